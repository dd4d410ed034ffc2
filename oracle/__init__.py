"""CPU oracle for the expert-FFN hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's algorithm for the path the
HIP library implements:

* ``gguf``   — GGUF block dequantisation (Q8_0, Q4_K, Q5_K, Q6_K; plus F32/F16),
  following ``tinyserve/gguf_dequant_torch.py:35-78,101-249``;
* ``mxfp4``  — MXFP4 (e2m1 nibbles + e8m0 block-32 scales) dequantisation,
  following ``tinyserve/mxfp4.py:5-53``;
* ``expert`` — expert FFN semantics (GPT-OSS clamped SwiGLU with biases, GGUF
  SiLU-gated), router top-k, the weighted top-k sum and the prefill grouping,
  following ``tinyserve/_model_hooks.py:376-476``, ``tinyserve/ggml_forward.py:88-151``,
  ``tinyserve/expert_pipeline.py:241-337`` and ``tinyserve/_fast_cache.pyx:60-85``;
* ``oracle.c`` — an independent scalar C restatement (per-element decoders written
  from the block-format definitions), built by ``oracle/Makefile`` into
  ``oracle/_build/liboracle.so``; used to brute-force check the vectorised
  restatement.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import, call, link or execute anything in this package, and only
as the checker (or the timed CPU baseline). The product path in
``tinyserve_amd`` never routes through it.

Pinning (how each function is checked; the tests under ``tests/`` do the checks):

* Q8_0: the reference's known values (``tests/test_gguf_dequant_torch.py:123-170``),
  golden vectors, and the C restatement.
* Q4_K: the reference's wire-format encoder + independent decoder test
  (``tests/test_gguf_dequant_torch.py:16-117,173-246``), golden vectors, C restatement.
* Q5_K, Q6_K: golden vectors written by ``tests/golden/make_golden.py`` from the
  reference's own ``gguf_dequant_torch`` (the reference has no known-answer test
  for them), C restatement, and closed-form special cases (all-zero quants, a
  single set bit).
* MXFP4: the reference's known values (``tests/test_mxfp4.py:8-61``), exact parity
  with HF ``convert_moe_packed_tensors`` (``tests/test_mxfp4.py:76-96``), golden
  vectors at the e8m0 extremes (0 and 255), C restatement.
* Expert/routing/grouping semantics: invariants (linearity in x, expert
  permutation, negative slots contribute zero, grouping is a permutation that
  preserves (token, k) order), closed forms on tiny inputs, and torch.topk /
  torch.softmax on the CPU for routing.
"""
