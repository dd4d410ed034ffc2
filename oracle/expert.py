"""Expert-FFN, routing and grouping semantics on the CPU (test oracle only).

All arithmetic is float32 on float32 copies of the (bf16) inputs: weights are
dequantised exactly (``oracle.gguf`` / ``oracle.mxfp4``), then every product is an
fp32 matmul, mirroring the reference's CPU check form
(``tests/test_ggml_ops.py:57-64``: fp32 dequant, fp32 matmul).

* MXFP4 / GPT-OSS expert: ``_FusedExpertTemplate.forward``
  (``tinyserve/_model_hooks.py:380-394``) with biases; interleaved gate/up rows
  (even = gate, odd = up), ``gate = min(gate, limit)``, ``up = clip(up, -limit, limit)``,
  ``h = (up + 1) * gate * sigmoid(alpha * gate)`` with ``limit = 7``, ``alpha = 1.702``
  (``tinyserve/expert_forward.py:30,185-187``).
* GGUF expert: ``GGMLExpertForward._fallback_forward``
  (``tinyserve/ggml_forward.py:117-151``): separate gate/up/down tensors,
  ``proj_shapes`` in ggml (ne0 = in, ne1 = out) order, ``h = silu(gate) * up``
  (the pipeline hard-codes SiLU, ``tinyserve/expert_pipeline.py:97``), no bias.
* Routing (``tinyserve/_model_hooks.py:456-473``): ``topk_then_softmax`` (GPT-OSS)
  and ``softmax_then_topk`` with renormalisation (Qwen3-MoE).
* Decode combine: ``out[t] += w[t,k] * y_k`` over the top-k, skipping slots < 0
  (``tinyserve/csrc/expert_loop.cpp:83-121``, ``tinyserve/expert_pipeline.py:266-281``).
* Prefill grouping: (token, k) pairs grouped by expert id, token-major within an
  expert (``tinyserve/_fast_cache.pyx:60-85``, ``tinyserve/expert_pipeline.py:303-333``).
"""
from __future__ import annotations

import numpy as np

from . import gguf as _gguf
from . import mxfp4 as _mx

SWIGLU_LIMIT = 7.0
SWIGLU_ALPHA = 1.702


def sigmoid(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-x) -> inf for very negative x gives the exact limit 0
        return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def gptoss_swiglu(gu: np.ndarray, limit: float = SWIGLU_LIMIT, alpha: float = SWIGLU_ALPHA) -> np.ndarray:
    gate = np.minimum(gu[..., 0::2], np.float32(limit))
    up = np.clip(gu[..., 1::2], np.float32(-limit), np.float32(limit))
    return ((up + np.float32(1.0)) * gate * sigmoid(gate * np.float32(alpha))).astype(np.float32)


def silu_gate(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    return (gate * sigmoid(gate) * up).astype(np.float32)


# ----------------------------------------------------------------------------- MXFP4
def mxfp4_expert_weights(e: dict) -> tuple[np.ndarray, np.ndarray]:
    """Dequantised (W_gu [2I, H], W_dn [H, I]) float32 of one MXFP4 expert dict with
    keys gate_up_blocks/gate_up_scales/down_blocks/down_scales."""
    wgu = _mx.dequant_mxfp4_no_transpose(e["gate_up_blocks"], e["gate_up_scales"], "f32")
    wdn = _mx.dequant_mxfp4_no_transpose(e["down_blocks"], e["down_scales"], "f32")
    return wgu, wdn


def mxfp4_expert_forward(x: np.ndarray, e: dict, weights=None) -> np.ndarray:
    """One GPT-OSS expert on x [T, H] (float32 values) -> [T, H] float32."""
    wgu, wdn = weights if weights is not None else mxfp4_expert_weights(e)
    x = np.asarray(x, dtype=np.float32).reshape(-1, wgu.shape[1])
    gu = x @ wgu.T
    if e.get("gate_up_bias") is not None:
        gu = gu + np.asarray(e["gate_up_bias"], dtype=np.float32)
    h = gptoss_swiglu(gu)
    y = h @ wdn.T
    if e.get("down_bias") is not None:
        y = y + np.asarray(e["down_bias"], dtype=np.float32)
    return y.astype(np.float32)


# ----------------------------------------------------------------------------- GGUF
def gguf_expert_weights(e: dict) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Dequantised (W_gate [I,H], W_up [I,H], W_down [H,I]) of one GGUF expert dict with
    keys gate/up/down (bytes), gate_type/up_type/down_type, hidden, inter."""
    H, I = e["hidden"], e["inter"]
    wg = _gguf.dequant_tensor(e["gate"], e["gate_type"], (I, H))
    wu = _gguf.dequant_tensor(e["up"], e["up_type"], (I, H))
    wd = _gguf.dequant_tensor(e["down"], e["down_type"], (H, I))
    return wg, wu, wd


def gguf_expert_forward(x: np.ndarray, e: dict, weights=None) -> np.ndarray:
    wg, wu, wd = weights if weights is not None else gguf_expert_weights(e)
    x = np.asarray(x, dtype=np.float32).reshape(-1, wg.shape[1])
    h = silu_gate(x @ wg.T, x @ wu.T)
    return (h @ wd.T).astype(np.float32)


# ----------------------------------------------------------------------------- routing
def _topk_order(v: np.ndarray) -> np.ndarray:
    """Per row, indices in torch.topk's order: NaN first, then descending value, ties (and
    NaNs among themselves) to the lower index."""
    v = np.asarray(v)
    n = v.shape[-1]
    out = np.empty(v.shape, dtype=np.int64)
    for r, row in zip(np.ndindex(v.shape[:-1]), v.reshape(-1, n)):
        nan = np.isnan(row)
        out[r] = np.lexsort((np.arange(n), -np.where(nan, 0.0, row), ~nan))
    return out


def route_topk_then_softmax(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """torch.topk(logits, k) then softmax over the k values (_model_hooks.py:466-473).
    Ties resolve to the lower expert index; NaN ranks above every number (torch.topk)."""
    logits = np.asarray(logits, dtype=np.float32)
    idx = _topk_order(logits)[..., :k]
    vals = np.take_along_axis(logits, idx, axis=-1).astype(np.float64)
    ex = np.exp(vals - vals.max(axis=-1, keepdims=True))
    w = ex / ex.sum(axis=-1, keepdims=True)
    return idx.astype(np.int64), w.astype(np.float32)


def route_softmax_then_topk(logits: np.ndarray, k: int, renormalize: bool = True):
    """softmax(fp32) -> topk -> renormalise (_model_hooks.py:456-465)."""
    logits = np.asarray(logits, dtype=np.float32).astype(np.float64)
    ex = np.exp(logits - logits.max(axis=-1, keepdims=True))
    p = ex / ex.sum(axis=-1, keepdims=True)
    idx = _topk_order(p)[..., :k]
    w = np.take_along_axis(p, idx, axis=-1)
    if renormalize:
        w = w / w.sum(axis=-1, keepdims=True)
    return idx.astype(np.int64), w.astype(np.float32)


# ----------------------------------------------------------------------------- combine
def moe_combine(x: np.ndarray, idx: np.ndarray, w: np.ndarray, expert_fwd) -> np.ndarray:
    """out[t] = sum_k w[t,k] * expert_fwd(idx[t,k], x[t]); idx < 0 contributes nothing."""
    x = np.asarray(x, dtype=np.float32)
    T = x.shape[0]
    out = np.zeros_like(x, dtype=np.float32)
    cache: dict[int, np.ndarray] = {}
    for t in range(T):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e < 0:
                continue
            out[t] += np.float32(w[t, j]) * expert_fwd(e, x[t : t + 1]).reshape(-1)
    return out


def moe_combine_grouped(x: np.ndarray, idx: np.ndarray, w: np.ndarray, expert_fwd) -> np.ndarray:
    """Prefill form: one batched forward per expert over its grouped tokens, then the
    weighted scatter (expert_pipeline.py:166-239)."""
    x = np.asarray(x, dtype=np.float32)
    out = np.zeros_like(x, dtype=np.float32)
    for eid, pairs in group_tokens_by_expert(idx).items():
        toks = np.array([p[0] for p in pairs])
        ks = np.array([p[1] for p in pairs])
        yb = expert_fwd(eid, x[toks])
        for i in range(len(pairs)):
            out[toks[i]] += np.float32(w[toks[i], ks[i]]) * yb[i]
    return out


def group_tokens_by_expert(idx: np.ndarray) -> dict[int, list[tuple[int, int]]]:
    """dict eid -> [(tok, k), ...] in token-major order (_fast_cache.pyx:60-85)."""
    groups: dict[int, list[tuple[int, int]]] = {}
    T, K = idx.shape
    for t in range(T):
        for j in range(K):
            groups.setdefault(int(idx[t, j]), []).append((t, j))
    return groups
