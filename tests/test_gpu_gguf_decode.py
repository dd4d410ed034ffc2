"""GGUF expert decode and matvec on the super-block kernels (gq_phase_a/b, gq_matvec_kernel)
against the oracle: routed calls (the in-kernel top-k and the table phase A hands to phase B),
expert counts that take several phase B rounds or leave waves idle, fp32 / fp16
activations (the bf16 hi/lo staging), missing slots, and the matvec's token-count limit
(ggml_forward.py:88-115, expert_loop.cpp:83-121, _model_hooks.py:456-473, ggml_ops.cu:461-569)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from oracle import gguf as og
from tests.helpers import assert_close_bf16, bf16_dev, dev_u8, metrics, to_f32
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_forward import gguf_expert_layout

pytestmark = pytest.mark.gpu


def _pool(rng, H, I, types, E):
    lay = synth.gguf_layout(H, I, *types)
    experts = [synth.make_gguf_expert(rng, H, I, *types) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_gguf_expert(e, lay) for e in experts])).cuda()
    L = gguf_expert_layout(lay, dict(zip(("gate", "up", "down"), types)), {"gate": (H, I), "up": (H, I), "down": (I, H)})
    return L, experts, pool


def _ref(experts, x, idx, w):
    return oex.moe_combine(x, idx, w, lambda e, xx: oex.gguf_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("mode", ["softmax_then_topk", "topk_then_softmax", "softmax_then_topk_no_renorm"])
@pytest.mark.parametrize("H,I,types,E,k,T", [
    (512, 256, (13, 13, 14), 128, 8, 1),   # the workload-4 routing shape at a small size
    (512, 256, (13, 13, 14), 64, 8, 4),    # four tokens routed in one launch
    (256, 512, (12, 12, 14), 40, 16, 2),   # k = 16: two rounds of phase B experts
    (256, 256, (8, 8, 8), 9, 5, 3),        # k = 5: phase B waves left idle, Q8_0
])
def test_gguf_decode_routed_vs_oracle(H, I, types, E, k, T, mode):
    rng = np.random.default_rng(H + I + E + k + T)
    L, experts, pool = _pool(rng, H, I, types, E)
    logits = synth.zipf_logits(rng, T, E)
    x_bits = synth.bf16_normal(rng, (T, H))
    y, idx, w = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                      torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, mode,
                                      return_routing=True)
    if mode == "topk_then_softmax":
        ridx, rw = oex.route_topk_then_softmax(logits, k)
    else:
        ridx, rw = oex.route_softmax_then_topk(logits, k, renormalize=(mode == "softmax_then_topk"))
    assert np.array_equal(idx.cpu().numpy(), ridx), "routing indices"
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), ridx, rw), f"routed gguf {types} k={k} T={T} {mode}")


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
@pytest.mark.parametrize("E,k", [(32, 4), (128, 8), (200, 16)])
def test_gguf_decode_routing_ties_and_nan(E, k):
    """Every phase A wave selects its own pair's expert (the rank alone, by a threshold
    search) while one wave per token writes the whole top-k table for phase B: both must
    rank NaN first, then descending logits, ties to the lower id (torch.topk's order), or
    a pair's h would belong to another expert than its weight. Rows: integer logits with
    many ties, all-equal logits, NaN and +inf (weights NaN, as torch's softmax gives), and
    a plain row; the outputs of the rows without NaN or inf are checked against the oracle."""
    rng = np.random.default_rng(E + k)
    H, I, T = 256, 256, 4
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), 6)
    logits = rng.normal(size=(T, E)).astype(np.float32)
    logits[0] = rng.integers(-2, 3, size=E).astype(np.float32)
    logits[1] = 0.0
    logits[2, 3] = np.nan
    logits[2, E - 1] = np.nan
    logits[2, 5] = np.inf
    ridx, rw = oex.route_topk_then_softmax(logits, k)
    es = torch.arange(E, dtype=torch.int32, device="cuda") % 6
    x_bits = synth.bf16_normal(rng, (T, H))
    y, idx, w = ops.moe_decode_routed(L, pool, es, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k,
                                      return_routing=True)
    assert np.array_equal(idx.cpu().numpy(), ridx), "routing indices"
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, equal_nan=True)
    ok = [0, 1, 3]
    ref = _ref([experts[e % 6] for e in range(E)], synth.bf16_to_f32(x_bits)[ok], ridx[ok], rw[ok])
    assert_close_bf16(y[ok], ref, f"gguf decode, ties and NaN, E={E} k={k}")


def test_gguf_decode_routed_repeats_and_missing_expert():
    """Repeated routed calls on one workspace agree; an expert without a resident slot
    contributes nothing (its weight stays in the normalisation, as in the reference)."""
    rng = np.random.default_rng(3)
    H, I, E, k = 512, 256, 32, 4
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), E)
    logits = synth.zipf_logits(rng, 2, E)
    x_bits = synth.bf16_normal(rng, (2, H))
    ridx, rw = oex.route_softmax_then_topk(logits, k)
    missing = int(ridx[0, 1])
    expert_slot = np.arange(E, dtype=np.int32)
    expert_slot[missing] = -1
    es = torch.from_numpy(expert_slot).cuda()
    ws = ops.moe_decode_workspace(L, 2, k, "cuda")
    outs = [ops.moe_decode_routed(L, pool, es, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k,
                                  "softmax_then_topk", workspace=ws) for _ in range(3)]
    for y in outs[1:]:
        assert torch.equal(y, outs[0])
    live_w = np.where(ridx == missing, 0.0, rw).astype(np.float32)
    assert_close_bf16(outs[0], _ref(experts, synth.bf16_to_f32(x_bits), ridx, live_w), "missing expert")


@pytest.mark.parametrize("types,H,I,T,x_dtype,pad", [
    ((12, 12, 14), 2880, 2880, 1, torch.bfloat16, 0),  # the workload-2 expert
    ((13, 13, 14), 2048, 768, 3, torch.bfloat16, 0),
    ((8, 8, 8), 512, 1024, 2, torch.float32, 0),
    ((14, 14, 14), 768, 512, 4, torch.float16, 0),
    ((12, 12, 8), 512, 512, 2, torch.bfloat16, 2),     # slots 2 bytes off 16-byte boundaries
    ((13, 13, 14), 1024, 512, 100, torch.bfloat16, 0),  # many tokens, one expert each
])
def test_gguf_decode_one_expert_stream_kernels(types, H, I, T, x_dtype, pad):
    """One expert per token (k = 1) runs on the sub-block stream kernels (gs_gate_up_kernel,
    gs_down_kernel): given slots, then routed from logits with the selection handed on."""
    rng = np.random.default_rng(H + I + T + pad)
    E = 6
    L, experts, pool = _pool(rng, H, I, types, E)
    if pad:
        pool = torch.cat([torch.zeros((E, pad), dtype=torch.uint8, device="cuda"), pool], dim=1).contiguous()
        L.slot_bytes += pad
        L.gate_off += pad
        L.up_off += pad
        L.down_off += pad
    x = rng.normal(0.0, 1.0, (T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(x_dtype)
    xf = xt.float().numpy()
    idx = rng.integers(0, E, size=(T, 1)).astype(np.int32)
    w = rng.uniform(0.5, 1.5, size=(T, 1)).astype(np.float32)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), xt.cuda(),
                       out_dtype=torch.float32)
    assert_close_bf16(y, _ref(experts, xf, idx, w), f"one-expert decode {types} H {H} I {I}")
    if T <= 4:
        logits = synth.zipf_logits(rng, T, E)
        y2, ridx, rw = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                             torch.from_numpy(logits).cuda(), xt.cuda(), 1, "softmax_then_topk",
                                             out_dtype=torch.float32, return_routing=True)
        eidx, ew = oex.route_softmax_then_topk(logits, 1)
        assert np.array_equal(ridx.cpu().numpy(), eidx)
        assert_close_bf16(y2, _ref(experts, xf, eidx, ew), f"one-expert routed decode {types}")


@pytest.mark.parametrize("H,I,types,x_dtype", [
    (2880, 2880, (13, 13, 14), torch.bfloat16),  # rows start inside units in both launches
    (2880, 2880, (12, 12, 14), torch.float32),   # the same through the hi / lo activation kernels
    (288, 96, (13, 13, 14), torch.bfloat16),     # rows of 2.25 / 0.75 half super-blocks
    (96, 288, (12, 12, 14), torch.float16),
    (320, 2880, (14, 14, 12), torch.bfloat16),   # Q6_K gate / up, Q4_K down
])
def test_gguf_decode_rows_straddling_units(H, I, types, x_dtype):
    """Several experts per token (the super-block kernels, half a K-quant super-block per
    lane) at row lengths that are not multiples of 128 values, so rows start inside units
    and a unit's sub-blocks go to two rows: against the fp32 oracle."""
    rng = np.random.default_rng(H + 3 * I + sum(types))
    E, k, T = 4, 3, 2
    L, experts, pool = _pool(rng, H, I, types, E)
    x = rng.normal(0.0, 1.0, (T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(x_dtype)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.2, 1.0, size=(T, k)).astype(np.float32)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), xt.cuda(),
                       out_dtype=torch.float32)
    assert_close_bf16(y, _ref(experts, xt.float().numpy(), idx, w), f"gguf decode {types} H {H} I {I} {x_dtype}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_gguf_decode_wide_activations(x_dtype):
    """fp32 / fp16 activations are staged as a bf16 hi/lo pair: the result follows the fp32
    oracle on the unrounded activations far more tightly than bf16 rounding would allow."""
    rng = np.random.default_rng(17)
    H, I, E, k, T = 2048, 256, 6, 3, 2
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), E)
    x = rng.normal(0.0, 1.0, (T, H)).astype(np.float32)
    xt = torch.from_numpy(x).to(x_dtype)
    xf = xt.float().numpy()
    idx, w = oex.route_softmax_then_topk(rng.normal(size=(T, E)).astype(np.float32), k)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(), xt.cuda(),
                       out_dtype=torch.float32)
    ref = _ref(experts, xf, idx, w)
    assert_close_bf16(y, ref, f"gguf decode x {x_dtype}")
    cos, rel = metrics(to_f32(y), ref)
    # h is rounded to bf16 between the two matrices (as in the reference), so the bar is that
    # rounding's, not fp32's: still well inside the decode bar
    assert cos > 0.99999 and rel < 3e-3, (cos, rel)


@pytest.mark.parametrize("T", [8, 9])
@pytest.mark.parametrize("gtype,x_dtype", [(8, torch.float32), (13, torch.float16), (14, torch.bfloat16)])
def test_gguf_matvec_token_limit(T, gtype, x_dtype):
    """T = 8 is the last count on the streaming matvec, T = 9 runs the row kernel: both
    match the fp32 oracle, in every activation dtype."""
    rng = np.random.default_rng(T * 100 + gtype)
    K, N = 1024, 96
    data = synth.make_gguf(rng, gtype, N * K)
    x = rng.normal(0.0, 1.0, (T, K)).astype(np.float32)
    xt = torch.from_numpy(x).to(x_dtype)
    ref = xt.float().numpy() @ og.dequant_tensor(data, gtype, (N, K)).T
    y = ops.gguf_matvec(xt.cuda(), dev_u8(data), gtype, N, K, out_dtype=torch.float32)
    assert y.shape == (T, N)
    cos, rel = metrics(to_f32(y), ref)
    # the activations enter the dot products as two int8 terms per 32-value block (about 16
    # significant bits relative to the block maximum): fp32-level accuracy, not bit-exact bf16
    assert cos > 0.999999 and rel < 1e-4, (cos, rel)


def test_gguf_decode_routed_workload4_full_size():
    """Workload 4 at its real shape: 128 Q5_K/Q6_K experts of hidden 2048, inter 768, top-8
    of softmax-renormalised logits, one token (the benchmark's configuration)."""
    wl = synth.workload(4)
    H, I, E, k = wl["hidden"], wl["inter"], wl["E"], wl["top_k"]
    pool = torch.from_numpy(wl["pool"]).cuda()
    L = gguf_expert_layout(wl["layout"], {"gate": 13, "up": 13, "down": 14}, {"gate": (H, I), "up": (H, I), "down": (I, H)})
    y, idx, w = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                      torch.from_numpy(wl["logits"]).cuda(), bf16_dev(wl["x_bits"]), k,
                                      "softmax_then_topk", return_routing=True)
    ridx, rw = oex.route_softmax_then_topk(wl["logits"], k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    assert_close_bf16(y, _ref(wl["experts"], synth.bf16_to_f32(wl["x_bits"]), ridx, rw), "workload 4")


def test_gguf_prefill_workload4_shapes():
    """tsa_moe_prefill over GGUF slots at workload-4 shapes, 64 tokens (the GGUF prefill
    runs the super-block decode over all the tokens' assignments at once)."""
    rng = np.random.default_rng(64)
    H, I, E, k, T = 2048, 768, 128, 8, 64
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), E)
    x_bits = synth.bf16_normal(rng, (T, H))
    idx, w = oex.route_softmax_then_topk(synth.zipf_logits(rng, T, E), k)
    y = ops.moe_prefill(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                        torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    ref = oex.moe_combine_grouped(synth.bf16_to_f32(x_bits), idx, w,
                                  lambda e, xx: oex.gguf_expert_forward(xx, experts[e]))
    assert_close_bf16(y, ref, "GGUF prefill, workload-4 shapes")


def test_gguf_decode_more_assignments_than_grid_rows():
    """T k above 65535 (one launch grid row per assignment): the decode runs token chunks."""
    rng = np.random.default_rng(65)
    H, I, E, k, T = 256, 256, 8, 8, 8200
    L, experts, pool = _pool(rng, H, I, (8, 8, 8), E)
    x_bits = synth.bf16_normal(rng, (T, H))
    idx = np.argsort(rng.random((T, E)), axis=1)[:, :k].astype(np.int32)  # k distinct experts per token
    w = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    ref = oex.moe_combine_grouped(synth.bf16_to_f32(x_bits), idx, w,
                                  lambda e, xx: oex.gguf_expert_forward(xx, experts[e]))
    assert_close_bf16(y, ref, "GGUF decode, T k = 65600")


def test_gguf_routed_decode_more_assignments_than_grid_rows():
    """The routed entry with T k above 65535: routed and decoded in token chunks."""
    rng = np.random.default_rng(67)
    H, I, E, k, T = 256, 256, 8, 8, 8200
    L, experts, pool = _pool(rng, H, I, (8, 8, 8), E)
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = synth.zipf_logits(rng, T, E)
    y, gidx, gw = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                        torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k,
                                        mode="softmax_then_topk", return_routing=True)
    idx, w = oex.route_softmax_then_topk(logits, k)
    assert np.array_equal(gidx.cpu().numpy(), idx)
    ref = oex.moe_combine_grouped(synth.bf16_to_f32(x_bits), idx, w,
                                  lambda e, xx: oex.gguf_expert_forward(xx, experts[e]))
    assert_close_bf16(y, ref, "routed GGUF decode, T k = 65600")


def test_ggml_expert_forward_other_activation():
    """GGMLExpertForward with a non-SiLU act_fn (here GELU) runs act_fn(gate) * up between the
    GGUF matvecs, as the reference passes any act_fn."""
    from tinyserve_amd.ggml_forward import GGMLExpertForward

    rng = np.random.default_rng(66)
    H, I = 512, 256
    types = {"gate": 12, "up": 12, "down": 14}
    lay = synth.gguf_layout(H, I, 12, 12, 14)
    e = synth.make_gguf_expert(rng, H, I, 12, 12, 14)
    packed = torch.from_numpy(synth.pack_gguf_expert(e, lay)).cuda()
    fwd = GGMLExpertForward(lay, types, torch.nn.GELU(), {"gate": (H, I), "up": (H, I), "down": (I, H)})
    x_bits = synth.bf16_normal(rng, (3, H))
    y = fwd.forward(packed, bf16_dev(x_bits))
    wg, wu, wd = oex.gguf_expert_weights(e)
    xf = synth.bf16_to_f32(x_bits)
    g = torch.nn.functional.gelu(torch.from_numpy(xf @ wg.T)).numpy()
    ref = (g * (xf @ wu.T)) @ wd.T
    assert_close_bf16(y, ref, "GELU-gated GGUF expert")
