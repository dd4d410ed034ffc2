"""GPU routing, fused MoE decode, grouping and prefill parity against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.helpers import DECODE_SYNC_BYTES, assert_close_bf16, bf16_dev, tiled_h, to_f32
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_forward import gguf_expert_layout, mxfp4_expert_layout

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------------------- routing
@pytest.mark.parametrize("mode,E,k,T", [("topk_then_softmax", 32, 4, 1), ("topk_then_softmax", 32, 4, 513),
                                        ("softmax_then_topk", 128, 8, 1), ("softmax_then_topk", 128, 8, 77),
                                        ("softmax_then_topk_no_renorm", 64, 6, 9), ("topk_then_softmax", 1000, 16, 3)])
def test_route_topk_vs_oracle(mode, E, k, T):
    rng = np.random.default_rng(E + k + T)
    logits = synth.zipf_logits(rng, T, E) if E <= 128 else rng.normal(size=(T, E)).astype(np.float32)
    idx, w = ops.route_topk(torch.from_numpy(logits).cuda(), k, mode)
    if mode == "topk_then_softmax":
        ridx, rw = oex.route_topk_then_softmax(logits, k)
    else:
        ridx, rw = oex.route_softmax_then_topk(logits, k, renormalize=(mode == "softmax_then_topk"))
    assert np.array_equal(idx.cpu().numpy(), ridx), "top-k indices must match exactly"
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    # torch.topk on the CPU gives the same set and order (no ties at these seeds)
    tv, ti = torch.topk(torch.from_numpy(logits), k, dim=-1)
    assert np.array_equal(ti.numpy(), ridx)


def test_route_ties_go_to_lower_index():
    logits = torch.zeros(2, 16, device="cuda")
    logits[1, 5] = 1.0
    idx, w = ops.route_topk(logits, 4)
    assert idx[0].tolist() == [0, 1, 2, 3]
    assert idx[1].tolist() == [5, 0, 1, 2]
    np.testing.assert_allclose(w[0].cpu().numpy(), 0.25, rtol=1e-6)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
@pytest.mark.parametrize("E,k", [(32, 4), (100, 8), (256, 16)])
def test_route_nan_logits_same_in_every_router(E, k):
    """NaN logits rank above every number (as torch.topk ranks them) in the standalone
    router and in the routing inside both MXFP4 decode paths; a selected NaN or +inf makes
    the token's weights NaN, as torch's softmax does. Row 3 has no NaN or inf: its output is
    checked against the oracle."""
    rng = np.random.default_rng(E + k)
    T = 4
    logits = rng.normal(size=(T, E)).astype(np.float32)
    logits[0, 3] = np.nan
    logits[1, 7] = np.nan
    logits[1, E - 1] = np.nan
    logits[2, 5] = np.inf
    ridx, rw = oex.route_topk_then_softmax(logits, k)
    idx, w = ops.route_topk(torch.from_numpy(logits).cuda(), k)
    assert np.array_equal(idx.cpu().numpy(), ridx), "standalone router"
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, equal_nan=True)
    for tiled in (False, True):
        H, I = (512, 512) if not tiled else (256, 128)
        rng2 = np.random.default_rng(7)
        experts = [synth.make_mxfp4_expert(rng2, H, I) for _ in range(6)]
        if tiled:
            lay = synth.mxfp4_tiled_layout(H, I)
            pool = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])
        else:
            lay = synth.mxfp4_layout(H, I)
            pool = np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])
        L = mxfp4_expert_layout(lay, tiled=tiled)
        es = torch.arange(E, dtype=torch.int32, device="cuda") % 6
        x_bits = synth.bf16_normal(rng, (T, H))
        y, gidx, gw = ops.moe_decode_routed(L, torch.from_numpy(pool).cuda(), es, torch.from_numpy(logits).cuda(),
                                            bf16_dev(x_bits), k, return_routing=True)
        torch.cuda.synchronize()
        what = "tiled" if tiled else "checkpoint order"
        assert np.array_equal(gidx.cpu().numpy(), ridx), f"{what} decode routing"
        np.testing.assert_allclose(gw.cpu().numpy(), rw, rtol=1e-5, equal_nan=True)
        ref = oex.moe_combine(synth.bf16_to_f32(x_bits)[3:], ridx[3:] % 6, rw[3:],
                              lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))
        assert_close_bf16(y[3:], ref, f"{what} decode, row without NaN")


# ----------------------------------------------------------------------------- decode
def _mx_setup(H, I, E, seed, bias=True):
    rng = np.random.default_rng(seed)
    lay = synth.mxfp4_layout(H, I, bias=bias)
    experts = [synth.make_mxfp4_expert(rng, H, I, bias=bias) for _ in range(E)]
    pool = np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])
    return rng, lay, experts, torch.from_numpy(pool).cuda()


def _mx_ref(experts, x, idx, w):
    return oex.moe_combine(x, idx, w, lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("H,I,E,k,T", [(256, 128, 6, 2, 1), (512, 384, 8, 4, 3), (256, 256, 4, 1, 2)])
def test_moe_decode_mxfp4_small(H, I, E, k, T):
    rng, lay, experts, pool = _mx_setup(H, I, E, seed=H + I + E + k + T)
    L = mxfp4_expert_layout(lay)
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = rng.normal(size=(T, E)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(logits, k)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                       bf16_dev(x_bits))
    ref = _mx_ref(experts, synth.bf16_to_f32(x_bits), idx, w)
    assert_close_bf16(y, ref, "mxfp4 decode")


def test_moe_decode_mxfp4_workload3_full():
    """The headline workload at full size: 32 experts, hidden 2880, top-4, routed on the GPU."""
    wl = synth.workload(3)
    L = mxfp4_expert_layout(wl["layout"])
    pool = torch.from_numpy(wl["pool"]).cuda()
    idx, w = ops.route_topk(torch.from_numpy(wl["logits"]).cuda(), 4, "topk_then_softmax")
    ridx, rw = oex.route_topk_then_softmax(wl["logits"], 4)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    x = bf16_dev(wl["x_bits"])
    y = ops.moe_decode(L, pool, idx, w, x)
    ref = _mx_ref(wl["experts"], synth.bf16_to_f32(wl["x_bits"]), ridx, rw)
    assert_close_bf16(y, ref, "workload 3")


def test_moe_decode_negative_slots_and_permutation():
    rng, lay, experts, pool = _mx_setup(256, 128, 5, seed=9)
    L = mxfp4_expert_layout(lay)
    x = bf16_dev(synth.bf16_normal(rng, (1, 256)))
    slots = torch.tensor([[-1, -1]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.5, 0.5]], device="cuda")
    y = ops.moe_decode(L, pool, slots, w, x, out_dtype=torch.float32)
    assert torch.count_nonzero(y).item() == 0
    s1 = torch.tensor([[1, -1, 3, 7]], dtype=torch.int32, device="cuda")  # 7 >= n_slots: skipped
    w1 = torch.tensor([[0.25, 0.9, 0.75, 0.3]], device="cuda")
    s2 = torch.tensor([[3, 1]], dtype=torch.int32, device="cuda")
    w2 = torch.tensor([[0.75, 0.25]], device="cuda")
    y1 = ops.moe_decode(L, pool, s1, w1, x, out_dtype=torch.float32)
    y2 = ops.moe_decode(L, pool, s2, w2, x, out_dtype=torch.float32)
    np.testing.assert_allclose(to_f32(y1), to_f32(y2), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("H,E,k,T,routed", [(512, 6, 4, 1, False), (512, 8, 4, 4, True), (1024, 5, 2, 2, True),
                                             (2048, 4, 4, 1, False), (512, 20, 6, 3, False)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
def test_fused_decode_intermediate_and_output(H, E, k, T, routed, x_dtype):
    """Checkpoint-order MXFP4 slots (H == I, T <= 4): the published intermediate h
    (workspace) and the output against the oracle. bf16 x runs the MFMA decode loading the
    checkpoint order lane by lane (h bf16 [T k, I]); fp32 x the single-launch VALU kernel
    (h fp32 [T, k, I])."""
    rng, lay, experts, pool = _mx_setup(H, H, E, seed=H + E + k + T)
    L = mxfp4_expert_layout(lay)
    x_bits = synth.bf16_normal(rng, (T, H))
    xf = synth.bf16_to_f32(x_bits)
    x = bf16_dev(x_bits) if x_dtype == torch.bfloat16 else torch.from_numpy(xf).cuda()
    logits = rng.normal(size=(T, E)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(logits, k)
    ws = ops.moe_decode_workspace(L, T, k, "cuda")
    ws.fill_(0xFF)  # the two-launch forms read nothing they did not write in the call
    if routed:
        y, gidx, gw = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                            torch.from_numpy(logits).cuda(), x, k, workspace=ws,
                                            return_routing=True)
        assert np.array_equal(gidx.cpu().numpy(), idx)
        np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5)
    else:
        y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                           x, workspace=ws)
    torch.cuda.synchronize()
    o = DECODE_SYNC_BYTES  # h follows the workspace's sync area
    if x_dtype == torch.bfloat16:
        h_gpu = tiled_h(ws, T * k, H).reshape(T, k, H)
    else:
        h_gpu = ws[o : o + T * k * H * 4].view(torch.float32).cpu().numpy().reshape(T, k, H)
    for t in range(T):
        for j in range(k):
            e = experts[idx[t, j]]
            wgu, _ = oex.mxfp4_expert_weights(e)
            h_ref = oex.gptoss_swiglu(xf[t : t + 1] @ wgu.T + e["gate_up_bias"]).reshape(-1)
            assert_close_bf16(h_gpu[t, j], h_ref, f"h[{t},{j}]")
    assert_close_bf16(y, _mx_ref(experts, xf, idx, w), "fused output")


def test_moe_decode_mxfp4_two_launch_path_T6():
    """T > 4 tokens take the two-launch kernels; same semantics."""
    rng, lay, experts, pool = _mx_setup(256, 128, 6, seed=31)
    L = mxfp4_expert_layout(lay)
    T, k = 6, 3
    x_bits = synth.bf16_normal(rng, (T, 256))
    idx, w = oex.route_topk_then_softmax(rng.normal(size=(T, 6)).astype(np.float32), k)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                       bf16_dev(x_bits))
    assert_close_bf16(y, _mx_ref(experts, synth.bf16_to_f32(x_bits), idx, w), "two-launch decode")


@pytest.mark.parametrize("T", [1, 3])
def test_moe_decode_routed_matches_oracle_and_repeats(T):
    """Routing fused into the decode launches; 12 back-to-back calls on one workspace with
    different inputs each time."""
    rng, lay, experts, pool = _mx_setup(512, 256, 8, seed=5 + T)
    L = mxfp4_expert_layout(lay)
    expert_slot = torch.arange(8, dtype=torch.int32, device="cuda")
    ws = ops.moe_decode_workspace(L, T, 4, "cuda")
    ws.fill_(0xFF)  # no initialisation needed: the decode keeps no state in it
    outs, refs = [], []
    for it in range(12):
        logits = rng.normal(size=(T, 8)).astype(np.float32)
        x_bits = synth.bf16_normal(rng, (T, 512))
        y, idx, w = ops.moe_decode_routed(L, pool, expert_slot, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), 4,
                                          workspace=ws, return_routing=True)
        ridx, rw = oex.route_topk_then_softmax(logits, 4)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5)
        outs.append(y)
        refs.append(_mx_ref(experts, synth.bf16_to_f32(x_bits), ridx, rw))
    torch.cuda.synchronize()
    for y, ref in zip(outs, refs):
        assert_close_bf16(y, ref, "routed decode")


def test_moe_decode_routed_missing_expert_slot():
    """expert_slot = -1 (not resident) contributes zero, as a negative slot does."""
    rng, lay, experts, pool = _mx_setup(256, 128, 4, seed=8)
    L = mxfp4_expert_layout(lay)
    logits = np.array([[3.0, 2.0, 1.0, 0.0]], dtype=np.float32)
    x_bits = synth.bf16_normal(rng, (1, 256))
    es = torch.tensor([0, -1, 2, 3], dtype=torch.int32, device="cuda")
    y = ops.moe_decode_routed(L, pool, es, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), 2, out_dtype=torch.float32)
    ridx, rw = oex.route_topk_then_softmax(logits, 2)
    ref = np.float32(rw[0, 0]) * oex.mxfp4_expert_forward(synth.bf16_to_f32(x_bits), experts[0])
    assert_close_bf16(y, ref, "missing slot")


def _gguf_ref(experts, x, idx, w):
    return oex.moe_combine(x, idx, w, lambda e, xx: oex.gguf_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("H,I,types,E,k,T", [
    (256, 256, (12, 12, 14), 3, 2, 1), (512, 256, (13, 13, 14), 6, 3, 2), (256, 512, (8, 8, 8), 4, 2, 1),
    (2880, 256, (12, 12, 14), 2, 2, 1), (512, 256, (14, 14, 12), 3, 3, 1),
])
def test_moe_decode_gguf_small(H, I, types, E, k, T):
    rng = np.random.default_rng(H + I + E + k)
    lay = synth.gguf_layout(H, I, *types)
    experts = [synth.make_gguf_expert(rng, H, I, *types) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_gguf_expert(e, lay) for e in experts])).cuda()
    L = gguf_expert_layout(lay, dict(zip(("gate", "up", "down"), types)), {"gate": (H, I), "up": (H, I), "down": (I, H)})
    x_bits = synth.bf16_normal(rng, (T, H))
    idx, w = oex.route_softmax_then_topk(rng.normal(size=(T, E)).astype(np.float32), k)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                       bf16_dev(x_bits))
    assert_close_bf16(y, _gguf_ref(experts, synth.bf16_to_f32(x_bits), idx, w), f"gguf decode {types}")


def test_moe_decode_gguf_workload4_full():
    wl = synth.workload(4)
    H, I = wl["hidden"], wl["inter"]
    L = gguf_expert_layout(wl["layout"], {"gate": 13, "up": 13, "down": 14},
                           {"gate": (H, I), "up": (H, I), "down": (I, H)})
    idx, w = ops.route_topk(torch.from_numpy(wl["logits"]).cuda(), 8, "softmax_then_topk")
    ridx, rw = oex.route_softmax_then_topk(wl["logits"], 8)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    y = ops.moe_decode(L, torch.from_numpy(wl["pool"]).cuda(), idx, w, bf16_dev(wl["x_bits"]))
    assert_close_bf16(y, _gguf_ref(wl["experts"], synth.bf16_to_f32(wl["x_bits"]), ridx, rw), "workload 4")


def test_single_expert_workload2_full():
    """Workload 2: one Q4_K/Q6_K expert with rows straddling super-blocks (K = 2880)."""
    wl = synth.workload(2)
    H, I = wl["hidden"], wl["inter"]
    L = gguf_expert_layout(wl["layout"], {"gate": 12, "up": 12, "down": 14},
                           {"gate": (H, I), "up": (H, I), "down": (I, H)})
    slot = torch.from_numpy(wl["slot"]).cuda().reshape(1, -1)
    one_s = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
    one_w = torch.ones((1, 1), device="cuda")
    y = ops.moe_decode(L, slot, one_s, one_w, bf16_dev(wl["x_bits"]))
    ref = oex.gguf_expert_forward(synth.bf16_to_f32(wl["x_bits"]), wl["expert"])
    assert_close_bf16(y, ref, "workload 2")


# ----------------------------------------------------------------------------- grouping / prefill
@pytest.mark.parametrize("T,k,E", [(2048, 4, 32), (37, 8, 128), (1, 1, 1), (3000, 2, 1000), (5000, 3, 64),
                                   (4096, 8, 1024), (1000, 4, 2)])  # the most experts; most lanes of a batch share one
def test_group_by_expert_vs_oracle(T, k, E):
    rng = np.random.default_rng(T + k + E)
    idx = rng.integers(0, E, size=(T, k)).astype(np.int32)
    if T > 10:
        idx[3, 0] = -1  # ignored
    counts, offsets, perm = ops.group_by_expert(torch.from_numpy(idx).cuda(), E)
    groups = oex.group_tokens_by_expert(idx)
    c, o, p = counts.cpu().numpy(), offsets.cpu().numpy(), perm.cpu().numpy()
    for e in range(E):
        pairs = groups.get(e, [])
        assert c[e] == len(pairs)
        got = p[o[e] : o[e] + c[e]]
        assert np.array_equal(got, np.array([t * k + j for t, j in pairs], dtype=np.int64)), e
    assert o[E] == int((idx >= 0).sum())


def test_moe_prefill_small_vs_oracle():
    rng, lay, experts, pool = _mx_setup(256, 128, 8, seed=77)
    L = mxfp4_expert_layout(lay)
    T, k = 64, 2
    logits = synth.zipf_logits(rng, T, 8)
    idx, w = oex.route_topk_then_softmax(logits, k)
    x_bits = synth.bf16_normal(rng, (T, 256))
    expert_slot = torch.arange(8, dtype=torch.int32, device="cuda")
    y = ops.moe_prefill(L, pool, expert_slot, torch.from_numpy(idx.astype(np.int32)).cuda(),
                        torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    ref = oex.moe_combine_grouped(synth.bf16_to_f32(x_bits), idx, w,
                                  lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))
    assert_close_bf16(y, ref, "prefill")
