"""MXFP4 experts in the 16-row MFMA tile order: device repack and the fused MFMA decode,
against the oracle (which reads the checkpoint order)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.helpers import assert_close_bf16, bf16_dev, tiled_h, to_f32
from tinyserve_amd import mx_tiles, ops, synth
from tinyserve_amd.expert_forward import mxfp4_expert_layout

pytestmark = pytest.mark.gpu


@pytest.fixture
def one_launch():
    ops.set_decode_options(0)
    yield
    ops.set_decode_options()


@pytest.fixture(params=[0, 1], ids=["one_launch", "two_launches"])
def form(request):
    """The tiled decode's form (tsa_set_decode_options), restored to the default after."""
    ops.set_decode_options(request.param)
    yield request.param
    ops.set_decode_options()


@pytest.mark.parametrize("N,K", [(16, 32), (64, 256), (5760, 2880), (48, 160), (2880, 2880), (32, 4096)])
def test_tile_repack_matches_host_packer(N, K):
    rng = np.random.default_rng(N + K)
    G = K // 32
    blocks = rng.integers(0, 256, (N, G, 16), dtype=np.uint8)
    scales = rng.integers(0, 256, (N, G), dtype=np.uint8)
    tb, ts = ops.mxfp4_tile(torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda())
    hb, hs = mx_tiles.tile_mxfp4(blocks, scales)
    assert ops.mxfp4_tile_sizes(N, K) == (hb.size, hs.size)
    assert np.array_equal(tb.cpu().numpy(), hb), "tiled blocks differ from the host packer"
    assert np.array_equal(ts.cpu().numpy(), hs), "tiled scales differ from the host packer"


def _setup(H, I, E, seed, bias=True):
    rng = np.random.default_rng(seed)
    lay = synth.mxfp4_tiled_layout(H, I, bias=bias)
    experts = [synth.make_mxfp4_expert(rng, H, I, bias=bias) for _ in range(E)]
    pool = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])
    return rng, mxfp4_expert_layout(lay, tiled=True), experts, torch.from_numpy(pool).cuda()


def _ref(experts, x, idx, w):
    return oex.moe_combine(x, idx, w, lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("H,I,E,k,T,routed", [
    (256, 128, 6, 2, 1, False), (512, 384, 8, 4, 3, True), (256, 256, 4, 1, 2, False), (1024, 512, 5, 2, 4, True),
    (2048, 2048, 4, 4, 1, True), (512, 1024, 20, 6, 3, False), (256, 128, 8, 3, 7, True), (768, 256, 16, 16, 2, False),
])
def test_tiled_decode_vs_oracle(H, I, E, k, T, routed, form):
    """Output and the published bf16 intermediate h (T > 4 runs in chunks of 4 tokens)."""
    rng, L, experts, pool = _setup(H, I, E, seed=H + 3 * I + E + k + T)
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = rng.normal(size=(T, E)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(logits, k)
    ws = ops.moe_decode_workspace(L, T, k, "cuda")
    ws.fill_(0xFF)  # no initialisation needed: the decode keeps no state in it
    if routed:
        y, gidx, gw = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                            torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, workspace=ws,
                                            return_routing=True)
        assert np.array_equal(gidx.cpu().numpy(), idx)
        np.testing.assert_allclose(gw.cpu().numpy(), w, rtol=1e-5)
    else:
        y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                           bf16_dev(x_bits), workspace=ws)
    torch.cuda.synchronize()
    xf = synth.bf16_to_f32(x_bits)
    assert_close_bf16(y, _ref(experts, xf, idx, w), "tiled decode")
    # h of the last launch's tokens (the chunk starting at 4 * floor((T-1)/4))
    t0 = 4 * ((T - 1) // 4)
    tc = T - t0
    h = tiled_h(ws, tc * k, I, one_launch=form == 0 and k <= 4).reshape(tc, k, I)
    for t in range(tc):
        for j in range(k):
            e = experts[idx[t0 + t, j]]
            wgu, _ = oex.mxfp4_expert_weights(e)
            h_ref = oex.gptoss_swiglu(xf[t0 + t : t0 + t + 1] @ wgu.T + e["gate_up_bias"]).reshape(-1)
            assert_close_bf16(h[t, j], h_ref, f"h[{t0 + t},{j}]")


@pytest.mark.parametrize("H,I,E,k,T,routed,small", [
    (256, 128, 6, 2, 1, False, False), (288, 96, 5, 2, 3, True, False),   # 9 and 3 blocks per row
    (2880, 2880, 8, 4, 1, True, False), (768, 256, 16, 16, 2, False, False),
    (256, 128, 8, 3, 7, True, False), (512, 1024, 6, 3, 2, True, True),     # 2 launch pairs; small |h|
    (256, 128, 6, 2, 65, False, False),                                   # past 64 tokens: the VALU kernels
])
def test_checkpoint_order_mfma_decode_vs_oracle(H, I, E, k, T, routed, small):
    """Checkpoint-order slots through the MFMA decode (each lane loads its 16-byte block of
    the [N, K/32, 16] array and its scale byte): output and the bf16 intermediate h."""
    rng = np.random.default_rng(H + 5 * I + E + k + T)
    lay = synth.mxfp4_layout(H, I, bias=not small)
    sc = dict(scale_lo=113, scale_hi=117) if small else {}
    experts = [synth.make_mxfp4_expert(rng, H, I, bias=not small, **sc) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])).cuda()
    L = mxfp4_expert_layout(lay)
    assert L.mx_tiled == 0
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = rng.normal(size=(T, E)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(logits, k)
    ws = ops.moe_decode_workspace(L, T, k, "cuda")
    ws.fill_(0xFF)
    if routed:
        y, gidx, _ = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                           torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, workspace=ws,
                                           return_routing=True)
        assert np.array_equal(gidx.cpu().numpy(), idx)
    else:
        y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                           bf16_dev(x_bits), workspace=ws)
    torch.cuda.synchronize()
    xf = synth.bf16_to_f32(x_bits)
    assert_close_bf16(y, _ref(experts, xf, idx, w), "checkpoint-order decode")
    if T <= 64:  # the last chunk's h (bf16 after the sync area)
        t0 = 4 * ((T - 1) // 4)
        tc = T - t0
        h = tiled_h(ws, tc * k, I).reshape(tc, k, I)
        for t in range(tc):
            for j in range(k):
                e = experts[idx[t0 + t, j]]
                wgu, _ = oex.mxfp4_expert_weights(e)
                pre = xf[t0 + t : t0 + t + 1] @ wgu.T + (0.0 if small else e["gate_up_bias"])
                assert_close_bf16(h[t, j], oex.gptoss_swiglu(pre).reshape(-1), f"h[{t0 + t},{j}]")


def test_tiled_equals_checkpoint_order_path():
    """Both layouts of the same experts give the same result (each checked against the oracle)."""
    H, I, E, k = 512, 256, 6, 3
    rng = np.random.default_rng(42)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    lay_r, lay_t = synth.mxfp4_layout(H, I), synth.mxfp4_tiled_layout(H, I)
    pool_r = torch.from_numpy(np.stack([synth.pack_mxfp4_expert(e, lay_r) for e in experts])).cuda()
    pool_t = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay_t) for e in experts])).cuda()
    x_bits = synth.bf16_normal(rng, (2, H))
    idx, w = oex.route_topk_then_softmax(rng.normal(size=(2, E)).astype(np.float32), k)
    s, wt = torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda()
    y_r = ops.moe_decode(mxfp4_expert_layout(lay_r), pool_r, s, wt, bf16_dev(x_bits), out_dtype=torch.float32)
    y_t = ops.moe_decode(mxfp4_expert_layout(lay_t, tiled=True), pool_t, s, wt, bf16_dev(x_bits),
                         out_dtype=torch.float32)
    ref = _ref(experts, synth.bf16_to_f32(x_bits), idx, w)
    assert_close_bf16(y_r, ref, "checkpoint order")
    assert_close_bf16(y_t, ref, "tile order")


def test_tiled_pool_from_device_repack():
    """Slots filled on the GPU with tsa_mxfp4_tile from checkpoint-order tensors."""
    H, I, E, k = 512, 512, 4, 2
    rng = np.random.default_rng(5)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    lay = synth.mxfp4_tiled_layout(H, I)
    pool = torch.zeros((E, lay.total_bytes), dtype=torch.uint8, device="cuda")
    for s, e in enumerate(experts):
        for mat, name in (("gate_up", "gate_up_proj"), ("down", "down_proj")):
            bo, bn = lay.offsets[name], lay.sizes[name]
            so, sn = lay.offsets[name + "_scales"], lay.sizes[name + "_scales"]
            ops.mxfp4_tile(torch.from_numpy(e[mat + "_blocks"]).cuda(), torch.from_numpy(e[mat + "_scales"]).cuda(),
                           out_blocks=pool[s, bo : bo + bn], out_scales=pool[s, so : so + sn])
        for name, key in (("gate_up_proj_bias", "gate_up_bias_bits"), ("down_proj_bias", "down_bias_bits")):
            o, n = lay.offsets[name], lay.sizes[name]
            pool[s, o : o + n] = torch.from_numpy(e[key].view(np.uint8).copy()).cuda()
    x_bits = synth.bf16_normal(rng, (1, H))
    idx, w = oex.route_topk_then_softmax(rng.normal(size=(1, E)).astype(np.float32), k)
    y = ops.moe_decode(mxfp4_expert_layout(lay, tiled=True), pool, torch.from_numpy(idx.astype(np.int32)).cuda(),
                       torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), idx, w), "device-repacked pool")


def test_tiled_decode_workload3_full_routed(form):
    """GPT-OSS-20B shapes (hidden = inter = 2880, 32 experts, top-4), routed in the launch."""
    wl = synth.workload(3)
    H, I, E = wl["hidden"], wl["inter"], wl["E"]
    lay = synth.mxfp4_tiled_layout(H, I)
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in wl["experts"]])).cuda()
    L = mxfp4_expert_layout(lay, tiled=True)
    y, idx, w = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                      torch.from_numpy(wl["logits"]).cuda(), bf16_dev(wl["x_bits"]), 4,
                                      return_routing=True)
    ridx, rw = oex.route_topk_then_softmax(wl["logits"], 4)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert_close_bf16(y, _ref(wl["experts"], synth.bf16_to_f32(wl["x_bits"]), ridx, rw), "workload 3 tiled")


@pytest.mark.parametrize("T", [1, 3])
def test_tiled_routed_repeats_and_missing_slots(T, form):
    """12 back-to-back launches on one workspace (counters must return to zero), with
    experts 2 and 5 not resident (expert_slot -1 contributes zero)."""
    H, I, E, k = 512, 256, 8, 4
    rng, L, experts, pool = _setup(H, I, E, seed=11 + T)
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    es[2] = -1
    es[5] = -1
    ws = ops.moe_decode_workspace(L, T, k, "cuda")
    ws.fill_(0xFF)  # no initialisation needed: the decode keeps no state in it
    outs, refs = [], []
    for _ in range(12):
        logits = rng.normal(size=(T, E)).astype(np.float32)
        x_bits = synth.bf16_normal(rng, (T, H))
        y = ops.moe_decode_routed(L, pool, es, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, workspace=ws)
        ridx, rw = oex.route_topk_then_softmax(logits, k)
        rw = np.where(np.isin(ridx, [2, 5]), 0.0, rw).astype(np.float32)
        outs.append(y)
        refs.append(_ref(experts, synth.bf16_to_f32(x_bits), ridx, rw))
    torch.cuda.synchronize()
    for y, ref in zip(outs, refs):
        assert_close_bf16(y, ref, "tiled routed repeat")


def test_tiled_routed_many_experts_separate_routing():
    """E > 256 routes in a separate launch, then runs the tiled kernel on the slots."""
    H, I, E, k = 256, 128, 300, 4
    rng, L, experts, pool = _setup(H, I, E, seed=300)
    logits = rng.normal(size=(2, E)).astype(np.float32)
    x_bits = synth.bf16_normal(rng, (2, H))
    y, idx, w = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                      torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, return_routing=True)
    ridx, rw = oex.route_topk_then_softmax(logits, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), ridx, rw), "E = 300")


def test_tiled_no_bias_and_f32_output():
    H, I, E, k = 256, 256, 4, 2
    rng, L, experts, pool = _setup(H, I, E, seed=3, bias=False)
    assert L.gate_bias_off == -1 and L.down_bias_off == -1
    x_bits = synth.bf16_normal(rng, (1, H))
    idx, w = oex.route_topk_then_softmax(rng.normal(size=(1, E)).astype(np.float32), k)
    y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                       bf16_dev(x_bits), out_dtype=torch.float32)
    assert y.dtype == torch.float32
    assert_close_bf16(to_f32(y), _ref(experts, synth.bf16_to_f32(x_bits), idx, w), "no bias")


def test_tiled_rejects_non_bf16_activations():
    H, I, E = 256, 128, 2
    rng, L, experts, pool = _setup(H, I, E, seed=1)
    x = torch.randn((1, H), device="cuda", dtype=torch.float32)
    s = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
    w = torch.ones((1, 1), device="cuda")
    with pytest.raises(RuntimeError, match="bf16 activations"):
        ops.moe_decode(L, pool, s, w, x)


@pytest.mark.parametrize("H,I,E,k,T", [(2880, 2880, 8, 4, 1), (512, 1024, 6, 3, 3)])
def test_tiled_decode_small_h(H, I, E, k, T, form):
    """Experts with e8m0 block scales 2^-14 .. 2^-10 and no biases: |gate_up| ~ 0.04, so
    |h| ~ 0.01 - 0.05 and y carries h's precision alone. Output and h against the oracle."""
    rng = np.random.default_rng(H + I + T)
    lay = synth.mxfp4_tiled_layout(H, I, bias=False)
    experts = [synth.make_mxfp4_expert(rng, H, I, bias=False, scale_lo=113, scale_hi=117) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])).cuda()
    L = mxfp4_expert_layout(lay, tiled=True)
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = rng.normal(size=(T, E)).astype(np.float32)
    ws = ops.moe_decode_workspace(L, T, k, "cuda")
    y, gidx, gw = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                        torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, workspace=ws,
                                        return_routing=True)
    torch.cuda.synchronize()
    idx, w = oex.route_topk_then_softmax(logits, k)
    assert np.array_equal(gidx.cpu().numpy(), idx)
    xf = synth.bf16_to_f32(x_bits)
    h = tiled_h(ws, T * k, I, one_launch=form == 0 and k <= 4).reshape(T, k, I)
    h_rms = []
    for t in range(T):
        for j in range(k):
            wgu, _ = oex.mxfp4_expert_weights(experts[idx[t, j]])
            h_ref = oex.gptoss_swiglu(xf[t : t + 1] @ wgu.T).reshape(-1)
            h_rms.append(float(np.sqrt(np.mean(h_ref.astype(np.float64) ** 2))))
            assert_close_bf16(h[t, j], h_ref, f"h[{t},{j}]")
    assert 0.003 < np.median(h_rms) < 0.06, f"h rms {h_rms} outside the small-h regime the test is for"
    assert_close_bf16(y, _ref(experts, xf, idx, w), "small-h decode")


@pytest.mark.parametrize("routed", [True, False])
def test_tiled_decode_outlier_channel(routed, form):
    """x with one channel 1000x the others (a different channel per token): each 32-value
    block of x has its own scale, so the other channels keep their bf16 precision."""
    H, I, E, k, T = 2880, 2880, 6, 4, 2
    rng = np.random.default_rng(77)
    lay = synth.mxfp4_tiled_layout(H, I)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])).cuda()
    L = mxfp4_expert_layout(lay, tiled=True)
    x = rng.normal(size=(T, H)).astype(np.float32) * np.float32(0.01)
    x[0, 17] = 10.0
    x[1, 2000] = -10.0
    u = x.view(np.uint32).astype(np.uint64)  # to bf16, round to nearest even
    x_bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    logits = rng.normal(size=(T, E)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(logits, k)
    xf = synth.bf16_to_f32(x_bits)
    ref = _ref(experts, xf, idx, w)
    if routed:
        y = ops.moe_decode_routed(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                  torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k)
    else:
        y = ops.moe_decode(L, pool, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                           bf16_dev(x_bits))
    torch.cuda.synchronize()
    assert_close_bf16(y, ref, "outlier channel")
    # the contribution of the small channels alone (outliers removed) must be carried too
    xs = xf.copy()
    xs[0, 17] = 0.0
    xs[1, 2000] = 0.0
    wl = [oex.mxfp4_expert_weights(e) for e in experts]
    for t in range(T):
        for j in range(k):
            wgu, _ = wl[idx[t, j]]
            full = xf[t] @ wgu.T
            small = xs[t] @ wgu.T
            assert np.abs(small).max() > 0.02 * np.abs(full).max(), "the small channels must matter"


def test_one_launch_wait_gives_up_then_workspace_heals():
    """A wait limit of 0 makes every down wave of the one-launch form give up at once (forced
    from the host; every workgroup still exits): the outputs are NaN and the workspace is
    poisoned, so later calls write NaN too, until its sync area is cleared."""
    H, I, E, k = 512, 256, 6, 4
    rng, L, experts, pool = _setup(H, I, E, seed=91)
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    ws = ops.moe_decode_workspace(L, 1, k, "cuda")

    def call():
        logits = rng.normal(size=(1, E)).astype(np.float32)
        x_bits = synth.bf16_normal(rng, (1, H))
        y = ops.moe_decode_routed(L, pool, es, torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, workspace=ws)
        idx, w = oex.route_topk_then_softmax(logits, k)
        return y, _ref(experts, synth.bf16_to_f32(x_bits), idx, w)

    try:
        ops.set_decode_options(0, 0)
        y, _ = call()
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all(), "a wait that gave up must leave NaN outputs"
        assert ops.decode_workspace_poisoned(ws)
        ops.set_decode_options(0)  # one launch, default wait limit
        y, _ = call()
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all(), "a poisoned workspace must keep writing NaN"
        assert ops.decode_workspace_poisoned(ws)
        ws.zero_()
        for _ in range(3):
            y, ref = call()
            torch.cuda.synchronize()
            assert_close_bf16(y, ref, "after clearing the sync area")
        assert not ops.decode_workspace_poisoned(ws)
    finally:
        ops.set_decode_options()


@pytest.mark.parametrize("routed", [True, False])
def test_one_launch_graph_replays(routed, one_launch):
    """One decode call captured in a HIP graph and replayed with new inputs each time (same
    kernel arguments, so the workspace's call counter alone tells the calls apart); eager
    calls on the same workspace in between. Every result against the oracle."""
    H, I, E, k = 512, 512, 8, 4
    rng, L, experts, pool = _setup(H, I, E, seed=123 + routed)
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    ws = ops.moe_decode_workspace(L, 1, k, "cuda")
    x = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    logits = torch.empty((1, E), dtype=torch.float32, device="cuda")
    slots = torch.empty((1, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((1, k), dtype=torch.float32, device="cuda")
    y = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")

    def run():
        if routed:
            ops.moe_decode_routed(L, pool, es, logits, x, k, workspace=ws, out=y)
        else:
            ops.moe_decode(L, pool, slots, wts, x, workspace=ws, out=y)

    def fill():
        lg = rng.normal(size=(1, E)).astype(np.float32)
        xb = synth.bf16_normal(rng, (1, H))
        idx, w = oex.route_topk_then_softmax(lg, k)
        x.copy_(bf16_dev(xb))
        logits.copy_(torch.from_numpy(lg))
        slots.copy_(torch.from_numpy(idx.astype(np.int32)))
        wts.copy_(torch.from_numpy(w))
        return _ref(experts, synth.bf16_to_f32(xb), idx, w)

    fill()
    run()  # warm up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            run()
    torch.cuda.synchronize()
    for i in range(6):
        ref = fill()
        torch.cuda.synchronize()
        if i % 3 == 2:
            run()  # an eager call between replays
        else:
            g.replay()
        torch.cuda.synchronize()
        assert_close_bf16(y, ref, f"replay {i}")
    assert not ops.decode_workspace_poisoned(ws)
