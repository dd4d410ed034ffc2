"""Batched prefill on the grouped MXFP4 MFMA GEMMs (tiled pools, bf16 activations), against
the oracle's grouped expert forward (expert_pipeline.py:166-239)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.helpers import assert_close_bf16, bf16_dev, to_f32
from tinyserve_amd import _lib, ops, synth
from tinyserve_amd.expert_forward import mxfp4_expert_layout

pytestmark = pytest.mark.gpu


def _pool(H, I, E, seed, bias=True, tiled=True, mfma=_lib.PREFILL_FP6):
    rng = np.random.default_rng(seed)
    experts = [synth.make_mxfp4_expert(rng, H, I, bias=bias) for _ in range(E)]
    if tiled:
        lay = synth.mxfp4_tiled_layout(H, I, bias=bias)
        pool = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])
    else:
        lay = synth.mxfp4_layout(H, I, bias=bias)
        pool = np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])
    return rng, mxfp4_expert_layout(lay, tiled=tiled, prefill_mfma=mfma), experts, torch.from_numpy(pool).cuda()


def _ref(experts, xf, idx, w):
    return oex.moe_combine_grouped(xf, idx, w, lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("H,I,E,k,T", [
    (256, 128, 8, 2, 64),      # one weight tile along N, two pieces along K
    (512, 384, 6, 4, 200),     # experts with more than 128 rows; a partial weight tile (768 rows)
    (2880, 2880, 4, 2, 45),    # the GPT-OSS shape: K % 128 = 64, 22.5 weight tiles of gate_up
    (256, 160, 5, 3, 333),     # K = 160 (two pieces, the second a quarter full)
    (1024, 256, 33, 1, 97),    # more experts than the tile table's first rows; k = 1
    (256, 128, 256, 8, 300),   # over 128 partial row tiles spread over the 8 XCD groups
])
@pytest.mark.parametrize("mfma", [_lib.PREFILL_FP6, _lib.PREFILL_BF16], ids=["fp6", "bf16"])
def test_prefill_tiled_vs_oracle(H, I, E, k, T, mfma):
    rng, L, experts, pool = _pool(H, I, E, seed=H + I + E + k + T, mfma=mfma)
    x_bits = synth.bf16_normal(rng, (T, H))
    idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
    y = ops.moe_prefill(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                        torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    assert y.dtype == torch.bfloat16 and y.shape == (T, H)
    assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), idx, w),
                      f"prefill H={H} I={I} E={E} k={k} T={T} mfma={mfma}")


def test_prefill_only_full_row_tiles():
    """Every expert gets exactly 128 or 256 rows: the tile table holds full entries only."""
    H, I, E, k, T = 512, 256, 5, 2, 384
    rng, L, experts, pool = _pool(H, I, E, seed=31)
    idx = np.array([[0, 1]] * 128 + [[0, 2]] * 128 + [[3, 4]] * 128)
    assert np.bincount(idx.reshape(-1), minlength=E).tolist() == [256, 128, 128, 128, 128]
    w = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    x_bits = synth.bf16_normal(rng, (T, H))
    y = ops.moe_prefill(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                        torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), idx, w), "prefill, full row tiles only")


def test_prefill_missing_experts_and_dropped_assignments():
    """Experts without a resident slot and assignments with idx < 0 contribute nothing."""
    H, I, E, k, T = 512, 256, 6, 3, 150
    rng, L, experts, pool = _pool(H, I, E, seed=5)
    x_bits = synth.bf16_normal(rng, (T, H))
    idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
    idx = idx.copy()
    idx[7, 1] = -1
    idx[100, 0] = -1
    expert_slot = np.arange(E, dtype=np.int32)
    expert_slot[2] = -1  # not resident
    y = ops.moe_prefill(L, pool, torch.from_numpy(expert_slot).cuda(), torch.from_numpy(idx.astype(np.int32)).cuda(),
                        torch.from_numpy(w).cuda(), bf16_dev(x_bits), out_dtype=torch.float32)
    live = (idx >= 0) & (expert_slot[np.maximum(idx, 0)] >= 0)
    ref = _ref(experts, synth.bf16_to_f32(x_bits), np.where(live, idx, -1), np.where(live, w, 0.0).astype(np.float32))
    assert_close_bf16(y, ref, "prefill with missing experts")


def test_prefill_tiled_matches_chunked_checkpoint_path():
    """The same experts as a checkpoint-order pool (fused decode over token chunks) agree."""
    H, I, E, k, T = 512, 256, 8, 4, 70
    rng, Lt, experts, pool_t = _pool(H, I, E, seed=11)
    _, Lc, experts_c, pool_c = _pool(H, I, E, seed=11, tiled=False)
    x_bits = synth.bf16_normal(rng, (T, H))
    idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
    args = (torch.arange(E, dtype=torch.int32, device="cuda"), torch.from_numpy(idx.astype(np.int32)).cuda(),
            torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    yt = ops.moe_prefill(Lt, pool_t, *args)
    yc = ops.moe_prefill(Lc, pool_c, *args)
    ref = _ref(experts, synth.bf16_to_f32(x_bits), idx, w)
    assert_close_bf16(yt, ref, "tiled")
    assert_close_bf16(yc, ref, "chunked")
    assert_close_bf16(yt, to_f32(yc), "tiled vs chunked")


def test_prefill_repeat_calls_and_smaller_batch():
    """A reused workspace gives the same answer, also for a smaller second batch."""
    H, I, E, k = 256, 256, 4, 2
    rng, L, experts, pool = _pool(H, I, E, seed=21)
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    ws = ops.moe_prefill_workspace(L, 300, k, E, "cuda")
    for T in (300, 300, 17):
        x_bits = synth.bf16_normal(rng, (T, H))
        idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
        y = ops.moe_prefill(L, pool, es, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                            bf16_dev(x_bits), workspace=ws)
        assert_close_bf16(y, _ref(experts, synth.bf16_to_f32(x_bits), idx, w), f"repeat T={T}")


def test_prefill_workload5_sampled_tokens():
    """The full batched-prefill workload (2048 tokens, top-4 of 32 Zipf-routed experts); the
    oracle checks a sample of tokens (each output row depends only on its own token)."""
    wl = synth.workload(5)
    H, I, E, k = wl["hidden"], wl["inter"], wl["E"], wl["top_k"]
    lay = synth.mxfp4_tiled_layout(H, I)
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in wl["experts"]])).cuda()
    L = mxfp4_expert_layout(lay, tiled=True)
    idx, w = oex.route_topk_then_softmax(wl["logits"], k)
    T = idx.shape[0]
    y = ops.moe_prefill(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                        torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(), bf16_dev(wl["x_bits"]))
    yf = to_f32(y)
    assert np.isfinite(yf).all()
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert counts.max() > 4 * 128 and counts.min() < 128, "Zipf routing gives multi-tile and partial-tile experts"
    rng = np.random.default_rng(0)
    toks = np.unique(np.concatenate([np.arange(8), np.arange(T - 8, T), rng.choice(T, 24, replace=False)]))
    xf = synth.bf16_to_f32(wl["x_bits"][toks])
    ref = np.zeros((len(toks), H), np.float32)
    for e in np.unique(idx[toks]):
        W = oex.mxfp4_expert_weights(wl["experts"][e])
        rows, js = np.nonzero(idx[toks] == e)
        ye = oex.mxfp4_expert_forward(xf[rows], wl["experts"][e], W)
        for r, j, v in zip(rows, js, ye):
            ref[r] += np.float32(w[toks[r], j]) * v
    assert_close_bf16(yf[toks], ref, "workload 5 sample")


def test_prefill_fp6_and_bf16_forms_agree_and_zero_blocks():
    """The fp6-term and bf16 GEMMs agree with each other and the oracle on activations with
    all-zero tokens, all-zero 32-blocks, tiny and large blocks (the fp6 scales span them)."""
    H, I, E, k, T = 512, 384, 6, 2, 96
    rng, L6, experts, pool = _pool(H, I, E, seed=77)
    Lb = mxfp4_expert_layout(synth.mxfp4_tiled_layout(H, I), tiled=True, prefill_mfma=_lib.PREFILL_BF16)
    x = synth.bf16_to_f32(synth.bf16_normal(rng, (T, H)))
    x[3] = 0.0                      # a zero token
    x[5, 64:96] = 0.0               # a zero block
    x[6, :32] *= 2.0 ** -60         # a tiny block
    x[7, 32:64] *= 2.0 ** 20        # a huge block
    x_bits = (x.view(np.uint32) >> 16).astype(np.uint16)  # exact: scaling by powers of two
    idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
    args = (torch.arange(E, dtype=torch.int32, device="cuda"), torch.from_numpy(idx.astype(np.int32)).cuda(),
            torch.from_numpy(w).cuda(), bf16_dev(x_bits))
    y6 = ops.moe_prefill(L6, pool, *args, out_dtype=torch.float32)
    yb = ops.moe_prefill(Lb, pool, *args, out_dtype=torch.float32)
    ref = _ref(experts, synth.bf16_to_f32(x_bits), idx, w)
    rows = [r for r in range(T) if r != 7]  # row 7 (its outputs are far larger) is checked on its own
    for y, form in ((y6, "fp6"), (yb, "bf16")):
        yf = to_f32(y)
        assert np.isfinite(yf).all()
        assert_close_bf16(yf[rows], ref[rows], f"{form} form")
        assert_close_bf16(yf[7:8], ref[7:8], f"{form} form, huge block")
        assert_close_bf16(yf[3:4], ref[3:4], f"{form} form, zero token")
