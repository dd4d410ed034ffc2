"""Grouped GGUF prefill (moe_prefill_gguf.hip: expert-major tiles, K-quant / Q8_0 blocks
decoded to bf16 in LDS, bf16 MFMA, combine in j order) against the oracle's fp32 expert
(ggml_forward.py:117-151 runs the batched expert with bf16 weights; the oracle's fp32 form
bounds that within the bf16 tolerance), over every block type, ragged and multi-tile
expert runs, experts that are not resident, repeated experts, a garbage-filled workspace,
rows that straddle super-blocks (K % 256 != 0), and the decode-kernel path that small
calls and unaligned layouts keep
(expert_pipeline.py:166-239)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.helpers import assert_close_bf16, bf16_dev
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_forward import gguf_expert_layout

pytestmark = pytest.mark.gpu


def _pool(rng, H, I, types, E, pad=0):
    lay = synth.gguf_layout(H, I, *types)
    experts = [synth.make_gguf_expert(rng, H, I, *types) for _ in range(E)]
    packed = np.stack([synth.pack_gguf_expert(e, lay) for e in experts])
    L = gguf_expert_layout(lay, dict(zip(("gate", "up", "down"), types)), {"gate": (H, I), "up": (H, I), "down": (I, H)})
    if pad:  # every matrix `pad` bytes further into a slot `pad` bytes longer
        packed = np.concatenate([np.zeros((E, pad), np.uint8), packed], axis=1)
        L.slot_bytes += pad
        L.gate_off += pad
        L.up_off += pad
        L.down_off += pad
    return L, experts, torch.from_numpy(np.ascontiguousarray(packed)).cuda()


def _rb(a: np.ndarray) -> np.ndarray:
    """float32 -> the nearest bf16 value (ties to even), as float32 (finite inputs)."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def _bf16_path_ref(experts, x, idx, w, es):
    """The reference's batched GGUF expert in its own roundings (ggml_forward.py:117-151):
    weights decoded exactly, then cast to bf16; h = act(gate, up) and every expert output
    rounded to bf16; the weighted sum over j in fp32. Products in float64. Also returns, per
    output, sum_j |w_j| sum_i |h_i W_d[n, i]|: where the GPU's fp32 sums round an h element
    to the neighbouring bf16 value, the output moves by a small part of that sum."""
    T, k = idx.shape
    y = np.zeros((T, x.shape[1]), np.float32)
    bound = np.zeros((T, x.shape[1]), np.float64)
    yk = np.zeros((T, k, x.shape[1]), np.float32)
    ak = np.zeros((T, k, x.shape[1]), np.float64)
    for e in np.unique(idx):
        s = es[e]
        if s < 0:
            continue
        wg, wu, wd = (_rb(m).astype(np.float64) for m in oex.gguf_expert_weights(experts[s]))
        tt, jj = np.nonzero(idx == e)
        xe = x[tt].astype(np.float64)
        h = _rb(oex.silu_gate((xe @ wg.T).astype(np.float32), (xe @ wu.T).astype(np.float32))).astype(np.float64)
        yk[tt, jj] = _rb((h @ wd.T).astype(np.float32))
        ak[tt, jj] = np.abs(h) @ np.abs(wd).T
    for j in range(k):
        live = np.array([es[e] >= 0 for e in idx[:, j]])
        y += np.where(live[:, None], w[:, j : j + 1] * yk[:, j], 0.0).astype(np.float32)
        bound += np.where(live[:, None], np.abs(w[:, j : j + 1]) * ak[:, j], 0.0)
    return y, bound


def _assert_elementwise(y, ref, bound, what, rtol=1e-2, sum_frac=4e-3):
    """Every element within rtol of its reference value plus sum_frac of its sum of absolute
    products: a block decoded from the wrong bytes moves the outputs it feeds by more."""
    g = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y, np.float32)
    err = np.abs(g.astype(np.float64) - ref) - (rtol * np.abs(ref) + sum_frac * bound)
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() <= 0, f"{what}: element {worst}: {g[worst]} vs {ref[worst]} (bound {bound[worst]:.4g})"


def _run(L, experts, pool, rng, T, k, E, expert_slot=None, idx=None, out_dtype=None, workspace=None,
         bf16_path=True, grouped=False):
    """One prefill call against the oracle; ``grouped``: also require that the grouped GEMMs
    ran (their bf16 weights put 99% of the outputs within 1e-5 of their absolute-product
    sums from the bf16-path reference; the decode kernels' exact weights land near 1e-3)."""
    H = L.hidden
    x_bits = synth.bf16_normal(rng, (T, H))
    if idx is None:
        idx, w = oex.route_softmax_then_topk(synth.zipf_logits(rng, T, E), k)
    else:
        w = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    es = np.arange(E, dtype=np.int32) if expert_slot is None else expert_slot
    y = ops.moe_prefill(L, pool, torch.from_numpy(es).cuda(), torch.from_numpy(idx.astype(np.int32)).cuda(),
                        torch.from_numpy(w).cuda(), bf16_dev(x_bits), out_dtype=out_dtype, workspace=workspace)

    def ffn(e, xx):
        s = es[e]
        return oex.gguf_expert_forward(xx, experts[s]) if s >= 0 else np.zeros_like(xx)

    x = synth.bf16_to_f32(x_bits)
    ref = oex.moe_combine_grouped(x, idx, w, ffn)
    yb, bound = _bf16_path_ref(experts, x, idx, w, es)
    _assert_elementwise(y, yb, bound, "element check", sum_frac=4e-3 if bf16_path else 8e-3)
    if grouped:  # a bf16 y against the reference rounded the same way
        yr = _rb(yb) if y.dtype == torch.bfloat16 else yb
        rel = np.abs(y.float().cpu().numpy().astype(np.float64) - yr) / np.maximum(bound, 1e-30)
        assert np.quantile(rel, 0.99) < 1e-5, f"not the grouped path: p99 {np.quantile(rel, 0.99):.3g}"
    return y, ref


@pytest.mark.parametrize("types", [(12, 12, 14), (13, 13, 14), (8, 8, 8), (14, 14, 14), (13, 13, 13), (12, 12, 8),
                                   (12, 12, 12), (8, 8, 14)])
def test_gguf_grouped_prefill_types(types):
    rng = np.random.default_rng(100 + sum(types))
    H, I, E, k, T = 512, 256, 16, 4, 40  # 160 assignments: ragged tiles of the 16 experts
    L, experts, pool = _pool(rng, H, I, types, E)
    y, ref = _run(L, experts, pool, rng, T, k, E, grouped=True)
    assert_close_bf16(y, ref, f"GGUF grouped prefill, types {types}")


def test_gguf_grouped_prefill_partial_column_tile():
    """inter 160: the gate_up launch's last column tile holds 32 of its 64 gate / up rows (the
    rest read zeros past the matrix and are not stored); the down rows then straddle."""
    rng = np.random.default_rng(12)
    H, I, E, k, T = 512, 160, 8, 4, 40
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), E)
    y, ref = _run(L, experts, pool, rng, T, k, E, grouped=True)
    assert_close_bf16(y, ref, "GGUF grouped prefill, partial column tile")


def test_gguf_grouped_prefill_multi_tile_and_fp32_out():
    """Few experts, many tokens: runs of several 64-row tiles plus a partial one; fp32 output."""
    rng = np.random.default_rng(7)
    H, I, E, k, T = 256, 512, 3, 2, 150
    L, experts, pool = _pool(rng, H, I, (12, 12, 14), E)
    y, ref = _run(L, experts, pool, rng, T, k, E, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    assert_close_bf16(y, ref, "GGUF grouped prefill, multi-tile runs")


def test_gguf_grouped_prefill_missing_and_repeated_experts():
    """expert_slot -1 (not resident: contributes zero) and several ids mapped to one slot;
    the workspace starts as 0xFF bytes (no call needs it cleared)."""
    rng = np.random.default_rng(8)
    H, I, E, k, T = 512, 512, 12, 4, 33
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), 6)
    es = np.array([0, -1, 2, 3, 1, 5, 4, 2, -1, 0, 3, 1], dtype=np.int32)
    ws = ops.moe_prefill_workspace(L, T, k, E, "cuda").fill_(0xFF)
    y, ref = _run(L, experts, pool, rng, T, k, E, expert_slot=es, workspace=ws)
    assert_close_bf16(y, ref, "GGUF grouped prefill, missing / repeated experts")


def test_gguf_grouped_prefill_many_expert_ids():
    """640 expert ids (the grouping kernel's tile table takes two experts per thread past
    512) over 32 resident slots, with every ninth id not resident: ids past 512 own tiles."""
    rng = np.random.default_rng(13)
    H, I, E, k, T = 256, 256, 640, 8, 96
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), 32)
    es = np.array([-1 if e % 9 == 4 else e % 32 for e in range(E)], dtype=np.int32)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    idx[: T // 2, 0] = 600 + (np.arange(T // 2) % 40)  # ids past 512 in many rows
    for t in range(T // 2):  # keep each token's ids distinct
        if (idx[t, 1:] == idx[t, 0]).any():
            idx[t, 1:][idx[t, 1:] == idx[t, 0]] = (idx[t, 0] + 1) % 512
    y, ref = _run(L, experts, pool, rng, T, k, E, expert_slot=es, idx=idx, grouped=True)
    assert_close_bf16(y, ref, "GGUF grouped prefill, 640 expert ids")


def test_gguf_grouped_prefill_workload4_shapes_long_prompt():
    """Workload-4 expert shapes (Q5_K gate/up 2048 -> 768, Q6_K down), 128 experts, top-8 of
    256 tokens: 2048 assignments over the grouped tiles."""
    rng = np.random.default_rng(9)
    H, I, E, k, T = 2048, 768, 128, 8, 256
    L, experts, pool = _pool(rng, H, I, (13, 13, 14), E)
    y, ref = _run(L, experts, pool, rng, T, k, E)
    assert_close_bf16(y, ref, "GGUF grouped prefill, workload-4 shapes, 256 tokens")


@pytest.mark.parametrize("pad,T", [(2, 40), (0, 8)])
def test_gguf_prefill_decode_path_cases(pad, T):
    """Slots whose K-quant blocks sit off a 16-byte boundary (pad 2), and calls with fewer
    than 64 assignments (T 8, k 4), keep the decode kernels; same results."""
    rng = np.random.default_rng(10 + pad + T)
    H, I, E, k = 512, 256, 16, 4
    L, experts, pool = _pool(rng, H, I, (12, 12, 14), E, pad=pad)
    y, ref = _run(L, experts, pool, rng, T, k, E, bf16_path=False)  # exact weights on this path
    assert_close_bf16(y, ref, f"GGUF prefill on the decode kernels (pad {pad}, T {T})")


def test_gguf_grouped_prefill_q6_q8_unaligned_base():
    """Q6_K / Q8_0 matrices at 2-byte (not 16-byte) offsets: the grouped path reads their
    windows from the 16-byte boundary below each row piece."""
    rng = np.random.default_rng(11)
    H, I, E, k, T = 512, 256, 8, 4, 48
    L, experts, pool = _pool(rng, H, I, (14, 14, 8), E, pad=6)
    y, ref = _run(L, experts, pool, rng, T, k, E)
    assert_close_bf16(y, ref, "GGUF grouped prefill, Q6_K / Q8_0 at 2-byte offsets")


@pytest.mark.parametrize("types,H,I,pad", [
    ((12, 12, 12), 288, 96, 0),     # 9 and 3 units per row: rows start at every unit of a super-block
    ((14, 14, 14), 288, 96, 0),
    ((13, 13, 14), 2880, 320, 0),   # 2880 % 256 = 64: gate/up rows straddle, down rows too (320 % 256)
    ((14, 14, 14), 320, 2880, 0),
    ((14, 14, 8), 320, 2880, 6),    # Q6_K / Q8_0 matrices at 2-byte offsets
    ((8, 8, 8), 288, 96, 0),        # Q8_0: whole blocks per row, the last K piece partial
    ((12, 12, 8), 2880, 320, 0),
])
def test_gguf_grouped_prefill_straddling_rows(types, H, I, pad):
    """K not a multiple of 256: a K-quant row starts inside a super-block and its K pieces
    cover two; the last piece of a row is partial (its other values belong to the next row)."""
    rng = np.random.default_rng(300 + H + I + sum(types) + pad)
    E, k, T = 8, 4, 40
    L, experts, pool = _pool(rng, H, I, types, E, pad=pad)
    y, ref = _run(L, experts, pool, rng, T, k, E, grouped=True)
    assert_close_bf16(y, ref, f"GGUF grouped prefill, straddling rows, types {types}, H {H}, I {I}")


def test_gguf_grouped_prefill_2880_wide_512_tokens():
    """Workload 2's expert (Q4_K gate/up 2880 -> 2880, Q6_K down) in an 8-expert layer, a
    512-token prefill with Zipf top-4: 2048 assignments, every row straddling."""
    rng = np.random.default_rng(2880)
    H = I = 2880
    E, k, T = 8, 4, 512
    L, experts, pool = _pool(rng, H, I, (12, 12, 14), E)
    y, ref = _run(L, experts, pool, rng, T, k, E, grouped=True)
    assert_close_bf16(y, ref, "GGUF grouped prefill, 2880-wide, 512 tokens")
