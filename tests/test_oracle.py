"""CPU checks that pin the oracle (no GPU): golden vectors written from the reference's
own dequantisers, known answers from the reference's tests, closed-form encoders written
from the block-format definitions, HF's MXFP4 converter, the independent scalar C
restatement, and closed forms / invariants for routing, activation and combine."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from oracle import expert as oex
from oracle import gguf as og
from oracle import mxfp4 as omx

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dequant_golden.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as g:
        return {k: g[k] for k in g.files}


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def _same(a, b) -> bool:
    """Bit-equal, except that any NaN matches any NaN (payloads carry no meaning)."""
    a, b = np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(_bits(a)[~na], _bits(b)[~nb])


# ----------------------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("name,t,shape", [("q5_k", 13, (24 * 256,)), ("q6_k", 14, (24 * 256,)),
                                          ("q4_k_k2880", 12, (4, 2880)), ("q6_k_k2880", 14, (4, 2880))])
def test_gguf_oracle_matches_reference_golden(golden, name, t, shape):
    """Bit-exact against tinyserve/gguf_dequant_torch.py (recorded by tests/golden/make_golden.py),
    including fp16-subnormal d/dmin and rows straddling super-blocks at K = 2880."""
    out = og.dequant_tensor(golden[f"{name}_data"], t, shape)
    ref = golden[f"{name}_out"].reshape(shape)
    assert _same(out, ref), f"{name}: oracle differs from the reference"


def test_mxfp4_oracle_matches_reference_golden(golden):
    """e8m0 extremes (0, 1, 254, 255) in bf16 and fp32, and the transposed form."""
    b, s = golden["mxfp4_blocks"], golden["mxfp4_scales"]
    bf = omx.dequant_mxfp4_no_transpose(b, s, "bf16")
    ref_bf = omx.bf16_from_bits(golden["mxfp4_out_bf16_bits"].view(np.uint16))
    assert _same(bf, ref_bf)
    assert np.isnan(ref_bf).sum() == 7 and np.isinf(ref_bf).any()  # 0 * 2^128 -> NaN, others -> +-inf
    assert _same(omx.dequant_mxfp4_no_transpose(b, s, "f32"), golden["mxfp4_out_f32"])
    assert _same(omx.dequant_mxfp4(b, s, "f32"), golden["mxfp4_T_out_f32"])


# ----------------------------------------------------------------------------- Q8_0 known answers
def test_q8_0_known_values():
    """The reference's Q8_0 known answers (tests/test_gguf_dequant_torch.py:123-170)."""
    q = np.arange(1, 33, dtype=np.int8)
    blk = struct.pack("<e", 2.0) + q.tobytes()
    np.testing.assert_array_equal(og.dequant_tensor(blk, 8, (32,)), q.astype(np.float32) * 2.0)
    q = np.array([-16, -8, 0, 8, 16] + [0] * 27, dtype=np.int8)
    blk = struct.pack("<e", 0.5) + q.tobytes()
    np.testing.assert_array_equal(og.dequant_tensor(blk, 8, (32,)), q.astype(np.float32) * 0.5)


def test_unsupported_type_raises():
    with pytest.raises(ValueError, match="99"):
        og.dequant_tensor(b"\x00" * 100, 99, (32,))


# ----------------------------------------------------------------------------- K-quant encoders
# Written from the block-format definitions: choose the integers, pack them, and compare the
# oracle against values computed from those integers directly (no bit unpacking involved).
def _pack_6bit(sc, mn) -> bytes:
    """12-byte scale/min field: j < 4 in bytes j / j+4 (low 6 bits); j >= 4 split into a
    low nibble in byte j+4 (sc) / its high nibble (min) and 2 high bits on bytes j-4 / j."""
    s = bytearray(12)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(s)


def _q4k_or_q5k(rng, five: bool):
    d, dmin = np.float16(rng.uniform(0.001, 0.05)), np.float16(rng.uniform(0.001, 0.05))
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 32 if five else 16, 256)
    qs = bytearray(128)
    qh = bytearray(32)
    for e in range(256):
        c, l = e // 64, e % 64
        lo = q[e] & 15
        if l < 32:
            qs[32 * c + l] |= lo
        else:
            qs[32 * c + l - 32] |= lo << 4
        if five and q[e] >> 4:
            qh[e % 32] |= 1 << (e // 32)
    blk = struct.pack("<ee", d, dmin) + _pack_6bit(sc, mn) + (bytes(qh) if five else b"") + bytes(qs)
    j = np.arange(256) // 32
    expect = (np.float32(d) * sc[j].astype(np.float32)) * q.astype(np.float32) - np.float32(dmin) * mn[j].astype(np.float32)
    return blk, expect.astype(np.float32)


@pytest.mark.parametrize("five", [False, True])
def test_q4k_q5k_encoder_closed_form(five):
    rng = np.random.default_rng(11 + five)
    blks, exps = zip(*[_q4k_or_q5k(rng, five) for _ in range(6)])
    out = og.dequant_tensor(b"".join(blks), 13 if five else 12, (6 * 256,))
    np.testing.assert_array_equal(_bits(out), _bits(np.concatenate(exps)))


def test_q6k_encoder_closed_form():
    rng = np.random.default_rng(6)
    blks, exps = [], []
    for _ in range(5):
        d = np.float16(rng.uniform(0.001, 0.05))
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        q = rng.integers(-32, 32, 256)
        u = (q + 32).astype(np.int64)
        ql, qh = bytearray(128), bytearray(64)
        for e in range(256):
            h, r = e // 128, e % 128
            t, l = r // 32, r % 32
            ql[64 * h + 32 * (t & 1) + l] |= (int(u[e]) & 15) << (4 * (t >> 1))
            qh[32 * h + l] |= (int(u[e]) >> 4) << (2 * t)
        blks.append(bytes(ql) + bytes(qh) + sc.tobytes() + struct.pack("<e", d))
        exps.append((np.float32(d) * sc[np.arange(256) // 16].astype(np.float32)) * q.astype(np.float32))
    out = og.dequant_tensor(b"".join(blks), 14, (5 * 256,))
    np.testing.assert_array_equal(_bits(out), _bits(np.concatenate(exps).astype(np.float32)))


def test_kquant_single_bit_cases():
    """A lone quant bit: only its element is non-zero (catches swapped index arithmetic)."""
    for t, ts in ((12, 144), (13, 176)):
        for e in (0, 31, 32, 63, 64, 200, 255):
            blk = bytearray(ts)
            blk[0:2] = struct.pack("<e", 1.0)
            blk[4:16] = _pack_6bit([1] * 8, [0] * 8)
            base = 48 if t == 13 else 16
            c, l = e // 64, e % 64
            blk[base + 32 * c + (l % 32)] = 1 if l < 32 else 16
            out = og.dequant_tensor(bytes(blk), t, (256,))
            assert out[e] == 1.0 and np.count_nonzero(out) == 1, (t, e)


# ----------------------------------------------------------------------------- MXFP4
def test_mxfp4_known_values():
    """The reference's MXFP4 known answers (tests/test_mxfp4.py:8-61)."""
    b = np.zeros((1, 1, 16), np.uint8)
    b[0, 0, :2] = [0x21, 0x43]
    out = omx.dequant_mxfp4(b, np.array([[127]], np.uint8), "f32")
    np.testing.assert_array_equal(out[:4, 0], [0.5, 1.0, 1.5, 2.0])
    b[0, 0, :2] = [0x02, 0x00]
    assert omx.dequant_mxfp4(b, np.array([[128]], np.uint8), "f32")[0, 0] == 2.0
    b[0, 0, :2] = [0x0A, 0x00]
    assert omx.dequant_mxfp4(b, np.array([[127]], np.uint8), "f32")[0, 0] == -1.0
    assert omx.dequant_mxfp4(np.zeros((4, 2, 16), np.uint8), np.full((4, 2), 127, np.uint8), "f32").shape == (64, 4)


def test_mxfp4_matches_hf_convert_moe_packed_tensors():
    """Exact parity with transformers' converter (tests/test_mxfp4.py:76-96)."""
    torch = pytest.importorskip("torch")
    mxi = pytest.importorskip("transformers.integrations.mxfp4")
    rng = np.random.default_rng(42)
    blocks = rng.integers(0, 256, (2, 32, 4, 16), dtype=np.uint8)
    scales = rng.integers(120, 135, (2, 32, 4), dtype=np.uint8)
    hf = mxi.convert_moe_packed_tensors(torch.from_numpy(blocks), torch.from_numpy(scales), dtype=torch.bfloat16)
    for i in range(2):
        ours = omx.bf16_bits(omx.dequant_mxfp4(blocks[i], scales[i], "bf16"))
        assert np.array_equal(ours.view(np.int16), hf[i].contiguous().view(torch.int16).numpy())


def test_mxfp4_matvec_is_dequant_times_x():
    rng = np.random.default_rng(3)
    b = rng.integers(0, 256, (24, 6, 16), dtype=np.uint8)
    s = rng.integers(119, 126, (24, 6), dtype=np.uint8)
    x = rng.normal(size=192).astype(np.float32)
    bias = rng.normal(size=24).astype(np.float32)
    w = omx.dequant_mxfp4_no_transpose(b, s, "f32").astype(np.float64)
    np.testing.assert_allclose(omx.ref_matvec(b, s, x, bias).reshape(-1), w @ x + bias, rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------------------- C restatement
@pytest.fixture(scope="module")
def coracle():
    from oracle import c_oracle

    try:
        c_oracle.build()
        return c_oracle
    except Exception as exc:  # pragma: no cover - gcc is part of the image
        pytest.skip(f"C oracle does not build: {exc}")


@pytest.mark.parametrize("t,K", [(8, 2880), (12, 2880), (13, 512), (14, 2880), (12, 256), (14, 768)])
def test_c_restatement_matches_numpy(coracle, t, K):
    from tinyserve_amd import synth

    rng = np.random.default_rng(t * K)
    N = 8  # N * K a whole number of blocks; at K = 2880 rows straddle super-blocks
    data = synth.make_gguf(rng, t, N * K)
    a = og.dequant_tensor(data, t, (N, K))
    b = coracle.gguf_dequant(data, t, N * K).reshape(N, K)
    assert np.array_equal(_bits(a), _bits(b))
    x = rng.normal(size=K).astype(np.float32)
    np.testing.assert_allclose(coracle.gguf_matvec(data, t, x, N, K), og.ref_matvec(data, x, t, N, K).reshape(-1),
                               rtol=1e-5, atol=1e-4)


def test_c_restatement_mxfp4(coracle, golden):
    b, s = golden["mxfp4_blocks"], golden["mxfp4_scales"]
    assert _same(omx.dequant_mxfp4_no_transpose(b, s, "f32"), coracle.mxfp4_dequant(b, s).reshape(6, 128))


# ----------------------------------------------------------------------------- routing
def test_routing_matches_torch_topk_softmax():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    lg = rng.normal(size=(64, 32)).astype(np.float32)
    idx, w = oex.route_topk_then_softmax(lg, 4)
    tv, ti = torch.topk(torch.from_numpy(lg), 4, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, torch.softmax(tv, dim=-1).numpy(), rtol=1e-6)
    lg = rng.normal(size=(16, 128)).astype(np.float32)
    idx, w = oex.route_softmax_then_topk(lg, 8)
    p = torch.softmax(torch.from_numpy(lg), dim=-1)
    tv, ti = torch.topk(p, 8, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, (tv / tv.sum(-1, keepdim=True)).numpy(), rtol=1e-5)
    _, w2 = oex.route_softmax_then_topk(lg, 8, renormalize=False)
    np.testing.assert_allclose(w2, tv.numpy(), rtol=1e-5)


def test_routing_ties_go_to_lower_index():
    idx, w = oex.route_topk_then_softmax(np.array([[0, 1, 1, 0, 1]], np.float32), 3)
    assert idx.tolist() == [[1, 2, 4]]
    np.testing.assert_allclose(w, [[1 / 3] * 3], rtol=1e-6)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
def test_routing_nan_and_inf_order_matches_torch_topk():
    """NaN ranks above every number and +-inf keep their places, as torch.topk orders them
    (rows without ties: torch leaves the order of equal values unspecified, and it varies
    with the row length; the oracle resolves ties to the lower index)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    for _ in range(200):
        E = int(rng.integers(2, 300))
        k = int(rng.integers(1, min(E, 16) + 1))
        lg = rng.normal(size=(3, E)).astype(np.float32)
        for r in range(3):
            for val, p in ((np.nan, 0.5), (np.inf, 0.3), (-np.inf, 0.3)):
                if rng.random() < p:
                    lg[r, rng.integers(E)] = val
        tv, ti = torch.topk(torch.from_numpy(lg), k, dim=-1)
        idx, w = oex.route_topk_then_softmax(lg, k)
        assert np.array_equal(idx, ti.numpy())
        np.testing.assert_allclose(w, torch.softmax(tv.double(), dim=-1).float().numpy(), rtol=1e-6, equal_nan=True)


# ----------------------------------------------------------------------------- activation / combine
def test_gptoss_swiglu_closed_forms():
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))  # noqa: E731
    gu = np.array([[0.0, 3.0, 10.0, 10.0, 2.0, -10.0, -3.0, 0.5]], np.float32)  # (gate, up) pairs
    h = oex.gptoss_swiglu(gu).reshape(-1)
    np.testing.assert_allclose(h, [0.0, (7 + 1) * 7 * sig(1.702 * 7), (-7 + 1) * 2 * sig(1.702 * 2),
                                   (0.5 + 1) * -3 * sig(1.702 * -3)], rtol=1e-6)


def test_silu_gate_closed_form():
    g, u = np.array([0.0, 1.0, -2.0], np.float32), np.array([5.0, 2.0, 3.0], np.float32)
    np.testing.assert_allclose(oex.silu_gate(g, u), g / (1 + np.exp(-g)) * u, rtol=1e-6)


def test_combine_invariants():
    rng = np.random.default_rng(1)
    mats = [rng.normal(size=(8, 8)).astype(np.float32) for _ in range(4)]
    fwd = lambda e, xx: np.tanh(xx @ mats[e].T)  # noqa: E731
    x = rng.normal(size=(3, 8)).astype(np.float32)
    idx = np.array([[0, 2], [3, 1], [2, 2]])
    w = rng.uniform(size=(3, 2)).astype(np.float32)
    base = oex.moe_combine(x, idx, w, fwd)
    np.testing.assert_allclose(oex.moe_combine(x, idx[:, ::-1], w[:, ::-1], fwd), base, rtol=1e-6)  # permutation
    np.testing.assert_allclose(oex.moe_combine(x, idx, 2 * w, fwd), 2 * base, rtol=1e-6)  # linear in weights
    neg = idx.copy()
    neg[:, 1] = -1
    np.testing.assert_allclose(oex.moe_combine(x, neg, w, fwd), oex.moe_combine(x, idx[:, :1], w[:, :1], fwd))
    np.testing.assert_allclose(oex.moe_combine_grouped(x, idx, w, fwd), base, rtol=1e-5, atol=1e-6)


def test_grouping_is_token_major_permutation():
    idx = np.array([[3, 1], [1, 3], [0, 1]])
    g = oex.group_tokens_by_expert(idx)
    assert g == {3: [(0, 0), (1, 1)], 1: [(0, 1), (1, 0), (2, 1)], 0: [(2, 0)]}
