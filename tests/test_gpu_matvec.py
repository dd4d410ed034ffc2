"""GPU dequant-matvec parity against the oracle (fp32 dequant, fp32 matmul)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gguf as og
from oracle import mxfp4 as omx
from tests.helpers import assert_close_bf16, bf16_dev, dev_u8, metrics, to_f32
from tinyserve_amd import ops, synth

pytestmark = pytest.mark.gpu


def _x(rng, T, K, dtype):
    x = rng.normal(0.0, 1.0, (T, K)).astype(np.float32)
    xt = torch.from_numpy(x).to(dtype)
    return xt.float().numpy(), xt.cuda()


# Reference test shapes (tests/test_ggml_ops.py:187-212) plus row-straddling K=2880 and
# the full workload-1 size.
@pytest.mark.parametrize("gtype,K,N", [
    (8, 64, 32), (8, 256, 64), (8, 2880, 2880),
    (12, 256, 32), (12, 512, 64), (12, 2880, 2880), (12, 2880, 96),
    (13, 256, 32), (13, 512, 64), (13, 2048, 768), (13, 2880, 40),
    (14, 256, 32), (14, 512, 64), (14, 768, 2048), (14, 2880, 2880), (14, 2880, 24),
])
@pytest.mark.parametrize("T", [1, 3])
def test_gguf_matvec_vs_oracle(gtype, K, N, T):
    rng = np.random.default_rng(42 + gtype * 100 + K + N + T)
    data = synth.make_gguf(rng, gtype, N * K)
    xf, xd = _x(rng, T, K, torch.float32)
    ref = xf @ og.dequant_tensor(data, gtype, (N, K)).T
    y = ops.gguf_matvec(xd, dev_u8(data), gtype, N, K)
    assert y.shape == (T, N) and y.dtype == torch.float32
    assert_close_bf16(y, ref, f"type {gtype} K {K} N {N} T {T}")
    cos, rel = metrics(to_f32(y), ref)  # fp32 output: much tighter than the bar
    assert rel < 1e-4, rel


@pytest.mark.parametrize("gtype", [8, 12, 14])
def test_gguf_matvec_bf16_in_out_unaligned(gtype):
    rng = np.random.default_rng(5)
    K, N = 512, 48
    data = synth.make_gguf(rng, gtype, N * K)
    xf, xd = _x(rng, 1, K, torch.bfloat16)
    ref = xf @ og.dequant_tensor(data, gtype, (N, K)).T
    y = ops.gguf_matvec(xd, dev_u8(data, offset=3), gtype, N, K)
    assert y.dtype == torch.bfloat16
    assert_close_bf16(y, ref)


@pytest.mark.parametrize("gtype,K,N", [(8, 512, 96), (12, 512, 96), (13, 2048, 64), (14, 768, 80)])
@pytest.mark.parametrize("offset", [2, 6, 10])
@pytest.mark.parametrize("T", [1, 3])
def test_gguf_matvec_2byte_aligned_weights(gtype, K, N, offset, T):
    """Weights 2 (not 16) bytes aligned: the stream matvec's buffer-to-LDS copies start at the
    16-byte boundary below each row range, so every row reads its own bytes."""
    rng = np.random.default_rng(300 + gtype + offset + T)
    data = synth.make_gguf(rng, gtype, N * K)
    xf, xd = _x(rng, T, K, torch.float32)
    ref = xf @ og.dequant_tensor(data, gtype, (N, K)).T
    y = ops.gguf_matvec(xd, dev_u8(data, offset=offset), gtype, N, K)
    cos, rel = metrics(to_f32(y), ref)
    assert rel < 1e-4, rel


def test_gguf_matvec_linear_in_x():
    """Size-independent property at workload-2 size: W(a x1 + b x2) = a W x1 + b W x2."""
    rng = np.random.default_rng(11)
    K = N = 2880
    data = dev_u8(synth.make_gguf(rng, 12, N * K))
    x1 = torch.from_numpy(rng.normal(size=(1, K)).astype(np.float32)).cuda()
    x2 = torch.from_numpy(rng.normal(size=(1, K)).astype(np.float32)).cuda()
    y1, y2 = ops.gguf_matvec(x1, data, 12, N, K), ops.gguf_matvec(x2, data, 12, N, K)
    y3 = ops.gguf_matvec(0.5 * x1 - 2.0 * x2, data, 12, N, K)
    cos, rel = metrics(to_f32(y3), to_f32(0.5 * y1 - 2.0 * y2))
    assert cos > 0.999999 and rel < 1e-4


@pytest.mark.parametrize("N,K,T,bias", [(5760, 2880, 1, True), (2880, 2880, 1, True), (64, 128, 1, True),
                                        (2880, 2880, 5, False), (768, 2048, 2, True)])
def test_mxfp4_matvec_vs_oracle(N, K, T, bias):
    rng = np.random.default_rng(N + K + T)
    blocks = rng.integers(0, 256, size=(N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(119, 126, size=(N, K // 32), dtype=np.uint8)
    b_bits = synth.bf16_normal(rng, (N,), 0.02) if bias else None
    xf, xd = _x(rng, T, K, torch.bfloat16)
    ref = xf @ omx.dequant_mxfp4_no_transpose(blocks, scales, "f32").T
    if bias:
        ref = ref + synth.bf16_to_f32(b_bits)
    y = ops.mxfp4_matvec(xd, torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(),
                         bf16_dev(b_bits) if bias else None)
    assert y.shape == (T, N) and y.dtype == torch.bfloat16
    assert_close_bf16(y, ref, f"mxfp4 N {N} K {K} T {T}")


@pytest.mark.parametrize("N,K,T,bias_dt,out_dt", [
    (5760, 2880, 1, torch.bfloat16, torch.bfloat16),  # workload 7: 22.5 pieces of 128 per row
    (100, 96, 3, torch.float32, torch.float32),        # 3 blocks per row, a partial 16-row slice
    (48, 4096, 8, None, torch.bfloat16),               # the largest K and a full column of 8 tokens
    (33, 2880, 9, torch.bfloat16, torch.float32),      # two token columns (8 + 1)
    (16, 32, 17, None, torch.float32),                 # one block per row, three token columns
    (64, 4128, 2, torch.bfloat16, torch.bfloat16),     # past the matrix-core form's K: the row kernel
])
def test_mxfp4_matvec_matrix_core_shapes(N, K, T, bias_dt, out_dt):
    """bf16 tokens take the matrix-core matvec (checkpoint-order blocks as the scaled MFMA's
    fp4 operand, x as block-scaled fp8 terms) up to K 4096: ragged rows, partial pieces,
    several token columns, bias dtypes and fp32 outputs."""
    rng = np.random.default_rng(N * 7 + K + T)
    blocks = rng.integers(0, 256, size=(N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(112, 132, size=(N, K // 32), dtype=np.uint8)
    xf, xd = _x(rng, T, K, torch.bfloat16)
    ref = xf @ omx.dequant_mxfp4_no_transpose(blocks, scales, "f32").T
    bias = None
    if bias_dt is not None:
        bf = rng.normal(0.0, 0.5, N).astype(np.float32)
        bias = torch.from_numpy(bf).to(bias_dt)
        ref = ref + bias.float().numpy()
        bias = bias.cuda()
    y = ops.mxfp4_matvec(xd, torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(), bias, out_dtype=out_dt)
    assert y.shape == (T, N) and y.dtype == out_dt
    assert_close_bf16(y, ref, f"mxfp4 N {N} K {K} T {T}")


@pytest.mark.parametrize("case", ["outlier_channel", "small_scales", "wide_scales"])
def test_mxfp4_matvec_matrix_core_precision(case):
    """The fp8 hi/lo terms keep each bf16 x value exactly unless it lies 2^9 below its
    32-block's maximum: an x channel 10^3 x the rest, weights with e8m0 scales near
    2^-14 (outputs ~1e-3), and scales over the whole e8m0 range but NaN."""
    rng = np.random.default_rng({"outlier_channel": 1, "small_scales": 2, "wide_scales": 3}[case])
    N, K, T = 320, 2880, 2
    blocks = rng.integers(0, 256, size=(N, K // 32, 16), dtype=np.uint8)
    lo, hi = {"outlier_channel": (119, 126), "small_scales": (111, 116), "wide_scales": (60, 190)}[case]
    scales = rng.integers(lo, hi, size=(N, K // 32), dtype=np.uint8)
    x = rng.normal(0.0, 1.0, (T, K)).astype(np.float32)
    if case == "outlier_channel":
        x[:, 1234] *= 1000.0
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ref = xt.float().numpy().astype(np.float64) @ omx.dequant_mxfp4_no_transpose(blocks, scales, "f32").T.astype(np.float64)
    y = ops.mxfp4_matvec(xt.cuda(), torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(), None,
                         out_dtype=torch.float32)
    cos, rel = metrics(to_f32(y), ref.astype(np.float32))
    assert cos >= 0.9999 and rel <= 1e-2, (case, cos, rel)


def test_mxfp4_matvec_f32_out_tight():
    rng = np.random.default_rng(2)
    N, K = 256, 2880
    blocks = rng.integers(0, 256, size=(N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(119, 126, size=(N, K // 32), dtype=np.uint8)
    xf, xd = _x(rng, 1, K, torch.float32)
    ref = xf @ omx.dequant_mxfp4_no_transpose(blocks, scales, "f32").T
    y = ops.mxfp4_matvec(xd, torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(), None)
    cos, rel = metrics(to_f32(y), ref)
    assert rel < 1e-4, rel


def test_unsupported_type_raises():
    act = torch.randn(1, 32, device="cuda")
    w = torch.zeros(100, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="Unsupported ggml_type"):
        ops.gguf_matvec(act, w, 99, 10, 32)


def test_weight_too_small_raises():
    act = torch.randn(1, 256, device="cuda")
    w = torch.zeros(100, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="weight_data too small"):
        ops.gguf_matvec(act, w, 12, 4, 256)
