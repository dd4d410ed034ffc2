"""numpy restatement of the reference's MXFP4 dequantiser (test oracle only).

Follows ``tinyserve/mxfp4.py:5-53``. A row of an MXFP4 matrix is ``G`` groups of
``B = 16`` bytes (32 e2m1 values) plus one e8m0 scale byte per group; byte ``j`` of
group ``g`` holds element ``32g + 2j`` in its low nibble and ``32g + 2j + 1`` in its
high nibble. The value is ``LUT[nibble] * 2**(scale - 127)``: the LUT value in the
requested dtype, times a float32 power of two (``torch.ldexp`` multiplies by
``torch.pow(2.0, e)``, a float32 tensor), rounded to the requested dtype. For the
e8m0 range 1..254 the result is exact in bf16/fp32; ``scale == 0`` gives float32
subnormal multipliers (still exact); ``scale == 255`` multiplies by +inf, so the
two zero codes give NaN and the others +/-inf.
"""
from __future__ import annotations

import numpy as np

# tinyserve/mxfp4.py:5-8
FP4_LUT = np.array(
    [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (round to nearest even), returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0  # torch's canonical bfloat16 NaN
    return r


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value, as float32."""
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e8m0_to_f32(scales: np.ndarray) -> np.ndarray:
    """float32 2**(s-127), the multiplier torch.ldexp uses (exact; 255 -> inf)."""
    si = np.asarray(scales).astype(np.int32) - 127
    return np.ldexp(np.float32(1.0), si).astype(np.float32)


def dequant_mxfp4_no_transpose(blocks: np.ndarray, scales: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """MXFP4 -> [N, K] values (mxfp4.py:20-44). Returns float32 holding values of ``dtype``."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    N, G, B = blocks.shape
    rows = N * G
    bf = blocks.reshape(rows, B)
    out = np.empty((rows, B * 2), dtype=np.float32)
    out[:, 0::2] = FP4_LUT[bf & 0x0F]
    out[:, 1::2] = FP4_LUT[bf >> 4]
    with np.errstate(invalid="ignore", over="ignore"):
        out = out * e8m0_to_f32(scales).reshape(rows, 1)
    if dtype == "bf16":
        out = bf16_round(out)
    elif dtype != "f32":
        raise ValueError(f"dtype must be 'bf16' or 'f32', got {dtype!r}")
    return out.reshape(N, G * B * 2)


def dequant_mxfp4(blocks: np.ndarray, scales: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """Transposed [K, N] form (mxfp4.py:47-53)."""
    return np.ascontiguousarray(dequant_mxfp4_no_transpose(blocks, scales, dtype).T)


def ref_matvec(blocks, scales, x, bias=None) -> np.ndarray:
    """fp32 dequant then fp32 matvec: y[N] = W[N,K] @ x + bias."""
    w = dequant_mxfp4_no_transpose(blocks, scales, "f32")
    y = w @ np.asarray(x, dtype=np.float32).reshape(-1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.astype(np.float32)
