"""Vectorised numpy restatement of the reference's GGUF dequantiser (test oracle only).

Follows ``tinyserve/gguf_dequant_torch.py`` (itself a port of city96/ComfyUI-GGUF):
the byte stream is cut into fixed-size blocks, each block is decoded to
``block_size`` float32 values, and the flat result is reshaped to ``shape``.
Element (n, k) of a GGUF matrix with ``shape = (N, K)`` is therefore flat index
``n*K + k`` of the block stream, even when K is not a multiple of the
super-block size (rows then straddle super-blocks).

Every arithmetic step keeps the reference's float32 operation order:
``d*sc`` and ``dmin*m`` are float32 products, the value is ``(d*sc)*q - dmin*m``
(two roundings at most, the first of which is exact for these magnitudes).
"""
from __future__ import annotations

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q5_K = 13
GGML_Q6_K = 14

# (block_elements, type_size_bytes) — gguf_dequant_torch.py:20-29 (hot-path types).
QUANT_SIZES: dict[int, tuple[int, int]] = {
    GGML_Q8_0: (32, 34),
    GGML_Q4_K: (256, 144),
    GGML_Q5_K: (256, 176),
    GGML_Q6_K: (256, 210),
}

QK_K = 256
K_SCALE_SIZE = 12


def _as_u8(data) -> np.ndarray:
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(data), dtype=np.uint8)
    arr = np.asarray(data)
    return np.ascontiguousarray(arr).view(np.uint8).reshape(-1)


def dequant_tensor(data, ggml_type: int, shape: tuple[int, ...]) -> np.ndarray:
    """Dequantise GGUF bytes to float32 of ``shape`` (gguf_dequant_torch.py:35-78)."""
    raw = _as_u8(data)
    if ggml_type == GGML_F32:
        return raw.view("<f4").astype(np.float32).reshape(shape)
    if ggml_type == GGML_F16:
        return raw.view("<f2").astype(np.float32).reshape(shape)
    if ggml_type not in QUANT_SIZES:
        raise ValueError(
            f"Unsupported GGML quantization type {ggml_type}. "
            f"Supported: [0, 1] + {sorted(QUANT_SIZES)}"
        )
    block_size, type_size = QUANT_SIZES[ggml_type]
    n_blocks = raw.size // type_size
    blocks = raw[: n_blocks * type_size].reshape(n_blocks, type_size)
    out = _DEQUANT[ggml_type](blocks)
    return out.reshape(shape).astype(np.float32, copy=False)


def _split(blocks: np.ndarray, *sizes: int) -> list[np.ndarray]:
    """Column split of [n, type_size] blocks (gguf_dequant_torch.py:95-98)."""
    out, off = [], 0
    for s in sizes:
        out.append(blocks[:, off : off + s])
        off += s
    out.append(blocks[:, off:])
    return out


def _f16(col: np.ndarray) -> np.ndarray:
    """[n, 2] little-endian fp16 bytes -> [n, 1] float32 (exact, subnormals kept)."""
    return np.ascontiguousarray(col).view("<f2").astype(np.float32)


def get_scale_min(scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Unpack the 12-byte 6-bit scale/min field (gguf_dequant_torch.py:101-111).

    Bytes 0-3 carry sc[0..3] (low 6 bits), bytes 4-7 carry m[0..3]; the top two
    bits of those eight bytes are bits 4-5 of sc[4..7] / m[4..7], whose low
    nibbles live in bytes 8-11 (low nibble sc, high nibble m).
    """
    n = scales.shape[0]
    s = scales.reshape(n, 3, 4)
    d, m, m_d = s[:, 0, :], s[:, 1, :], s[:, 2, :]
    sc = np.concatenate([d & 0x3F, (m_d & 0x0F) | ((d >> 2) & 0x30)], axis=-1)
    mn = np.concatenate([m & 0x3F, (m_d >> 4) | ((m >> 2) & 0x30)], axis=-1)
    return sc.reshape(n, 8), mn.reshape(n, 8)


def _dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    # gguf_dequant_torch.py:118-122
    d, x = _split(blocks, 2)
    return _f16(d) * np.ascontiguousarray(x).view(np.int8).astype(np.float32)


def _dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    # gguf_dequant_torch.py:187-203
    n = blocks.shape[0]
    d, dmin, scales, qs = _split(blocks, 2, 2, K_SCALE_SIZE)
    d, dmin = _f16(d), _f16(dmin)
    sc, m = get_scale_min(scales)
    dd = (d * sc.astype(np.float32)).reshape(n, 8, 1)
    dm = (dmin * m.astype(np.float32)).reshape(n, 8, 1)
    q = qs.reshape(n, 4, 1, 32) >> np.array([0, 4], dtype=np.uint8).reshape(1, 1, 2, 1)
    q = (q & 0x0F).reshape(n, 8, 32).astype(np.float32)
    return (dd * q - dm).reshape(n, QK_K)


def _dequant_q5_k(blocks: np.ndarray) -> np.ndarray:
    # gguf_dequant_torch.py:206-227
    n = blocks.shape[0]
    d, dmin, scales, qh, qs = _split(blocks, 2, 2, K_SCALE_SIZE, QK_K // 8)
    d, dmin = _f16(d), _f16(dmin)
    sc, m = get_scale_min(scales)
    dd = (d * sc.astype(np.float32)).reshape(n, 8, 1)
    dm = (dmin * m.astype(np.float32)).reshape(n, 8, 1)
    ql = qs.reshape(n, 4, 1, 32) >> np.array([0, 4], dtype=np.uint8).reshape(1, 1, 2, 1)
    qh = qh.reshape(n, 1, 1, 32) >> np.arange(8, dtype=np.uint8).reshape(1, 1, 8, 1)
    ql = (ql & 0x0F).reshape(n, 8, 32)
    qh = (qh & 0x01).reshape(n, 8, 32)
    q = (ql | (qh << 4)).astype(np.float32)
    return (dd * q - dm).reshape(n, QK_K)


def _dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    # gguf_dequant_torch.py:230-249
    n = blocks.shape[0]
    ql, qh, scales, d = _split(blocks, QK_K // 2, QK_K // 4, QK_K // 16)
    sc = np.ascontiguousarray(scales).view(np.int8).astype(np.float32)
    dd = (_f16(d) * sc).reshape(n, QK_K // 16, 1)
    ql = ql.reshape(n, 2, 1, 64) >> np.array([0, 4], dtype=np.uint8).reshape(1, 1, 2, 1)
    ql = (ql & 0x0F).reshape(n, 8, 32)
    qh = qh.reshape(n, 2, 1, 32) >> np.array([0, 2, 4, 6], dtype=np.uint8).reshape(1, 1, 4, 1)
    qh = (qh & 0x03).reshape(n, 8, 32)
    q = (ql | (qh << 4)).astype(np.int8) - np.int8(32)
    q = q.reshape(n, QK_K // 16, 16).astype(np.float32)
    return (dd * q).reshape(n, QK_K)


_DEQUANT = {
    GGML_Q8_0: _dequant_q8_0,
    GGML_Q4_K: _dequant_q4_k,
    GGML_Q5_K: _dequant_q5_k,
    GGML_Q6_K: _dequant_q6_k,
}


def ref_matvec(weight_bytes, x: np.ndarray, ggml_type: int, N: int, K: int) -> np.ndarray:
    """fp32 dequant then fp32 matvec, the reference's check form
    (``tests/test_ggml_ops.py:57-64``): y = x[1,K] @ W[N,K]^T."""
    w = dequant_tensor(weight_bytes, ggml_type, (N, K))
    xf = np.asarray(x, dtype=np.float32).reshape(1, K)
    return (xf @ w.T).reshape(N)
