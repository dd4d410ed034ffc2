"""Shared test helpers: tolerance checks and host<->device conversions."""
from __future__ import annotations

import numpy as np
import torch

# Output bar for float results (after the GPU result is rounded to bf16):
# cosine >= 0.9999 and max|gpu - ref| / max|ref| <= 1e-2.
COS_MIN = 0.9999
REL_MAX = 1e-2

def to_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def metrics(gpu: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    g = np.asarray(gpu, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    denom = np.linalg.norm(g) * np.linalg.norm(r)
    cos = float(g @ r / denom) if denom > 0 else float(np.array_equal(g, r))
    rel = float(np.abs(g - r).max() / max(np.abs(r).max(), 1e-30))
    return cos, rel


def assert_close_bf16(gpu: torch.Tensor | np.ndarray, ref: np.ndarray, what: str = "") -> None:
    if isinstance(gpu, torch.Tensor):
        gpu = to_f32(gpu.to(torch.bfloat16))
    cos, rel = metrics(gpu, ref)
    assert cos >= COS_MIN and rel <= REL_MAX, f"{what}: cosine {cos:.7f} (>= {COS_MIN}), max rel err {rel:.3e} (<= {REL_MAX})"


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit equality of float arrays, with NaNs equal to NaNs."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def dev_u8(arr: np.ndarray, offset: int = 0, device: str = "cuda") -> torch.Tensor:
    """Upload bytes; with offset > 0 the returned view starts `offset` bytes into a larger
    allocation (an unaligned base pointer)."""
    arr = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    buf = torch.zeros(arr.size + offset, dtype=torch.uint8)
    buf[offset:] = torch.from_numpy(arr.copy())
    return buf.to(device)[offset:]


def bf16_dev(bits: np.ndarray, device: str = "cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16).to(device)


DECODE_SYNC_BYTES = 32 << 10  # the decode workspace's leading sync area


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """OCP fp8 e4m3 (bias 7, no infinities, 0x7F / 0xFF NaN) -> float32, exact."""
    c = np.asarray(codes, dtype=np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e, m = (c >> 3) & 15, c & 7
    v = sign * np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    v[(c & 0x7F) == 0x7F] = np.nan
    return v.astype(np.float32)


def tiled_h(ws: torch.Tensor, pairs: int, inter: int, one_launch: bool = False) -> np.ndarray:
    """The intermediate h [pairs, inter] the tiled decode wrote to its workspace (right after
    the sync area), as float32. Two launches: bf16 [pairs][inter]. One launch: per pair the
    down dot's operands, hi and lo fp8 terms [inter] each and the A-scale table (block b's
    e8m0 byte at 4 (4 (b / 16) + b % 4) + (b % 16) / 4), padded to 256 bytes."""
    o = DECODE_SYNC_BYTES
    if not one_launch:
        raw = ws[o : o + pairs * 2 * inter].cpu().numpy().view(np.uint16).reshape(pairs, inter)
        return (raw.astype(np.uint32) << 16).view(np.float32)
    pb = (2 * inter + 96 + 255) // 256 * 256
    raw = ws[o : o + pairs * pb].cpu().numpy().view(np.uint8).reshape(pairs, pb)
    b = np.arange(inter // 32)
    tb = 4 * (4 * (b // 16) + b % 4) + (b % 16) // 4
    scale = np.exp2(raw[:, 2 * inter + tb].astype(np.float64) - 127.0)  # [pairs, blocks]
    v = e4m3_to_f32(raw[:, :inter]).astype(np.float64) + e4m3_to_f32(raw[:, inter : 2 * inter])
    return (v * np.repeat(scale, 32, axis=1)).astype(np.float32)
