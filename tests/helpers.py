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


def tiled_h(ws: torch.Tensor, pairs: int, inter: int) -> np.ndarray:
    """The intermediate h [pairs, inter] (bf16) the tiled decode wrote at the start of its
    workspace, as float32."""
    raw = ws[: pairs * 2 * inter].cpu().numpy().view(np.uint16).reshape(pairs, inter)
    return (raw.astype(np.uint32) << 16).view(np.float32)
