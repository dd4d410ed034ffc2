"""torch (CPU) restatement of the reference's dequantise-then-matmul path, used only as the
timed CPU baseline of bench.py (test infrastructure; never imported by the library).

Follows the same reference functions as the numpy oracle, in torch as the reference
runs them on the CPU: ``tinyserve/gguf_dequant_torch.py`` (whole-tensor vectorised block
decode for Q8_0 / Q4_K / Q5_K / Q6_K) and ``tinyserve/mxfp4.py:20-44`` (LUT lookup, then
ldexp by the e8m0 scale), followed by float32 matmuls in the form of
``tests/test_ggml_ops.py:57-64`` and the expert FFN of ``tinyserve/expert_forward.py``.
``tests/test_oracle_torch.py`` pins every function here bit-for-bit to the numpy oracle
(which the golden vectors pin to the reference).
"""
from __future__ import annotations

import numpy as np
import torch

from . import gguf as _gguf

QK_K = 256
_LUT = torch.tensor([+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                    dtype=torch.float32)


def as_u8(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy())


def _f16(col: torch.Tensor) -> torch.Tensor:
    return col.contiguous().view(torch.float16).float()


def _split(blocks: torch.Tensor, *sizes: int) -> list[torch.Tensor]:
    out, off = [], 0
    for s in sizes:
        out.append(blocks[:, off : off + s])
        off += s
    out.append(blocks[:, off:])
    return out


def _scale_min(scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    n = scales.shape[0]
    s = scales.reshape(n, 3, 4)
    d, m, m_d = s[:, 0, :], s[:, 1, :], s[:, 2, :]
    sc = torch.cat([d & 0x3F, (m_d & 0x0F) | ((d >> 2) & 0x30)], dim=-1)
    mn = torch.cat([m & 0x3F, (m_d >> 4) | ((m >> 2) & 0x30)], dim=-1)
    return sc, mn


def _q8_0(b: torch.Tensor) -> torch.Tensor:
    d, x = _split(b, 2)
    return _f16(d) * x.contiguous().view(torch.int8).float()


def _q4_k(b: torch.Tensor) -> torch.Tensor:
    n = b.shape[0]
    d, dmin, scales, qs = _split(b, 2, 2, 12)
    sc, m = _scale_min(scales)
    dd = (_f16(d) * sc.float()).reshape(n, 8, 1)
    dm = (_f16(dmin) * m.float()).reshape(n, 8, 1)
    q = qs.reshape(n, 4, 1, 32) >> torch.tensor([0, 4], dtype=torch.uint8).reshape(1, 1, 2, 1)
    q = (q & 0x0F).reshape(n, 8, 32).float()
    return (dd * q - dm).reshape(n, QK_K)


def _q5_k(b: torch.Tensor) -> torch.Tensor:
    n = b.shape[0]
    d, dmin, scales, qh, qs = _split(b, 2, 2, 12, QK_K // 8)
    sc, m = _scale_min(scales)
    dd = (_f16(d) * sc.float()).reshape(n, 8, 1)
    dm = (_f16(dmin) * m.float()).reshape(n, 8, 1)
    ql = qs.reshape(n, 4, 1, 32) >> torch.tensor([0, 4], dtype=torch.uint8).reshape(1, 1, 2, 1)
    qh = qh.reshape(n, 1, 1, 32) >> torch.arange(8, dtype=torch.uint8).reshape(1, 1, 8, 1)
    q = ((ql & 0x0F).reshape(n, 8, 32) | ((qh & 0x01).reshape(n, 8, 32) << 4)).float()
    return (dd * q - dm).reshape(n, QK_K)


def _q6_k(b: torch.Tensor) -> torch.Tensor:
    n = b.shape[0]
    ql, qh, scales, d = _split(b, QK_K // 2, QK_K // 4, QK_K // 16)
    dd = (_f16(d) * scales.contiguous().view(torch.int8).float()).reshape(n, QK_K // 16, 1)
    ql = ql.reshape(n, 2, 1, 64) >> torch.tensor([0, 4], dtype=torch.uint8).reshape(1, 1, 2, 1)
    qh = qh.reshape(n, 2, 1, 32) >> torch.tensor([0, 2, 4, 6], dtype=torch.uint8).reshape(1, 1, 4, 1)
    q = ((ql & 0x0F).reshape(n, 8, 32) | ((qh & 0x03).reshape(n, 8, 32) << 4)).to(torch.int16) - 32
    return (dd * q.reshape(n, QK_K // 16, 16).float()).reshape(n, QK_K)


_DEQUANT = {_gguf.GGML_Q8_0: _q8_0, _gguf.GGML_Q4_K: _q4_k, _gguf.GGML_Q5_K: _q5_k, _gguf.GGML_Q6_K: _q6_k}


def gguf_dequant(data: torch.Tensor, ggml_type: int, shape) -> torch.Tensor:
    """uint8 GGUF bytes -> float32 ``shape`` (whole tensor at once)."""
    be, ts = _gguf.QUANT_SIZES[ggml_type]
    n = data.numel() // ts
    return _DEQUANT[ggml_type](data[: n * ts].reshape(n, ts)).reshape(shape)


def mxfp4_dequant(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """[N, G, 16] uint8 + [N, G] uint8 -> float32 [N, 32 G]: LUT[nibble] * 2**(scale - 127)."""
    N, G, B = blocks.shape
    lo, hi = _LUT[(blocks & 0x0F).long()], _LUT[(blocks >> 4).long()]
    vals = torch.stack([lo, hi], dim=-1).reshape(N, G, 2 * B)
    return torch.ldexp(vals, scales.to(torch.int32).unsqueeze(-1) - 127).reshape(N, G * 2 * B)


def gptoss_swiglu(gu: torch.Tensor, limit: float = 7.0, alpha: float = 1.702) -> torch.Tensor:
    g = gu[..., 0::2].clamp(max=limit)
    u = gu[..., 1::2].clamp(min=-limit, max=limit)
    return (u + 1.0) * g * torch.sigmoid(alpha * g)


def mxfp4_expert_weights(e: dict) -> tuple[torch.Tensor, torch.Tensor]:
    return (mxfp4_dequant(e["gate_up_blocks"], e["gate_up_scales"]), mxfp4_dequant(e["down_blocks"], e["down_scales"]))


def mxfp4_expert_ffn(x: torch.Tensor, wgu: torch.Tensor, wdn: torch.Tensor, bgu=None, bdn=None) -> torch.Tensor:
    gu = x @ wgu.T
    if bgu is not None:
        gu = gu + bgu
    y = gptoss_swiglu(gu) @ wdn.T
    return y + bdn if bdn is not None else y


def gguf_expert_weights(e: dict) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    H, I = e["hidden"], e["inter"]
    return (gguf_dequant(e["gate"], e["gate_type"], (I, H)), gguf_dequant(e["up"], e["up_type"], (I, H)),
            gguf_dequant(e["down"], e["down_type"], (H, I)))


def gguf_expert_ffn(x: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    return (torch.nn.functional.silu(x @ wg.T) * (x @ wu.T)) @ wd.T


def torch_expert(e: dict) -> dict:
    """An expert dict (synth's numpy form) with its byte arrays as torch uint8 tensors."""
    out = dict(e)
    for k in ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales"):
        if k in e:
            out[k] = torch.from_numpy(np.ascontiguousarray(e[k]))
    for k in ("gate", "up", "down"):
        if k in e:
            out[k] = as_u8(e[k])
    for k in ("gate_up_bias", "down_bias"):
        if e.get(k) is not None:
            out[k] = torch.from_numpy(np.asarray(e[k], dtype=np.float32))
    return out
