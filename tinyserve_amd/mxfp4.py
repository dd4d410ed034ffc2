"""MXFP4 (e2m1 values, e8m0 block-32 scales) on the HIP library.

The names of tinyserve/mxfp4.py:5-53 (``FP4_LUT``, ``get_lut``,
``dequant_mxfp4_no_transpose(..., out=None)``, ``dequant_mxfp4``) and the vecmat of
tinyserve/_model_hooks.py:105-116 (``mxfp4_linear``, the ``_mxfp4_linear`` backend):
blocks ``[N, G, 16]`` uint8 (byte j holds element 2j in its low nibble) and scales
``[N, G]`` uint8, value = FP4_LUT[nibble] * 2**(scale - 127). The dequantisation runs as
one kernel, bit-exact against the reference's lookup + ldexp; device tensors only.
"""
from __future__ import annotations

import torch

from . import ops

# The 16 e2m1 code values in code order (the sign is bit 3), as a bfloat16 CPU tensor.
FP4_LUT = torch.tensor([+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                       dtype=torch.bfloat16)
FP4_VALUES = FP4_LUT.tolist()

_luts: dict[tuple, torch.Tensor] = {}


def get_lut(dtype: torch.dtype, device) -> torch.Tensor:
    """FP4_LUT as `dtype` on `device` (one cached copy per pair)."""
    key = (dtype, torch.device(device))
    lut = _luts.get(key)
    if lut is None:
        lut = _luts[key] = FP4_LUT.to(dtype=dtype, device=key[1])
    return lut


def dequant_mxfp4_no_transpose(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16,
                               out: torch.Tensor | None = None) -> torch.Tensor:
    """[N, G, 16] + [N, G] -> [N, 32 G] (the F.linear weight layout). With `out` (a contiguous
    tensor of N * 32 G elements of `dtype`, any shape) the values are written into it and
    the returned tensor is a [N, 32 G] view of it."""
    return ops.mxfp4_dequant(blocks, scales, dtype=dtype, transpose=False, out=out)


def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[N, G, 16] + [N, G] -> [32 G, N] (transposed, as the reference returns it)."""
    return ops.mxfp4_dequant(blocks, scales, dtype=dtype, transpose=True)


def mxfp4_linear(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor,
                 bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., K] @ deq(W)^T + bias -> [..., N] in x's dtype, fused (no dequantised weight)."""
    return ops.mxfp4_matvec(x, blocks, scales, bias)
