"""MXFP4 (e2m1 values, e8m0 block-32 scales) on the HIP library.

Same functions as tinyserve/mxfp4.py:5-53 (``FP4_VALUES``, ``dequant_mxfp4_no_transpose``,
``dequant_mxfp4``) and the vecmat of tinyserve/_model_hooks.py:105-116
(``mxfp4_linear``, the ``_mxfp4_linear`` backend): blocks ``[N, G, 16]`` uint8 (byte j
holds element 2j in its low nibble) and scales ``[N, G]`` uint8, value =
LUT[nibble] * 2**(scale - 127), computed bit-exactly on the GPU. Device tensors only.
"""
from __future__ import annotations

import torch

from . import ops

FP4_VALUES = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def dequant_mxfp4_no_transpose(blocks: torch.Tensor, scales: torch.Tensor,
                               dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[N, G, 16] + [N, G] -> [N, 32 G] (the Linear weight layout)."""
    return ops.mxfp4_dequant(blocks, scales, dtype=dtype, transpose=False)


def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[N, G, 16] + [N, G] -> [32 G, N] (transposed, as the reference returns it)."""
    return ops.mxfp4_dequant(blocks, scales, dtype=dtype, transpose=True)


def mxfp4_linear(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor,
                 bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., K] @ deq(W)^T + bias -> [..., N] in x's dtype, fused (no dequantised weight)."""
    return ops.mxfp4_matvec(x, blocks, scales, bias)
