"""``torch.ops.tinyserve_ggml.ggml_mul_mat_vec`` on the HIP library.

Same schema, semantics and error texts as the reference op
(tinyserve/csrc/ggml_ops.cu:461-574): ``ggml_mul_mat_vec(Tensor activation, Tensor
weight_data, int ggml_type, int out_features, int in_features) -> Tensor`` multiplies
the first ``in_features`` elements of the flattened activation by the GGUF matrix in
``weight_data`` (which may be larger than needed: padded slots) and returns ``[1,
out_features]`` in the activation's dtype, on the current stream. It is computed by
``tsa_gguf_matvec``; there is no CPU path.

``register()`` defines the op once per process (skipped if another library already
defined ``tinyserve_ggml::ggml_mul_mat_vec``), so ``GGMLLinear`` / ``GGMLExpertForward``
and any caller of the reference op find it under the same name.
"""
from __future__ import annotations

import torch

from . import _lib, ops

_LIB = None
SCHEMA = "ggml_mul_mat_vec(Tensor activation, Tensor weight_data, int ggml_type, int out_features, int in_features) -> Tensor"


def ggml_mul_mat_vec(activation: torch.Tensor, weight_data: torch.Tensor, ggml_type: int, out_features: int,
                     in_features: int) -> torch.Tensor:
    if not activation.is_cuda:
        raise RuntimeError("activation must be on CUDA")
    if not weight_data.is_cuda:
        raise RuntimeError("weight_data must be on CUDA")
    if weight_data.dtype != torch.uint8:
        raise RuntimeError("weight_data must be uint8")
    be, ts = ops.gguf_block_info(int(ggml_type))  # raises "Unsupported ggml_type: ..."
    if in_features % be:
        raise RuntimeError(f"in_features ({in_features}) must be divisible by block_elements ({be})")
    expected = out_features * (in_features // be) * ts
    if weight_data.numel() < expected:
        raise RuntimeError(f"weight_data too small: got {weight_data.numel()} bytes, expected {expected}")
    x = activation.reshape(-1)
    if x.numel() < in_features:
        raise RuntimeError(f"activation too small: got {x.numel()} elements, expected {in_features}")
    y = ops.gguf_matvec(x[:in_features].reshape(1, in_features), weight_data, int(ggml_type), int(out_features),
                        int(in_features), out_dtype=activation.dtype)
    return y.reshape(1, out_features)


def register() -> bool:
    """Define ``torch.ops.tinyserve_ggml.ggml_mul_mat_vec`` (idempotent). Returns True
    when the op is available afterwards."""
    global _LIB
    if _LIB is not None:
        return True
    if hasattr(torch.ops, "tinyserve_ggml") and hasattr(torch.ops.tinyserve_ggml, "ggml_mul_mat_vec"):
        return True
    _lib.load()  # fail loudly here if the HIP library is missing
    lib = torch.library.Library("tinyserve_ggml", "DEF")
    lib.define(SCHEMA)
    lib.impl("ggml_mul_mat_vec", ggml_mul_mat_vec, "CompositeExplicitAutograd")
    _LIB = lib
    return True
