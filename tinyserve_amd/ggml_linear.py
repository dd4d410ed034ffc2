"""``GGMLLinear``: nn.Linear over raw GGUF quantised weights, on the HIP matvec.

Mirrors tinyserve/ggml_linear.py:20-173 (``_check_ggml``, ``GGMLLinear``,
``replace_linear_with_ggml``) with the same constructor and forward contract. Every
batch size goes through ``tsa_gguf_matvec`` (one launch handles all tokens; the
reference loops one op call per token for batch > 1, :86-100) and there is no CPU
fallback: without the HIP library the constructor's first forward raises.
"""
from __future__ import annotations

import logging

import torch
import torch.nn as nn

from . import _lib, ops

logger = logging.getLogger(__name__)

_HAS_GGML: bool | None = None


def _check_ggml() -> bool:
    """True when the HIP library loads and ``torch.ops.tinyserve_ggml`` is registered."""
    global _HAS_GGML
    if _HAS_GGML is None:
        from . import ggml_ops

        try:
            _HAS_GGML = ggml_ops.register()
        except (OSError, RuntimeError) as exc:
            logger.error("tinyserve_amd HIP library unavailable: %s", exc)
            _HAS_GGML = False
    return _HAS_GGML


class GGMLLinear(nn.Module):
    """An ``nn.Linear`` stand-in whose weight stays in its GGUF encoding (Q8_0 / Q4_K / Q5_K /
    Q6_K bytes) on the GPU; every forward runs the HIP GGUF matvec on it."""

    def __init__(self, raw_bytes: bytes | torch.Tensor, ggml_type: int, out_features: int, in_features: int,
                 bias: torch.Tensor | None = None, device: torch.device | str = "cuda"):
        super().__init__()
        data = raw_bytes if isinstance(raw_bytes, torch.Tensor) else torch.tensor(bytearray(raw_bytes), dtype=torch.uint8)
        self._qweight = data.reshape(-1).to(device=device)
        self._ggml_type = int(ggml_type)
        self.out_features, self.in_features = int(out_features), int(in_features)
        self.bias = None if bias is None else nn.Parameter(bias.to(device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not _check_ggml():
            raise RuntimeError("GGMLLinear needs the tinyserve_amd HIP library (build it with __graft_entry__.build())")
        lead = x.shape[:-1]
        out = ops.gguf_matvec(x.reshape(-1, self.in_features), self._qweight, self._ggml_type, self.out_features,
                              self.in_features, out_dtype=x.dtype)
        if self.bias is not None:
            out = out + self.bias
        return out.reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        names = {8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"ggml_type={names.get(self._ggml_type, '?')}, qweight={self._qweight.shape[0]} bytes, "
                f"bias={self.bias is not None}")


def replace_linear_with_ggml(model: nn.Module, raw_weights: dict[str, tuple[bytes, int, tuple[int, int]]],
                             device: torch.device | str = "cuda") -> int:
    """Replace ``nn.Linear`` modules named in ``raw_weights`` (path -> (bytes, ggml_type,
    (out_features, in_features))) by ``GGMLLinear``; returns the number replaced. Paths that
    do not resolve to an ``nn.Linear`` are skipped; meta-device biases are dropped."""
    replaced = 0
    for name, (raw, ggml_type, shape) in raw_weights.items():
        parent_path, _, attr = name.rpartition(".")
        parent = model
        for p in parent_path.split(".") if parent_path else []:
            parent = getattr(parent, p, None)
            if parent is None:
                break
        if parent is None:
            continue
        old = getattr(parent, attr, None)
        if not isinstance(old, nn.Linear):
            continue
        bias = old.bias
        if bias is not None and bias.device.type == "meta":
            bias = None
        setattr(parent, attr, GGMLLinear(raw, ggml_type, shape[0], shape[1], bias=bias, device=device))
        replaced += 1
    logger.info("GGMLLinear now backs %d linear layer(s)", replaced)
    return replaced
