"""Packed-expert slot layout: named tensors at fixed byte offsets of one flat buffer.

``TensorLayout`` keeps the contract of the reference's class of the same name
(tinyserve/expert_store.py:57-77): offsets are assigned in the insertion order of
``tensor_specs``; ``sizes`` are element count times element size; ``total_bytes`` is
the slot size. The resident slot pool (``ExpertCache``) stores experts in exactly
this layout, in the weights' native formats (no repacking).
"""
from __future__ import annotations

import torch


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


class TensorLayout:
    """Describes how named tensors are packed into a flat byte buffer."""

    def __init__(self, tensor_specs: dict[str, tuple[tuple[int, ...], torch.dtype]]):
        self.specs = tensor_specs
        self.offsets: dict[str, int] = {}
        self.sizes: dict[str, int] = {}
        offset = 0
        for name, (shape, dtype) in tensor_specs.items():
            n = 1
            for d in shape:
                n *= int(d)
            nbytes = n * _element_size(dtype)
            self.offsets[name] = offset
            self.sizes[name] = nbytes
            offset += nbytes
        self.total_bytes = offset

    @staticmethod
    def from_tensors(tensors: dict[str, torch.Tensor]) -> "TensorLayout":
        return TensorLayout({name: (tuple(t.shape), t.dtype) for name, t in tensors.items()})


def pack_tensors(dest: torch.Tensor, layout: TensorLayout, tensors: dict[str, torch.Tensor]) -> None:
    """Copy each tensor's raw bytes to its offset in ``dest`` (uint8, >= total_bytes)."""
    for name, t in tensors.items():
        off, nb = layout.offsets[name], layout.sizes[name]
        dest[off : off + nb].copy_(t.contiguous().reshape(-1).view(torch.uint8))


class ExpertBuffer:
    """One expert's packed bytes on a device (tinyserve/expert_store.py:84-112)."""

    def __init__(self, layout: TensorLayout, device: torch.device | str):
        self.layout = layout
        self.packed = torch.empty(layout.total_bytes, dtype=torch.uint8, device=device)

    def get_tensor(self, name: str) -> torch.Tensor:
        shape, dtype = self.layout.specs[name]
        off, nb = self.layout.offsets[name], self.layout.sizes[name]
        return self.packed[off : off + nb].view(dtype).view(shape)
