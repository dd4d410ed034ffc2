"""Packed-expert slot layout: named tensors at fixed byte offsets of one flat buffer.

``TensorLayout`` keeps the contract of the reference's class of the same name
(tinyserve/expert_store.py:57-77): offsets are assigned in the insertion order of
``tensor_specs``; ``sizes`` are element count times element size; ``total_bytes`` is
the slot size. The resident slot pool (``ExpertCache``) stores experts in exactly this
layout. MXFP4 checkpoints can be kept in their checkpoint order or repacked once, at
load time, into the 16-row MFMA tile order the fast decode and prefill kernels read
(``ExpertStore.from_safetensors(..., tiled=True)``); GGUF experts keep their ggml bytes.
"""
from __future__ import annotations

import itertools
import math

import torch


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


class TensorLayout:
    """Byte map of one packed expert slot: each named tensor's (offset, size) in the slot,
    tensors placed back to back in the order of ``tensor_specs``."""

    def __init__(self, tensor_specs: dict[str, tuple[tuple[int, ...], torch.dtype]]):
        self.specs = tensor_specs
        names = list(tensor_specs)
        sizes = [math.prod(int(d) for d in shape) * _element_size(dtype) for shape, dtype in tensor_specs.values()]
        self.sizes: dict[str, int] = dict(zip(names, sizes))
        self.offsets: dict[str, int] = dict(zip(names, itertools.accumulate([0] + sizes[:-1])))
        self.total_bytes = sum(sizes)

    @staticmethod
    def from_tensors(tensors: dict[str, torch.Tensor]) -> "TensorLayout":
        """The layout that packs these tensors (their shapes and dtypes, in dict order)."""
        specs = {}
        for name, t in tensors.items():
            specs[name] = (tuple(t.shape), t.dtype)
        return TensorLayout(specs)


def pack_tensors(dest: torch.Tensor, layout: TensorLayout, tensors: dict[str, torch.Tensor]) -> None:
    """Copy each tensor's raw bytes to its offset in ``dest`` (uint8, >= total_bytes)."""
    for name, t in tensors.items():
        off, nb = layout.offsets[name], layout.sizes[name]
        dest[off : off + nb].copy_(t.contiguous().reshape(-1).view(torch.uint8))


def mxfp4_tiled_specs(specs: dict) -> dict:
    """The slot specs with both MXFP4 matrices in the 16-row MFMA tile order (mx_tiles): the
    blocks keep their shape and size, each scale tensor becomes [rows / 16, tile-scale bytes];
    the key order is kept. Raises ValueError for specs without MXFP4 blocks and scales or
    with shapes the tile order cannot hold (rows % 16, columns % 32)."""
    from .mx_tiles import tile_sizes

    out = dict(specs)
    for mat in ("gate_up_proj", "down_proj"):
        if mat not in specs or mat + "_scales" not in specs:
            raise ValueError(f"tiled slots need MXFP4 {mat} blocks and scales (found {sorted(specs)})")
        shape, dtype = specs[mat]
        if len(shape) != 3 or shape[2] != 16 or dtype != torch.uint8:
            raise ValueError(f"{mat}: MXFP4 blocks must be uint8 [rows, K / 32, 16] (got {shape}, {dtype})")
        N, G, _ = shape
        _, sb = tile_sizes(N, 32 * G)
        out[mat + "_scales"] = ((N // 16, sb // (N // 16)), torch.uint8)
    return out


class ExpertBuffer:
    """One expert's packed bytes on a device (tinyserve/expert_store.py:84-112)."""

    def __init__(self, layout: TensorLayout, device: torch.device | str):
        self.layout = layout
        self.packed = torch.empty(layout.total_bytes, dtype=torch.uint8, device=device)

    def get_tensor(self, name: str) -> torch.Tensor:
        shape, dtype = self.layout.specs[name]
        off, nb = self.layout.offsets[name], self.layout.sizes[name]
        return self.packed[off : off + nb].view(dtype).view(shape)


class ExpertStore:
    """Every MoE layer's experts as packed slots in host memory, ``_data`` [layers, experts,
    expert_bytes] (tinyserve/expert_store.py:115-130: same attributes; the reference's
    INT4 cache, FP8 and disk-offload options are out of scope here)."""

    def __init__(self, data: torch.Tensor, layout: TensorLayout, num_layers: int, num_experts: int,
                 layer_indices: list[int] | None = None, tiled: bool = False):
        self._data = data
        self.layout = layout
        self._bf16_layout = layout
        self.num_layers = num_layers
        self.num_experts = num_experts
        self.expert_bytes = layout.total_bytes
        self.buffer_expert_bytes = layout.total_bytes
        self.layer_indices = list(layer_indices) if layer_indices is not None else list(range(num_layers))
        self.tiled = tiled

    @classmethod
    def from_safetensors(cls, model_dir: str, moe_block_attr: str = "mlp", expert_list_attr: str = "experts",
                         layer_indices: list[int] | None = None, tiled: bool = False) -> tuple["ExpertStore", int]:
        """Expert tensors straight from a local safetensors checkpoint
        (tinyserve/expert_store.py:290-400): keys ``*.layers.<i>.<moe_block_attr>.<expert_list_attr>.<name>``
        with a leading expert dimension; a ``_blocks`` suffix is dropped (``gate_up_proj_blocks``
        -> ``gate_up_proj``, so MXFP4 checkpoints give ``gate_up_proj`` / ``gate_up_proj_scales``
        / ``gate_up_proj_bias`` / ``down_proj`` ...), and the slot keeps the checkpoint's key
        order. ``tiled``: MXFP4 matrices are stored in the 16-row MFMA tile order of the fast
        decode instead (mx_tiles.tile_mxfp4; their scale tensors become the tile-scale areas).
        Returns (store, num_experts)."""
        import json
        import os
        import re

        from safetensors import safe_open

        index = os.path.join(model_dir, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                shards = sorted(set(json.load(f)["weight_map"].values()))
        else:
            shards = sorted(f for f in os.listdir(model_dir) if f.endswith(".safetensors"))
        prefix = f"{moe_block_attr}.{expert_list_attr}."
        pat = re.compile(r"layers\.(\d+)\." + re.escape(prefix) + r"(.+)$")
        layer_tensors: dict[int, dict[str, torch.Tensor]] = {}
        for shard in shards:
            with safe_open(os.path.join(model_dir, shard), framework="pt", device="cpu") as f:
                for key in f.keys():
                    m = pat.search(key)
                    if m is None:
                        continue
                    li = int(m.group(1))
                    if layer_indices is not None and li not in layer_indices:
                        continue
                    layer_tensors.setdefault(li, {})[re.sub(r"_blocks$", "", m.group(2))] = f.get_tensor(key)
        layers = sorted(layer_tensors) if layer_indices is None else [li for li in layer_indices if li in layer_tensors]
        if not layers:
            raise ValueError(f"No expert tensors found in {model_dir} (pattern *.layers.<i>.{prefix}*)")
        first = layer_tensors[layers[0]]
        num_experts = int(next(iter(first.values())).shape[0])
        specs = {n: (tuple(t.shape[1:]), t.dtype) for n, t in first.items()}
        if tiled:
            specs = mxfp4_tiled_specs(specs)
        layout = TensorLayout(specs)
        data = torch.empty((len(layers), num_experts, layout.total_bytes), dtype=torch.uint8,
                           pin_memory=torch.cuda.is_available())
        host = data.numpy()
        for si, li in enumerate(layers):
            tensors = layer_tensors[li]
            if set(tensors) != set(specs):
                raise ValueError(f"layer {li}: expert tensors {sorted(tensors)} differ from {sorted(specs)}")
            for e in range(num_experts):
                parts = {n: t[e].contiguous() for n, t in tensors.items()}
                if tiled:
                    from .mx_tiles import tile_mxfp4

                    for mat in ("gate_up_proj", "down_proj"):
                        tb, ts = tile_mxfp4(parts[mat].numpy(), parts[mat + "_scales"].numpy())
                        parts[mat] = torch.from_numpy(tb)
                        parts[mat + "_scales"] = torch.from_numpy(ts)
                for n, t in parts.items():
                    off, nb = layout.offsets[n], layout.sizes[n]
                    host[si, e, off : off + nb] = t.reshape(-1).view(torch.uint8).numpy()
            del layer_tensors[li]
        return cls(data, layout, len(layers), num_experts, layers, tiled), num_experts

    def get_expert_data(self, layer_idx: int, expert_idx: int) -> torch.Tensor:
        """Packed bytes of expert ``expert_idx`` of store layer ``layer_idx`` (CPU)."""
        return self._data[layer_idx, expert_idx]

    def allocate_buffer(self, device: torch.device | str) -> ExpertBuffer:
        return ExpertBuffer(self.layout, device)

    def copy_to_buffer(self, buf: ExpertBuffer, layer_idx: int, expert_idx: int, non_blocking: bool = False) -> None:
        buf.packed.copy_(self._data[layer_idx, expert_idx], non_blocking=non_blocking)

    def copy_to_buffer_slot(self, cache, slot: int, layer_idx: int, expert_idx: int) -> None:
        """Copy into row ``slot`` of a slot pool (an object with ``_packed`` [slots, bytes], or the tensor)."""
        getattr(cache, "_packed", cache)[slot].copy_(self._data[layer_idx, expert_idx])

    def load_layer(self, layer_idx: int, device: torch.device | str = "cuda") -> torch.Tensor:
        """All experts of store layer ``layer_idx`` as a [num_experts, expert_bytes] pool (expert e in slot e)."""
        return self._data[layer_idx].to(device)

    def expert_layout(self, act_fn=None):
        """The kernels' tsa_expert_layout of these slots (MXFP4 checkpoints)."""
        from .expert_forward import mxfp4_expert_layout

        return mxfp4_expert_layout(self.layout, act_fn, self.expert_bytes, tiled=self.tiled)
