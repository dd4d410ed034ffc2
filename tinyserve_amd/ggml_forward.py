"""``GGMLExpertForward``: one GGUF expert (gate ‖ up ‖ down raw bytes) on the HIP library.

Mirrors tinyserve/ggml_forward.py:27-151: same constructor (``layout``, ``ggml_types``,
``act_fn``, ``proj_shapes`` in ggml (ne0 = in, ne1 = out) order), same
``forward(packed, h, layer_idx=-1)``, the per-layer type override
(``_layer_ggml_types``, :79-81) and the "actual bytes" of a padded slot (:94-101).
With gate and up in one type (the usual case) the whole FFN is one fused
``tsa_moe_decode`` over a one-slot pool, for any batch size; mixed gate/up types fall
back to three ``tsa_gguf_matvec`` launches and a torch SiLU product on the GPU. There
is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib, ops
from .expert_forward import _is_silu
from .expert_store import TensorLayout

_BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def _check_ggml() -> bool:
    from .ggml_linear import _check_ggml as check

    return check()


class GGMLExpertForward:
    def __init__(self, layout: TensorLayout, ggml_types: dict[str, int], act_fn, proj_shapes: dict[str, tuple[int, int]]):
        self._ggml_types = ggml_types
        self._act_fn = act_fn
        self._proj_shapes = proj_shapes
        self._gate_off = layout.offsets["gate"]
        self._up_off = layout.offsets["up"]
        self._down_off = layout.offsets["down"]
        self._has_ggml = _check_ggml()
        self._silu = _is_silu(act_fn)
        self._layouts: dict[tuple, _lib.ExpertLayout] = {}
        self._ones: dict[tuple, tuple[torch.Tensor, torch.Tensor]] = {}

    @staticmethod
    def _actual_bytes(shape: tuple[int, int], t: int) -> int:
        be, ts = _BLOCK[t]
        return shape[0] * shape[1] // be * ts

    def _layout(self, types: dict[str, int], slot_bytes: int) -> _lib.ExpertLayout:
        key = (types["gate"], types["up"], types["down"], slot_bytes)
        L = self._layouts.get(key)
        if L is None:
            H, I = self._proj_shapes["gate"]
            L = _lib.ExpertLayout()
            L.format, L.act = _lib.EXPERT_GGUF, _lib.ACT_SILU
            L.hidden, L.inter, L.slot_bytes = H, I, slot_bytes
            L.gate_type, L.up_type, L.down_type = types["gate"], types["up"], types["down"]
            L.bias_dtype = _lib.BF16
            L.gate_off, L.up_off, L.down_off = self._gate_off, self._up_off, self._down_off
            L.gate_scales_off = L.down_scales_off = L.gate_bias_off = L.down_bias_off = -1
            self._layouts[key] = L
        return L

    def forward(self, packed: torch.Tensor, h: torch.Tensor, layer_idx: int = -1) -> torch.Tensor:
        if not self._has_ggml:
            raise RuntimeError("GGMLExpertForward needs the tinyserve_amd HIP library")
        types = self._ggml_types
        if layer_idx >= 0 and layer_idx in getattr(self, "_layer_ggml_types", {}):
            types = self._layer_ggml_types[layer_idx]
        H = self._proj_shapes["gate"][0]
        h2 = h.reshape(-1, H)
        # a SiLU gate with equal gate/up types is the fused decode kernel; any other act_fn
        # (or mixed gate/up types) runs the three GGUF matvecs with act_fn(gate) * up between
        if self._silu and types["gate"] == types["up"]:
            L = self._layout(types, packed.numel())
            T = h2.shape[0]
            key = (h.device, T)
            if key not in self._ones:
                self._ones[key] = (torch.zeros((T, 1), dtype=torch.int32, device=h.device),
                                   torch.ones((T, 1), dtype=torch.float32, device=h.device))
            s, w = self._ones[key]
            return ops.moe_decode(L, packed.reshape(1, -1), s, w, h2).reshape(h.shape)
        gs, us, ds = self._proj_shapes["gate"], self._proj_shapes["up"], self._proj_shapes["down"]
        g = packed[self._gate_off : self._gate_off + self._actual_bytes(gs, types["gate"])]
        u = packed[self._up_off : self._up_off + self._actual_bytes(us, types["up"])]
        d = packed[self._down_off : self._down_off + self._actual_bytes(ds, types["down"])]
        go = ops.gguf_matvec(h2, g, types["gate"], gs[1], gs[0], out_dtype=torch.float32)
        uo = ops.gguf_matvec(h2, u, types["up"], us[1], us[0], out_dtype=torch.float32)
        act = torch.nn.functional.silu if self._silu or self._act_fn is None else self._act_fn
        hid = (act(go) * uo).to(h.dtype)
        return ops.gguf_matvec(hid, d, types["down"], ds[1], ds[0], out_dtype=h.dtype).reshape(h.shape)
