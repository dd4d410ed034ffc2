"""Expert forward over packed native-format slots (MXFP4 and GGUF).

Keeps the builder entry points of tinyserve/expert_forward.py for the quantised
layouts: ``_build_mxfp4_inline_forward(layout, act_fn)`` returns ``(packed, h) -> y``
(tinyserve/expert_forward.py:197-246), and ``fast_expert_forward`` is the fused top-k
loop of tinyserve/csrc/expert_loop.cpp:41-123, here one HIP call per layer with the
slots and weights kept on the device.

One deliberate difference: the reference's MXFP4 inline forward drops the expert
biases (tinyserve/expert_forward.py:224-244) while its template forward and HF's
GPT-OSS experts add them (tinyserve/_model_hooks.py:380-394); the kernels here follow
the template forward and add ``gate_up_proj_bias`` / ``down_proj_bias`` when the
layout holds them.

BF16 (unquantised) expert layouts are outside this library's scope:
``_build_inline_forward`` returns None for them.
"""
from __future__ import annotations

import torch

from . import _lib, ops
from .expert_store import TensorLayout

# sigmoid(1.702 x) ~ GELU(x): GPT-OSS SwiGLU coefficient (tinyserve/expert_forward.py:30).
_QUICK_GELU_COEFF = 1.702
_SWIGLU_LIMIT = 7.0

_BIAS_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _is_silu(act_fn) -> bool:
    if act_fn is None:
        return False
    if isinstance(act_fn, torch.nn.SiLU) or act_fn is torch.nn.functional.silu:
        return True
    name = getattr(act_fn, "__name__", "") or type(act_fn).__name__
    return name.lower() in ("silu", "silu_", "siluactivation")


def mxfp4_expert_layout(layout: TensorLayout, act_fn=None, slot_bytes: int | None = None,
                        swiglu_limit: float = _SWIGLU_LIMIT, swiglu_alpha: float = _QUICK_GELU_COEFF,
                        tiled: bool = False) -> _lib.ExpertLayout:
    """tsa_expert_layout of a GPT-OSS MXFP4 slot (gate_up_proj[_scales/_bias], down_proj[...]);
    ``tiled`` marks matrices stored in the 16-row MFMA tile order (synth.mxfp4_tiled_layout)."""
    specs = layout.specs
    gu_shape = tuple(specs["gate_up_proj"][0])
    dn_shape = tuple(specs["down_proj"][0])
    two_i = gu_shape[0]
    hidden = (gu_shape[1] * gu_shape[2] * 2) if len(gu_shape) == 3 else gu_shape[1] * 2
    inter = (dn_shape[1] * dn_shape[2] * 2) if len(dn_shape) == 3 else dn_shape[1] * 2
    if two_i != 2 * inter or dn_shape[0] != hidden:
        raise ValueError(f"inconsistent MXFP4 expert shapes: gate_up {gu_shape}, down {dn_shape}")
    L = _lib.ExpertLayout()
    L.format = _lib.EXPERT_MXFP4
    if act_fn is None:
        L.act = _lib.ACT_SWIGLU_OAI
    elif _is_silu(act_fn):
        raise NotImplementedError("MXFP4 experts with a chunked SiLU gate are not supported; GPT-OSS uses SwiGLU")
    else:
        raise NotImplementedError(f"unsupported activation {act_fn!r}")
    L.hidden, L.inter = hidden, inter
    L.slot_bytes = slot_bytes or layout.total_bytes
    L.gate_type = L.up_type = L.down_type = 0
    L.gate_off = L.up_off = layout.offsets["gate_up_proj"]
    L.gate_scales_off = layout.offsets["gate_up_proj_scales"]
    L.down_off = layout.offsets["down_proj"]
    L.down_scales_off = layout.offsets["down_proj_scales"]
    L.gate_bias_off = layout.offsets.get("gate_up_proj_bias", -1)
    L.down_bias_off = layout.offsets.get("down_proj_bias", -1)
    bias_dt = specs.get("gate_up_proj_bias", specs.get("down_proj_bias", (None, torch.bfloat16)))[1]
    L.bias_dtype = _BIAS_DTYPES[bias_dt]
    L.swiglu_limit, L.swiglu_alpha = float(swiglu_limit), float(swiglu_alpha)
    L.mx_tiled = int(bool(tiled))
    return L


def gguf_expert_layout(layout: TensorLayout, ggml_types: dict, proj_shapes: dict,
                       slot_bytes: int | None = None) -> _lib.ExpertLayout:
    """tsa_expert_layout of a GGUF slot with ``gate``/``up``/``down`` raw bytes.

    ``proj_shapes`` are ggml (ne0 = in, ne1 = out): gate/up (H, I), down (I, H)
    (tinyserve/mmap_store.py:80-84, tinyserve/ggml_forward.py:105-115)."""
    H, I = int(proj_shapes["gate"][0]), int(proj_shapes["gate"][1])
    if tuple(proj_shapes["up"]) != (H, I) or tuple(proj_shapes["down"]) != (I, H):
        raise ValueError(f"inconsistent GGUF expert shapes {proj_shapes}")
    L = _lib.ExpertLayout()
    L.format = _lib.EXPERT_GGUF
    L.act = _lib.ACT_SILU
    L.hidden, L.inter = H, I
    L.slot_bytes = slot_bytes or layout.total_bytes
    L.gate_type, L.up_type, L.down_type = int(ggml_types["gate"]), int(ggml_types["up"]), int(ggml_types["down"])
    L.gate_off, L.up_off, L.down_off = layout.offsets["gate"], layout.offsets["up"], layout.offsets["down"]
    L.gate_scales_off = L.down_scales_off = -1
    L.gate_bias_off = L.down_bias_off = -1
    L.bias_dtype = _lib.BF16
    L.swiglu_limit, L.swiglu_alpha = _SWIGLU_LIMIT, _QUICK_GELU_COEFF
    return L


def build_expert_layout(layout: TensorLayout, act_fn=None, ggml_types: dict | None = None,
                        proj_shapes: dict | None = None, slot_bytes: int | None = None) -> _lib.ExpertLayout | None:
    """The kernel-side layout of a packed expert, or None for unquantised layouts."""
    if "gate_up_proj_scales" in layout.specs:
        return mxfp4_expert_layout(layout, act_fn, slot_bytes)
    if ggml_types is not None and {"gate", "up", "down"} <= set(layout.specs):
        return gguf_expert_layout(layout, ggml_types, proj_shapes, slot_bytes)
    return None


def _build_inline_forward(layout, act_fn):
    """BF16 fused-expert layouts are outside this library's scope (see module doc)."""
    return None


def _build_mxfp4_inline_forward(layout: TensorLayout, act_fn):
    """``(packed [expert_bytes] u8, h [T, H]) -> [T, H]`` for an MXFP4 slot; None otherwise."""
    if "gate_up_proj_scales" not in layout.specs:
        return None
    L = mxfp4_expert_layout(layout, act_fn)
    one = {}

    def _forward(packed: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
        T = h.reshape(-1, L.hidden).shape[0]
        key = (h.device, T)
        if key not in one:
            one[key] = (torch.zeros((T, 1), dtype=torch.int32, device=h.device),
                        torch.ones((T, 1), dtype=torch.float32, device=h.device))
        slots, w = one[key]
        return ops.moe_decode(L, packed.reshape(1, -1), slots, w, h)

    return _forward


def fast_expert_forward(hidden_states: torch.Tensor, expert_slots: torch.Tensor, routing_weights: torch.Tensor,
                        cache_packed: torch.Tensor, layout: _lib.ExpertLayout,
                        workspace: torch.Tensor | None = None) -> torch.Tensor:
    """sum_j w_j * FFN(cache_packed[slot_j], hidden) with slot < 0 skipped
    (tinyserve/csrc/expert_loop.cpp:41-123); one fused HIP call, no host sync."""
    return ops.moe_decode(layout, cache_packed, expert_slots.reshape(hidden_states.reshape(-1, layout.hidden).shape[0], -1),
                          routing_weights, hidden_states, workspace=workspace)
