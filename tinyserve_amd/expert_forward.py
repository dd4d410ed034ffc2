"""Expert forward over packed slots (MXFP4 and GGUF) and the reference's builder entry points.

The functions of tinyserve/expert_forward.py with the same names and arguments:

* ``swap_weights_and_forward(template, buf, h)`` / ``_precompute_param_refs(template,
  layout)`` / ``forward_from_packed(template, packed, refs, h)`` (:33-106): bind a
  packed expert's tensors to a template module's parameters (by copy into storage the
  template owns, or by zero-copy views) and call the template. With the template modules
  defined here (``MXFP4ExpertModule``, ``GGUFExpertModule``), whose parameters are the
  slot's quantised tensors, the forward runs on this library's kernels.
* ``_build_inline_forward(layout, act_fn)`` (:109-194): ``(packed, h) -> y`` for an
  unquantised (bf16/fp16/fp32) fused-expert slot with ``F.linear``; None for quantised
  slots. Unquantised experts are not this library's hot path; this is plain torch on the GPU.
* ``_build_mxfp4_inline_forward(layout, act_fn)`` (:197-246): ``(packed, h) -> y`` for an
  MXFP4 slot, one fused decode call (the closure's ``expert_layout`` attribute is the
  kernel layout, used by the batched paths).
* ``_build_gpu_int4_forward`` (:249-262): None, as in the reference (MXFP4 slots run on
  the MXFP4 kernels directly).
* ``_build_cpp_layout_args(layout, act_fn)`` (:277-338): the keyword arguments of
  ``fast_expert_forward`` for a slot layout (``{"layout": tsa_expert_layout}`` for MXFP4;
  None where no kernel layout follows from the TensorLayout alone: GGUF needs its ggml
  types, unquantised slots have no kernel).
* ``fast_expert_forward`` is the fused top-k loop of tinyserve/csrc/expert_loop.cpp:41-123,
  one HIP call per layer with the slots and weights kept on the device.

One deliberate difference: the reference's MXFP4 inline forward drops the expert biases
(tinyserve/expert_forward.py:224-244) while its template forward and HF's GPT-OSS experts
add them (tinyserve/_model_hooks.py:380-394); the kernels here follow the template forward
and add ``gate_up_proj_bias`` / ``down_proj_bias`` when the layout holds them.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, ops
from .expert_store import TensorLayout

# sigmoid(1.702 x) ~ GELU(x): GPT-OSS SwiGLU coefficient (tinyserve/expert_forward.py:30).
_QUICK_GELU_COEFF = 1.702
_SWIGLU_LIMIT = 7.0
# rows up to which the MXFP4 inline forward uses the decode kernels
_INLINE_DECODE_ROWS = 8

_BIAS_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def _is_silu(act_fn) -> bool:
    if act_fn is None:
        return False
    if isinstance(act_fn, torch.nn.SiLU) or act_fn is torch.nn.functional.silu:
        return True
    name = getattr(act_fn, "__name__", "") or type(act_fn).__name__
    return name.lower() in ("silu", "silu_", "siluactivation")


def _mx_tiled_specs(layout: TensorLayout) -> bool:
    """Whether an MXFP4 layout's scales have the tiled shape [rows / 16, tile scale bytes]
    (the checkpoint shape is [rows, K / 32])."""
    from .mx_tiles import tile_scale_bytes

    gu, gs = layout.specs["gate_up_proj"][0], layout.specs["gate_up_proj_scales"][0]
    if len(gu) != 3:
        return False
    return tuple(gs) == (gu[0] // 16, tile_scale_bytes(gu[1] * 32))


def mxfp4_expert_layout(layout: TensorLayout, act_fn=None, slot_bytes: int | None = None,
                        swiglu_limit: float = _SWIGLU_LIMIT, swiglu_alpha: float = _QUICK_GELU_COEFF,
                        tiled: bool = False, prefill_mfma: int = 0) -> _lib.ExpertLayout:
    """tsa_expert_layout of a GPT-OSS MXFP4 slot (gate_up_proj[_scales/_bias], down_proj[...]);
    ``tiled`` marks matrices stored in the 16-row MFMA tile order (synth.mxfp4_tiled_layout);
    a layout whose scale tensors have the tiled shape is taken as tiled in any case.
    ``prefill_mfma``: _lib.PREFILL_FP6 (fp4 weights x two fp6 activation terms on the scaled
    MFMA, the default) or _lib.PREFILL_BF16 (weights expanded to bf16) for the prefill GEMMs."""
    specs = layout.specs
    tiled = tiled or _mx_tiled_specs(layout)
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
    if prefill_mfma not in (_lib.PREFILL_FP6, _lib.PREFILL_BF16):
        raise ValueError(f"prefill_mfma must be PREFILL_FP6 or PREFILL_BF16, got {prefill_mfma}")
    L.prefill_mfma = int(prefill_mfma)
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


# ----------------------------------------------------------------------------- template modules
def _param_owner(module: nn.Module, dotted: str) -> tuple[nn.Module, str]:
    *path, leaf = dotted.split(".")
    for part in path:
        module = getattr(module, part)
    return module, leaf


_template_storage: dict[int, dict[str, torch.Tensor]] = {}


def swap_weights_and_forward(template: nn.Module, buf, hidden_states: torch.Tensor) -> torch.Tensor:
    """Copy every tensor of ``buf`` (an ExpertBuffer: ``layout``, ``get_tensor``) into the
    template's parameter of that name and call the template. The parameters are first
    pointed at storage the template owns (allocated once per template), so the copy never
    writes into a cache slot that forward_from_packed left the parameters viewing."""
    with torch.no_grad():
        own = _template_storage.setdefault(id(template), {})
        for name, (shape, dtype) in buf.layout.specs.items():
            owner, leaf = _param_owner(template, name)
            param = getattr(owner, leaf)
            dst = own.get(name)
            if dst is None or tuple(dst.shape) != tuple(shape) or dst.dtype != dtype or dst.device != param.device:
                dst = own[name] = torch.empty(shape, dtype=dtype, device=param.device)
            dst.copy_(buf.get_tensor(name))
            param.data = dst
    return template(hidden_states)


def _precompute_param_refs(template: nn.Module, layout: TensorLayout) -> list:
    """(parameter, byte offset, byte size, shape, dtype) per slot tensor, resolved once."""
    refs = []
    for name, (shape, dtype) in layout.specs.items():
        owner, leaf = _param_owner(template, name)
        refs.append((getattr(owner, leaf), layout.offsets[name], layout.sizes[name], tuple(shape), dtype))
    return refs


def forward_from_packed(template: nn.Module, packed: torch.Tensor, param_refs: list,
                        hidden_states: torch.Tensor) -> torch.Tensor:
    """Point the template's parameters at views of the packed slot (no copy) and call it."""
    for param, off, nbytes, shape, dtype in param_refs:
        param.data = packed[off : off + nbytes].view(dtype).view(shape)
    return template(hidden_states)


def _gptoss_swiglu(gate_up: torch.Tensor, limit: float = _SWIGLU_LIMIT, alpha: float = _QUICK_GELU_COEFF):
    """GPT-OSS activation on interleaved (gate, up) columns, in fp32."""
    g = gate_up[..., 0::2].float().clamp(max=limit)
    u = gate_up[..., 1::2].float().clamp(min=-limit, max=limit)
    return (u + 1.0) * g * torch.sigmoid(alpha * g)


class MXFP4ExpertModule(nn.Module):
    """A GPT-OSS MXFP4 expert whose parameters are the slot's tensors (the names and shapes
    of an MXFP4 TensorLayout: ``gate_up_proj[_scales][_bias]``, ``down_proj[...]``), so a
    packed slot binds to it through forward_from_packed / swap_weights_and_forward. The
    forward runs the MXFP4 vecmat kernel for both projections (bf16 in and out, like the
    reference's bf16 experts) and the clamped SwiGLU between them."""

    def __init__(self, layout: TensorLayout, device=None, swiglu_limit: float = _SWIGLU_LIMIT,
                 swiglu_alpha: float = _QUICK_GELU_COEFF):
        super().__init__()
        if _mx_tiled_specs(layout):
            raise NotImplementedError("the MXFP4 template forward takes checkpoint-layout slots; tiled slots run "
                                      "through the fused kernels (_build_mxfp4_inline_forward, moe_decode, moe_prefill)")
        for name, (shape, dtype) in layout.specs.items():
            self.register_parameter(name, nn.Parameter(torch.zeros(shape, dtype=dtype, device=device),
                                                       requires_grad=False))
        self._limit, self._alpha = float(swiglu_limit), float(swiglu_alpha)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        gb = getattr(self, "gate_up_proj_bias", None)
        db = getattr(self, "down_proj_bias", None)
        gate_up = ops.mxfp4_matvec(h, self.gate_up_proj, self.gate_up_proj_scales, gb)
        act = _gptoss_swiglu(gate_up, self._limit, self._alpha).to(h.dtype)
        return ops.mxfp4_matvec(act, self.down_proj, self.down_proj_scales, db)


class GGUFExpertModule(nn.Module):
    """A GGUF expert whose parameters ``gate`` / ``up`` / ``down`` are the slot's raw ggml
    block bytes (uint8, the names of a GGUF slot layout), for forward_from_packed /
    swap_weights_and_forward; the forward runs the GGUF matvec kernel per projection and
    ``act_fn(gate) * up`` between them (tinyserve/ggml_forward.py:88-115 semantics).
    ``proj_shapes`` in ggml order: gate/up (H, I), down (I, H)."""

    def __init__(self, layout: TensorLayout, ggml_types: dict, proj_shapes: dict, act_fn=None, device=None):
        super().__init__()
        for name in ("gate", "up", "down"):
            shape, dtype = layout.specs[name]
            self.register_parameter(name, nn.Parameter(torch.zeros(shape, dtype=dtype, device=device),
                                                       requires_grad=False))
        self._types = {k: int(v) for k, v in ggml_types.items()}
        self._H, self._I = int(proj_shapes["gate"][0]), int(proj_shapes["gate"][1])
        self._act = act_fn if act_fn is not None else nn.SiLU()

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        H, I = self._H, self._I
        g = ops.gguf_matvec(h, self.gate.reshape(-1), self._types["gate"], I, H, out_dtype=torch.float32)
        u = ops.gguf_matvec(h, self.up.reshape(-1), self._types["up"], I, H, out_dtype=torch.float32)
        act = (self._act(g) * u).to(h.dtype)
        return ops.gguf_matvec(act, self.down.reshape(-1), self._types["down"], H, I)


# ----------------------------------------------------------------------------- inline builders
def _build_inline_forward(layout: TensorLayout, act_fn):
    """``(packed, h) -> y`` for an unquantised fused-expert slot (``gate_up_proj`` and
    ``down_proj`` as bf16/fp16/fp32 matrices, biases optional) with F.linear; None for
    quantised slots (MXFP4 has _build_mxfp4_inline_forward, GGUF has GGMLExpertForward).
    A matrix stored [in, out] is transposed as the reference's template does
    (tinyserve/expert_forward.py:131-149): gate_up maps hidden = min(shape) to 2 inter, so it
    is transposed when its first dimension is hidden; down maps inter = max(gate_up) / 2 to
    hidden, so it is transposed when its first dimension is inter. A square down matrix
    (hidden == inter, as in GPT-OSS) takes gate_up's orientation: the reference transposes
    it always, which is the same for checkpoints that store both [in, out] (HF GPT-OSS), and
    right also for ones that store both [out, in]. act_fn None: the GPT-OSS clamped SwiGLU
    on interleaved (gate, up) columns; otherwise act_fn(gate) * up on the two halves."""
    specs = layout.specs
    if "gate_up_proj" not in specs or "down_proj" not in specs or "gate_up_proj_scales" in specs:
        return None
    gu_shape, gu_dtype = specs["gate_up_proj"]
    dn_shape, _ = specs["down_proj"]
    if gu_dtype not in (torch.bfloat16, torch.float16, torch.float32) or len(gu_shape) != 2 or len(dn_shape) != 2:
        return None
    hidden, gated = min(gu_shape), max(gu_shape) // 2
    if set(dn_shape) != {hidden, gated}:
        return None
    gu_transposed = gu_shape[0] == hidden
    dn_transposed = gu_transposed if dn_shape[0] == dn_shape[1] else dn_shape[0] == gated
    has_bias = "gate_up_proj_bias" in specs and "down_proj_bias" in specs

    def view(packed, name):
        shape, dtype = specs[name]
        off = layout.offsets[name]
        return packed[off : off + layout.sizes[name]].view(dtype).view(shape)

    def _forward(packed: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
        w = view(packed, "gate_up_proj")
        gate_up = F.linear(h, w.t() if gu_transposed else w, view(packed, "gate_up_proj_bias") if has_bias else None)
        if act_fn is None:
            act = _gptoss_swiglu(gate_up).to(gate_up.dtype)
        else:
            gate, up = gate_up.chunk(2, dim=-1)
            act = act_fn(gate) * up
        w = view(packed, "down_proj")
        return F.linear(act, w.t() if dn_transposed else w, view(packed, "down_proj_bias") if has_bias else None)

    return _forward


def _build_gpu_int4_forward(layout, act_fn):
    """None, as in the reference (its INT4 conversion path is disabled); MXFP4 slots run
    on the MXFP4 kernels directly."""
    return None


def _build_cpp_layout_args(layout: TensorLayout, act_fn):
    """Keyword arguments of fast_expert_forward for slots of this layout: the kernel layout
    of an MXFP4 slot; None where the TensorLayout alone fixes no kernel layout (GGUF slots
    need their ggml types, see gguf_expert_layout; unquantised slots have no kernel)."""
    if "gate_up_proj_scales" not in layout.specs:
        return None
    return {"layout": mxfp4_expert_layout(layout, act_fn)}


def _build_mxfp4_inline_forward(layout: TensorLayout, act_fn):
    """``(packed [expert_bytes] u8, h [T, H]) -> [T, H]`` for an MXFP4 slot; None otherwise."""
    if "gate_up_proj_scales" not in layout.specs:
        return None
    L = mxfp4_expert_layout(layout, act_fn)
    one = {}

    def _forward(packed: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
        # every row through slot 0 with weight 1: the decode kernels for a few rows, the
        # grouped prefill GEMMs beyond that
        T = h.reshape(-1, L.hidden).shape[0]
        key = (h.device, T)
        if key not in one:
            one[key] = (torch.zeros((T, 1), dtype=torch.int32, device=h.device),
                        torch.ones((T, 1), dtype=torch.float32, device=h.device))
        slots, w = one[key]
        pool = packed.reshape(1, -1)
        if T <= _INLINE_DECODE_ROWS:
            return ops.moe_decode(L, pool, slots, w, h)
        return ops.moe_prefill(L, pool, slots[:1, 0], slots, w, h)

    _forward.expert_layout = L
    return _forward


def fast_expert_forward(hidden_states: torch.Tensor, expert_slots: torch.Tensor, routing_weights: torch.Tensor,
                        cache_packed: torch.Tensor, layout: _lib.ExpertLayout,
                        workspace: torch.Tensor | None = None) -> torch.Tensor:
    """sum_j w_j * FFN(cache_packed[slot_j], hidden) with slot < 0 skipped
    (tinyserve/csrc/expert_loop.cpp:41-123); one fused HIP call, no host sync."""
    return ops.moe_decode(layout, cache_packed, expert_slots.reshape(hidden_states.reshape(-1, layout.hidden).shape[0], -1),
                          routing_weights, hidden_states, workspace=workspace)
