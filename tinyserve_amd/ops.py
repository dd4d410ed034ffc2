"""torch-facing wrappers of the C ABI: device tensors in, device tensors out.

Every function enqueues on the current HIP stream of the tensors' device and returns
without synchronising. Inputs must already be on the GPU; nothing here falls back to
a CPU implementation.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


# ----------------------------------------------------------------------------- GGUF
def gguf_block_info(ggml_type: int) -> tuple[int, int]:
    be, ts = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.load().tsa_gguf_block_info(int(ggml_type), ctypes.byref(be), ctypes.byref(ts)))
    return be.value, ts.value


def gguf_dequant(data: torch.Tensor, ggml_type: int, shape, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Bit-exact dequantisation of raw GGUF bytes (uint8, on the GPU) to ``shape``."""
    _lib.require_device(data, what="data")
    if data.dtype != torch.uint8:
        raise RuntimeError("data must be uint8")
    data = data.contiguous()
    shape = tuple(int(s) for s in shape)
    n = 1
    for s in shape:
        n *= s
    out = torch.empty(shape, dtype=dtype, device=data.device)
    _lib.check(_lib.load().tsa_gguf_dequant(int(ggml_type), data.data_ptr(), data.numel(), n, out.data_ptr(),
                                            _lib.tsa_dtype(dtype), _stream(data)))
    return out


def gguf_matvec(x: torch.Tensor, w: torch.Tensor, ggml_type: int, out_features: int, in_features: int,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y[T, N] = x[T, K] @ deq(W)^T for an N x K GGUF matrix stored as raw bytes."""
    _lib.require_device(x, what="activation")
    _lib.require_device(w, what="weight_data")
    if w.dtype != torch.uint8:
        raise RuntimeError("weight_data must be uint8")
    K, N = int(in_features), int(out_features)
    x2 = x.reshape(-1, K) if x.numel() % K == 0 else x.reshape(1, -1)
    x2 = x2.contiguous()
    T = x2.shape[0]
    y = torch.empty((T, N), dtype=out_dtype or x.dtype, device=x.device)
    w = w.contiguous()
    _lib.check(_lib.load().tsa_gguf_matvec(int(ggml_type), w.data_ptr(), w.numel(), x2.data_ptr(),
                                           _lib.tsa_dtype(x2.dtype), T, K, y.data_ptr(), _lib.tsa_dtype(y.dtype), N,
                                           _stream(x)))
    return y


# ----------------------------------------------------------------------------- MXFP4
def mxfp4_dequant(blocks: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.bfloat16,
                  transpose: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """Bit-exact MXFP4 dequantisation: blocks [N, G, 16] + scales [N, G] -> [N, 32G] (or [32G, N])."""
    _lib.require_device(blocks, scales, what="blocks/scales")
    N = blocks.shape[0]
    G = scales.shape[-1] if scales.dim() > 1 else scales.numel() // max(N, 1)
    K = G * 32
    blocks, scales = blocks.contiguous(), scales.contiguous()
    shape = (K, N) if transpose else (N, K)
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=blocks.device)
    elif not out.is_contiguous() or out.numel() != N * K or out.dtype != dtype:
        raise ValueError("out must be a contiguous tensor of N*K elements of the requested dtype")
    _lib.check(_lib.load().tsa_mxfp4_dequant(blocks.data_ptr(), scales.data_ptr(), N, K, out.data_ptr(),
                                             _lib.tsa_dtype(dtype), int(transpose), _stream(blocks)))
    return out.view(shape)


def mxfp4_tile_sizes(N: int, K: int) -> tuple[int, int]:
    """(blocks_bytes, scales_bytes) of an [N, K] MXFP4 matrix in the 16-row MFMA tile order."""
    bb, sb = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.load().tsa_mxfp4_tile_sizes(N, K, ctypes.byref(bb), ctypes.byref(sb)))
    return bb.value, sb.value


def mxfp4_tile(blocks: torch.Tensor, scales: torch.Tensor, out_blocks: torch.Tensor | None = None,
               out_scales: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Repack MXFP4 blocks [N, G, 16] + scales [N, G] (checkpoint order) into the 16-row
    MFMA tile order the fast decode reads (uint8 tensors of mxfp4_tile_sizes bytes)."""
    _lib.require_device(blocks, scales, what="blocks/scales")
    N = blocks.shape[0]
    K = blocks[0].numel() * 2
    bb, sb = mxfp4_tile_sizes(N, K)
    blocks, scales = blocks.contiguous(), scales.contiguous()
    if out_blocks is None:
        out_blocks = torch.empty(bb, dtype=torch.uint8, device=blocks.device)
    if out_scales is None:
        out_scales = torch.empty(sb, dtype=torch.uint8, device=blocks.device)
    if out_blocks.numel() * out_blocks.element_size() < bb or out_scales.numel() * out_scales.element_size() < sb:
        raise ValueError(f"outputs too small: need {bb} and {sb} bytes")
    _lib.check(_lib.load().tsa_mxfp4_tile(blocks.data_ptr(), scales.data_ptr(), N, K, out_blocks.data_ptr(),
                                          out_scales.data_ptr(), _stream(blocks)))
    return out_blocks, out_scales


def mxfp4_matvec(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y[T, N] = x[T, K] @ deq(W)^T + bias with W in MXFP4 ([N, G, 16] or [N, 16G] blocks)."""
    _lib.require_device(x, blocks, scales, what="tensor")
    N = blocks.shape[0]
    K = blocks[0].numel() * 2
    x2 = x.reshape(-1, K).contiguous()
    T = x2.shape[0]
    y = torch.empty((T, N), dtype=out_dtype or x.dtype, device=x.device)
    blocks, scales = blocks.contiguous(), scales.contiguous()
    b = None if bias is None else bias.contiguous()
    _lib.check(_lib.load().tsa_mxfp4_matvec(blocks.data_ptr(), scales.data_ptr(), _lib.ptr(b),
                                            _lib.tsa_dtype(b.dtype) if b is not None else 0, x2.data_ptr(),
                                            _lib.tsa_dtype(x2.dtype), T, y.data_ptr(), _lib.tsa_dtype(y.dtype), N, K,
                                            _stream(x)))
    return y


# ----------------------------------------------------------------------------- routing
ROUTE_MODES = {
    "topk_then_softmax": _lib.ROUTE_TOPK_SOFTMAX,
    "softmax_then_topk": _lib.ROUTE_SOFTMAX_TOPK_RENORM,
    "softmax_then_topk_no_renorm": _lib.ROUTE_SOFTMAX_TOPK,
}


def route_topk(logits: torch.Tensor, top_k: int, mode: str = "topk_then_softmax") -> tuple[torch.Tensor, torch.Tensor]:
    """(idx int32 [T, k], weights float32 [T, k]) from router logits [T, E]."""
    _lib.require_device(logits, what="logits")
    lg = logits.reshape(-1, logits.shape[-1]).contiguous()
    T, E = lg.shape
    idx = torch.empty((T, top_k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=lg.device)
    _lib.check(_lib.load().tsa_route_topk(lg.data_ptr(), _lib.tsa_dtype(lg.dtype), T, E, int(top_k),
                                          ROUTE_MODES[mode], idx.data_ptr(), w.data_ptr(), _stream(lg)))
    return idx, w


def router_logits(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The router linear on the GPU: [T, E] = x [T, H] @ weight [E, H]^T (+ bias), fp32
    accumulation, rounded once to ``out_dtype`` (default: the weight's dtype, as
    ``F.linear`` returns it)."""
    _lib.require_device(x, weight, *([bias] if bias is not None else []), what="tensor")
    E, H = weight.shape
    x2 = x.reshape(-1, H).contiguous()
    w = weight.contiguous()
    b = bias.contiguous() if bias is not None else None
    out = torch.empty((x2.shape[0], E), dtype=out_dtype or weight.dtype, device=x.device)
    _lib.check(_lib.load().tsa_router_logits(
        x2.data_ptr(), _lib.tsa_dtype(x2.dtype), x2.shape[0], H, w.data_ptr(), _lib.tsa_dtype(w.dtype), _lib.ptr(b),
        _lib.tsa_dtype(b.dtype) if b is not None else 0, E, out.data_ptr(), _lib.tsa_dtype(out.dtype), _stream(x)))
    return out


# ----------------------------------------------------------------------------- MoE
def _n_slots(pool: torch.Tensor, layout: _lib.ExpertLayout) -> int:
    """Whole slots of ``layout.slot_bytes`` in a contiguous uint8 pool (the kernels index
    slot * slot_bytes, so the pool must hold them all)."""
    if pool.dtype != torch.uint8 or not pool.is_contiguous():
        raise RuntimeError("the expert pool must be a contiguous uint8 tensor")
    n = pool.numel() // int(layout.slot_bytes)
    if n < 1:
        raise RuntimeError(f"expert pool of {pool.numel()} bytes holds no {layout.slot_bytes}-byte slot")
    return n


def moe_decode_workspace_size(layout: _lib.ExpertLayout, T: int, k: int) -> int:
    """Bytes of the decode workspace for T tokens, k experts each; validates the layout
    (host only, raises RuntimeError with the library's message)."""
    n = ctypes.c_int64()
    _lib.check(_lib.load().tsa_moe_decode_workspace_size(ctypes.byref(layout), int(T), int(k), ctypes.byref(n)))
    return n.value


def moe_decode_workspace(layout: _lib.ExpertLayout, T: int, k: int, device) -> torch.Tensor:
    """Decode workspace, zeroed: its leading sync area (the one-launch MXFP4 decode's call
    counter and workgroup flags) must hold one value in every word before the first call."""
    return torch.zeros(max(moe_decode_workspace_size(layout, T, k), 1), dtype=torch.uint8, device=device)


def set_decode_options(tiled_form: int = 1, wait_limit: int = 1 << 18) -> None:
    """Process-wide: the tiled MXFP4 decode in two launches (1, the default) or one (0), and
    the polls a one-launch wait makes before it gives up (tsa_set_decode_options)."""
    _lib.check(_lib.load().tsa_set_decode_options(int(tiled_form), int(wait_limit)))


def decode_workspace_poisoned(workspace: torch.Tensor) -> bool:
    """True if a one-launch wait gave up on this workspace (synchronises the current stream)."""
    out = ctypes.c_int()
    _lib.check(_lib.load().tsa_moe_decode_workspace_status(workspace.data_ptr(), workspace.numel(), ctypes.byref(out),
                                                           _lib.stream_handle(workspace.device)))
    return bool(out.value)


def moe_decode(layout: _lib.ExpertLayout, pool: torch.Tensor, slots: torch.Tensor, weights: torch.Tensor,
               x: torch.Tensor, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
               out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y[t] = sum_j weights[t, j] * FFN_{slots[t, j]}(x[t]) over the resident slot pool."""
    _lib.require_device(pool, slots, weights, x, what="tensor")
    H = layout.hidden
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    slots = slots.reshape(T, -1).to(torch.int32).contiguous()
    weights = weights.reshape(T, -1).to(torch.float32).contiguous()
    k = slots.shape[1]
    n_slots = _n_slots(pool, layout)
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype or x.dtype, device=x.device)
    if workspace is None:
        workspace = moe_decode_workspace(layout, T, k, x.device)
    _lib.check(_lib.load().tsa_moe_decode(ctypes.byref(layout), pool.data_ptr(), n_slots, slots.data_ptr(),
                                          weights.data_ptr(), T, k, x2.data_ptr(), _lib.tsa_dtype(x2.dtype),
                                          out.data_ptr(), _lib.tsa_dtype(out.dtype), workspace.data_ptr(),
                                          workspace.numel(), _stream(x)))
    return out


def moe_decode_routed(layout: _lib.ExpertLayout, pool: torch.Tensor, expert_slot: torch.Tensor, logits: torch.Tensor,
                      x: torch.Tensor, top_k: int, mode: str = "topk_then_softmax", out: torch.Tensor | None = None,
                      workspace: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                      return_routing: bool = False):
    """Router top-k + fused expert FFN in one call (a single launch for MXFP4, T <= 4)."""
    _lib.require_device(pool, expert_slot, logits, x, what="tensor")
    H = layout.hidden
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    lg = logits.reshape(T, -1).contiguous()
    E = lg.shape[1]
    expert_slot = expert_slot.to(torch.int32).contiguous()
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype or x.dtype, device=x.device)
    if workspace is None:
        workspace = moe_decode_workspace(layout, T, top_k, x.device)
    idx = torch.empty((T, top_k), dtype=torch.int32, device=x.device) if return_routing else None
    w = torch.empty((T, top_k), dtype=torch.float32, device=x.device) if return_routing else None
    _lib.check(_lib.load().tsa_moe_decode_routed(
        ctypes.byref(layout), pool.data_ptr(), _n_slots(pool, layout), expert_slot.data_ptr(), E, lg.data_ptr(),
        _lib.tsa_dtype(lg.dtype), ROUTE_MODES[mode], T, int(top_k), x2.data_ptr(), _lib.tsa_dtype(x2.dtype),
        out.data_ptr(), _lib.tsa_dtype(out.dtype), _lib.ptr(idx), _lib.ptr(w), workspace.data_ptr(), workspace.numel(),
        _stream(x)))
    return (out, idx, w) if return_routing else out


def moe_decode_gated(layout: _lib.ExpertLayout, pool: torch.Tensor, expert_slot: torch.Tensor, x: torch.Tensor,
                     router_weight: torch.Tensor, router_bias: torch.Tensor | None, top_k: int,
                     mode: str = "topk_then_softmax", **kw):
    """Hidden states to the weighted expert sum without leaving the GPU: the router linear
    (router_logits), then moe_decode_routed on its logits (keyword arguments pass through)."""
    logits = router_logits(x, router_weight, router_bias)
    return moe_decode_routed(layout, pool, expert_slot, logits, x, top_k, mode, **kw)


def group_by_expert(idx: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(counts [E], offsets [E+1], perm [n_valid]) — expert-major, token-major within an expert."""
    _lib.require_device(idx, what="idx")
    idx2 = idx.reshape(idx.shape[0], -1).to(torch.int32).contiguous()
    T, k = idx2.shape
    counts = torch.empty(num_experts, dtype=torch.int32, device=idx.device)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=idx.device)
    perm = torch.empty(max(T * k, 1), dtype=torch.int32, device=idx.device)
    _lib.check(_lib.load().tsa_group_by_expert(idx2.data_ptr(), T, k, int(num_experts), counts.data_ptr(),
                                               offsets.data_ptr(), perm.data_ptr(), _stream(idx)))
    return counts, offsets, perm[: T * k]


def moe_prefill_workspace(layout: _lib.ExpertLayout, T: int, k: int, E: int, device) -> torch.Tensor:
    n = ctypes.c_int64()
    _lib.check(_lib.load().tsa_moe_prefill_workspace_size(ctypes.byref(layout), int(T), int(k), int(E),
                                                          ctypes.byref(n)))
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=device)


def moe_prefill(layout: _lib.ExpertLayout, pool: torch.Tensor, expert_slot: torch.Tensor, idx: torch.Tensor,
                weights: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Batched (prefill) MoE: out[t] = sum_j weights[t, j] * FFN_{expert_slot[idx[t, j]]}(x[t])."""
    _lib.require_device(pool, expert_slot, idx, weights, x, what="tensor")
    H = layout.hidden
    x2 = x.reshape(-1, H).contiguous()
    T = x2.shape[0]
    idx = idx.reshape(T, -1).to(torch.int32).contiguous()
    weights = weights.reshape(T, -1).to(torch.float32).contiguous()
    expert_slot = expert_slot.to(torch.int32).contiguous()
    k, E = idx.shape[1], expert_slot.numel()
    n_slots = _n_slots(pool, layout)
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype or x.dtype, device=x.device)
    if workspace is None:
        workspace = moe_prefill_workspace(layout, T, k, E, x.device)
    _lib.check(_lib.load().tsa_moe_prefill(ctypes.byref(layout), pool.data_ptr(), n_slots, expert_slot.data_ptr(), E,
                                           idx.data_ptr(), weights.data_ptr(), T, k, x2.data_ptr(),
                                           _lib.tsa_dtype(x2.dtype), out.data_ptr(), _lib.tsa_dtype(out.dtype),
                                           workspace.data_ptr(), workspace.numel(), _stream(x)))
    return out
