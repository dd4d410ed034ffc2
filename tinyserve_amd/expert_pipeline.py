"""``ExpertPipeline`` over an all-resident expert cache, and the MoE block hook.

Keeps tinyserve/expert_pipeline.py's constructor, ``ExpertPipeline(store, template, device,
staging_buffer_a, staging_buffer_b, transfer_stream, compute_stream, cache=None,
shared_stream=None, ram_cache=None, cpu_expert=None, max_top_k=8)`` (:58-138), and its two
entry points, ``execute_layer_experts(hidden_states, layer_idx, expert_indices,
routing_weights)`` (decode, :140-164) and ``execute_layer_experts_batched(...)`` (prefill,
:166-239), plus the attributes the reference's ExpertBatcher reads (``store``,
``template``, ``cache``, ``staging_buffer_a``, ``_inline_fwd``, ``_param_refs``).

What differs is the mechanism. The reference double-buffers PCIe transfers into an LRU pool
sized for a small card and loops over experts in Python (with ``.tolist()`` host syncs).
One MI355X holds every expert of the target models in its 288 GB, so the first time a
layer runs all its experts are copied into the cache (``ensure_resident``); from then on a
decode layer is one ``tsa_moe_decode`` call and a prefill layer one ``tsa_moe_prefill``
call over the cache's slot pool, with the expert -> slot lookup done on the device.
``execute_layer_logits`` goes from router logits to the weighted sum in one
``tsa_moe_decode_routed`` call (the routing runs inside the decode kernels).

``install_offloaded_forward`` replaces a MoE block's forward as the reference's hook does
(tinyserve/_model_hooks.py:479-568), with the reference's routing modes: router logits (an
``nn.Linear`` router on the router kernel) routed inside the decode kernels or by the device
top-k, or the model's own router's result (``router_native``); then the experts through the
pipeline, with the block's shared expert (if any) on ``pipeline.shared_stream`` joined by an
event. ``execute_batched_experts`` and ``schedule_prefetch`` complete the interface the
reference's hook and batcher call.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .expert_cache import ExpertCache
from .expert_forward import (_build_cpp_layout_args, _build_gpu_int4_forward, _build_inline_forward,
                             _build_mxfp4_inline_forward, _precompute_param_refs, mxfp4_expert_layout)


class ExpertPipeline:
    def __init__(self, store, template: nn.Module | None = None, device="cuda", staging_buffer_a=None,
                 staging_buffer_b=None, transfer_stream=None, compute_stream=None, cache: ExpertCache | None = None,
                 shared_stream=None, ram_cache=None, cpu_expert=None, max_top_k: int = 8,
                 tile_mxfp4: bool = True):
        self.store = store
        self.template = template
        self.device = torch.device(device)
        self.staging_buffer_a = staging_buffer_a if staging_buffer_a is not None else store.allocate_buffer(self.device)
        self.staging_buffer_b = staging_buffer_b
        self.transfer_stream = transfer_stream
        self.compute_stream = compute_stream
        self.ram_cache = ram_cache
        self.cpu_expert = cpu_expert
        self.max_top_k = max_top_k
        self.cache_bias = 0.0
        self.profiler = None
        self._native_quant = hasattr(store, "ggml_types")
        # MXFP4 experts kept in checkpoint order by the store are tiled on their way into the
        # cache, so the cache's slots run the tiled decode and grouped prefill GEMMs
        self._tiled_layout = (self._mxfp4_tiled_cache_layout(store, cache, getattr(template, "_act_fn", None))
                              if tile_mxfp4 and not self._native_quant and self.device.type == "cuda" else None)
        self.cache_layout = self._tiled_layout or store.layout
        if cache is None:  # room for every expert of every layer
            n = store.num_layers * store.num_experts
            cache = ExpertCache(n, self.cache_layout.total_bytes, self.device, num_layers=max(self._layer_ids()) + 1,
                                num_experts=store.num_experts)
        self.cache = cache
        self.shared_stream = shared_stream if shared_stream is not None else (
            torch.cuda.Stream(self.device) if self.device.type == "cuda" else None)
        if self._native_quant:
            from .ggml_forward import GGMLExpertForward

            self._act_fn = nn.SiLU()
            self._nq_forward = GGMLExpertForward(store.layout, store.ggml_types, self._act_fn,
                                                 getattr(store, "proj_shapes", {}))
            self._param_refs = None
            self._inline_fwd = None
            self._cpp_layout_args = None
        else:
            self._act_fn = getattr(template, "_act_fn", None)
            self._param_refs = _precompute_param_refs(template, store.layout) if template is not None else None
            self._inline_fwd = (_build_inline_forward(store.layout, self._act_fn)
                                or _build_mxfp4_inline_forward(self.cache_layout, self._act_fn)
                                or _build_gpu_int4_forward(store.layout, self._act_fn))
            self._cpp_layout_args = _build_cpp_layout_args(self.cache_layout, self._act_fn)
        self._kernel_layouts: dict[int, object] = {}
        self._decode_ws: dict[tuple, torch.Tensor] = {}

    def _layer_ids(self) -> list[int]:
        """The layer_idx values the store answers to: a GGUF store's block numbers, else
        0 .. num_layers - 1 (ExpertStore indexes its layers by position)."""
        layers = getattr(self.store, "layers", None)
        return list(layers) if layers else list(range(self.store.num_layers))

    # ---- residency and layouts
    @staticmethod
    def _mxfp4_tiled_cache_layout(store, cache, act_fn):
        """The slot layout of a cache that holds the store's MXFP4 experts in the tile order,
        or None: the store is not MXFP4, already tiled, the tiled kernels do not take its
        shapes, or a given cache's slots are too small for the tiled bytes."""
        from .expert_forward import _mx_tiled_specs
        from .expert_store import TensorLayout, mxfp4_tiled_specs

        layout = getattr(store, "layout", None)
        if (layout is None or "gate_up_proj_scales" not in layout.specs or "down_proj_scales" not in layout.specs
                or getattr(store, "tiled", False) or _mx_tiled_specs(layout)):
            return None
        try:
            tiled = TensorLayout(mxfp4_tiled_specs(layout.specs))
            if cache is not None and cache.expert_bytes < tiled.total_bytes:
                return None
            ops.moe_decode_workspace_size(mxfp4_expert_layout(tiled, act_fn, tiled.total_bytes, tiled=True), 1, 1)
        except (ValueError, NotImplementedError, RuntimeError):
            return None
        return tiled

    def kernel_layout(self, layer_idx: int):
        """The kernels' tsa_expert_layout of this layer's slots (GGUF layers may differ in type)."""
        L = self._kernel_layouts.get(layer_idx)
        if L is None:
            if self._native_quant:
                L = self.store.expert_layout(layer_idx)
            elif self._tiled_layout is not None:
                L = mxfp4_expert_layout(self._tiled_layout, self._act_fn, self.cache.expert_bytes, tiled=True)
            else:
                L = self.store.expert_layout(self._act_fn)
            self._kernel_layouts[layer_idx] = L
        return L

    def ensure_resident(self, layer_idx: int) -> None:
        """Copy every expert of the layer that has no slot yet into the cache (host work on
        the first call for a layer only; afterwards a check of the host slot map)."""
        E = self.store.num_experts
        cache = self.cache
        if cache.layer_resident(layer_idx, E):
            return
        for e in range(E):
            if not cache.contains(layer_idx, e):
                slot = cache.allocate(layer_idx, e)
                if self._tiled_layout is not None:
                    self._copy_tiled(slot, layer_idx, e)
                else:
                    self.store.copy_to_buffer_slot(cache, slot, layer_idx, e)
        cache.flush_slot_updates()

    def _copy_tiled(self, slot: int, layer_idx: int, expert_idx: int) -> None:
        """One checkpoint-order MXFP4 expert into a tiled cache slot: its bytes to the device
        staging buffer, both matrices repacked into the slot by the tiling kernel
        (tsa_mxfp4_tile), the other tensors (biases) copied as they are. Stream-ordered on
        the current stream, like the kernels that read the slot."""
        buf = self.staging_buffer_a
        self.store.copy_to_buffer(buf, layer_idx, expert_idx)
        dst, tl = self.cache._packed[slot], self._tiled_layout
        for name in tl.specs:
            if name.endswith("_scales") and name[: -len("_scales")] in ("gate_up_proj", "down_proj"):
                continue
            off, nb = tl.offsets[name], tl.sizes[name]
            if name in ("gate_up_proj", "down_proj"):
                so, sn = tl.offsets[name + "_scales"], tl.sizes[name + "_scales"]
                ops.mxfp4_tile(buf.get_tensor(name), buf.get_tensor(name + "_scales"),
                               out_blocks=dst[off : off + nb], out_scales=dst[so : so + sn])
            else:
                dst[off : off + nb].copy_(buf.packed[buf.layout.offsets[name] : buf.layout.offsets[name] + nb])

    def _workspace(self, L, T: int, k: int) -> torch.Tensor:
        key = (int(L.hidden), int(L.inter), int(L.format), T, k)
        ws = self._decode_ws.get(key)
        if ws is None:
            ws = self._decode_ws[key] = ops.moe_decode_workspace(L, T, k, self.device)
        return ws

    # ---- the reference's entry points
    def execute_layer_experts(self, hidden_states: torch.Tensor, layer_idx: int, expert_indices: torch.Tensor,
                              routing_weights: torch.Tensor) -> torch.Tensor:
        """sum_j w[t, j] * expert_{idx[t, j]}(h[t]) for every token; one fused decode call."""
        self.ensure_resident(layer_idx)
        L = self.kernel_layout(layer_idx)
        h = hidden_states.reshape(-1, L.hidden)
        T = h.shape[0]
        idx = expert_indices.reshape(T, -1)
        k = idx.shape[1]
        slots = self.cache.lookup_slots(layer_idx, idx)
        w = routing_weights.reshape(T, k).to(torch.float32)
        y = ops.moe_decode(L, self.cache._packed, slots, w, h, workspace=self._workspace(L, T, k))
        return y.view(hidden_states.shape)

    def execute_layer_experts_batched(self, hidden_states: torch.Tensor, layer_idx: int,
                                      expert_indices: torch.Tensor, routing_weights: torch.Tensor) -> torch.Tensor:
        """The same sum for a prefill batch: one grouped tsa_moe_prefill call."""
        self.ensure_resident(layer_idx)
        L = self.kernel_layout(layer_idx)
        h = hidden_states.reshape(-1, L.hidden)
        T = h.shape[0]
        if T == 0:
            return hidden_states.clone()
        idx = expert_indices.reshape(T, -1).to(torch.int32)
        w = routing_weights.reshape(T, -1).to(torch.float32)
        y = ops.moe_prefill(L, self.cache._packed, self.cache.expert_slot(layer_idx), idx, w, h)
        return y.to(hidden_states.dtype).view(hidden_states.shape)

    def execute_layer_logits(self, hidden_states: torch.Tensor, layer_idx: int, router_logits: torch.Tensor,
                             top_k: int, mode: str = "topk_then_softmax", return_routing: bool = False):
        """Router logits [T, E] -> the weighted expert sum in one routed decode call."""
        self.ensure_resident(layer_idx)
        L = self.kernel_layout(layer_idx)
        h = hidden_states.reshape(-1, L.hidden)
        T = h.shape[0]
        res = ops.moe_decode_routed(L, self.cache._packed, self.cache.expert_slot(layer_idx),
                                    router_logits.reshape(T, -1), h, top_k, mode,
                                    workspace=self._workspace(L, T, top_k), return_routing=return_routing)
        if return_routing:
            y, idx, w = res
            return y.view(hidden_states.shape), idx, w
        return res.view(hidden_states.shape)


    # ---- the rest of the reference's pipeline interface
    def execute_batched_experts(self, items, layer_idx: int) -> list[torch.Tensor]:
        """Expert-level batching over several requests (tinyserve/expert_pipeline.py:706-719):
        delegates to ExpertBatcher, which runs one grouped call for the whole batch."""
        from .expert_batcher import ExpertBatcher

        return ExpertBatcher(self).batch_execute(items, layer_idx)

    def schedule_prefetch(self, layer_idx: int, expert_ids=None) -> None:
        """The reference's prefetch of predicted experts (tinyserve/expert_pipeline.py:721-):
        with every expert resident it only makes sure the layer's experts have slots; the
        predicted ids (a list or a device tensor) are not read, so nothing synchronises."""
        if self.cache is not None:
            self.ensure_resident(layer_idx)


_SOFTMAX_ORDERS = ("topk_then_softmax", "softmax_then_topk", "router_native")


def _native_route(result, top_k: int, dtype: torch.dtype):
    """(top_idx, weights, logits or None) from what a model's own router returned, as
    tinyserve/_model_hooks.py:429-455 reads it: a tensor of logits (sigmoid, then top-k of
    the sigmoid values), a (logits, weights, indices) triple (HF GPT-OSS / Qwen3-MoE
    routers), or a pair (full weights and indices, or indices and weights). All of it runs
    on the router's device; weights come back in ``dtype``."""
    if isinstance(result, torch.Tensor):
        w, idx = torch.topk(torch.sigmoid(result), top_k, dim=-1)
        return idx, w.to(dtype), None
    if len(result) == 3:
        logits, w, idx = result
        return idx, w.to(dtype), logits
    first, second = result
    if second.dtype in (torch.int32, torch.int64):
        w_full, idx = first, second
        w = w_full.gather(-1, idx) if w_full.shape[-1] > top_k else w_full
    else:
        idx, w = first, second
    return idx, w.to(dtype), None


def _router_linear(router: nn.Module):
    """The router's (weight, bias) if it is a plain nn.Linear the router kernel can run
    (tsa_router_logits: bf16 / fp16 / fp32 weights on the GPU, in_features a multiple of 8),
    else None (the model's module is called)."""
    if type(router) is not nn.Linear or router.weight.device.type != "cuda":
        return None
    if router.weight.dtype not in (torch.bfloat16, torch.float16, torch.float32) or router.in_features % 8:
        return None
    return router.weight, router.bias


def install_offloaded_forward(moe_block: nn.Module, pipeline: ExpertPipeline, layer_idx: int, router_attr: str,
                              top_k: int, returns_router_logits: bool = False,
                              softmax_order: str = "topk_then_softmax", next_pipeline=None, next_route=None,
                              next_fate_fn=None, adaptive_fate: bool = True, is_first_layer: bool = False,
                              all_pipelines=None, routed_decode_tokens: int = 4) -> None:
    """Replace ``moe_block.forward`` (tinyserve/_model_hooks.py:479-568) with the same
    arguments.

    Routing (tinyserve/_model_hooks.py:424-476): ``"topk_then_softmax"`` (GPT-OSS) and
    ``"softmax_then_topk"`` (renormalised unless the block's ``norm_topk_prob`` is False)
    start from router logits: an ``nn.Linear`` router runs on the router kernel
    (tsa_router_logits), any other router module is called; up to ``routed_decode_tokens``
    tokens then take one routed decode call (top-k and softmax inside the decode kernels),
    longer inputs the device top-k and one batched prefill call. ``"router_native"`` calls the
    model's router and reads its result as the reference does (``_native_route``), then runs
    the decode or prefill call on those experts and weights (weights in the hidden dtype, as
    the reference passes them).

    The block's ``shared_experts`` / ``shared_expert`` runs on ``pipeline.shared_stream``,
    joined by an event. For one-token decode with ``next_pipeline`` and a ``next_route`` /
    ``next_fate_fn`` given, ``next_pipeline.schedule_prefetch(layer_idx + 1, ...)`` is called
    as the reference calls it, and likewise ``all_pipelines[layer_idx + hop]`` for hops 2 and 3;
    with every expert resident these only check residency. ``returns_router_logits`` returns
    ``(out, logits)``, logits None when a native router gives none."""
    if softmax_order not in _SOFTMAX_ORDERS:
        raise ValueError(f"unsupported softmax_order {softmax_order!r}; expected one of {_SOFTMAX_ORDERS}")
    renormalize = getattr(moe_block, "norm_topk_prob", True)
    mode = ("topk_then_softmax" if softmax_order == "topk_then_softmax" else
            "softmax_then_topk" if renormalize else "softmax_then_topk_no_renorm")
    router = getattr(moe_block, router_attr)
    linear = _router_linear(router) if softmax_order != "router_native" else None
    shared = getattr(moe_block, "shared_experts", None) or getattr(moe_block, "shared_expert", None)
    prefetch_fn = next_fate_fn if next_fate_fn is not None else next_route

    def offloaded_forward(hidden_states: torch.Tensor, **_kwargs):
        hidden = hidden_states.shape[-1]
        flat = hidden_states.reshape(-1, hidden)
        T = flat.shape[0]
        shared_out = shared_event = None
        main = torch.cuda.current_stream(flat.device)
        if shared is not None:
            side = pipeline.shared_stream
            side.wait_stream(main)
            with torch.cuda.stream(side):
                shared_out = shared(flat)
                shared_event = torch.cuda.Event()
                shared_event.record(side)
            # tensors crossing streams: keep their memory until both streams are done with it
            flat.record_stream(side)
            shared_out.record_stream(main)
        if softmax_order == "router_native":
            idx, w, logits = _native_route(router(flat), top_k, flat.dtype)
            if T <= routed_decode_tokens:
                out = pipeline.execute_layer_experts(flat, layer_idx, idx, w)
            else:
                out = pipeline.execute_layer_experts_batched(flat, layer_idx, idx, w)
        else:
            logits = ops.router_logits(flat, *linear) if linear is not None else router(flat)
            if T <= routed_decode_tokens:
                out = pipeline.execute_layer_logits(flat, layer_idx, logits, top_k, mode)
            else:
                idx, w = ops.route_topk(logits.float(), top_k, mode)
                out = pipeline.execute_layer_experts_batched(flat, layer_idx, idx, w.to(flat.dtype))
        out = out.to(flat.dtype)
        if shared_event is not None:
            main.wait_event(shared_event)
            out = out + shared_out
        if T == 1 and next_pipeline is not None and prefetch_fn is not None:
            next_pipeline.schedule_prefetch(layer_idx + 1, None)
        if T == 1 and all_pipelines is not None:
            for hop in (2, 3):
                if layer_idx + hop < len(all_pipelines):
                    all_pipelines[layer_idx + hop].schedule_prefetch(layer_idx + hop, None)
        out = out.view(hidden_states.shape)
        return (out, logits) if returns_router_logits else out

    moe_block.forward = offloaded_forward
