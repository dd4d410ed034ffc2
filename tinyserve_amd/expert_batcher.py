"""Expert-level batching across concurrent requests (tinyserve/expert_batcher.py:17-85).

``BatchItem`` and ``ExpertBatcher(pipeline).batch_execute(items, layer_idx)`` keep the
reference's contract: every request brings ``hidden_states [1, H]``, its top-k
``expert_indices`` and ``routing_weights``; the result is one ``[1, H]`` output per
request, ``sum_k w_k * FFN_k(h)``.

``pipeline`` is shaped like the reference's ExpertPipeline: ``cache`` (lookup /
allocate / get_packed / ``_packed``), ``store`` (copy_to_buffer), ``staging_buffer_a``,
``template`` + ``_param_refs`` and ``_inline_fwd``. Two paths:

* kernel path: when the experts' packed format has a kernel layout (``pipeline.kernel_layout(layer)``,
  or an ``expert_layout`` attribute on ``pipeline._inline_fwd``, which
  ``_build_mxfp4_inline_forward`` sets) and the cache has the device slot table
  (``expert_slot``), every expert of the layer is made resident once and the whole batch
  is one ``tsa_moe_prefill`` call: requests stacked, ids mapped to slots on the device,
  grouped by expert inside the library. No per-expert Python loop, no host sync.
* generic path, for unquantised (bf16 / f16 / f32) experts: the reference's per-expert
  loop, hits through ``_inline_fwd`` or ``forward_from_packed``, misses through the staging
  buffer and ``swap_weights_and_forward``, then cached.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .expert_forward import forward_from_packed, swap_weights_and_forward


@dataclass
class BatchItem:
    hidden_states: torch.Tensor  # [1, hidden_dim]
    expert_indices: torch.Tensor  # [top_k]
    routing_weights: torch.Tensor  # [top_k]
    request_idx: int


class ExpertBatcher:
    def __init__(self, pipeline):
        self._pipeline = pipeline

    def _kernel_layout(self, layer_idx: int):
        p = self._pipeline
        if not hasattr(getattr(p, "cache", None), "expert_slot"):
            return None
        if hasattr(p, "kernel_layout"):
            return p.kernel_layout(layer_idx)
        return getattr(getattr(p, "_inline_fwd", None), "expert_layout", None)

    def _make_resident(self, layer_idx: int) -> None:
        """Every expert of the layer gets a cache slot (the reference's miss path, once per expert)."""
        p = self._pipeline
        if hasattr(p, "ensure_resident"):
            p.ensure_resident(layer_idx)
            return
        cache, store = p.cache, p.store
        if cache.layer_resident(layer_idx, store.num_experts):
            return
        buf = p.staging_buffer_a
        for e in range(store.num_experts):
            if not cache.contains(layer_idx, e):
                store.copy_to_buffer(buf, layer_idx, e, non_blocking=False)
                cache.get_packed(cache.allocate(layer_idx, e)).copy_(buf.packed)
        cache.flush_slot_updates()

    def batch_execute(self, items: list[BatchItem], layer_idx: int) -> list[torch.Tensor]:
        if not items:
            return []
        L = self._kernel_layout(layer_idx)
        if L is None:
            return self._batch_execute_loop(items, layer_idx)
        p = self._pipeline
        self._make_resident(layer_idx)
        h = torch.cat([it.hidden_states.reshape(1, -1) for it in items], dim=0)
        idx = torch.stack([it.expert_indices.reshape(-1).to(torch.int32) for it in items]).to(h.device)
        w = torch.stack([it.routing_weights.reshape(-1).to(torch.float32) for it in items]).to(h.device)
        y = ops.moe_prefill(L, p.cache._packed, p.cache.expert_slot(layer_idx), idx, w, h)
        return [y[i : i + 1].to(items[i].hidden_states.dtype) for i in range(len(items))]

    # ---- unquantised experts: the reference's loop over experts
    def _batch_execute_loop(self, items: list[BatchItem], layer_idx: int) -> list[torch.Tensor]:
        groups: dict[int, list[tuple[int, float]]] = {}
        for i, it in enumerate(items):
            for eid, wt in zip(it.expert_indices.reshape(-1).tolist(), it.routing_weights.reshape(-1).tolist()):
                groups.setdefault(int(eid), []).append((i, float(wt)))
        outputs = [torch.zeros_like(it.hidden_states) for it in items]
        p = self._pipeline
        cache = getattr(p, "cache", None)
        for eid, members in groups.items():
            h = torch.cat([items[i].hidden_states.reshape(1, -1) for i, _ in members], dim=0)
            out = None
            if cache is not None:
                slot = cache.lookup(layer_idx, eid)
                if slot is not None:
                    packed = cache.get_packed(slot)
                    if p._inline_fwd is not None:
                        out = p._inline_fwd(packed, h)
                    else:
                        out = forward_from_packed(p.template, packed, p._param_refs, h)
            if out is None:
                out = self._load_and_forward(h, layer_idx, eid)
            for r, (i, wt) in enumerate(members):
                outputs[i] += wt * out[r : r + 1].to(outputs[i].dtype)
        return outputs

    def _load_and_forward(self, h: torch.Tensor, layer_idx: int, eid: int) -> torch.Tensor:
        p = self._pipeline
        buf = p.staging_buffer_a
        p.store.copy_to_buffer(buf, layer_idx, eid, non_blocking=False)
        out = swap_weights_and_forward(p.template, buf, h)
        if getattr(p, "cache", None) is not None:
            p.cache.get_packed(p.cache.allocate(layer_idx, eid)).copy_(buf.packed)
        return out
