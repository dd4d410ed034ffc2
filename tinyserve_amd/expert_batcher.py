"""Expert-level batching across concurrent requests (tinyserve/expert_batcher.py:17-85).

``BatchItem`` and ``ExpertBatcher(pipeline).batch_execute(items, layer_idx)`` keep the
reference's contract: every request brings ``hidden_states [1, H]``, its top-k
``expert_indices`` and ``routing_weights``; the result is one ``[1, H]`` output per
request, ``sum_k w_k * FFN_k(h)``. Here the whole batch is one device-side call: the
requests' rows are stacked, expert ids map to resident slots through the pipeline's
``expert_slot`` table, and ``tsa_moe_prefill`` groups by expert and runs the grouped
FFN, so there is no per-expert Python loop and no host sync.

``pipeline`` needs ``layout`` (a ``tsa_expert_layout``), ``pool`` (the resident slot
pool, uint8 ``[n_slots, slot_bytes]``) and ``expert_slot(layer_idx)`` returning an int32
``[E]`` device tensor (-1 for experts that are not resident: they contribute zero, as
slot < 0 does in tinyserve/csrc/expert_loop.cpp:85).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops


@dataclass
class BatchItem:
    hidden_states: torch.Tensor  # [1, hidden_dim]
    expert_indices: torch.Tensor  # [top_k]
    routing_weights: torch.Tensor  # [top_k]
    request_idx: int


class ExpertBatcher:
    def __init__(self, pipeline):
        self._pipeline = pipeline

    def batch_execute(self, items: list[BatchItem], layer_idx: int) -> list[torch.Tensor]:
        if not items:
            return []
        p = self._pipeline
        h = torch.cat([it.hidden_states.reshape(1, -1) for it in items], dim=0)
        idx = torch.stack([it.expert_indices.reshape(-1).to(torch.int32) for it in items]).to(h.device)
        w = torch.stack([it.routing_weights.reshape(-1).to(torch.float32) for it in items]).to(h.device)
        es = p.expert_slot(layer_idx)
        y = ops.moe_prefill(p.layout, p.pool, es, idx, w, h)
        return [y[i : i + 1].to(items[i].hidden_states.dtype) for i in range(len(items))]
