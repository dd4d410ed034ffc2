"""Resident expert slot pool on the GPU (tinyserve/expert_cache.py:14-261, all-resident form).

The reference's ``ExpertCache`` is an LRU over a slot pool sized to what an 8-16 GB card
holds. One MI355X has 288 GB of HBM, which holds every expert of the models this library
targets, so this cache has no eviction policy: ``allocate`` takes a free slot and a full
pool is an error. The interface is the reference's: ``lookup`` / ``contains`` /
``allocate`` / ``flush_slot_updates`` / ``lookup_slots`` / ``get_packed`` /
``store_from_buffer`` / ``load_to_buffer``, the ``_packed`` pool ``[capacity,
expert_bytes]`` uint8 and the hit statistics. What this build adds for the kernels:
``expert_slot(layer)`` is the layer's int32 ``[num_experts]`` device table (slot or -1)
that ``tsa_moe_decode_routed`` / ``tsa_moe_prefill`` read, and ``layer_resident`` says
whether every expert of a layer has a slot.
"""
from __future__ import annotations

import numpy as np
import torch


class ExpertCache:
    def __init__(self, capacity: int, expert_bytes: int, device, policy: str = "resident", num_layers: int = 1,
                 num_experts: int = 1):
        if capacity <= 0 or expert_bytes <= 0:
            raise ValueError(f"capacity ({capacity}) and expert_bytes ({expert_bytes}) must be positive")
        self.capacity = int(capacity)
        self.expert_bytes = int(expert_bytes)
        self.device = torch.device(device)
        self.policy = policy  # accepted for signature compatibility; nothing is ever evicted
        self._packed = torch.empty(self.capacity, self.expert_bytes, dtype=torch.uint8, device=self.device)
        self._slot_of: dict[tuple[int, int], int] = {}
        self._next_free = 0
        self._released: list[int] = []
        self.hits = 0
        self.misses = 0
        self._layer_hits: dict[int, int] = {}
        self._layer_misses: dict[int, int] = {}
        # (layer, expert) -> slot: host copy (written by allocate) and device copy (read by
        # the kernels), synchronised by flush_slot_updates
        self._map_cpu = np.full((max(num_layers, 1), max(num_experts, 1)), -1, dtype=np.int32)
        self._map = torch.from_numpy(self._map_cpu.copy()).to(self.device)
        self._dirty = False

    # ---- host-side bookkeeping
    def lookup(self, layer_idx: int, expert_idx: int) -> int | None:
        slot = self._slot_of.get((layer_idx, expert_idx))
        if slot is None:
            self.misses += 1
            self._layer_misses[layer_idx] = self._layer_misses.get(layer_idx, 0) + 1
        else:
            self.hits += 1
            self._layer_hits[layer_idx] = self._layer_hits.get(layer_idx, 0) + 1
        return slot

    def contains(self, layer_idx: int, expert_idx: int) -> bool:
        return (layer_idx, expert_idx) in self._slot_of

    def begin_pass(self) -> None:
        """Policy hook of the reference (least-stale rotation); nothing to rotate here."""

    def _grow_map(self, layer_idx: int, expert_idx: int) -> None:
        nl, ne = self._map_cpu.shape
        if layer_idx < nl and expert_idx < ne:
            return
        grown = np.full((max(nl, layer_idx + 1), max(ne, expert_idx + 1)), -1, dtype=np.int32)
        grown[:nl, :ne] = self._map_cpu
        self._map_cpu = grown
        self._map = torch.from_numpy(grown.copy()).to(self.device)
        self._dirty = False

    def allocate(self, layer_idx: int, expert_idx: int) -> int:
        """A slot for (layer, expert): its existing one, else a free one. The pool never
        evicts: allocating past ``capacity`` raises."""
        key = (layer_idx, expert_idx)
        slot = self._slot_of.get(key)
        if slot is not None:
            return slot
        if self._released:
            slot = self._released.pop()
        elif self._next_free < self.capacity:
            slot = self._next_free
            self._next_free += 1
        else:
            raise RuntimeError(f"ExpertCache is full ({self.capacity} slots) and keeps every expert resident; "
                               f"create it with a capacity for all experts")
        self._slot_of[key] = slot
        self._grow_map(layer_idx, expert_idx)
        self._map_cpu[layer_idx, expert_idx] = slot
        self._dirty = True
        return slot

    def release(self, layer_idx: int, expert_idx: int) -> None:
        """Give (layer, expert)'s slot back (the caller decides; there is no policy)."""
        slot = self._slot_of.pop((layer_idx, expert_idx), None)
        if slot is not None:
            self._released.append(slot)
            self._map_cpu[layer_idx, expert_idx] = -1
            self._dirty = True

    def flush_slot_updates(self) -> None:
        """Copy the host slot map to the device (lookup_slots and expert_slot call it)."""
        if self._dirty:
            self._map.copy_(torch.from_numpy(self._map_cpu))
            self._dirty = False

    def layer_resident(self, layer_idx: int, num_experts: int | None = None) -> bool:
        """True when every expert of the layer (num_experts of them, default the map's width)
        has a slot."""
        n = self._map_cpu.shape[1] if num_experts is None else num_experts
        if layer_idx >= self._map_cpu.shape[0] or n > self._map_cpu.shape[1]:
            return False
        return bool((self._map_cpu[layer_idx, :n] >= 0).all())

    # ---- device-side tables for the kernels
    def lookup_slots(self, layer_idx: int, expert_ids: torch.Tensor) -> torch.Tensor:
        """Slots of ``expert_ids`` (any shape, on the device) as int32 on the device; -1 for
        experts without a slot and for ids outside the table. No host sync."""
        self.flush_slot_updates()
        if layer_idx >= self._map.shape[0]:
            return torch.full(expert_ids.shape, -1, dtype=torch.int32, device=self.device)
        row = self._map[layer_idx]
        ids = expert_ids.to(device=self.device, dtype=torch.int64)
        inside = (ids >= 0) & (ids < row.numel())
        return torch.where(inside, row[ids.clamp(0, row.numel() - 1)], torch.full_like(row[:1], -1))

    def expert_slot(self, layer_idx: int) -> torch.Tensor:
        """The layer's int32 [num_experts] device table: slot of each expert or -1."""
        self.flush_slot_updates()
        return self._map[layer_idx]

    # ---- slot contents
    def get_packed(self, slot: int) -> torch.Tensor:
        return self._packed[slot]

    def store_from_buffer(self, slot: int, buf) -> None:
        self._packed[slot].copy_(buf.packed)

    def load_to_buffer(self, slot: int, buf) -> None:
        buf.packed.copy_(self._packed[slot])

    # ---- statistics
    @property
    def hit_rate(self) -> float:
        total = self.hits + self.misses
        return self.hits / total if total else 0.0

    def get_layer_stats(self) -> dict[int, dict]:
        out = {}
        for li in sorted(set(self._layer_hits) | set(self._layer_misses)):
            h, m = self._layer_hits.get(li, 0), self._layer_misses.get(li, 0)
            out[li] = {"hits": h, "misses": m, "hit_rate": h / (h + m) if h + m else 0.0}
        return out

    def reset_stats(self) -> None:
        self.hits = self.misses = 0
        self._layer_hits.clear()
        self._layer_misses.clear()

    def clear(self) -> None:
        """Forget every slot assignment (the pool's bytes are left as they are)."""
        self._slot_of.clear()
        self._next_free = 0
        self._released.clear()
        self._map_cpu[:] = -1
        self._dirty = True
        self.reset_stats()
