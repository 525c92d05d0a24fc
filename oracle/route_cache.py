"""Test oracle (test infrastructure only: imported by tests/, never by the product).

Restatements of the reference's route-aware slot retention, written the way the reference
computes it, so the product's different mechanics are checked against it:
  - route_quotas: RouteCachePolicy.rebalance's heap allocation of slots to layers
    (runtime/deepseek_v4_ssd/route_cache.py:68-95); the product sorts all marginal values;
  - RouteArena: ExpertCache's route-mode eviction with per-layer heaps of
    (score, last access, version, layer, expert), lazily invalidated, tiers of over-quota /
    other layers (expert_cache.py:1131-1181, :1870-1886); the native cache scans slots.
"""
from __future__ import annotations

import heapq

import numpy as np


def route_quotas(scores: np.ndarray, capacity: int) -> np.ndarray:
    """route_cache.py:84-94: a heap grants each next slot to the layer whose next sorted
    score is largest; ties to the lower rank, then the lower layer."""
    layers, experts = scores.shape
    order = np.sort(scores, axis=1)[:, ::-1]
    quotas = np.zeros(layers, np.int64)
    heap = [(-float(order[l, 0]), 0, l) for l in range(layers)]
    heapq.heapify(heap)
    for _ in range(capacity):
        _, rank, l = heapq.heappop(heap)
        quotas[l] += 1
        rank += 1
        if rank < experts:
            heapq.heappush(heap, (-float(order[l, rank]), rank, l))
    return quotas


class RouteArena:
    """Slots of (layer, expert) with route-mode eviction. plan() mirrors the native cache's
    plan: free slots in order; a resident expert is a hit; the experts handed out by the
    current plan are protected (expert_cache.py:1790-1826)."""

    def __init__(self, slots: int, layers: int, experts: int):
        self.slots, self.layers, self.experts = slots, layers, experts
        self.entries = {}           # (layer, expert) -> [slot, last_access, version]
        self.free = list(range(slots))
        self.heaps = [[] for _ in range(layers)]
        self.counts = [0] * layers
        self.clock = 0
        self.scores = np.zeros((layers, experts))
        self.quotas = np.zeros(layers, np.int64)

    def set_route(self, scores, quotas):
        """A rebalance: new scores re-key every entry (_rebuild_route_heap_locked, :1133-1141)."""
        self.scores = np.array(scores, np.float64)
        self.quotas = np.array(quotas, np.int64)
        self.heaps = [[] for _ in range(self.layers)]
        for (l, e), entry in self.entries.items():
            entry[2] += 1
            self.heaps[l].append((float(self.scores[l, e]), entry[1], entry[2], l, e))
        for h in self.heaps:
            heapq.heapify(h)

    def _touch(self, l, e):
        entry = self.entries[(l, e)]
        self.clock += 1
        entry[1] = self.clock
        entry[2] += 1
        heapq.heappush(self.heaps[l], (float(self.scores[l, e]), entry[1], entry[2], l, e))

    def _evict(self, protected, incoming):
        tiers = ([], [])
        for l in range(self.layers):
            if not self.counts[l]:
                continue
            eligible = self.counts[l] > self.quotas[l] or (l == incoming and self.counts[l] >= self.quotas[l])
            tiers[0 if eligible else 1].append(l)
        held, candidates = [], []
        for tier in tiers:
            for l in tier:
                heap = self.heaps[l]
                while heap:
                    item = heapq.heappop(heap)
                    entry = self.entries.get((l, item[4]))
                    if entry is None or (float(self.scores[l, item[4]]), entry[1], entry[2]) != item[:3]:
                        continue
                    held.append(item)
                    if (l, item[4]) in protected:
                        continue
                    candidates.append(item)
                    break
            if candidates:
                break
        winner = min(candidates) if candidates else None
        for item in held:
            if item != winner:
                heapq.heappush(self.heaps[item[3]], item)
        if winner is None:
            raise RuntimeError("the expert cache is too small for one step")
        return winner[3], winner[4]

    def plan(self, layer, experts):
        protected, slots, missing = set(), [], []
        for e in experts:
            key = (layer, e)
            if key in self.entries:
                self._touch(layer, e)
            else:
                if self.free:
                    slot = self.free.pop(0)
                else:
                    victim = self._evict(protected, layer)
                    slot = self.entries.pop(victim)[0]
                    self.counts[victim[0]] -= 1
                self.entries[key] = [slot, 0, 0]
                self.counts[layer] += 1
                self._touch(layer, e)
                missing.append((e, slot))
            protected.add(key)
            slots.append(self.entries[key][0])
        return slots, missing
