"""Route-history retention policy for the HBM slot cache: the reference's RouteCachePolicy
(runtime/deepseek_v4_ssd/route_cache.py:12-120), same constructor, methods and arrays.

Per (layer, expert) it keeps two exponentially decayed decode routing rates (half-lives
16 and 256 tokens) and the current prompt's routing counts as a weak prior. Every
16 x layers decode tokens (and when a prefill ends) it rebalances: retention score =
(0.75 short + 0.25 long + prior) x the layer's relative read cost, and the cache's slots
are split over layers by marginal value (each next slot goes to the largest remaining
score). The scores and quotas drive the native cache's eviction in route mode
(wm_slot_cache_set_route); they never change routing.
"""
from __future__ import annotations

import math

import numpy as np


class RouteCachePolicy:
    short_half_life = 16
    long_half_life = 256
    rebalance_tokens = 16

    def __init__(self, layers: int, experts: int, slots: int, top_k: int):
        if min(layers, experts, slots, top_k) < 1 or top_k > experts:
            raise ValueError("invalid route cache dimensions")
        self.layers, self.experts, self.top_k = layers, experts, top_k
        self.capacity = min(slots, layers * experts)
        shape = (layers, experts)
        self.short = np.zeros(shape, np.float64)
        self.long = np.zeros(shape, np.float64)
        self.prefill = np.zeros(shape, np.float64)
        self.scores = np.zeros(shape, np.float64)
        self.prefill_tokens = np.zeros(layers, np.int64)
        self.decode_tokens = np.zeros(layers, np.int64)
        self.request_decode_tokens = np.zeros(layers, np.int64)
        self.read_cost = np.zeros(layers, np.float64)
        self.read_samples = np.zeros(layers, np.int64)
        self.quotas = np.zeros(layers, np.int64)
        self.rebalances = 0
        self._last_rebalance = 0
        self.rebalance()

    def begin_prefill(self) -> None:
        """A new prompt: its routes become the prior; decode history is kept."""
        self.prefill[:] = 0.0
        self.prefill_tokens[:] = 0
        self.request_decode_tokens[:] = 0

    def observe(self, layer: int, selected, phase: str) -> bool:
        """Routes of one layer (token-major, top_k per token). True when it rebalanced."""
        ids = np.asarray(selected, np.int32).reshape(-1)
        if not 0 <= layer < self.layers or (ids.size and (ids.min() < 0 or ids.max() >= self.experts)):
            raise ValueError("invalid routed expert")
        if ids.size == 0:
            return False
        tokens = max(1, math.ceil(ids.size / self.top_k))
        if phase == "prefill":
            self.prefill[layer] += np.bincount(ids, minlength=self.experts)
            self.prefill_tokens[layer] += tokens
            return False
        # token j of the batch (0-based) is tokens - 1 - j tokens old at the end of it
        age = tokens - 1 - np.arange(ids.size) // self.top_k
        for hist, half_life in ((self.short, self.short_half_life), (self.long, self.long_half_life)):
            keep = 2.0 ** (-1.0 / half_life)
            hist[layer] *= keep ** tokens
            hist[layer] += np.bincount(ids, weights=(1.0 - keep) * keep ** age, minlength=self.experts)
        self.decode_tokens[layer] += tokens
        self.request_decode_tokens[layer] += tokens
        total = int(self.decode_tokens.sum())
        if total - self._last_rebalance >= self.rebalance_tokens * self.layers:
            self._last_rebalance = total
            self.rebalance()
            return True
        return False

    def record_read(self, layer: int, seconds: float) -> None:
        """One expert read's duration: a running mean (weight 0.05 after the first)."""
        if not math.isfinite(seconds) or seconds <= 0:
            return
        if self.read_samples[layer] == 0:
            self.read_cost[layer] = seconds
        else:
            self.read_cost[layer] += 0.05 * (seconds - self.read_cost[layer])
        self.read_samples[layer] += 1

    def rebalance(self) -> None:
        prior = self.prefill / np.maximum(self.prefill_tokens, 1)[:, None]
        prior *= (0.1 * np.exp2(-self.request_decode_tokens / 32.0))[:, None]
        rates = 0.75 * self.short + 0.25 * self.long + prior
        sampled = self.read_samples > 0
        typical = float(np.median(self.read_cost[sampled])) if sampled.any() else 1.0
        cost = np.where(sampled, self.read_cost, typical)
        cost = np.clip(cost / max(typical, 1e-9), 0.5, 2.0)
        self.scores[:] = rates * cost[:, None]
        # Each layer's scores, sorted down, are its marginal value per extra slot. The
        # capacity goes to the largest values overall; equal values go to the lower rank
        # first, then to the lower layer (so ties spread over layers before deepening one).
        ranked = -np.sort(-self.scores, axis=1)
        value = ranked.reshape(-1)
        rank = np.tile(np.arange(self.experts), self.layers)
        layer = np.repeat(np.arange(self.layers), self.experts)
        order = np.lexsort((layer, rank, -value))[:self.capacity]
        self.quotas[:] = np.bincount(layer[order], minlength=self.layers)
        self.rebalances += 1

    def snapshot(self) -> dict:
        arrays = [v for v in vars(self).values() if isinstance(v, np.ndarray)]
        return {
            "short_half_life_tokens": self.short_half_life,
            "long_half_life_tokens": self.long_half_life,
            "rebalance_tokens": self.rebalance_tokens,
            "rebalances": self.rebalances,
            "history_survives_eviction": True,
            "history_scope": "loaded model lifetime; includes observed speculative/replay routes",
            "metadata_array_bytes": sum(a.nbytes for a in arrays),
            "layers": [{
                "layer": l,
                "target_slots": int(self.quotas[l]),
                "decode_observed_tokens": int(self.decode_tokens[l]),
                "prefill_observed_tokens": int(self.prefill_tokens[l]),
                "history_experts": int(np.count_nonzero(self.short[l] + self.long[l])),
                "read_cost_seconds": float(self.read_cost[l]),
                "read_samples": int(self.read_samples[l]),
                "predicted_retained_value": float(np.sort(self.scores[l])[::-1][:self.quotas[l]].sum()),
            } for l in range(self.layers)],
        }
