"""Routing and the local expert backend, on the device.

Mirrors the routed part of ``moelan/model.py``: ``route`` (154-167, softmax
83-86), ``group_by_expert`` (226-236), ``ExpertBackend`` / ``LocalBackend``
(243-278), and a layer call that runs all of it on the device for prompts
(``moe_layer``: router product 597, routing 603, expert call 606).
"""

from __future__ import annotations

import time
from collections import Counter

import numpy as np

from . import kernels


def route(logits, top_k: int, normalize: bool):
    """Softmax router, top-k selection: (expert ids (n,k) int32, weights (n,k) f32)."""
    return kernels.route(logits, top_k, normalize)


def group_by_expert(idx, w, num_experts: int | None = None):
    """(n,k) routing -> experts, offsets, rows, weights (rows grouped per expert)."""
    return kernels.group_by_expert(idx, w, num_experts)


class ExpertBackend:
    """Computes sum_k w_k * expert_k(x) for routed rows. Records routing heat."""

    def __init__(self):
        self.heat: Counter = Counter()
        self.last: dict[int, list[int]] = {}
        self.moe_time = 0.0

    def moe(self, layer: int, x, idx, w):
        t0 = time.perf_counter()
        idx_h = idx.cpu().numpy() if kernels.is_device(idx) else np.asarray(idx)
        for e in idx_h.reshape(-1):
            self.heat[(layer, int(e))] += 1
        self.last[layer] = idx_h[-1].tolist()
        y = self._moe(layer, x, idx, w)
        self.moe_time += time.perf_counter() - t0
        return y

    def _moe(self, layer, x, idx, w):  # pragma: no cover - interface
        raise NotImplementedError

    def close(self) -> None:
        pass


class LocalBackend(ExpertBackend):
    """All experts resident in this GPU's HBM."""

    def __init__(self, store):
        super().__init__()
        self.store = store

    def _moe(self, layer, x, idx, w):
        experts, offsets, rows, weights = group_by_expert(idx, w)
        to_np = (lambda a: a.cpu().numpy()) if kernels.is_device(experts) else np.asarray
        experts, offsets, rows, weights = map(to_np, (experts, offsets, rows, weights))
        groups = [(experts[i], rows[offsets[i]:offsets[i + 1]], weights[offsets[i]:offsets[i + 1]])
                  for i in range(len(experts))]
        return self.store.compute(layer, x, groups)


def moe_layer(x, router, table, top_k: int, normalize: bool, H: int, I: int, gs: int, out=None, workspace=None):
    """A whole MoE layer on the device for many rows (prompts): router product,
    routing, grouping, the grouped MFMA expert FFN and the weighted combine.
    ``table``: the layer's expert table (ExpertStore.layer_table)."""
    return kernels.prefill_layer(x, router, table, top_k, normalize, H, I, gs, out, workspace)
