"""The routed part of a MoE layer, as moelan's model module exposes it.

moelan's ``model.py`` holds the router's top-k selection (``route``,
moelan/model.py:154-167, with its softmax 83-86), the grouping of routed rows
by expert (``group_by_expert``, 226-236) and the expert backends the layers
call (``ExpertBackend`` / ``LocalBackend``, 243-278). The same names are here
so that moelan's layer code can import them from this package: the routing
functions are the device kernels of :mod:`distributedmoellm_amd.kernels`
under moelan's names, and :func:`moe_layer` runs a prompt's whole MoE layer
(router product, routing, grouping, expert FFN, weighted sum; moelan/model.py:
597-606) as one device call.
"""

from __future__ import annotations

import time
from collections import Counter

import numpy as np

from . import kernels


def route(logits, top_k: int, normalize: bool):
    """Top-k experts per row of router logits: (ids (n, k) int32, gate weights
    (n, k) f32), on the device."""
    return kernels.route(logits, top_k, normalize)


def group_by_expert(idx, w, num_experts: int | None = None):
    """Routing (n, k) regrouped per expert: (experts, offsets, rows, weights),
    the rows of expert i being rows[offsets[i]:offsets[i + 1]]."""
    return kernels.group_by_expert(idx, w, num_experts)


def _host(a) -> np.ndarray:
    return a.cpu().numpy() if kernels.is_device(a) else np.asarray(a)


class ExpertBackend:
    """What a MoE layer calls for its routed experts: ``moe(layer, x, idx, w)``
    returns, per row r of x, the sum over j of w[r, j] times expert idx[r, j]
    applied to x[r]. Every call also counts how often each (layer, expert) was
    picked (``heat``), keeps the experts the last row picked (``last``) and
    adds its wall time to ``moe_time``; subclasses supply ``_moe``."""

    def __init__(self):
        self.heat: Counter = Counter()
        self.last: dict[int, list[int]] = {}
        self.moe_time = 0.0

    def moe(self, layer: int, x, idx, w):
        start = time.perf_counter()
        picks = _host(idx)
        ids, counts = np.unique(picks, return_counts=True)
        self.heat.update({(layer, int(e)): int(c) for e, c in zip(ids, counts)})
        self.last[layer] = picks[-1].tolist()
        result = self._moe(layer, x, idx, w)
        self.moe_time += time.perf_counter() - start
        return result

    def _moe(self, layer, x, idx, w):  # pragma: no cover - interface
        raise NotImplementedError

    def close(self) -> None:
        """Release what the backend holds (nothing for the local one)."""


class LocalBackend(ExpertBackend):
    """Every routed expert served by one ExpertStore (here: resident in this
    GPU's HBM): the routing is regrouped per expert and handed to
    ``store.compute``."""

    def __init__(self, store):
        super().__init__()
        self.store = store

    def _moe(self, layer, x, idx, w):
        experts, offsets, rows, weights = (_host(a) for a in group_by_expert(idx, w))
        cuts = offsets[1:-1]
        groups = list(zip(experts, np.split(rows, cuts), np.split(weights, cuts)))
        return self.store.compute(layer, x, groups)


def moe_layer(x, router, table, top_k: int, normalize: bool, H: int, I: int, gs: int, out=None, workspace=None):
    """A prompt's whole MoE layer in one device call: router product, routing,
    grouping, the grouped MFMA expert FFN and the weighted sum. ``table``: the
    layer's device expert table (``ExpertStore.layer_table``)."""
    return kernels.prefill_layer(x, router, table, top_k, normalize, H, I, gs, out, workspace)
