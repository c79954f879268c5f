"""A HIP device tier for moelan's own expert store.

moelan's ExpertStore gives the experts a GPU holds to the object in
``store.gpu`` (moelan/experts.py:655-667; its torch tier is
moelan/accel.py:75-188), through this protocol:

- ``add(key, expert) -> bool``: hold an expert (False when the budget is full);
- ``key in tier`` and ``tier.experts``: what it holds;
- ``launch_held(layer, x, groups) -> (handle | None, other groups)``: queue the
  (expert, rows, weights) groups whose experts it holds;
- ``collect(handle, out)``: add their weighted outputs into ``out``;
- ``release()``, ``calibrate(...)``, ``stats()``.

:class:`HipTier` implements it on the HIP kernels. Its int4 experts stay in
their packed bytes in HBM (the torch tier widens each to a dense f16 copy,
four times the bytes), and a layer's held int4 groups run as ONE layer call
(``moe_q4``) on the current stream; the sum comes back through a pinned host
buffer asynchronously, so the caller computes its own share meanwhile. Other
formats (int8 group-quantized, GGUF blocks, f32) run one expert at a time on
their own device kernels and join the same deterministic combine.
"""

from __future__ import annotations

import threading
import time

import numpy as np

from . import gguf as G
from . import kernels
from .experts import Expert, F32Matrix, GroupQuant, Packed4, upload_experts


def _native_matrix(m):
    """One of moelan's matrix objects as this package's own: int4 ``Packed4``
    (raw, s, gs, shape, offset), int8 ``GroupQuant`` (q, s, gs), GGUF
    ``QuantMatrix`` (raw, qtype, shape) and ``Stacked`` (parts), ``F32Matrix``
    (w); anything else with ``dequant()`` (e.g. a 16-bit matrix) is widened
    to f32. The host arrays are taken as they are (views, no copy)."""
    if isinstance(m, (Packed4, GroupQuant, F32Matrix, G.QuantMatrix, G.Stacked)):
        return m
    if hasattr(m, "parts"):
        return G.Stacked(*(_native_matrix(p) for p in m.parts))
    if all(hasattr(m, a) for a in ("raw", "s", "gs", "shape", "offset")):
        return Packed4(np.ascontiguousarray(m.raw), np.ascontiguousarray(m.s), int(m.gs), tuple(m.shape),
                       bool(m.offset))
    if all(hasattr(m, a) for a in ("q", "s", "gs")):
        return GroupQuant(np.ascontiguousarray(m.q), np.ascontiguousarray(m.s), int(m.gs))
    if all(hasattr(m, a) for a in ("raw", "qtype", "shape")):
        return G.QuantMatrix(np.ascontiguousarray(m.raw), int(m.qtype), int(m.shape[1]))
    if hasattr(m, "w"):
        return F32Matrix(m.w)
    return F32Matrix(np.asarray(m.dequant(), np.float32))


class HipTier:
    """Experts held in HBM for a moelan ExpertStore (``store.gpu = HipTier(...)``).

    ``spec`` names the device ("hip" or "cuda", optionally ":<index>"; only the
    current device is used) and ``budget_bytes`` bounds the HBM its experts take.
    """

    def __init__(self, spec: str = "hip", budget_bytes: int = 1 << 40):
        kernels._need()
        import torch
        self.torch = torch
        self.spec = spec
        self.device = kernels.device()
        self.name = f"hip: {torch.cuda.get_device_name(self.device)}"
        self.budget = int(budget_bytes)
        self.experts: dict = {}            # (layer, expert) -> Expert in HBM
        self.used = 0
        self.lock = threading.RLock()
        self.calls = 0
        self.busy_s = 0.0
        self.share = 0.0                   # target share of routed work, from calibrate()
        self.gpu_ms = self.cpu_ms = None
        self._spare: dict = {}             # (rows, cols) -> pinned result buffers not in use

    def __contains__(self, key) -> bool:
        return tuple(key) in self.experts

    def expert_bytes(self, inter: int, hidden: int, gs: int = 32) -> int:
        """HBM of one int4 expert: 3*inter*hidden/2 packed bytes and their f32 scales."""
        return 3 * inter * hidden // 2 + 3 * inter * hidden // gs * 4

    def add(self, key, expert, over_budget: bool = False) -> bool:
        """Hold one expert (any of moelan's formats) in HBM. False if it does
        not fit in the budget (unless ``over_budget``)."""
        e = Expert(_native_matrix(expert.gu), _native_matrix(expert.down), int(expert.inter))
        size = e.nbytes
        with self.lock:
            if self.used + size > self.budget and not over_budget:
                return False
            upload_experts([e])
            if isinstance(e.gu, Packed4) and isinstance(e.down, Packed4):
                e.fused = kernels.q4_expert_ptrs(e) or False
            self.experts[tuple(key)] = e
            self.used += size
        return True

    def _result_buffer(self, shape):
        """A pinned host buffer for one launch's result (kept for reuse after collect)."""
        free = self._spare.get(shape)
        if free:
            return free.pop()
        return self.torch.empty(shape, dtype=self.torch.float32, pin_memory=True)

    def launch(self, layer: int, x, groups):
        """Queue the given (expert, rows, weights) groups, all held here; returns a handle."""
        torch = self.torch
        t0 = time.perf_counter()
        with self.lock:
            xd = kernels.to_device(np.ascontiguousarray(x, np.float32), torch.float32)
            n, H = xd.shape
            od = torch.zeros((n, H), dtype=torch.float32, device=xd.device)
            fused: dict = {}
            ys, yrows, yw = [], [], []
            keep = []
            for expert, rows, weights in groups:
                e = self.experts[(layer, int(expert))]
                keep.append(e)
                rows = np.asarray(rows, np.int32)
                weights = np.asarray(weights, np.float32)
                if e.fused:
                    fused.setdefault((e.inter, e.gu.gs), []).append((e.fused, rows, weights))
                else:
                    rt = torch.as_tensor(rows.astype(np.int64), device=xd.device)
                    ys.append(e(xd.index_select(0, rt)))
                    yrows.append(rows)
                    yw.append(weights)
            kernels.combine(od, ys, yrows, yw)
            for (inter, gs), items in fused.items():
                kernels.moe_q4(xd, items, H, inter, gs, od)
            host = self._result_buffer((n, H)) if n * H else None
            done = torch.cuda.Event()
            if host is not None:
                host.copy_(od, non_blocking=True)
            done.record()
            self.calls += 1
        return host, done, t0, keep

    def launch_held(self, layer: int, x, groups):
        """Launch those of ``groups`` whose experts are held here; returns
        (handle or None, the other groups)."""
        groups = list(groups)
        with self.lock:
            mine = [g for g in groups if (layer, int(g[0])) in self.experts]
            if not mine:
                return None, groups
            rest = [g for g in groups if (layer, int(g[0])) not in self.experts]
            return self.launch(layer, x, mine), rest

    def collect(self, handle, out: np.ndarray) -> None:
        """Wait for a launch and add its weighted sum into ``out`` (host array)."""
        host, done, t0, _ = handle
        done.synchronize()
        if host is not None:
            out += host.numpy()
            with self.lock:
                self._spare.setdefault(tuple(host.shape), []).append(host)
        self.busy_s += time.perf_counter() - t0

    def release(self) -> None:
        """Free the held experts' HBM."""
        with self.lock:
            self.experts.clear()
            self.used = 0
        self.torch.cuda.empty_cache()

    def calibrate(self, sample_expert, cpu_expert_fn, hidden: int, repeats: int = 12) -> float:
        """Time one expert with one input row here and on the host
        (``cpu_expert_fn``) and set ``share`` = cpu / (gpu + cpu), the part of
        the routed work this tier should carry so both finish together."""
        probe = (-1, 0)                      # layer -1: never routed to
        self.add(probe, sample_expert, over_budget=True)
        x = np.random.default_rng(0).standard_normal((1, hidden)).astype(np.float32)
        groups = [(0, np.array([0], np.int32), np.ones(1, np.float32))]

        def here():
            o = np.zeros_like(x)
            self.collect(self.launch(-1, x, groups), o)
        for _ in range(3):
            here()
            cpu_expert_fn(x)
        t0 = time.perf_counter()
        for _ in range(repeats):
            here()
        g = (time.perf_counter() - t0) / repeats
        t0 = time.perf_counter()
        for _ in range(repeats):
            cpu_expert_fn(x)
        c = (time.perf_counter() - t0) / repeats
        with self.lock:
            e = self.experts.pop(probe)
            self.used -= e.nbytes
        self.calls, self.busy_s = 0, 0.0
        self.gpu_ms, self.cpu_ms = g * 1e3, c * 1e3
        self.share = c / (g + c)
        return self.share

    def stats(self) -> dict:
        return {"device": self.name, "experts": len(self.experts), "used_bytes": self.used,
                "budget_bytes": self.budget, "share": round(self.share, 3),
                "gpu_ms_per_expert": self.gpu_ms, "cpu_ms_per_expert": self.cpu_ms,
                "calls": self.calls, "busy_s": round(self.busy_s, 3)}


__all__ = ["HipTier"]
