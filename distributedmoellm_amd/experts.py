"""Expert matrices and the expert store, resident in HBM.

Mirrors the matrix protocol and expert classes of ``moelan/experts.py``
(``matmul_t(x) == x @ W.T``, ``dequant()``, ``nbytes``: 66-69; ``GroupQuant``
125-167, ``Packed4`` 170-236, ``Expert`` 247-263, ``ExpertStore.compute``
641-670) with every product computed by the HIP kernels of
:mod:`distributedmoellm_amd.kernels`. A matrix keeps what it was given
(numpy, possibly a read-only memory map, or a device tensor) and uploads one
device copy on first use, which it keeps: packed bytes and scales stay
resident in HBM and are never widened to a full-precision copy.
"""

from __future__ import annotations

import numpy as np

from . import kernels

FORMATS = ("f32", "int8", "int4", "native")   # resident formats (moelan/experts.py:40)


def _dev_or_none(a):
    return a if kernels.is_device(a) else None


def default_threads() -> int:
    """Loader threads of a store when none are given (moelan/experts.py:50-51)."""
    import os
    return max(1, min(8, (os.cpu_count() or 2) // 2))


class F32Matrix:
    """A full-precision (rows, cols) weight (moelan/experts.py:72-89). Its
    product is a library f32 GEMM on one device copy, made on first use."""

    __slots__ = ("w", "_dev")

    def __init__(self, w):
        self.w = w if kernels.is_device(w) else np.ascontiguousarray(w, dtype=np.float32)
        self._dev = None

    def device_arrays(self):
        if self._dev is None:
            import torch
            self._dev = (kernels.to_device(self.w, torch.float32),)
        return self._dev

    def host_arrays(self):
        """The host array device_arrays() uploads, with its device shape."""
        return [(self.w, tuple(self.w.shape))]

    @property
    def shape(self):
        return tuple(self.w.shape)

    def matmul_t(self, x):
        import torch
        (w,) = self.device_arrays()
        y = torch.matmul(kernels.to_device(x, torch.float32), w.t())
        return kernels._ret(y, x)

    def dequant(self):
        return self.w

    @property
    def nbytes(self):
        return int(self.w.nbytes) if not kernels.is_device(self.w) else self.w.numel() * 4


class GroupQuant:
    """int8 values with one f32 (or f16) scale per ``gs`` inputs of each output row."""

    __slots__ = ("q", "s", "gs", "_dev")

    def __init__(self, q, s, gs: int):
        self.q, self.s, self.gs = q, s, gs
        self._dev = None

    @classmethod
    def quantize(cls, w: np.ndarray, gs: int = 64) -> "GroupQuant":
        """moelan/experts.py:133-142 (host-side, load time)."""
        O, I = w.shape
        if I % gs:
            gs = I
        g = w.reshape(O, I // gs, gs)
        amax = np.abs(g).max(axis=2)
        s = np.where(amax == 0, 1.0, amax / 127.0).astype(np.float32)
        q = np.clip(np.rint(g / s[:, :, None]), -127, 127).astype(np.int8).reshape(O, I)
        return cls(q, s, gs)

    def device_arrays(self):
        if self._dev is None:
            import torch
            O, I = self.q.shape
            self._dev = (kernels.to_device(self.q, torch.int8).reshape(O, I),
                         kernels.to_device(self.s).reshape(O, I // self.gs))
        return self._dev

    def host_arrays(self):
        """The host arrays device_arrays() uploads, with their device shapes."""
        O, I = self.q.shape
        return [(self.q, (O, I)), (self.s, (O, I // self.gs))]

    @property
    def shape(self):
        return tuple(self.q.shape)

    def dequant(self):
        import torch
        q, s = self.device_arrays()
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        kernels.q8_dequant(q, s, self.gs, out)
        return out if _dev_or_none(self.q) is not None else out.cpu().numpy()

    def matmul_t(self, x):
        q, s = self.device_arrays()
        return kernels.q8_matmul_t(x, q, s, self.gs)

    @property
    def nbytes(self):
        return int(self.q.nbytes + self.s.nbytes)


class Packed4:
    """Colibri's int4: two signed 4-bit values per byte (low nibble = even
    column), one scale per ``gs`` inputs; ``offset`` means the bytes were XOR-ed
    with 0x88 once (resident copies), so nibbles read as u = v + 8."""

    __slots__ = ("raw", "s", "gs", "shape", "offset", "_dev")

    def __init__(self, raw, s, gs: int, shape: tuple[int, int], offset: bool = False):
        self.raw, self.s, self.gs, self.shape, self.offset = raw, s, gs, tuple(shape), offset
        self._dev = None

    def device_arrays(self):
        """(raw uint8 [O, I/2], scales [O, I/gs]) on the device, uploaded once."""
        if self._dev is None:
            import torch
            O, I = self.shape
            self._dev = (kernels.to_device(self.raw, torch.uint8).reshape(O, I // 2),
                         kernels.to_device(self.s).reshape(O, I // self.gs))
        return self._dev

    def host_arrays(self):
        """The host arrays device_arrays() uploads, with their device shapes."""
        O, I = self.shape
        return [(self.raw, (O, I // 2)), (self.s, (O, I // self.gs))]

    def resident(self) -> "Packed4":
        """A copy in offset form (moelan/experts.py:188-191), XOR-ed once on the
        host at load time and uploaded."""
        raw = self.raw.cpu().numpy() if kernels.is_device(self.raw) else np.asarray(self.raw)
        s = self.s.cpu().numpy() if kernels.is_device(self.s) else np.array(self.s)
        raw = np.ascontiguousarray(raw if self.offset else np.bitwise_xor(raw, 0x88))
        p = Packed4(raw, s, self.gs, self.shape, True)
        p.device_arrays()
        return p

    def to_int8(self) -> GroupQuant:
        """int8 values v = u - 8 with the same scales (moelan/experts.py:205-211); load-time, on the host."""
        raw = self.raw.cpu().numpy() if kernels.is_device(self.raw) else np.asarray(self.raw)
        rr = raw if self.offset else np.bitwise_xor(raw, 0x88)
        O, I = self.shape
        u = np.empty((O, I // 2, 2), np.int16)
        u[:, :, 0] = rr.reshape(O, I // 2) & 15
        u[:, :, 1] = rr.reshape(O, I // 2) >> 4
        s = self.s.cpu().numpy() if kernels.is_device(self.s) else np.array(self.s)
        return GroupQuant((u.reshape(O, I) - 8).astype(np.int8), s, self.gs)

    def dequant(self):
        import torch
        raw, s = self.device_arrays()
        out = torch.empty(self.shape, dtype=torch.float32, device=raw.device)
        kernels.q4_dequant(raw, s, self.gs, self.offset, out)
        return out if _dev_or_none(self.raw) is not None else out.cpu().numpy()

    def matmul_t(self, x):
        raw, s = self.device_arrays()
        return kernels.q4_matmul_t(x, raw, s, self.gs, self.offset)

    @property
    def nbytes(self):
        return int(self.raw.nbytes + self.s.nbytes)


class Expert:
    """A SwiGLU expert with gate and up fused into one (2*inter, hidden) matrix
    (moelan/experts.py:247-263)."""

    __slots__ = ("gu", "down", "inter", "fused")

    def __init__(self, gu, down, inter: int):
        self.gu, self.down, self.inter = gu, down, inter
        self.fused = None   # q4_expert_ptrs() once asked (False: not that kind)

    def __call__(self, x):
        """down(silu(gate(x)) * up(x)); int4 experts run as one fused layer call."""
        import torch
        if isinstance(self.gu, Packed4) and isinstance(self.down, Packed4):
            ptrs = kernels.q4_expert_ptrs(self)
            if ptrs is not None:
                xd = kernels.to_device(x, torch.float32)
                n, H = xd.shape
                out = torch.zeros((n, H), dtype=torch.float32, device=xd.device)
                rows = np.arange(n, dtype=np.int32)
                # float activations, as the reference's per-matrix expert call
                kernels.moe_q4(xd, [(ptrs, rows, np.ones(n, np.float32))], H, self.inter, self.gu.gs, out,
                               int8=False)
                return out if kernels.is_device(x) else out.cpu().numpy()
        h = self.gu.matmul_t(kernels.to_device(x, torch.float32))
        a = silu_mul(h, self.inter)
        y = self.down.matmul_t(a)
        return y if kernels.is_device(x) else y.cpu().numpy()

    @property
    def nbytes(self):
        return self.gu.nbytes + self.down.nbytes


def silu_mul(h, inter: int):
    """silu(h[:, :inter]) * h[:, inter:] on the device (HIP kernel)."""
    import torch
    from . import _lib
    hd = kernels.to_device(h, torch.float32)
    n = hd.shape[0]
    a = torch.empty((n, inter), dtype=torch.float32, device=hd.device)
    _lib.call("moe_silu_mul", hd.data_ptr(), hd.shape[1], n, inter, a.data_ptr(), inter, kernels.stream_handle())
    return a


def synthetic_expert(hidden: int, inter: int, fmt: str, gs: int = 32, rng=None, scale_dtype=np.float16) -> Expert:
    """A random expert of the given shape (host arrays), drawn as the benchmark
    configurations say: int4 nibbles uniform, scales |N(0,0.02)|/8; int8 uniform
    in [-127, 127], scales |N(0,0.02)|/127 (cf. moelan/experts.py:322-339)."""
    rng = rng or np.random.default_rng(0)

    def mat(o, i):
        if fmt == "int4":
            raw = rng.integers(0, 256, (o, i // 2), dtype=np.uint8)
            s = (np.abs(rng.normal(0.0, 0.02, (o, i // gs))) / 8).astype(scale_dtype)
            return Packed4(raw, s, gs, (o, i))
        if fmt == "int8":
            q = rng.integers(-127, 128, (o, i), dtype=np.int8)
            s = (np.abs(rng.normal(0.0, 0.02, (o, i // gs))) / 127).astype(scale_dtype)
            return GroupQuant(q, s, gs)
        raise ValueError(f"unknown expert format {fmt!r}")
    return Expert(mat(2 * inter, hidden), mat(hidden, inter), inter)


def _matrices(e: Expert):
    for m in (e.gu, e.down):
        yield from getattr(m, "parts", (m,))


_TORCH_OF = {np.dtype(np.uint8): "uint8", np.dtype(np.int8): "int8", np.dtype(np.float16): "float16",
             np.dtype(np.float32): "float32"}


_STAGES: dict = {}   # staging bytes -> two pinned host buffers, kept for the process


def _staging(stage_bytes: int):
    """Two pinned host buffers of ``stage_bytes``, made once and written
    through once (first writes to new pinned pages run at a fraction of the
    speed of later ones)."""
    import torch
    st = _STAGES.get(stage_bytes)
    if st is None:
        bufs = [torch.empty(stage_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        views = [b.numpy() for b in bufs]
        for v in views:
            v.fill(0)
        st = _STAGES[stage_bytes] = (bufs, views)
    return st


def upload_experts(experts, stage_bytes: int = 32 << 20) -> None:
    """Device copies of many experts' matrices in few transfers: the matrices
    are packed (256-byte aligned) into a pinned staging buffer, which goes to
    one device allocation in one asynchronous copy; each matrix keeps views
    of that allocation (it is freed when the last of them goes). Two staging
    buffers alternate, so packing the next batch out of the (memory-mapped)
    source overlaps the transfer of the last. Matrices already on the device,
    or larger than a staging buffer, take device_arrays(). Not thread-safe:
    the staging buffers are shared by every call in the process."""
    import torch
    todo = []
    for e in experts:
        for part in _matrices(e):
            if getattr(part, "_dev", None) is not None or not hasattr(part, "host_arrays"):
                continue
            arrs = part.host_arrays()
            if any(kernels.is_device(a) or np.asarray(a).dtype not in _TORCH_OF for a, _ in arrs):
                part.device_arrays()
                continue
            todo.append((part, arrs))
    if not todo:
        return
    dev = kernels.device()
    stages, views = _staging(stage_bytes)
    done = [None, None]
    slot, used, batch = 0, 0, []

    def flush():
        # host copies of the batch in parallel pieces (numpy drops the GIL), then its transfers
        pieces = []
        for part, arrs, offs, total, base in batch:
            for (a, _), off in zip(arrs, offs):
                b = np.asarray(a).reshape(-1).view(np.uint8)
                for lo in range(0, b.size, 4 << 20):
                    pieces.append((views[slot][base + off + lo:base + off + min(b.size, lo + (4 << 20))],
                                   b[lo:lo + (4 << 20)]))
        list(_copy_pool().map(lambda p: np.copyto(p[0], p[1]), pieces))
        if not batch:
            return
        # one device allocation and one transfer for the batch; each matrix keeps views of it
        n = batch[-1][4] + batch[-1][3]
        d = torch.empty(n, dtype=torch.uint8, device=dev)
        d.copy_(stages[slot][:n], non_blocking=True)
        for part, arrs, offs, total, base in batch:
            part._dev = tuple(d[base + off:base + off + np.asarray(a).nbytes]
                              .view(getattr(torch, _TORCH_OF[np.asarray(a).dtype])).reshape(shape)
                              for (a, shape), off in zip(arrs, offs))
        batch.clear()

    for part, arrs in todo:
        offs, total = [], 0
        for a, _ in arrs:
            offs.append(total)
            total += (np.asarray(a).nbytes + 255) // 256 * 256
        if total > stage_bytes:
            part.device_arrays()
            continue
        if used + total > stage_bytes:            # switch buffers; wait until the other one is free
            flush()
            done[slot] = torch.cuda.Event()
            done[slot].record()
            slot, used = slot ^ 1, 0
            if done[slot] is not None:
                done[slot].synchronize()
        batch.append((part, arrs, offs, total, used))
        used += total
    flush()
    torch.cuda.current_stream().synchronize()     # the staging buffers are free again


_POOL = None


def _copy_pool():
    global _POOL
    if _POOL is None:
        from concurrent.futures import ThreadPoolExecutor
        _POOL = ThreadPoolExecutor(8, thread_name_prefix="moehip-stage")
    return _POOL


def to_format(e: Expert, fmt: str, gs: int = 64) -> Expert:
    """An expert in a resident format (moelan/experts.py:276-301): ``native``
    keeps the file's encoding; ``int4`` keeps colibri's bytes as they are (the
    kernels read them with their XOR); ``int8`` widens int4 nibbles to int8
    and rounds f32 matrices to int8 in groups of ``gs``; ``f32`` widens any
    matrix to full precision (on the device)."""
    if fmt == "native":
        return e
    if fmt not in FORMATS:
        raise ValueError(f"unknown expert format {fmt!r}")

    def conv(m):
        if fmt == "f32":
            return m if isinstance(m, F32Matrix) else F32Matrix(m.dequant())
        if fmt == "int4":
            if isinstance(m, Packed4):
                return m
            raise ValueError("int4 residency needs an int4 checkpoint (e.g. a colibri container)")
        if isinstance(m, Packed4):
            return m.to_int8()
        if isinstance(m, GroupQuant):
            return m
        if isinstance(m, F32Matrix):
            w = m.w.cpu().numpy() if kernels.is_device(m.w) else m.w
            return GroupQuant.quantize(w, gs)
        raise ValueError(f"int8 residency of a {type(m).__name__} matrix is not provided")
    return Expert(conv(e.gu), conv(e.down), e.inter)


class ExpertStore:
    """Experts by (layer, expert) in HBM and the per-layer compute call
    (moelan/experts.py:538-670).

    Tiers, as the reference's (HBM where it has RAM):
    - ``pinned``: uploaded by :meth:`pin`, kept until unpinned;
    - ``lru``: experts read on demand from a source that copies, at most
      ``lru_size`` (0: none kept);
    - ``mapped``: experts read on demand as views of a memory-mapped file
      (``zero_copy`` sources), at most ``map_size``; each keeps the device
      copy it made on first use while it is listed.
    Hits count pinned and LRU experts, misses the others (as the reference).
    ``sources`` may also be a dict {(layer, expert): Expert} of experts to pin.
    The arguments are the reference's (moelan/experts.py:538-540): ``threads``
    read experts out of their sources in parallel in :meth:`pin`, ``gs`` is the
    group of the int8 format's rounding of f32 matrices.
    """

    def __init__(self, sources=None, fmt: str = "int4", lru_size: int = 0, threads: int | None = None,
                 gs: int = 64, map_size: int = 4096):
        from collections import OrderedDict
        if fmt not in FORMATS:
            raise ValueError(f"format must be one of {FORMATS}")
        self.fmt, self.gs = fmt, gs
        self.lru_size, self.map_size = lru_size, map_size
        self.threads = threads or default_threads()
        self.pinned: dict = {}
        self.lru: OrderedDict = OrderedDict()
        self.mapped: OrderedDict = OrderedDict()
        self.hits = 0
        self.misses = 0
        if isinstance(sources, dict):
            self.sources = []
            self.pinned.update({tuple(k): e for k, e in sources.items()})
        else:
            self.sources = [s for s in (sources or []) if s is not None]

    def _read_from(self, key, fmt: str | None = None):
        for src in self.sources:
            if src.has(key):
                e = src.load(key)
                return (to_format(e, fmt, self.gs) if fmt else e), src
        raise KeyError(f"expert {key} is not available on this node")

    def can_serve(self, key) -> bool:
        key = tuple(key)
        return key in self.pinned or any(s.has(key) for s in self.sources)

    def pin(self, items) -> None:
        """Pin experts and upload their arrays now: keys (read from the
        sources, ``threads`` at a time, moelan/experts.py:581-590) or
        ((layer, expert), Expert) pairs."""
        given, keys = [], []
        for it in items:
            if len(it) == 2 and isinstance(it[1], Expert):
                given.append((tuple(it[0]), it[1]))
            elif tuple(it) not in self.pinned and tuple(it) not in keys:
                keys.append(tuple(it))

        def read(key):
            e = self.lru.pop(key, None) or self.mapped.pop(key, None)
            return key, (to_format(e, self.fmt, self.gs) if e is not None else self._read_from(key, self.fmt)[0])
        if self.threads > 1 and len(keys) > 1:
            from concurrent.futures import ThreadPoolExecutor
            with ThreadPoolExecutor(min(self.threads, len(keys)), thread_name_prefix="moehip-read") as pool:
                loaded = list(pool.map(read, keys))
        else:
            loaded = [read(k) for k in keys]
        for key, e in given + loaded:
            self.pinned[key] = e
        upload_experts([e for _, e in given + loaded])

    def unpin_all_except(self, keep) -> None:
        keep = {tuple(k) for k in keep}
        for key in list(self.pinned):
            if key not in keep:
                del self.pinned[key]

    def forget(self, keys) -> None:
        """Drop every reference to ``keys`` (their device copies go with them)."""
        for k in keys:
            k = tuple(k)
            self.pinned.pop(k, None)
            self.lru.pop(k, None)
            self.mapped.pop(k, None)

    def get(self, key):
        """The expert for ``key`` (moelan/experts.py:610-635)."""
        key = tuple(key)
        e = self.pinned.get(key)
        if e is not None:
            self.hits += 1
            return e
        e = self.lru.get(key)
        if e is not None:
            self.lru.move_to_end(key)
            self.hits += 1
            return e
        e = self.mapped.get(key)
        if e is not None:
            self.mapped.move_to_end(key)
            self.misses += 1
            return e
        self.misses += 1
        e, src = self._read_from(key)
        if getattr(src, "zero_copy", False):
            self.mapped[key] = e
            while len(self.mapped) > self.map_size:
                self.mapped.popitem(last=False)
        elif self.lru_size > 0:
            self.lru[key] = e
            while len(self.lru) > self.lru_size:
                self.lru.popitem(last=False)
        return e

    def resident_bytes(self) -> int:
        return sum(e.nbytes for e in self.pinned.values()) + sum(e.nbytes for e in self.lru.values())

    def compute(self, layer: int, x, groups, mfma: bool = True):
        """Weighted sum of the routed experts' outputs for the given rows
        (moelan/experts.py:641-670). ``groups``: (expert, rows, weights) per
        expert. int4 experts with at least ``kernels.MFMA_FROM`` rows (prompt
        reading) run as one grouped MFMA GEMM (f16 operands); the other int4
        experts as one fused f32 layer call; other formats one by one. All
        weighted sums go through the deterministic combine kernel. Returns the
        type of ``x``."""
        import torch
        groups = list(groups)
        xd = kernels.to_device(x, torch.float32)
        out = torch.zeros(xd.shape, dtype=torch.float32, device=xd.device)
        # ``keep`` holds every expert whose device addresses go into the layer
        # call until it is enqueued: a later get() may drop an earlier expert
        # from the bounded tiers, and its freed blocks could be handed to the
        # next upload before the call reads them (moelan/experts.py:732-735)
        items, keep, H, shape = [], [], xd.shape[1], None
        big = []
        ys, yrows, yw = [], [], []
        for expert, rows, weights in groups:
            e = self.get((layer, int(expert)))
            if kernels.FUSED and e.fused is None:
                ok = isinstance(e.gu, Packed4) and isinstance(e.down, Packed4)
                e.fused = (kernels.q4_expert_ptrs(e) if ok else None) or False
            dims = (e.inter, e.gu.gs) if e.fused else None
            if (mfma and e.fused and len(rows) >= kernels.MFMA_FROM and H % 128 == 0 and e.inter % 128 == 0
                    and e.gu.gs % 32 == 0):
                big.append((e, rows, weights))
                continue
            if kernels.FUSED and e.fused and (shape is None or dims == shape):
                shape = dims
                keep.append(e)
                items.append((e.fused, rows, weights))
                continue
            rows_t = torch.as_tensor(np.asarray(rows, np.int64), device=xd.device)
            ys.append(e(xd.index_select(0, rows_t)))
            yrows.append(rows)
            yw.append(weights)
        for inter, gs in sorted({(e.inter, e.gu.gs) for e, _, _ in big}):
            sel = [(e, r, w) for e, r, w in big if (e.inter, e.gu.gs) == (inter, gs)]
            table = kernels.expert_table([e for e, _, _ in sel])
            eoff = np.zeros(len(sel) + 1, np.int32)
            np.cumsum([len(r) for _, r, _ in sel], out=eoff[1:])
            rows_all = np.concatenate([np.asarray(r, np.int32) for _, r, _ in sel])
            y = kernels.grouped_ffn(xd, table, eoff, rows_all, H, inter, gs)
            ys.append(y)
            yrows.append(rows_all)
            yw.append(np.concatenate([np.asarray(w, np.float32) for _, _, w in sel]))
        kernels.combine(out, ys, yrows, yw, consume=True)   # the outputs are this call's own
        if items:
            kernels.moe_q4(xd, items, H, shape[0], shape[1], out)
        del keep   # the call is enqueued: stream order protects the blocks from here on
        return out if kernels.is_device(x) else out.cpu().numpy()

    def layer_table(self, layer: int, num_experts: int):
        """Device table of all int4 experts of a layer (expert id -> descriptor), for the prefill layer call."""
        return kernels.expert_table([self.get((layer, e)) for e in range(num_experts)])
