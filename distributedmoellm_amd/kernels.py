"""The compute kernels of moelan's routed-expert path, on an MI355X.

Same module surface as ``moelan/kernels.py`` (flags 19-32, functions 920-1032)
so that ``experts.py`` / ``gguf.py`` style callers can select it as their
backend; every function runs hand-written HIP kernels (libmoehip.so, C ABI in
include/moehip.h) on the current ROCm device.

Arrays may be numpy (host: copied to the device for the call, results copied
back, as a drop-in) or torch tensors already on the device (no copies; the
result stays on the device). There is no CPU fallback: without the library or
a GPU ``ENABLED`` is False, ``WHY_DISABLED`` says why, and every kernel call
raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import sys
import warnings

import numpy as np

from . import _lib

ENABLED = False
WHY_DISABLED = ""
MAX_ROWS = 1 << 30          # every size runs on the device
ROW_DECODE_FROM = 4         # kept for callers that split on it (moelan/kernels.py:22)
BLAS_FROM = 8               # idem (moelan/kernels.py:23): the store sends such groups to the big-group path
FUSED = os.environ.get("MOELAN_FUSED", "1") != "0"
# The layer call rounds activations to int8 per group of 64 (or a multiple up to
# 512), as moelan's int8-activation kernels do (moelan/kernels.py:28-31);
# MOELAN_INT8_ACT=0 keeps them float (exact to the int4 weights).
INT8_ACT = os.environ.get("MOELAN_INT8_ACT", "1") != "0"
AVX2 = False

try:
    import torch
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

if os.environ.get("MOELAN_KERNELS", "1") == "0":
    WHY_DISABLED = "MOELAN_KERNELS=0"
elif torch is None:
    WHY_DISABLED = "torch is not importable"
elif _lib.load() is None:
    WHY_DISABLED = _lib.why_not()
elif _lib.lib().moe_device_count() < 1 or not torch.cuda.is_available():
    WHY_DISABLED = "no HIP device is visible"
else:
    _rc = _lib.lib().moe_init(torch.cuda.current_device())
    if _rc == 0:
        ENABLED = True
    else:
        WHY_DISABLED = _lib.last_error()


def warn_if_slow(stream=None) -> bool:
    """Print a loud notice when the HIP kernels are off. Returns True if so."""
    if ENABLED:
        return False
    stream = stream or sys.stderr
    bar = "!" * 78
    print(f"{bar}\n moelan's HIP expert kernels are OFF ({WHY_DISABLED}).\n"
          f" The routed-expert path cannot run on this machine.\n{bar}", file=stream, flush=True)
    return True


def _need() -> None:
    if not ENABLED:
        raise RuntimeError(f"HIP expert kernels are not available: {WHY_DISABLED}")


# ---------------------------------------------------------------- buffers

def device():
    return torch.device("cuda", torch.cuda.current_device())


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def is_device(a) -> bool:
    return torch is not None and isinstance(a, torch.Tensor) and a.is_cuda


def to_device(a, dtype=None):
    """A contiguous device tensor with the contents of ``a`` (numpy or torch)."""
    if isinstance(a, torch.Tensor):
        t = a if a.is_cuda else a.to(device())
    else:
        arr = np.ascontiguousarray(a)
        with warnings.catch_warnings():   # read-only memory maps: only read for the copy
            warnings.simplefilter("ignore")
            t = torch.from_numpy(arr)
        t = t.to(device())
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _f32(x):
    return to_device(x, torch.float32)


def _scale_kind(s) -> int:
    dt = s.dtype if isinstance(s, torch.Tensor) else np.dtype(s.dtype)
    if dt in (torch.float16, np.float16):
        return 1
    if dt in (torch.float32, np.float32):
        return 0
    raise TypeError(f"scales must be float32 or float16, not {dt}")


def _ret(y, like):
    """Results leave as they came: device tensors stay, numpy callers get numpy."""
    return y if is_device(like) else y.cpu().numpy()


def _ptr(t) -> int:
    return t.data_ptr()


# ---------------------------------------------------------------- one matrix

def q4_matmul_t(x, raw, s, gs: int, offset: bool):
    """x @ W.T for colibri int4 bytes; ``offset`` means raw was XOR-ed with 0x88."""
    _need()
    xd = _f32(x)
    if xd.dim() != 2:
        raise ValueError("x must be 2-D (rows, columns)")
    rd, sd = to_device(raw, torch.uint8), to_device(s)
    n, I = xd.shape
    O = rd.shape[0]
    if rd.numel() != O * (I // 2) or sd.numel() != O * (I // gs):
        raise ValueError(f"int4 matrix of {tuple(rd.shape)} bytes / {tuple(sd.shape)} scales does not match x {tuple(xd.shape)}, gs={gs}")
    y = torch.empty((n, O), dtype=torch.float32, device=xd.device)
    _lib.call("moe_q4_matmul_t", _ptr(xd), n, _ptr(rd), _ptr(sd), _scale_kind(sd), O, I, gs,
              1 if offset else 0, _ptr(y), stream_handle())
    return _ret(y, x)


def q8_matmul_t(x, q, s, gs: int):
    _need()
    xd = _f32(x)
    qd, sd = to_device(q, torch.int8), to_device(s)
    n, I = xd.shape
    O = qd.shape[0]
    if qd.numel() != O * I or sd.numel() != O * (I // gs):
        raise ValueError(f"int8 matrix {tuple(qd.shape)} / scales {tuple(sd.shape)} does not match x {tuple(xd.shape)}")
    y = torch.empty((n, O), dtype=torch.float32, device=xd.device)
    _lib.call("moe_q8_matmul_t", _ptr(xd), n, _ptr(qd), _ptr(sd), _scale_kind(sd), O, I, gs, _ptr(y),
              stream_handle())
    return _ret(y, x)


def gguf_matmul_t(x, raw, qtype: int, cols: int):
    """x @ W.T for a GGUF block-quantized W given as (rows, row bytes)."""
    _need()
    xd = _f32(x)
    rd = to_device(raw, torch.uint8)
    n = xd.shape[0]
    O = rd.shape[0]
    _check_gguf(rd, qtype, cols)
    if xd.shape[1] != cols:
        raise ValueError(f"x has {xd.shape[1]} columns, the matrix {cols}")
    y = torch.empty((n, O), dtype=torch.float32, device=xd.device)
    _lib.call("moe_gguf_matmul_t", _ptr(xd), n, _ptr(rd), int(qtype), O, int(cols), _ptr(y), stream_handle())
    return _ret(y, x)


# quantized GGUF type id -> (values, bytes) per block (moelan/gguf.py:36-42)
_GGUF_BLOCKS = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84),
                11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def _check_gguf(rd, qtype: int, cols: int) -> None:
    if qtype not in _GGUF_BLOCKS:
        raise ValueError(f"GGUF type {qtype} is not a quantized type ({sorted(_GGUF_BLOCKS)})")
    per, size = _GGUF_BLOCKS[qtype]
    if cols % per or rd.numel() != rd.shape[0] * (cols // per) * size:
        raise ValueError(f"GGUF rows of {rd.numel() // max(rd.shape[0], 1)} bytes do not hold {cols} type-{qtype} values")


def _check_out(out, O: int, I: int) -> None:
    if tuple(out.shape) != (O, I):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(O, I)}")


# ---------------------------------------------------------------- dequant

def _into(out, y):
    if is_device(out):
        out.copy_(y.view(out.shape))
    else:
        out[...] = y.cpu().numpy().reshape(out.shape)
    return out


def q4_dequant(raw, s, gs: int, offset: bool, out):
    _need()
    rd, sd = to_device(raw, torch.uint8), to_device(s)
    O, I = rd.shape[0], rd.numel() // rd.shape[0] * 2
    _check_out(out, O, I)
    if sd.numel() != O * (I // gs):
        raise ValueError(f"{sd.numel()} scales for a {O}x{I} matrix with groups of {gs}")
    y = out if (is_device(out) and out.is_contiguous() and out.dtype == torch.float32) else \
        torch.empty((O, I), dtype=torch.float32, device=rd.device)
    _lib.call("moe_q4_dequant", _ptr(rd), _ptr(sd), _scale_kind(sd), O, I, gs, 1 if offset else 0, _ptr(y),
              stream_handle())
    return out if y is out else _into(out, y)


def q8_dequant(q, s, gs: int, out):
    _need()
    qd, sd = to_device(q, torch.int8), to_device(s)
    O, I = qd.shape
    _check_out(out, O, I)
    if sd.numel() != O * (I // gs):
        raise ValueError(f"{sd.numel()} scales for a {O}x{I} matrix with groups of {gs}")
    y = out if (is_device(out) and out.is_contiguous() and out.dtype == torch.float32) else \
        torch.empty((O, I), dtype=torch.float32, device=qd.device)
    _lib.call("moe_q8_dequant", _ptr(qd), _ptr(sd), _scale_kind(sd), O, I, gs, _ptr(y), stream_handle())
    return out if y is out else _into(out, y)


def gguf_dequant(raw, qtype: int, out):
    _need()
    rd = to_device(raw, torch.uint8)
    O, cols = out.shape
    if rd.shape[0] != O:
        raise ValueError(f"{rd.shape[0]} GGUF rows for an output of {O} rows")
    _check_gguf(rd, qtype, cols)
    y = out if (is_device(out) and out.is_contiguous() and out.dtype == torch.float32) else \
        torch.empty((O, cols), dtype=torch.float32, device=rd.device)
    _lib.call("moe_gguf_dequant", _ptr(rd), int(qtype), O, cols, _ptr(y), stream_handle())
    return out if y is out else _into(out, y)


# ---------------------------------------------------------------- one layer

def int8_act_for(H: int, I: int, gs: int) -> bool:
    """Whether :func:`moe_q4` runs experts of this shape with int8 activations
    (moelan/kernels.py:920-922; groups of up to 512 here)."""
    return INT8_ACT and gs % 64 == 0 and gs <= 512 and H % gs == 0 and I % gs == 0


class HostCopies:
    """Device copies of host arrays that callers hand over again and again:
    the int4 matrices of moelan's own store, numpy views of a memory map with
    no device side of their own. A copy is keyed by the array's address,
    size, dtype and shape, and lives while some host array with that key
    does (weak references), so a view made again of the same mapped bytes
    finds the copy instead of uploading it again, and memory the host frees
    takes its copy with it. The host arrays are taken as fixed once handed
    over (moelan's are read-only maps or load-time copies)."""

    def __init__(self):
        import threading
        self._lock = threading.RLock()
        self._copies: dict = {}     # key -> [device tensor, live host arrays]
        self._watch: dict = {}      # id(host array) -> (weakref, key)
        self.uploads = 0            # arrays copied to the device so far
        self.upload_bytes = 0

    def get(self, a, dtype=None):
        """The device copy of host array ``a`` (made now if there is none)."""
        import weakref
        a = a if isinstance(a, np.ndarray) else np.asarray(a)
        key = (a.__array_interface__["data"][0], a.nbytes, a.dtype.str, a.shape)
        with self._lock:
            ent = self._copies.get(key)
            if ent is None:
                ent = self._copies[key] = [to_device(a, dtype), 0]
                self.uploads += 1
                self.upload_bytes += a.nbytes
            w = self._watch.get(id(a))
            if w is None or w[0]() is not a:
                self._watch[id(a)] = (weakref.ref(a, lambda r, i=id(a): self._gone(i, r)), key)
                ent[1] += 1
            # a weak-reference callback run meanwhile (garbage collection in
            # this thread) may have dropped the entry while ``a`` lives on
            self._copies[key] = ent
            return ent[0]

    def _gone(self, ident, ref) -> None:
        with self._lock:
            w = self._watch.get(ident)
            if w is None or w[0] is not ref:
                return
            del self._watch[ident]
            ent = self._copies.get(w[1])
            if ent is not None:
                ent[1] -= 1
                if ent[1] <= 0:
                    del self._copies[w[1]]

    def __len__(self) -> int:
        return len(self._copies)

    def nbytes(self) -> int:
        with self._lock:
            return sum(t.numel() * t.element_size() for t, _ in self._copies.values())


HOST_COPIES = HostCopies()


def _q4_arrays(m):
    """(raw uint8 [O, I/2], scales [O, I/gs]) of an int4 matrix on the device:
    its own device arrays, or for a matrix with host arrays only (moelan's
    Packed4: ``raw``, ``s``, ``gs``, ``shape``, ``offset``) the host copy cache's."""
    if hasattr(m, "device_arrays"):
        return m.device_arrays()
    O, I = m.shape
    raw, s = np.asarray(m.raw), np.asarray(m.s)
    if raw.dtype != np.uint8 or raw.size != O * I // 2 or s.size != O * (I // m.gs) or \
            s.dtype not in (np.float32, np.float16):
        return None
    return HOST_COPIES.get(raw).reshape(O, I // 2), HOST_COPIES.get(s).reshape(O, I // m.gs)


def q4_expert_ptrs(e):
    """What :func:`moe_q4` needs of one int4 expert: the device addresses of its
    four arrays, the XOR for its nibbles and whether its scales are f16; None if
    it does not qualify (moelan/kernels.py:929-939). Experts whose matrices
    hold host arrays only get device copies from :data:`HOST_COPIES`, made
    once per host array."""
    gu, dn = e.gu, e.down
    if not all(hasattr(m, a) for m in (gu, dn) for a in ("raw", "s", "gs", "shape", "offset")):
        return None
    if gu.gs != dn.gs or gu.offset != dn.offset:
        return None
    ga, da = _q4_arrays(gu), _q4_arrays(dn)
    if ga is None or da is None or ga[1].dtype != da[1].dtype:
        return None
    (gr, gsc), (dr, dsc) = ga, da
    return (gr.data_ptr(), gsc.data_ptr(), dr.data_ptr(), dsc.data_ptr(), 0 if gu.offset else 0x88,
            1 if gsc.dtype == torch.float16 else 0)


def pair_lists(rows, weights):
    """(poff, prow, pw, rrow, rptr, rpair) of a layer call, host int32/f32 arrays:
    pairs in item order, then the pairs of each touched row in ascending order."""
    k = len(rows)
    counts = np.array([len(r) for r in rows], np.int64)
    P = int(counts.sum())
    prow = np.concatenate([np.asarray(r, np.int64).reshape(-1) for r in rows]).astype(np.int32) if P else \
        np.zeros(0, np.int32)
    pw = np.concatenate([np.asarray(w, np.float32).reshape(-1) for w in weights]) if P else np.zeros(0, np.float32)
    poff = np.zeros(k + 1, np.int32)
    np.cumsum(counts, out=poff[1:])
    order = np.argsort(prow, kind="stable")
    rrow, starts = np.unique(prow[order], return_index=True)
    rptr = np.append(starts, P).astype(np.int32)
    return poff, prow, pw, rrow.astype(np.int32), rptr, order.astype(np.int32)


def upload_small(host: np.ndarray):
    """A small host array onto the device (as bytes, uint8) without waiting: staged in freshly
    allocated pinned memory (torch's pinned allocator keeps that block until
    the copy has run) and copied asynchronously on the current stream, so the
    host goes on queueing work instead of waiting for the stream to drain, as a
    copy from pageable memory would."""
    arr = np.ascontiguousarray(host)
    pinned = torch.empty(arr.nbytes, dtype=torch.uint8, pin_memory=True)
    pinned.numpy()[:] = arr.reshape(-1).view(np.uint8)
    return pinned.to(device(), non_blocking=True)


def upload_parts(parts):
    """Host byte strings into one device buffer (one asynchronous copy),
    256-byte aligned parts; returns (buffer, [device address of each part])."""
    offs, pos = [], 0
    for b in parts:
        offs.append(pos)
        pos += (len(b) + 255) // 256 * 256
    host = np.zeros(max(pos, 256), np.uint8)
    for o, b in zip(offs, parts):
        host[o:o + len(b)] = np.frombuffer(b, np.uint8)
    buf = upload_small(host)
    base = buf.data_ptr()
    return buf, [base + o for o in offs]


def combine(out, ys, rows, weights, consume: bool = False) -> None:
    """out[rows_i] += ys_i * weights_i for each i, per row in the given order
    (HIP combine kernel); ``ys`` are device tensors [len(rows_i), H].
    ``consume``: a single contiguous f32 ``ys[0]`` is the kernel's scratch
    as it is (its contents are lost) instead of a copy."""
    _need()
    if not ys:
        return
    H = out.shape[1]
    if consume and len(ys) == 1 and ys[0].dtype == torch.float32 and ys[0].is_contiguous():
        y = ys[0].reshape(-1, H)
    else:
        y = torch.cat([t.reshape(-1, H) for t in ys], 0).contiguous()
    _, _, pw, rrow, rptr, rpair = pair_lists(rows, weights)
    buf, (pw_p, rrow_p, rptr_p, rpair_p) = upload_parts([pw.tobytes(), rrow.tobytes(), rptr.tobytes(),
                                                         rpair.tobytes()])
    # y is a temporary here: the kernel may use it as scratch
    max_pairs = int(np.diff(rptr).max())
    _lib.call("moe_combine", _ptr(y), H, pw_p, rrow_p, rptr_p, rpair_p, len(rrow), max_pairs, _ptr(out),
              out.shape[1], H, stream_handle())


class LayerMeta:
    """A layer call's pair lists on the device, in one upload: the expert table,
    pairs per expert (poff, prow, pw) and pairs per touched row (rrow, rptr, rpair)."""

    def __init__(self, ptrs, rows, weights):
        k = len(ptrs)
        poff, prow, pw, rrow, rptr, rpair = pair_lists(rows, weights)
        table = (_lib.Q4Expert * max(k, 1))()
        for i, p in enumerate(ptrs):
            table[i] = _lib.Q4Expert(p[0], p[1], p[2], p[3], p[4], p[5] if len(p) > 5 else 0)
        self.ptrs = [tuple(p) for p in ptrs]
        self.buf, addrs = upload_parts([bytes(table), poff.tobytes(), prow.tobytes(), pw.tobytes(), rrow.tobytes(),
                                        rptr.tobytes(), rpair.tobytes()])
        (self.table, self.poff, self.prow, self.pw, self.rrow, self.rptr, self.rpair) = addrs
        counts = np.diff(poff)
        self.k, self.P, self.nr = k, int(poff[-1]), len(rrow)
        self.max_rows = int(counts.max()) if k else 0
        self.row_hi = int(prow.max()) + 1 if self.P else 0   # rows of x / out the call touches
        if self.P and int(prow.min()) < 0:
            raise ValueError("negative row index")


def moe_q4(x, items, H: int, I: int, gs: int, out, int8: bool | None = None) -> None:
    """Add ``sum_e w * expert_e(x[rows])`` into ``out`` for int4 experts in one
    call (moelan/kernels.py:942-968). ``items``: (ptrs from
    :func:`q4_expert_ptrs`, rows, gate weights) per expert; the experts'
    device arrays must stay alive until the call has run. Activations are
    rounded to int8 when :func:`int8_act_for` says so (``int8`` overrides)."""
    _need()
    if not items:
        return
    meta = LayerMeta([p for p, _, _ in items], [r for _, r, _ in items], [w for _, _, w in items])
    moe_q4_run(x, meta, H, I, gs, out, int8=int8)


def moe_q4_run(x, meta: LayerMeta, H: int, I: int, gs: int, out, workspace=None, int8: bool | None = None) -> None:
    """The layer call on pair lists already on the device."""
    _need()
    xd = _f32(x)
    od = out if (is_device(out) and out.dtype == torch.float32 and out.is_contiguous()) else _f32(out)
    if xd.shape[1] != H or od.shape[1] != H:
        raise ValueError(f"x and out need {H} columns, have {xd.shape[1]} and {od.shape[1]}")
    if meta.row_hi > min(xd.shape[0], od.shape[0]):
        raise ValueError(f"row {meta.row_hi - 1} is out of range for x/out of {xd.shape[0]}/{od.shape[0]} rows")
    for p in meta.ptrs:
        if not all(p[:4]):
            raise ValueError("null expert address")
    if int8 is None:
        int8 = int8_act_for(H, I, gs)
    elif int8 and not (gs % 64 == 0 and gs <= 512 and H % gs == 0 and I % gs == 0):
        raise ValueError(f"int8 activations need groups of 64 (or a multiple up to 512) dividing H and I, not {gs}")
    if int8:
        name, need = "moe_q4_layer_i8", _lib.lib().moe_q4_layer_i8_workspace(max(meta.P, 1), H, I, gs)
    else:
        name, need = "moe_q4_layer", _lib.lib().moe_q4_layer_workspace(max(meta.P, 1), H, I)
    ws = workspace if workspace is not None and workspace.numel() >= need else \
        torch.empty(need, dtype=torch.uint8, device=xd.device)
    _lib.call(name, _ptr(xd), xd.shape[1], meta.table, None, meta.k, meta.poff, meta.prow, meta.pw,
              meta.P, meta.rrow, meta.rptr, meta.rpair, meta.nr, _ptr(od), od.shape[1], H, I, gs,
              meta.max_rows, _ptr(ws), ws.numel(), stream_handle())
    if od is not out:
        _into(out, od)


def round_q8(x, gs: int):
    """Rows of ``x`` rounded to int8 per group of ``gs`` (moelan/kernels.py:
    833-852): (q int8 (n, K), scales f32 (n, K/gs), 8 * group sums int32).
    ``q`` keeps the columns in their own order (the device stores each 32-column
    chunk as even columns then odd ones; this reorders it back)."""
    _need()
    xd = _f32(x)
    n, K = xd.shape
    q = torch.empty((n, K), dtype=torch.int8, device=xd.device)
    d = torch.empty((n, K // gs), dtype=torch.float32, device=xd.device)
    s8 = torch.empty((n, K // gs), dtype=torch.int32, device=xd.device)
    _lib.call("moe_round_q8", _ptr(xd), K, None, n, K, int(gs), _ptr(q), _ptr(d), _ptr(s8), stream_handle())
    q = q.view(n, K // 32, 2, 16).transpose(2, 3).reshape(n, K)
    if is_device(x):
        return q, d, s8
    return q.cpu().numpy(), d.cpu().numpy(), s8.cpu().numpy()


# ---------------------------------------------------------------- prompt reading

MFMA_FROM = 16   # rows per expert from which the store uses the MFMA grouped GEMM (f16 operands)


def _i32(a):
    if is_device(a) or isinstance(a, torch.Tensor):
        return to_device(a, torch.int32)
    arr = np.ascontiguousarray(a, np.int32)
    return upload_small(arr).view(torch.int32).reshape(arr.shape)


def router_logits(x, router):
    """logits = x @ router.T in f32 on the device (moelan/model.py:597)."""
    _need()
    xd, rd = _f32(x), _f32(router)
    T, H = xd.shape
    E = rd.shape[0]
    if rd.shape[1] != H:
        raise ValueError(f"router has {rd.shape[1]} columns, x {H}")
    out = torch.empty((T, E), dtype=torch.float32, device=xd.device)
    need = _lib.lib().moe_router_logits_workspace(T, E, H)
    ws = torch.empty(max(need, 4), dtype=torch.uint8, device=xd.device)
    _lib.call("moe_router_logits", _ptr(xd), H, _ptr(rd), T, E, H, _ptr(out), _ptr(ws), ws.numel(), stream_handle())
    return _ret(out, x)


def route(logits, top_k: int, normalize: bool):
    """Softmax top-k router (moelan/model.py:160-167): (idx int32 (n,k), w f32 (n,k))."""
    _need()
    ld = _f32(logits)
    T, E = ld.shape
    idx = torch.empty((T, top_k), dtype=torch.int32, device=ld.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=ld.device)
    _lib.call("moe_route", _ptr(ld), T, E, int(top_k), 1 if normalize else 0, _ptr(idx), _ptr(w), stream_handle())
    return (idx, w) if is_device(logits) else (idx.cpu().numpy(), w.cpu().numpy())


def group_by_expert(idx, w, num_experts: int | None = None, with_pos: bool = False):
    """Stable grouping by expert (moelan/model.py:226-236): experts, offsets, rows, weights.
    ``num_experts`` bounds the expert ids (default: max id + 1)."""
    _need()
    idd, wd = _i32(idx), _f32(w)
    T, k = idd.shape
    E = int(num_experts) if num_experts is not None else int(idd.max().item()) + 1
    dev = idd.device
    eoff = torch.empty(E + 1, dtype=torch.int32, device=dev)
    rows = torch.empty(T * k, dtype=torch.int32, device=dev)
    wts = torch.empty(T * k, dtype=torch.float32, device=dev)
    pos = torch.empty(T * k, dtype=torch.int32, device=dev)
    experts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    n_used = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("moe_group_by_expert", _ptr(idd), _ptr(wd), T, k, E, _ptr(eoff), _ptr(rows), _ptr(wts), _ptr(pos),
              _ptr(experts), _ptr(offsets), _ptr(n_used), stream_handle())
    nu = int(n_used.item())
    total = int(offsets[nu].item())  # picks with a valid expert id (all of them for router output)
    res = (experts[:nu], offsets[:nu + 1], rows[:total], wts[:total])
    if not is_device(idx):
        res = tuple(t.cpu().numpy() for t in res)
    if with_pos:
        return res + ((eoff, pos),)
    return res


_TABLES: "OrderedDict" = None   # descriptors -> their device table, the last few built
_TABLES_KEEP = 16


def expert_table(experts) -> "torch.Tensor":
    """A device array of moe_q4_expert descriptors for int4 experts (None entries: zeros).
    Tables are kept by their contents (device addresses), so a layer's
    repeated calls upload it once; callers only read them."""
    global _TABLES
    from collections import OrderedDict
    descs = []
    for i, e in enumerate(experts):
        if e is None:
            descs.append(None)
            continue
        p = getattr(e, "fused", None) or q4_expert_ptrs(e)
        if p is None:
            raise ValueError(f"expert {i} is not an int4 expert with matching gate|up / down layout")
        if any(a % 16 for a in p[:4]):
            raise ValueError(f"expert {i}: weight arrays must be 16-byte aligned in HBM")
        descs.append(tuple(p))
    key = tuple(descs)
    if _TABLES is None:
        _TABLES = OrderedDict()
    hit = _TABLES.get(key)
    if hit is not None and hit.device == device():
        _TABLES.move_to_end(key)
        return hit
    table = (_lib.Q4Expert * max(len(experts), 1))()
    for i, p in enumerate(descs):
        if p is not None:
            table[i] = _lib.Q4Expert(*p)
    t = upload_small(np.frombuffer(bytes(table), np.uint8))
    _TABLES[key] = t
    while len(_TABLES) > _TABLES_KEEP:
        _TABLES.popitem(last=False)
    return t


def grouped_ffn(x, table, eoff, rows, H: int, I: int, gs: int):
    """y[q] = expert_e(x[rows[q]]) for each grouped row (MFMA path, f16 operands)."""
    _need()
    xd = _f32(x)
    eo, rw = _i32(eoff), _i32(rows)
    P = rw.numel()
    nexp = eo.numel() - 1
    y = torch.empty((P, H), dtype=torch.float32, device=xd.device)
    if P == 0:
        return y
    need = _lib.lib().moe_q4_grouped_ffn_workspace(P, H, I)
    ws = torch.empty(need, dtype=torch.uint8, device=xd.device)
    _lib.call("moe_q4_grouped_ffn", _ptr(xd), xd.shape[1], _ptr(table), nexp, _ptr(eo), _ptr(rw), P, H, I, gs,
              _ptr(y), H, _ptr(ws), ws.numel(), stream_handle())
    return y


def prefill_layer(x, router, table, top_k: int, normalize: bool, H: int, I: int, gs: int, out=None, workspace=None):
    """One MoE layer over x's rows on the device: router, route, group, grouped
    expert FFN, weighted combine (MoEModel._ffn + LocalBackend + ExpertStore.compute)."""
    _need()
    xd, rd = _f32(x), _f32(router)
    T = xd.shape[0]
    E = rd.shape[0]
    od = out if out is not None else torch.empty((T, H), dtype=torch.float32, device=xd.device)
    need = _lib.lib().moe_prefill_workspace(T, E, top_k, H, I)
    ws = workspace if workspace is not None and workspace.numel() >= need else \
        torch.empty(need, dtype=torch.uint8, device=xd.device)
    _lib.call("moe_prefill_layer", _ptr(xd), xd.shape[1], _ptr(rd), T, E, int(top_k), 1 if normalize else 0,
              _ptr(table), H, I, gs, _ptr(od), od.shape[1], _ptr(ws), ws.numel(), stream_handle())
    return od if is_device(x) else od.cpu().numpy()


def q4_matmul_t_mfma(x, raw, s, gs: int, offset: bool):
    """x @ W.T for int4 bytes on many rows through the f16 MFMA path (~1e-3 relative)."""
    _need()
    xd = _f32(x)
    rd, sd = to_device(raw, torch.uint8), to_device(s)
    n, I = xd.shape
    O = rd.shape[0]
    if rd.numel() != O * (I // 2) or sd.numel() != O * (I // gs):
        raise ValueError("int4 matrix does not match x")
    y = torch.empty((n, O), dtype=torch.float32, device=xd.device)
    _lib.call("moe_q4_gemm", _ptr(xd), n, _ptr(rd), _ptr(sd), _scale_kind(sd), O, I, gs, 1 if offset else 0, _ptr(y),
              stream_handle())
    return _ret(y, x)
