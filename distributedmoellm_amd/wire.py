"""Activations on the wire between a coordinator and its workers, on the device.

Mirrors ``moelan/protocol.py``'s ``WIRE_FORMATS``, ``WIRE_GROUP``,
``encode_rows`` and ``decode_rows`` (90-123), and the compute step of the
worker's ``moe`` op (``moelan/worker.py:337-354``): x decoded into HBM, the
store's layer call, y's touched rows encoded straight from HBM. The sockets
and message framing around them stay the reference's.

Arrays may be numpy (copied to the device and back, as a drop-in) or torch
tensors on the device (no copies). Encoding is bit-exact with the reference
for finite values; f16 rounds to nearest even as numpy's ``astype``.
"""

from __future__ import annotations

import numpy as np

from . import _lib, kernels

WIRE_FORMATS = ("f32", "f16", "int8")
WIRE_GROUP = 64   # int8: one scale per this many values (moelan/protocol.py:93)
_CODE = {"f32": 0, "f16": 1, "int8": 2}


def wire_group(d: int) -> int:
    """Values per int8 scale for rows of d values (moelan/protocol.py:108)."""
    return WIRE_GROUP if d % WIRE_GROUP == 0 else d


def encode_rows(a, wire: str, name: str, rows=None) -> dict:
    """``{name: rows of a}`` in the wire format (moelan/protocol.py:99-114):
    f16, or int8 with ``name + "_scale"`` f32 (n, d / wire_group(d)), or f32.
    ``rows`` selects (gathers) rows of ``a`` first, on the device."""
    import torch
    if wire not in _CODE:
        raise ValueError(f"wire format must be one of {WIRE_FORMATS}, not {wire!r}")
    kernels._need()
    ad = kernels._f32(a)
    if ad.dim() != 2:
        raise ValueError(f"expected rows (n, d), got shape {tuple(ad.shape)}")
    rd = None if rows is None else kernels.to_device(np.asarray(rows, np.int32) if not kernels.is_device(rows)
                                                      else rows, torch.int32)
    n = ad.shape[0] if rd is None else rd.numel()
    d = ad.shape[1]
    if rd is not None and n and (int(rd.min()) < 0 or int(rd.max()) >= ad.shape[0]):
        raise ValueError(f"rows out of range for {ad.shape[0]} rows")
    dtype = {"f32": torch.float32, "f16": torch.float16, "int8": torch.int8}[wire]
    out = torch.empty((n, d), dtype=dtype, device=ad.device)
    scale = torch.empty((n, d // wire_group(d)), dtype=torch.float32, device=ad.device) if wire == "int8" else None
    _lib.call("moe_wire_encode", kernels._ptr(ad), ad.stride(0), None if rd is None else kernels._ptr(rd), n, d,
              _CODE[wire], kernels._ptr(out), None if scale is None else kernels._ptr(scale),
              kernels.stream_handle())
    res = {name: out}
    if scale is not None:
        res[name + "_scale"] = scale
    if not kernels.is_device(a):
        res = {k: v.cpu().numpy() for k, v in res.items()}
    return res


def decode_rows(arrays: dict, name: str, out=None, rows=None):
    """f32 rows from ``arrays[name]`` (and ``name + "_scale"`` for int8),
    moelan/protocol.py:116-123. With ``out`` (a device f32 tensor) and ``rows``
    the decoded row r goes to ``out[rows[r]]`` instead of a new array."""
    import torch
    kernels._need()
    a = arrays[name]
    host = not kernels.is_device(a)
    if host:
        a = np.ascontiguousarray(a)
    ad = kernels.to_device(a)
    if ad.dtype == torch.int8:
        wire = 2
        sd = kernels._f32(arrays[name + "_scale"]).contiguous()
    elif ad.dtype == torch.float16:
        wire, sd = 1, None
    else:
        wire, sd = 0, None
        ad = ad.to(torch.float32)
    ad = ad.contiguous()
    n, d = ad.shape
    if wire == 2 and tuple(sd.shape) != (n, d // wire_group(d)):
        raise ValueError(f"{name}_scale has shape {tuple(sd.shape)}, expected {(n, d // wire_group(d))}")
    rd = None
    if out is None:
        out = torch.empty((n, d), dtype=torch.float32, device=ad.device)
        if rows is not None:
            raise ValueError("rows needs an out to scatter into")
    else:
        if not (kernels.is_device(out) and out.dtype == torch.float32 and out.stride(1) == 1 and out.shape[1] == d):
            raise ValueError("out must be a device f32 tensor of rows of the same width")
        if rows is not None:
            rd = kernels.to_device(np.asarray(rows, np.int32) if not kernels.is_device(rows) else rows, torch.int32)
            if rd.numel() != n or (n and (int(rd.min()) < 0 or int(rd.max()) >= out.shape[0])):
                raise ValueError("rows must give one row of out for every decoded row")
        elif out.shape[0] < n:
            raise ValueError(f"out has {out.shape[0]} rows, {n} decoded")
    _lib.call("moe_wire_decode", kernels._ptr(ad), None if sd is None else kernels._ptr(sd), wire, n, d,
              None if rd is None else kernels._ptr(rd), kernels._ptr(out), out.stride(0), kernels.stream_handle())
    return out.cpu().numpy() if (host and rows is None) else out


def worker_moe(store, layer: int, arrays: dict, wire: str = "f32"):
    """The compute step of the worker's ``moe`` op (moelan/worker.py:337-354):
    x decoded on the device, the layer's groups from ``experts`` / ``offsets``
    / ``rows`` / ``weights``, ``store.compute``, then y's touched rows encoded
    in ``wire``. Returns the reply's arrays: the encoded ``y`` and ``rows``."""
    x = decode_rows(arrays, "x")
    if not kernels.is_device(x):
        x = kernels.to_device(x)
    experts, offsets = np.asarray(arrays["experts"]), np.asarray(arrays["offsets"])
    rows = np.asarray(arrays["rows"])
    weights = np.asarray(arrays["weights"]).astype(np.float32, copy=False)
    groups = [(int(experts[i]), rows[offsets[i]:offsets[i + 1]], weights[offsets[i]:offsets[i + 1]])
              for i in range(len(experts))]
    y = store.compute(layer, x, groups)
    touched = np.unique(rows).astype(np.int32)
    return dict(encode_rows(y, wire, "y", rows=touched), rows=touched)
