"""GGUF block-quantized expert matrices on the device.

Mirrors ``moelan/gguf.py``'s quantized-matrix part: ``QTYPES`` (36-42),
``dequantize`` (258-275), ``QuantMatrix`` (278-314), ``Stacked`` (317-333),
``random_blocks`` (547-555) and ``synthetic_expert`` (558-564). The rows keep
their GGUF bytes (one device copy, uploaded on first use); every quantized
type (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) runs on the
HIP kernels. F32 / F16 / BF16 tensors are not expert weights here.
"""

from __future__ import annotations

import numpy as np

from . import kernels

# ggml type id -> (name, elements per block, bytes per block)
QTYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
          6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84),
          11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
          14: ("Q6_K", 256, 210), 30: ("BF16", 1, 2)}
QTYPE_IDS = {v[0]: k for k, v in QTYPES.items()}
QUANTIZED = {k for k, v in QTYPES.items() if v[1] > 1}
SUPPORTED = QUANTIZED   # the types these kernels run

# offsets of the f16 scale fields in each block (moelan/gguf.py:543-545)
_SCALE_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 10: (80, 82), 11: (108,),
                 12: (0, 2), 13: (0, 2), 14: (208,)}


def dequantize(raw, qtype: int, cols: int, out=None):
    """(rows, row bytes) quantized -> (rows, cols) float32, bit-exact."""
    if qtype not in SUPPORTED:
        raise ValueError(f"GGUF type {QTYPES.get(qtype, (qtype,))[0]} is not supported on the device")
    if out is None:
        if kernels.is_device(raw):
            import torch
            out = torch.empty((raw.shape[0], cols), dtype=torch.float32, device=raw.device)
        else:
            out = np.empty((raw.shape[0], cols), np.float32)
    return kernels.gguf_dequant(raw, qtype, out)


class QuantMatrix:
    """A GGUF-quantized (rows, cols) weight, multiplied straight from its bytes."""

    __slots__ = ("raw", "qtype", "shape", "_dev")

    def __init__(self, raw, qtype: int, cols: int):
        if qtype not in SUPPORTED:
            raise ValueError(f"GGUF type {QTYPES.get(qtype, (qtype,))[0]} is not supported on the device")
        self.raw, self.qtype = raw, qtype
        self.shape = (raw.shape[0], cols)
        self._dev = None

    def device_arrays(self):
        if self._dev is None:
            import torch
            self._dev = (kernels.to_device(self.raw, torch.uint8).reshape(self.raw.shape[0], -1),)
        return self._dev

    def host_arrays(self):
        """The host array device_arrays() uploads, with its device shape."""
        return [(self.raw, (self.raw.shape[0], -1))]

    def matmul_t(self, x):
        return kernels.gguf_matmul_t(x, self.device_arrays()[0], self.qtype, self.shape[1])

    def dequant(self):
        r = self.device_arrays()[0]
        y = dequantize(r, self.qtype, self.shape[1])
        return y if kernels.is_device(self.raw) else y.cpu().numpy()

    @property
    def nbytes(self) -> int:
        return int(self.raw.nbytes)


class Stacked:
    """Gate and up projections side by side: (gate rows + up rows, cols)."""

    __slots__ = ("parts",)

    def __init__(self, *parts):
        self.parts = parts

    def matmul_t(self, x):
        import torch
        ys = [p.matmul_t(x) for p in self.parts]
        if kernels.is_device(ys[0]):
            return torch.cat(ys, dim=1)
        return np.concatenate(ys, axis=1)

    def dequant(self):
        import torch
        ds = [p.dequant() for p in self.parts]
        return torch.cat(ds, 0) if kernels.is_device(ds[0]) else np.concatenate(ds, 0)

    @property
    def nbytes(self):
        return sum(p.nbytes for p in self.parts)


def random_blocks(rows: int, cols: int, qtype: int, rng=None, scale: float | None = 0.01) -> np.ndarray:
    """Random but well-behaved quantized rows: every byte uniform, the f16 scale
    fields set to ``scale`` (None: each drawn from |N(0, 0.01)|)."""
    rng = rng or np.random.default_rng(0)
    _, block, size = QTYPES[qtype]
    raw = rng.integers(0, 256, (rows, cols // block, size), dtype=np.uint8)
    fields = _SCALE_FIELDS.get(qtype, ())
    for off in fields:
        if scale is None:
            v = np.abs(rng.normal(0.0, 0.01, (rows, cols // block))).astype(np.float16)
        else:
            v = np.full((rows, cols // block), scale, np.float16)
        raw[:, :, off:off + 2] = v.view(np.uint8).reshape(rows, cols // block, 2)
    return raw.reshape(rows, cols // block * size)


def synthetic_expert(hidden: int, inter: int, types: list[str], rng=None, scale=None):
    """A random expert in the given GGUF types (gate, up, down)."""
    from .experts import Expert
    rng = rng or np.random.default_rng(0)
    g, u, d = (QTYPE_IDS[t] for t in types)

    def mk(q, o, i):
        return QuantMatrix(random_blocks(o, i, q, rng, scale=scale), q, i)
    return Expert(Stacked(mk(g, inter, hidden), mk(u, inter, hidden)), mk(d, hidden, inter), inter)
