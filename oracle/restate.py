"""CPU restatement of moelan's routed-expert arithmetic: the oracle.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, as the checker; the product package
(distributedmoellm_amd) never imports, links or runs anything under oracle/.

Each function restates one reference function (file:line of moelan 0.1.0) in
numpy. ``exact`` variants compute in float64 from the exactly decoded weights
(the value the f32 kernels approximate); the others keep the reference's own
f32 formulas where it matters (bit-exact decoders).

Pinning (what checks each function independently of this restatement) is
listed in tests/test_oracle.py; a function without such a check would be
marked "parity unpinned" here, and none is.
"""

from __future__ import annotations

import numpy as np

# ggml type id -> (name, values per block, bytes per block)   moelan/gguf.py:36-42
QTYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
          6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84),
          11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
          14: ("Q6_K", 256, 210), 30: ("BF16", 1, 2)}
Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 2, 3, 6, 7, 8, 10, 11, 12, 13, 14


# ------------------------------------------------------------------ int4 / int8

def q4_unpack(raw: np.ndarray, offset: bool) -> np.ndarray:
    """Unsigned nibbles u = v + 8 as uint8 [O, I]: low nibble -> even column.
    moelan/experts.py:193-203 (XOR 0x88 unless ``offset``)."""
    rr = raw if offset else np.bitwise_xor(raw, 0x88)
    O, half = rr.shape
    u = np.empty((O, half, 2), np.uint8)
    np.bitwise_and(rr, 15, out=u[:, :, 0])
    np.right_shift(rr, 4, out=u[:, :, 1])
    return u.reshape(O, 2 * half)


def q4_values(raw: np.ndarray, offset: bool) -> np.ndarray:
    """Signed int4 values v in -8..7 as int8 [O, I] (Packed4.to_int8, moelan/experts.py:205-211)."""
    return (q4_unpack(raw, offset).astype(np.int16) - 8).astype(np.int8)


def q4_dequant(raw, s, gs: int, offset: bool) -> np.ndarray:
    """f32 W = float32(u - 8) * s, one rounding. moelan/kernels.py:215-228."""
    v = q4_values(raw, offset).astype(np.float32)
    O, I = v.shape
    s32 = np.asarray(s).astype(np.float32).reshape(O, I // gs)
    return (v.reshape(O, I // gs, gs) * s32[:, :, None]).reshape(O, I)


def q8_dequant(q, s, gs: int) -> np.ndarray:
    """f32 W = float32(q) * s. moelan/kernels.py:230-237."""
    O, I = q.shape
    s32 = np.asarray(s).astype(np.float32).reshape(O, I // gs)
    return (q.astype(np.float32).reshape(O, I // gs, gs) * s32[:, :, None]).reshape(O, I)


def q4_dequant64(raw, s, gs: int, offset: bool) -> np.ndarray:
    """W = v * s in float64 with no rounding (the value every f32 path approximates)."""
    v = q4_values(raw, offset).astype(np.float64)
    O, I = v.shape
    s64 = np.asarray(s).astype(np.float64).reshape(O, I // gs)
    return (v.reshape(O, I // gs, gs) * s64[:, :, None]).reshape(O, I)


def q8_dequant64(q, s, gs: int) -> np.ndarray:
    O, I = q.shape
    s64 = np.asarray(s).astype(np.float64).reshape(O, I // gs)
    return (q.astype(np.float64).reshape(O, I // gs, gs) * s64[:, :, None]).reshape(O, I)


def matmul_t_exact(x, W) -> np.ndarray:
    """x @ W.T in float64 (the exact value the f32 kernels approximate)."""
    return np.asarray(x, np.float64) @ np.asarray(W, np.float64).T


def q4_matmul_t(x, raw, s, gs: int, offset: bool) -> np.ndarray:
    """x @ W.T for colibri int4 (moelan/kernels.py:1018-1027, _q4 :85-106), float64."""
    return matmul_t_exact(x, q4_dequant64(raw, s, gs, offset))


def q4_matmul_t_f32(x, raw, s, gs: int, offset: bool) -> np.ndarray:
    """The reference's own f32 formula: sum_g s*sum(u*x) - 8*(group sums of x) @ s.T
    (moelan/kernels.py:1024-1026 and the numpy path moelan/experts.py:222-232)."""
    x = np.ascontiguousarray(x, np.float32)
    u = q4_unpack(raw, offset).astype(np.float32)
    O, I = u.shape
    s32 = np.asarray(s, np.float32).reshape(O, I // gs)
    f = (u.reshape(O, I // gs, gs) * s32[:, :, None]).reshape(O, I)
    y = x @ f.T
    y -= np.float32(8.0) * (x.reshape(-1, I // gs, gs).sum(2) @ s32.T)
    return y


def q8_matmul_t(x, q, s, gs: int) -> np.ndarray:
    """x @ W.T for int8 group-quantized W (moelan/kernels.py:1030-1032), float64."""
    return matmul_t_exact(x, q8_dequant64(q, s, gs))


# ------------------------------------------------------------------ GGUF

def gguf_f16(lo, hi) -> np.ndarray:
    """moelan/kernels.py:244-255: IEEE half, except exponent 31 (Inf and NaN) -> signed inf."""
    h = np.asarray(lo).astype(np.uint16) | (np.asarray(hi).astype(np.uint16) << 8)
    v = h.view(np.float16).astype(np.float32)
    special = (h & 0x7C00) == 0x7C00
    return np.where(special, np.where(h & 0x8000, np.float32(-np.inf), np.float32(np.inf)), v).astype(np.float32)


def dq_q8_0(raw: np.ndarray, cols: int) -> np.ndarray:
    """(rows, 34*nb) -> (rows, cols): d * q. moelan/kernels.py:262-268."""
    rows = raw.shape[0]
    b = raw.reshape(rows, cols // 32, 34)
    d = gguf_f16(b[:, :, 0], b[:, :, 1])
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (d[:, :, None] * q).reshape(rows, cols)


def scale_min_k4(j: int, s: np.ndarray):
    """Sub-block j's 6-bit scale and min from the 12 packed bytes (moelan/kernels.py:310-316).
    ``s`` is (..., 12) uint8; returns int32 arrays."""
    s = s.astype(np.int32)
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    sc = (s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4)
    m = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, m


def dq_q4_k(raw: np.ndarray, cols: int) -> np.ndarray:
    """(rows, 144*nb) -> (rows, cols). moelan/kernels.py:318-336: for k = 0..3,
    byte 16+32k+l gives value 64k+l (low nibble, sub-block 2k) and 64k+32+l
    (high nibble, sub-block 2k+1); w = (d*sc)*q - dmin*m, f32, no contraction."""
    rows = raw.shape[0]
    nb = cols // 256
    b = raw.reshape(rows, nb, 144)
    d = gguf_f16(b[:, :, 0], b[:, :, 1])
    dmin = gguf_f16(b[:, :, 2], b[:, :, 3])
    sc = b[:, :, 4:16]
    qs = b[:, :, 16:].reshape(rows, nb, 4, 32).astype(np.int32)
    out = np.empty((rows, nb, 4, 64), np.float32)
    for k in range(4):
        s1, m1 = scale_min_k4(2 * k, sc)
        s2, m2 = scale_min_k4(2 * k + 1, sc)
        d1, mm1 = d * s1.astype(np.float32), dmin * m1.astype(np.float32)
        d2, mm2 = d * s2.astype(np.float32), dmin * m2.astype(np.float32)
        lo = (qs[:, :, k, :] & 15).astype(np.float32)
        hi = (qs[:, :, k, :] >> 4).astype(np.float32)
        out[:, :, k, :32] = d1[:, :, None] * lo - mm1[:, :, None]
        out[:, :, k, 32:] = d2[:, :, None] * hi - mm2[:, :, None]
    return out.reshape(rows, cols)


def _blocks(raw: np.ndarray, cols: int, qtype: int) -> np.ndarray:
    _, per, size = QTYPES[qtype]
    return np.asarray(raw).reshape(raw.shape[0], cols // per, size)


def _f32(v) -> np.ndarray:
    return np.asarray(v).astype(np.float32)


def dq_q4_0(raw: np.ndarray, cols: int) -> np.ndarray:
    """18-byte blocks (moelan/kernels.py:270-278): f16 d, 16 bytes; byte j holds
    value j (low nibble) and j+16 (high); w = d * (q - 8)."""
    b = _blocks(raw, cols, Q4_0)
    d = gguf_f16(b[..., 0], b[..., 1])[..., None]
    q = b[..., 2:18].astype(np.int32)
    return np.concatenate([d * _f32((q & 15) - 8), d * _f32((q >> 4) - 8)], -1).reshape(raw.shape[0], cols)


def dq_q4_1(raw: np.ndarray, cols: int) -> np.ndarray:
    """20-byte blocks (moelan/kernels.py:280-289): f16 d, f16 min, 16 bytes; w = d * q + min."""
    b = _blocks(raw, cols, Q4_1)
    d = gguf_f16(b[..., 0], b[..., 1])[..., None]
    mn = gguf_f16(b[..., 2], b[..., 3])[..., None]
    q = b[..., 4:20].astype(np.int32)
    return np.concatenate([d * _f32(q & 15) + mn, d * _f32(q >> 4) + mn], -1).reshape(raw.shape[0], cols)


def dq_q5(raw: np.ndarray, cols: int, with_min: bool) -> np.ndarray:
    """Q5_0 (22 bytes: d, 32-bit qh, 16 bytes) and Q5_1 (24 bytes: d, min, qh, 16
    bytes), moelan/kernels.py:291-308: value j (< 16) is the low nibble of byte j
    with qh bit j as bit 4, value j+16 the high nibble with qh bit j+16; Q5_0
    subtracts 16. w = d * q + min (min 0.0 for Q5_0, so -0.0 becomes +0.0)."""
    qt = Q5_1 if with_min else Q5_0
    b = _blocks(raw, cols, qt)
    d = gguf_f16(b[..., 0], b[..., 1])[..., None]
    mn = gguf_f16(b[..., 2], b[..., 3])[..., None] if with_min else np.float32(0.0)
    h0 = 4 if with_min else 2
    qh = (b[..., h0].astype(np.int64) | (b[..., h0 + 1].astype(np.int64) << 8)
          | (b[..., h0 + 2].astype(np.int64) << 16) | (b[..., h0 + 3].astype(np.int64) << 24))[..., None]
    q = b[..., h0 + 4:h0 + 20].astype(np.int64)
    j = np.arange(16)
    off = 0 if with_min else 16
    x0 = ((q & 15) | (((qh >> j) << 4) & 0x10)) - off
    x1 = ((q >> 4) | ((qh >> (j + 12)) & 0x10)) - off
    return np.concatenate([d * _f32(x0) + mn, d * _f32(x1) + mn], -1).astype(np.float32).reshape(raw.shape[0], cols)


def dq_q2_k(raw: np.ndarray, cols: int) -> np.ndarray:
    """84-byte superblocks (moelan/kernels.py:389-415): 16 scale bytes (low
    nibble scale, high nibble min, one per 16 values), 64 bytes of 2-bit values,
    f16 d at 80, dmin at 82. Value n*128 + 32j + 16s + l is bits 2j of byte
    16 + 32n + 16s + l, with scale byte 8n + 2j + s; w = (d*sc)*q - dmin*m."""
    b = _blocks(raw, cols, Q2_K)
    rows, nb = b.shape[:2]
    d = gguf_f16(b[..., 80], b[..., 81])
    dmin = gguf_f16(b[..., 82], b[..., 83])
    out = np.empty((rows, nb, 2, 4, 2, 16), np.float32)
    for n in range(2):
        for j in range(4):
            for s_ in range(2):
                sc = b[..., 8 * n + 2 * j + s_].astype(np.int32)
                dl, ml = d * _f32(sc & 15), dmin * _f32(sc >> 4)
                q = (b[..., 16 + 32 * n + 16 * s_:16 + 32 * n + 16 * s_ + 16].astype(np.int32) >> (2 * j)) & 3
                out[:, :, n, j, s_] = dl[..., None] * _f32(q) - ml[..., None]
    return out.reshape(rows, cols)


def q3_k_scales(sb: np.ndarray) -> np.ndarray:
    """The 16 six-bit scales (minus 32) of Q3_K from its 12 bytes (moelan/kernels.py:
    418-431; the same rule as _q3_scale :634-641): scale i takes byte (i & 7)'s low
    (i < 8) or high nibble and bits 2*(i // 4) of byte 8 + i % 4 above them."""
    s = sb.astype(np.int32)
    out = np.empty(s.shape[:-1] + (16,), np.int32)
    for i in range(16):
        lo = s[..., i & 7]
        lo = (lo & 15) if i < 8 else (lo >> 4)
        out[..., i] = (lo | (((s[..., 8 + i % 4] >> (2 * (i // 4))) & 3) << 4)) - 32
    return out


def dq_q3_k(raw: np.ndarray, cols: int) -> np.ndarray:
    """110-byte superblocks (moelan/kernels.py:416-454): 32 hmask bytes, 64 bytes of
    2-bit values, 12 scale bytes, f16 d at 108. Value y = n*128 + 32j + 16s + l:
    bits 2j of byte 32 + 32n + 16s + l, minus 4 unless bit (4n + j) of hmask byte
    16s + l is set; scale 8n + 2j + s; w = (d*sc) * v."""
    b = _blocks(raw, cols, Q3_K)
    rows, nb = b.shape[:2]
    d = gguf_f16(b[..., 108], b[..., 109])
    scales = q3_k_scales(b[..., 96:108])
    out = np.empty((rows, nb, 2, 4, 2, 16), np.float32)
    for n in range(2):
        for j in range(4):
            for s_ in range(2):
                dl = d * _f32(scales[..., 8 * n + 2 * j + s_])
                q = (b[..., 32 + 32 * n + 16 * s_:48 + 32 * n + 16 * s_].astype(np.int32) >> (2 * j)) & 3
                h = (b[..., 16 * s_:16 * s_ + 16].astype(np.int32) >> (4 * n + j)) & 1
                out[:, :, n, j, s_] = dl[..., None] * _f32(q - np.where(h != 0, 0, 4))
    return out.reshape(rows, cols)


def dq_q5_k(raw: np.ndarray, cols: int) -> np.ndarray:
    """176-byte superblocks (moelan/kernels.py:338-362): d, dmin, 12 scale bytes
    (as Q4_K), 32 qh bytes at 16, 128 nibble bytes at 48. For k = 0..3, byte
    48 + 32k + l gives value 64k + l (low nibble, qh bit 2k) and 64k + 32 + l
    (high nibble, qh bit 2k+1) of qh byte l; w = (d*sc) * (q + 16h) - dmin*m."""
    b = _blocks(raw, cols, Q5_K)
    rows, nb = b.shape[:2]
    d = gguf_f16(b[..., 0], b[..., 1])
    dmin = gguf_f16(b[..., 2], b[..., 3])
    sc = b[..., 4:16]
    qh = b[..., 16:48].astype(np.int32)
    qs = b[..., 48:].reshape(rows, nb, 4, 32).astype(np.int32)
    out = np.empty((rows, nb, 4, 64), np.float32)
    for k in range(4):
        s1, m1 = scale_min_k4(2 * k, sc)
        s2, m2 = scale_min_k4(2 * k + 1, sc)
        d1, mm1 = d * _f32(s1), dmin * _f32(m1)
        d2, mm2 = d * _f32(s2), dmin * _f32(m2)
        lo = (qs[:, :, k] & 15) + np.where(qh & (1 << (2 * k)), 16, 0)
        hi = (qs[:, :, k] >> 4) + np.where(qh & (2 << (2 * k)), 16, 0)
        out[:, :, k, :32] = d1[..., None] * _f32(lo) - mm1[..., None]
        out[:, :, k, 32:] = d2[..., None] * _f32(hi) - mm2[..., None]
    return out.reshape(rows, cols)


def dq_q6_k(raw: np.ndarray, cols: int) -> np.ndarray:
    """210-byte superblocks (moelan/kernels.py:363-388): 128 ql bytes, 64 qh bytes,
    16 int8 scales at 192, f16 d at 208. In half n (128 values), for l < 32:
    values l, l+32, l+64, l+96 are the low nibble of ql[64n+l], of ql[64n+l+32],
    the high nibble of ql[64n+l], of ql[64n+l+32], each with bits 2t..2t+1 of
    qh[32n+l] as bits 4-5, minus 32; scale 8n + l//16 + 2t; w = d * (sc * q)
    (the integer product first)."""
    b = _blocks(raw, cols, Q6_K)
    rows, nb = b.shape[:2]
    d = gguf_f16(b[..., 208], b[..., 209])[..., None]
    sc = b[..., 192:208].view(np.int8).astype(np.int32)
    out = np.empty((rows, nb, 2, 4, 32), np.float32)
    l = np.arange(32)
    for n in range(2):
        a = b[..., 64 * n:64 * n + 32].astype(np.int32)
        c = b[..., 64 * n + 32:64 * n + 64].astype(np.int32)
        h = b[..., 128 + 32 * n:160 + 32 * n].astype(np.int32)
        qs = (((a & 15) | (((h >> 0) & 3) << 4)) - 32, ((c & 15) | (((h >> 2) & 3) << 4)) - 32,
              ((a >> 4) | (((h >> 4) & 3) << 4)) - 32, ((c >> 4) | (((h >> 6) & 3) << 4)) - 32)
        for t in range(4):
            s_ = sc[..., 8 * n + l // 16 + 2 * t]
            out[:, :, n, t] = d * _f32(s_ * qs[t])
    return out.reshape(rows, cols)


def gguf_dequant(raw: np.ndarray, qtype: int, cols: int) -> np.ndarray:
    """moelan/kernels.py:455-476 (_gguf_row dispatch): every quantized type."""
    dec = {Q8_0: dq_q8_0, Q4_K: dq_q4_k, Q4_0: dq_q4_0, Q4_1: dq_q4_1, Q2_K: dq_q2_k, Q3_K: dq_q3_k,
           Q5_K: dq_q5_k, Q6_K: dq_q6_k, Q5_0: lambda r, c: dq_q5(r, c, False),
           Q5_1: lambda r, c: dq_q5(r, c, True)}
    if qtype not in dec:
        raise ValueError(f"qtype {qtype} is not a quantized GGUF type")
    return dec[qtype](np.asarray(raw), cols)


def gguf_matmul_t(x, raw, qtype: int, cols: int) -> np.ndarray:
    """x @ W.T from GGUF rows (moelan/kernels.py:981-998), float64 on the decoded weights."""
    return matmul_t_exact(x, gguf_dequant(raw, qtype, cols))


# offsets of the f16 scale fields of each block   moelan/gguf.py:543-545
SCALE_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 10: (80, 82), 11: (108,),
                12: (0, 2), 13: (0, 2), 14: (208,)}


def random_blocks(rows: int, cols: int, qtype: int, rng, scale=None) -> np.ndarray:
    """Random GGUF rows with small f16 scale fields, as moelan/gguf.py:547-555
    (there a constant; ``scale`` None draws each d / dmin from |N(0, 0.01)|)."""
    _, block, size = QTYPES[qtype]
    raw = rng.integers(0, 256, (rows, cols // block, size), dtype=np.uint8)
    fields = SCALE_FIELDS[qtype]
    for off in fields:
        if scale is None:
            v = np.abs(rng.normal(0.0, 0.01, (rows, cols // block))).astype(np.float16)
        else:
            v = np.full((rows, cols // block), scale, np.float16)
        raw[:, :, off:off + 2] = v.view(np.uint8).reshape(rows, cols // block, 2)
    return raw.reshape(rows, cols // block * size)


# ------------------------------------------------------------------ wire format

WIRE_GROUP = 64


def wire_encode(a, wire: str):
    """encode_rows (moelan/protocol.py:99-114) in numpy: f16 by numpy's cast (round
    to nearest even); int8 per row in groups of 64 values (the whole row when 64
    does not divide it): s = max|g| / 127 in f32 (1 where that is 0), q =
    clip(rint(g / s), -127, 127) with rint rounding half to even. Returns the
    wire array, and for int8 also the (n, d / gs) f32 scales."""
    a = np.asarray(a, np.float32)
    if wire == "f16":
        with np.errstate(over="ignore"):
            return a.astype(np.float16)
    if wire == "f32":
        return a.copy()
    n, d = a.shape
    gs = WIRE_GROUP if d % WIRE_GROUP == 0 else d
    g = a.reshape(n, d // gs, gs)
    sc = (np.abs(g).max(axis=2) / np.float32(127.0)).astype(np.float32)
    sc[sc == 0] = np.float32(1.0)
    q = np.clip(np.rint((g / sc[:, :, None]).astype(np.float32)), -127, 127).astype(np.int8)
    return q.reshape(n, d), sc


def wire_decode(q, sc=None) -> np.ndarray:
    """decode_rows (moelan/protocol.py:116-123): q * s in f32 for int8, else a cast."""
    q = np.asarray(q)
    if q.dtype == np.int8:
        n, d = q.shape
        return (q.reshape(n, sc.shape[1], -1).astype(np.float32) * np.asarray(sc, np.float32)[:, :, None]).reshape(n, d)
    return q.astype(np.float32)


# ------------------------------------------------------------------ experts

def silu(x):
    """moelan/experts.py:62-63."""
    return x / (1.0 + np.exp(-x))


def expert_exact(x, Wgu, Wdn, inter: int) -> np.ndarray:
    """SwiGLU expert (moelan/experts.py:256-259) in float64 on decoded weights."""
    h = matmul_t_exact(x, Wgu)
    a = silu(h[:, :inter]) * h[:, inter:]
    return a @ np.asarray(Wdn, np.float64).T


def store_compute(x, groups, expert_fn) -> np.ndarray:
    """ExpertStore.compute semantics (moelan/experts.py:641-670, 707-727):
    out = 0; for each (expert, rows, weights): out[rows] += e(x[rows]) * w.
    ``expert_fn(e, xrows)`` evaluates expert e; float64 accumulate."""
    out = np.zeros(np.shape(x), np.float64)
    for e, rows, w in groups:
        rows = np.asarray(rows)
        out[rows] += expert_fn(e, np.asarray(x)[rows]) * np.asarray(w, np.float64)[:, None]
    return out


def moe_q4(x, items, out) -> np.ndarray:
    """moe_q4 semantics (moelan/kernels.py:942-968): out[uniq] += sum over items of
    w * expert(x[rows]); items are (expert_fn, rows, w). Returns the new out (float64)."""
    res = np.asarray(out, np.float64).copy()
    for fn, rows, w in items:
        rows = np.asarray(rows)
        res[rows] += fn(np.asarray(x)[rows]) * np.asarray(w, np.float64)[:, None]
    return res


# ------------------------------------------------------------------ int8 activations

def round_q8(v, gs: int):
    """_round_q8 (moelan/kernels.py:833-852): a row rounded to int8 per group of gs.
    Returns (q int32 [K] in column order, d f32 [K/gs] the group scales, s8 int32
    [K/gs] = 8 * the sum of the group's q). f32 arithmetic as written: m = max |v|,
    sc = m / 127 (1 when m == 0), inv = 1 / sc, q = floor(v * inv + 0.5) with the
    product and the sum each rounded to f32."""
    v = np.asarray(v, np.float32)
    G = v.shape[0] // gs
    vg = v.reshape(G, gs)
    m = np.abs(vg).max(axis=1).astype(np.float32)
    sc = np.where(m > 0, m / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    prod = (vg * inv[:, None]).astype(np.float32)
    q = np.floor((prod + np.float32(0.5)).astype(np.float32)).astype(np.int32)
    s8 = (8 * q.sum(axis=1)).astype(np.int32)
    return q.reshape(-1), sc, s8


def q4i8_matvec(q, d, s8, raw, s, gs: int, offset: bool) -> np.ndarray:
    """One matrix against one int8-rounded row, as _moe_q4i's inner loop
    (moelan/kernels.py:882-895, 898-911) with _q4c64 (:807-831): per group the
    exact sum of unsigned nibble * q, then acc += f32(isum - s8[g]) *
    (s[o, g] * d[g]) over the groups in order, in f32."""
    u = q4_unpack(raw, offset).astype(np.int64)
    O, I = u.shape
    G = I // gs
    isum = (u.reshape(O, G, gs) * np.asarray(q, np.int64).reshape(G, gs)[None]).sum(2)
    sw = np.asarray(s).astype(np.float32).reshape(O, G)
    t = (isum - np.asarray(s8, np.int64)[None, :]).astype(np.float32) * \
        (sw * np.asarray(d, np.float32)[None, :]).astype(np.float32)
    acc = np.zeros(O, np.float32)
    for g in range(G):
        acc = (acc + t[:, g].astype(np.float32)).astype(np.float32)
    return acc


def moe_q4i(x, items, out, H: int, I: int, gs: int) -> np.ndarray:
    """moe_q4 with int8 activations (moelan/kernels.py:942-968 when int8_act_for
    holds; _moe_q4i :854-917): each distinct row of x rounded to int8 per group;
    per pair the gate|up product, SiLU(gate) * up in f32, that rounded to int8
    per group, the down product; then part[r] += w * y[p] in pair order (f32)
    and out[uniq] += part. items: (raw_gu, s_gu, raw_dn, s_dn, offset, rows, w)."""
    x = np.asarray(x, np.float32)
    rows = np.concatenate([np.asarray(it[5]) for it in items]).astype(np.int64)
    uniq, prow = np.unique(rows, return_inverse=True)
    rq = {int(r): round_q8(x[r], gs) for r in uniq}
    part = np.zeros((len(uniq), H), np.float32)
    p = 0
    for raw_gu, s_gu, raw_dn, s_dn, offset, rws, w in items:
        for j, r in enumerate(np.asarray(rws)):
            q, d, s8 = rq[int(r)]
            h = q4i8_matvec(q, d, s8, raw_gu, s_gu, gs, offset)
            g0, up = h[:I], h[I:]
            act = (g0 / (np.float32(1.0) + np.exp(-g0)) * up).astype(np.float32)
            qa, da, s8a = round_q8(act, gs)
            y = q4i8_matvec(qa, da, s8a, raw_dn, s_dn, gs, offset)
            k = int(prow[p])
            part[k] = (part[k] + np.float32(np.asarray(w, np.float32)[j]) * y).astype(np.float32)
            p += 1
    res = np.asarray(out, np.float32).copy()
    res[uniq] = (res[uniq] + part).astype(np.float32)
    return res


# ------------------------------------------------------------------ routing

def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """moelan/model.py:83-86 (in the input dtype)."""
    x = x - x.max(axis=axis, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=axis, keepdims=True)


def top_k(scores: np.ndarray, k: int) -> np.ndarray:
    """moelan/model.py:154-157: the k largest, largest first, ties to the lower index."""
    return np.argsort(-scores, axis=-1, kind="stable")[:, :k]


def route(logits: np.ndarray, k: int, normalize: bool):
    """moelan/model.py:160-167: f32 softmax, stable top-k, gather, renormalise."""
    probs = softmax(logits.astype(np.float32), axis=-1)
    idx = top_k(probs, k)
    w = np.take_along_axis(probs, idx, axis=-1)
    if normalize:
        w = w / w.sum(-1, keepdims=True)
    return idx.astype(np.int32), w.astype(np.float32)


def group_by_expert(idx: np.ndarray, w: np.ndarray):
    """moelan/model.py:226-236: stable sort of the flattened picks by expert ->
    experts (unique, ascending), offsets, rows (token of each pick), weights."""
    k = idx.shape[1]
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    experts, starts = np.unique(flat[order], return_index=True)
    offsets = np.append(starts, len(flat)).astype(np.int32)
    rows = (order // k).astype(np.int32)
    weights = w.reshape(-1)[order].astype(np.float32)
    return experts.astype(np.int32), offsets, rows, weights


def groups_of(idx, w):
    """LocalBackend._moe (moelan/model.py:274-278): (expert, rows, weights) per expert."""
    experts, offsets, rows, weights = group_by_expert(idx, w)
    return [(int(experts[i]), rows[offsets[i]:offsets[i + 1]], weights[offsets[i]:offsets[i + 1]])
            for i in range(len(experts))]


def moe_layer_exact(x, router_w, experts, k: int, normalize: bool = True, logits=None):
    """One MoE layer (moelan/model.py:597-606 with LocalBackend): logits = x @ R.T
    (f32, as the reference), route, group, weighted sum of the experts (float64).
    ``experts[e] = (Wgu, Wdn, inter)`` decoded. Returns (out, idx, w, logits)."""
    if logits is None:
        logits = np.asarray(x, np.float32) @ np.asarray(router_w, np.float32).T
    idx, w = route(logits, k, normalize)
    groups = groups_of(idx, w)
    out = store_compute(x, groups, lambda e, xr: expert_exact(xr, *experts[e]))
    return out, idx, w, logits
