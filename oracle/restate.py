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
Q8_0, Q4_K = 8, 12


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


def gguf_dequant(raw: np.ndarray, qtype: int, cols: int) -> np.ndarray:
    """moelan/kernels.py:455-476 (_gguf_row dispatch) for the two types on this path."""
    if qtype == Q8_0:
        return dq_q8_0(raw, cols)
    if qtype == Q4_K:
        return dq_q4_k(raw, cols)
    raise ValueError(f"qtype {qtype} is not on this path")


def gguf_matmul_t(x, raw, qtype: int, cols: int) -> np.ndarray:
    """x @ W.T from GGUF rows (moelan/kernels.py:981-998), float64 on the decoded weights."""
    return matmul_t_exact(x, gguf_dequant(raw, qtype, cols))


def random_blocks(rows: int, cols: int, qtype: int, rng, scale=None) -> np.ndarray:
    """Random GGUF rows with small f16 scale fields, as moelan/gguf.py:547-555
    (there a constant; ``scale`` None draws each d / dmin from |N(0, 0.01)|)."""
    _, block, size = QTYPES[qtype]
    raw = rng.integers(0, 256, (rows, cols // block, size), dtype=np.uint8)
    fields = {8: (0,), 12: (0, 2)}[qtype]
    for off in fields:
        if scale is None:
            v = np.abs(rng.normal(0.0, 0.01, (rows, cols // block))).astype(np.float16)
        else:
            v = np.full((rows, cols // block), scale, np.float16)
        raw[:, :, off:off + 2] = v.view(np.uint8).reshape(rows, cols // block, 2)
    return raw.reshape(rows, cols // block * size)


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
