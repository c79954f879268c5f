"""Pins the oracle (oracle/restate.py) before anything is compared with it.

Every oracle function is checked here against something other than its own
formula: the reference's literal test vectors (tests/golden/), layouts built
by independent packers written from the published formats, one-hot inputs
whose answer is a weight column, brute-force loops, and special values. A
plausible slip (swapped nibbles, a dropped -8, a transposed scale index, a
wrong 6-bit scale unpacking, a flipped tie rule) fails one of these.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import restate as R

GOLDEN = Path(__file__).parent / "golden"


# ---------------------------------------------------------------- routing

def test_route_and_grouping_literal():
    """The reference's own known answer (tests/test_moelan.py:64-72)."""
    g = json.loads((GOLDEN / "route_literal.json").read_text())
    logits = np.array(g["logits"], np.float32)
    idx, w = R.route(logits, g["top_k"], True)
    assert idx.tolist() == g["idx"]
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    experts, offsets, rows, weights = R.group_by_expert(idx, w)
    assert experts.tolist() == g["experts"]
    assert rows[offsets[2]:offsets[3]].tolist() == g["rows_of_expert_3"]


def _topk_loop(p, k):
    """Selection by repeated max with an explicit rule: larger wins, then lower index."""
    out = []
    for row in p:
        taken = []
        for _ in range(k):
            best = None
            for j, v in enumerate(row):
                if j in taken:
                    continue
                if best is None or v > row[best]:
                    best = j
            taken.append(best)
        out.append(taken)
    return np.array(out)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_route_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((17, 12)).astype(np.float32)
    logits[3, :] = 0.5                   # a row of exact ties
    logits[5, [2, 7, 9]] = 2.0          # ties among the winners
    idx, w = R.route(logits, 4, True)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.array_equal(idx, _topk_loop(R.softmax(logits.astype(np.float32)), 4))
    assert idx[3].tolist() == [0, 1, 2, 3] and idx[5, :3].tolist() == [2, 7, 9]
    want = np.take_along_axis(p, idx, 1)
    want /= want.sum(1, keepdims=True)
    np.testing.assert_allclose(w, want, rtol=1e-6)
    idx2, w2 = R.route(logits, 4, False)
    np.testing.assert_allclose(w2, np.take_along_axis(p, idx2, 1), rtol=1e-6)


def test_group_by_expert_brute_force():
    rng = np.random.default_rng(3)
    n, k, E = 40, 4, 9
    idx = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    w = rng.random((n, k)).astype(np.float32)
    experts, offsets, rows, weights = R.group_by_expert(idx, w)
    want_e = sorted(set(idx.reshape(-1).tolist()))
    assert experts.tolist() == want_e
    for i, e in enumerate(want_e):
        toks = [t for t in range(n) for j in range(k) if idx[t, j] == e]
        ws = [w[t, j] for t in range(n) for j in range(k) if idx[t, j] == e]
        assert rows[offsets[i]:offsets[i + 1]].tolist() == toks
        assert weights[offsets[i]:offsets[i + 1]].tolist() == ws
    assert offsets[-1] == n * k


# ---------------------------------------------------------------- int4 / int8

def _pack_like_reference_test(v):
    """Packing as written in the reference's test (tests/test_moelan.py:251-252)."""
    nib = (v & 15).astype(np.uint8)
    return nib[:, 0::2] | (nib[:, 1::2] << 4)


@pytest.mark.parametrize("rows", [1, 3, 4, 17])
def test_int4_layout_matches_reference_test(rows):
    """tests/test_moelan.py:245-258: W built from the signed values, not from bytes."""
    rng = np.random.default_rng(rows)
    O, I, gs = 96, 128, 32
    v = rng.integers(-8, 8, (O, I))
    s = rng.random((O, I // gs)).astype(np.float32)
    raw = _pack_like_reference_test(v)
    W = (v.reshape(O, -1, gs) * s[:, :, None]).reshape(O, I).astype(np.float32)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    assert np.array_equal(R.q4_dequant(raw, s, gs, False), W)
    assert np.array_equal(R.q4_dequant(raw ^ 0x88, s, gs, True), W)          # resident (XOR-ed) copy
    assert np.array_equal(R.q4_values(raw, False), v.astype(np.int8))
    W64 = (v.reshape(O, -1, gs) * s[:, :, None].astype(np.float64)).reshape(O, I)
    np.testing.assert_allclose(R.q4_matmul_t(x, raw, s, gs, False), x.astype(np.float64) @ W64.T, rtol=1e-12)
    ref = R.q4_matmul_t(x, raw, s, gs, False)
    got = R.q4_matmul_t_f32(x, raw, s, gs, False)   # the reference's unsigned-nibble formula
    assert np.linalg.norm(got - ref) <= 1e-5 * np.linalg.norm(ref)


def test_int4_one_hot_reads_columns():
    """x = e_c gives W[:, c] exactly: pins nibble order, sign and scale index."""
    rng = np.random.default_rng(5)
    O, I, gs = 8, 64, 32
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 8).astype(np.float16)
    for c in (0, 1, 2, 31, 32, 33, 63):
        x = np.zeros((1, I), np.float32)
        x[0, c] = 1.0
        byte = raw[:, c // 2]
        nib = (byte & 15) if c % 2 == 0 else (byte >> 4)
        v = np.where(nib >= 8, nib.astype(np.int32) - 16, nib.astype(np.int32))   # two's complement
        want = v * s[:, c // gs].astype(np.float64)
        assert np.array_equal(R.q4_matmul_t(x, raw, s, gs, False)[0], want)


def test_int8_closed_form():
    rng = np.random.default_rng(6)
    O, I, gs = 5, 64, 16
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = rng.random((O, I // gs)).astype(np.float32)
    W = R.q8_dequant(q, s, gs)
    for o in range(O):
        for c in range(I):
            assert W[o, c] == np.float32(np.float32(q[o, c]) * s[o, c // gs])
    x = rng.standard_normal((3, I)).astype(np.float32)
    want = [[sum(float(x[r, c]) * float(q[o, c]) * float(s[o, c // gs]) for c in range(I)) for o in range(O)]
            for r in range(3)]
    np.testing.assert_allclose(R.q8_matmul_t(x, q, s, gs), want, rtol=1e-12)


# ---------------------------------------------------------------- GGUF

def test_gguf_f16_rule():
    """moelan/kernels.py:244-255: normal and subnormal halves exact; exponent 31 -> +-inf (NaN too)."""
    bits = np.array([0x3C00, 0xC000, 0x0001, 0x03FF, 0x7BFF, 0x7C00, 0x7E00, 0xFC00, 0xFE01], np.uint16)
    got = R.gguf_f16(bits & 0xFF, bits >> 8)
    want = [1.0, -2.0, 2.0 ** -24, 1023 * 2.0 ** -24, 65504.0, np.inf, np.inf, -np.inf, -np.inf]
    assert got.tolist() == want


def _pack_q4k_scales(sc, m):
    """The 12-byte packing of eight 6-bit (scale, min) pairs as llama.cpp's
    quantize_row_q4_K writes it: j < 4 in the low six bits of bytes j and j+4;
    j >= 4 in the nibbles of byte j+4 with their top two bits in the top bits
    of bytes j-4 (scale) and j (min)."""
    out = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            out[j] |= sc[j]
            out[j + 4] |= m[j]
        else:
            out[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (m[j] >> 4) << 6
    return out


def _q4k_block(d, dmin, sc, m, q):
    """One 144-byte block from its fields; q = 256 values 0..15 in value order."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    blk[4:16] = _pack_q4k_scales(sc, m)
    for k in range(4):
        lo, hi = q[64 * k:64 * k + 32], q[64 * k + 32:64 * k + 64]
        blk[16 + 32 * k:48 + 32 * k] = lo | (hi << 4)
    return blk


def test_q4k_scale_unpack_round_trip():
    rng = np.random.default_rng(7)
    for _ in range(50):
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        packed = _pack_q4k_scales(sc, m)
        for j in range(8):
            a, b = R.scale_min_k4(j, packed)
            assert (int(a), int(b)) == (sc[j], m[j])


def test_q4k_known_blocks():
    # d = 1, dmin = 0: value = sub-block scale * nibble, integers, exact
    sc, m = np.arange(1, 9), np.arange(10, 18)
    q = np.full(256, 1, np.uint8)
    blk = _q4k_block(1.0, 0.0, sc, m, q)
    w = R.dq_q4_k(blk[None, :], 256)[0]
    assert w.tolist() == [float(sc[i // 32]) for i in range(256)]
    # the value index of every nibble: q = index % 16, d = 1, one scale, no min
    q = (np.arange(256) % 16).astype(np.uint8)
    blk = _q4k_block(1.0, 0.0, np.full(8, 1), np.zeros(8, int), q)
    assert R.dq_q4_k(blk[None, :], 256)[0].tolist() == (np.arange(256) % 16).astype(float).tolist()
    # the min: d = 0.5, dmin = 0.25, scale 2, min 3 -> 0.5*2*q - 0.75
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, 256).astype(np.uint8)
    blk = _q4k_block(0.5, 0.25, np.full(8, 2), np.full(8, 3), q)
    np.testing.assert_array_equal(R.dq_q4_k(blk[None, :], 256)[0], q.astype(np.float32) - np.float32(0.75))


def test_q8_0_known_blocks():
    q = (np.arange(32) - 16).astype(np.int8)
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:] = q.view(np.uint8)
    row = np.concatenate([blk, blk])
    w = R.dq_q8_0(row[None, :], 64)[0]
    assert w.tolist() == (0.5 * np.concatenate([q, q]).astype(float)).tolist()


def test_gguf_matmul_one_hot():
    rng = np.random.default_rng(9)
    for qt, cols in ((8, 64), (12, 512)):
        raw = R.random_blocks(3, cols, qt, rng)
        W = R.gguf_dequant(raw, qt, cols)
        for c in (0, 1, 31, 32, cols - 1):
            x = np.zeros((1, cols), np.float32)
            x[0, c] = 1
            assert np.array_equal(R.gguf_matmul_t(x, raw, qt, cols)[0], W[:, c].astype(np.float64))


# ---------------------------------------------------------------- experts / layer

def test_expert_and_store_semantics():
    """SwiGLU and out[rows] += e(x[rows]) * w against per-token loops."""
    rng = np.random.default_rng(10)
    H, I, E = 16, 8, 5
    Ws = {e: (rng.standard_normal((2 * I, H)), rng.standard_normal((H, I)), I) for e in range(E)}
    x = rng.standard_normal((6, H))
    groups = [(0, np.array([0, 2]), np.array([0.5, 0.25])), (3, np.array([2, 5]), np.array([1.0, 2.0]))]
    got = R.store_compute(x, groups, lambda e, xr: R.expert_exact(xr, *Ws[e]))
    want = np.zeros_like(x)
    for e, rows, w in groups:
        Wgu, Wdn, inter = Ws[e]
        for r, wt in zip(rows, w):
            g = Wgu[:inter] @ x[r]
            u = Wgu[inter:] @ x[r]
            a = g / (1 + np.exp(-g)) * u
            want[r] += wt * (Wdn @ a)
    np.testing.assert_allclose(got, want, rtol=1e-12)


def test_moe_layer_matches_token_loop():
    rng = np.random.default_rng(11)
    H, I, E, k, T = 16, 8, 6, 2, 7
    Ws = {e: (rng.standard_normal((2 * I, H)), rng.standard_normal((H, I)), I) for e in range(E)}
    Rw = rng.standard_normal((E, H)).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    out, idx, w, logits = R.moe_layer_exact(x, Rw, Ws, k)
    for t in range(T):
        lg = (x[t].astype(np.float64) @ Rw.T.astype(np.float64))
        order = sorted(range(E), key=lambda j: (-lg[j], j))[:k]
        assert idx[t].tolist() == order
        want = sum(w[t, j] * R.expert_exact(x[t:t + 1], *Ws[order[j]])[0] for j in range(k))
        np.testing.assert_allclose(out[t], want, rtol=1e-6)


# ------------------------------------------------------------------ int8 activations

def test_round_q8_rounds_half_up_and_bounds():
    """_round_q8 (moelan/kernels.py:833-852) pinned by what it must do: a group whose
    largest |v| is 127 has scale 1, so halves round up (floor(v + 0.5): 2.5 -> 3,
    -2.5 -> -2, unlike numpy's round-half-even); every group's largest |v| maps to
    127; the round trip is within half a step; a zero group has scale 1."""
    v = np.zeros(128, np.float32)
    v[:6] = [127.0, 2.5, -2.5, 0.5, -0.5, -127.0]
    q, d, s8 = R.round_q8(v, 64)
    assert d[0] == np.float32(1.0) and d[1] == np.float32(1.0)        # group 1 is all zero
    assert q[:6].tolist() == [127, 3, -2, 1, 0, -127]
    assert (q[64:] == 0).all() and s8[1] == 0
    assert s8[0] == 8 * int(q[:64].sum())
    rng = np.random.default_rng(30)
    for gs in (64, 128):
        x = (rng.standard_normal(512) * rng.uniform(0.01, 100, 512)).astype(np.float32)
        q, d, s8 = R.round_q8(x, gs)
        qg, xg = q.reshape(-1, gs), x.reshape(-1, gs).astype(np.float64)
        assert (np.abs(qg) <= 127).all()
        assert (np.abs(qg).max(axis=1) == 127).all()
        err = np.abs(xg - qg * d.astype(np.float64)[:, None])
        assert (err <= d.astype(np.float64)[:, None] * (0.5 + 1e-5)).all()
        np.testing.assert_array_equal(s8, 8 * qg.sum(axis=1))


def test_q4i8_matvec_one_hot_and_float64():
    """The int8-activation product: a one-hot q (d = 1, s8 = 8) reads column k as
    (u - 8) * s exactly; random rows agree with a float64 sum to f32 rounding."""
    rng = np.random.default_rng(31)
    O, I, gs = 12, 256, 64
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 8).astype(np.float16)
    W = R.q4_dequant64(raw, s, gs, False)
    for k in (0, 1, 63, 64, 255):
        q = np.zeros(I, np.int32)
        q[k] = 1
        d = np.ones(I // gs, np.float32)
        s8 = np.zeros(I // gs, np.int32)
        s8[k // gs] = 8
        y = R.q4i8_matvec(q, d, s8, raw, s, gs, False)
        np.testing.assert_array_equal(y.astype(np.float64), W[:, k])
    x = rng.standard_normal(I).astype(np.float32)
    q, d, s8 = R.round_q8(x, gs)
    want = W @ (q.astype(np.float64) * np.repeat(d.astype(np.float64), gs))
    got = R.q4i8_matvec(q, d, s8, raw, s, gs, False)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7 * np.abs(want).max())


def test_moe_q4i_close_to_float_layer():
    """The int8-activation layer call against the exact float one, with the bounds
    of the reference's own test (tests/test_fused.py:106-112): norm-wise 3e-2, per
    row 5e-2, cosine > 0.999."""
    rng = np.random.default_rng(32)
    H, I, gs = 256, 128, 64
    ex = []
    for _ in range(4):
        ex.append((rng.integers(0, 256, (2 * I, H // 2), dtype=np.uint8),
                   (np.abs(rng.normal(0, 0.02, (2 * I, H // gs))) / 8).astype(np.float16),
                   rng.integers(0, 256, (H, I // 2), dtype=np.uint8),
                   (np.abs(rng.normal(0, 0.02, (H, I // gs))) / 8).astype(np.float16)))
    x = rng.standard_normal((6, H)).astype(np.float32)
    sel = [(0, [0]), (1, [0, 3]), (2, [1, 2, 3]), (3, [5])]
    items = [(*ex[e], False, np.array(rows), rng.uniform(0.1, 1, len(rows)).astype(np.float32)) for e, rows in sel]
    got = R.moe_q4i(x, items, np.zeros((6, H), np.float32), H, I, gs)
    fitems = [(lambda xr, e=e: R.expert_exact(xr, R.q4_dequant64(ex[e][0], ex[e][1], gs, False),
                                               R.q4_dequant64(ex[e][2], ex[e][3], gs, False), I), rows, w)
              for (e, _), (_, _, _, _, _, rows, w) in zip(sel, items)]
    want = R.moe_q4(x, fitems, np.zeros((6, H)))
    assert np.linalg.norm(got - want) < 3e-2 * np.linalg.norm(want)
    assert float((want * got).sum() / np.sqrt((want * want).sum() * (got * got).sum())) > 0.999
    for r in range(6):
        if np.abs(want[r]).max() > 0:
            assert np.linalg.norm(got[r] - want[r]) < 5e-2 * np.linalg.norm(want[r])


# ---------------------------------------------------------------- wire format

def test_wire_int8_known_answers():
    """encode_rows int8 (moelan/protocol.py:104-110) pinned by what it must do: a
    group whose largest |v| is 127 has scale exactly 1, so q = rint(v) with ties
    to even (2.5 -> 2, 3.5 -> 4, -2.5 -> -2); a zero group has scale 1 and q 0;
    rows whose width 64 does not divide take one scale for the whole row."""
    a = np.zeros((2, 128), np.float32)
    a[0, :6] = [127.0, 2.5, 3.5, -2.5, 0.5, -127.0]
    q, s = R.wire_encode(a, "int8")
    assert s.shape == (2, 2) and s[0, 0] == 1.0 and s[0, 1] == 1.0 and s[1, 0] == 1.0
    assert q[0, :6].tolist() == [127, 2, 4, -2, 0, -127]
    assert (q[1] == 0).all()
    b = np.zeros((1, 96), np.float32)
    b[0, 0], b[0, 95] = 254.0, -1.0
    q, s = R.wire_encode(b, "int8")
    assert s.shape == (1, 1) and s[0, 0] == np.float32(2.0)
    assert q[0, 0] == 127 and q[0, 95] == 0          # -0.5 rounds to even 0


def test_wire_int8_error_bound_and_range():
    """decode(encode(a)) is within half a step of a, every |q| <= 127 and each
    group's largest |v| maps to +-127."""
    rng = np.random.default_rng(40)
    a = (rng.standard_normal((9, 256)) * rng.uniform(1e-3, 1e3, (9, 1))).astype(np.float32)
    q, s = R.wire_encode(a, "int8")
    back = R.wire_decode(q, s)
    err = np.abs(back - a).reshape(9, 4, 64)
    assert (err <= s[:, :, None] * 0.5 * (1 + 1e-6)).all()
    assert (np.abs(q.reshape(9, 4, 64)).max(axis=2) == 127).all()


def test_wire_f16_rounding():
    """f16 on the wire is numpy's cast: round to nearest even, overflow past
    65520 to inf, gradual underflow."""
    v = np.array([65504.0, 65519.0, 65520.0, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 2 ** -24, 2 ** -25,
                  3 * 2 ** -26, -0.0], np.float32)
    h = R.wire_encode(v[None, :], "f16")[0].astype(np.float64)
    assert h[0] == 65504 and h[1] == 65504 and np.isinf(h[2])
    assert h[3] == 1.0 and h[4] == 1 + 2 ** -9
    assert h[5] == 2 ** -24 and h[6] == 0 and h[7] == 2 ** -24
    assert np.signbit(h[8])
