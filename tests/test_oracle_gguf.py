"""Pins the oracle's decoders of the other GGUF block types (Q4_0, Q4_1, Q5_0,
Q5_1, Q2_K, Q3_K, Q5_K, Q6_K; moelan/kernels.py:270-453) without the
reference's gguf-py check, which cannot run here.

Each type gets a packer written from llama.cpp's quantize_row_*_ref layouts
(ggml-quants.c): values and scales -> bytes, one value at a time. Random
values are packed, decoded by the oracle, and compared bit-exactly with the
value each field says (d * sc * q - dmin * m in the reference's f32 order). A
decoder that reads a nibble from the wrong half, a high bit from the wrong
byte or position, a scale for the wrong 16 or 32 values, or drops an offset
fails these round trips, because the packers place every value by its own
index arithmetic.
"""

import numpy as np
import pytest

from oracle import restate as R

F32 = np.float32


def f16(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def h(v):
    """What an f16 field holds, as f32."""
    return F32(np.float16(v))


def pack_k4_scales(sc, m):
    """Eight 6-bit (scale, min) pairs in 12 bytes, as quantize_row_q4_K / q5_K."""
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


def pack_q4_0(d, L):
    """L: 32 values 0..15 (q + 8). Byte j: value j low, value j + 16 high."""
    b = np.zeros(18, np.uint8)
    b[0:2] = f16(d)
    for j in range(32):
        b[2 + j % 16] |= L[j] << (4 * (j // 16))
    return b


def pack_q4_1(d, mn, L):
    b = np.zeros(20, np.uint8)
    b[0:2], b[2:4] = f16(d), f16(mn)
    for j in range(32):
        b[4 + j % 16] |= L[j] << (4 * (j // 16))
    return b


def pack_q5(d, mn, L):
    """L: 32 values 0..31. Low four bits as Q4_0/Q4_1's nibbles, bit 4 of value j
    in bit j of the 32-bit qh. mn None: Q5_0 (22 bytes), else Q5_1 (24 bytes)."""
    b = np.zeros(22 if mn is None else 24, np.uint8)
    b[0:2] = f16(d)
    h0 = 2
    if mn is not None:
        b[2:4] = f16(mn)
        h0 = 4
    qh = 0
    for j in range(32):
        b[h0 + 4 + j % 16] |= (L[j] & 15) << (4 * (j // 16))
        qh |= ((L[j] >> 4) & 1) << j
    b[h0:h0 + 4] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    return b


def pack_q2_k(d, dmin, sc, m, L):
    """L: 256 values 0..3; sc, m: 16 four-bit values, one per 16 values. Byte
    16 + v // 128 * 32 + v % 32 holds value v in bits 2 * (v % 128 // 32)."""
    b = np.zeros(84, np.uint8)
    for i in range(16):
        b[i] = sc[i] | (m[i] << 4)
    for v in range(256):
        b[16 + (v // 128) * 32 + v % 32] |= L[v] << (2 * ((v % 128) // 32))
    b[80:82], b[82:84] = f16(d), f16(dmin)
    return b


def pack_q3_k(d, s, q):
    """q: 256 values -4..3; s: 16 scales -32..31. L = q + 4: bit 2 of value v in
    bit v // 32 of hmask byte v % 32, bits 0-1 packed as Q2_K's; scale i = s + 32
    in six bits: low four in byte i (i < 8) or the high nibble of byte i - 8,
    top two at bits 2 * (i // 4) of byte 8 + i % 4."""
    b = np.zeros(110, np.uint8)
    L = np.asarray(q) + 4
    for v in range(256):
        if L[v] > 3:
            b[v % 32] |= 1 << (v // 32)
        b[32 + (v // 128) * 32 + v % 32] |= (L[v] & 3) << (2 * ((v % 128) // 32))
    for i in range(16):
        l6 = int(s[i]) + 32
        if i < 8:
            b[96 + i] |= l6 & 0xF
        else:
            b[96 + i - 8] |= (l6 & 0xF) << 4
        b[96 + 8 + i % 4] |= (l6 >> 4) << (2 * (i // 4))
    b[108:110] = f16(d)
    return b


def pack_q5_k(d, dmin, sc, m, L):
    """L: 256 values 0..31; sc, m: eight 6-bit values, one per 32 values. For the
    64-value group k: value 64k + j (j < 32) low nibble of byte 48 + 32k + j and
    qh byte j bit 2k; value 64k + 32 + j high nibble and bit 2k + 1."""
    b = np.zeros(176, np.uint8)
    b[0:2], b[2:4] = f16(d), f16(dmin)
    b[4:16] = pack_k4_scales(sc, m)
    for v in range(256):
        k, r = v // 64, v % 64
        j, hi = r % 32, r // 32
        b[48 + 32 * k + j] |= (L[v] & 15) << (4 * hi)
        b[16 + j] |= ((L[v] >> 4) & 1) << (2 * k + hi)
    return b


def pack_q6_k(d, sc, q):
    """q: 256 values -32..31; sc: 16 int8 scales, one per 16 values. L = q + 32.
    In half n, value 128n + 32t + l (l < 32): low four bits in ql byte
    64n + l + 32 * (t % 2), nibble t // 2; top two bits at bits 2t of qh byte
    128 + 32n + l."""
    b = np.zeros(210, np.uint8)
    L = np.asarray(q) + 32
    for v in range(256):
        n, r = v // 128, v % 128
        t, l = r // 32, r % 32
        b[64 * n + l + 32 * (t % 2)] |= (L[v] & 15) << (4 * (t // 2))
        b[128 + 32 * n + l] |= (L[v] >> 4) << (2 * t)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = f16(d)
    return b


def decode(blocks, qtype):
    raw = np.concatenate(blocks)[None, :]
    return R.gguf_dequant(raw, qtype, R.QTYPES[qtype][1] * len(blocks))[0]


@pytest.mark.parametrize("seed", range(4))
def test_q4_0_q4_1_round_trip(seed):
    rng = np.random.default_rng(seed)
    L = rng.integers(0, 16, (3, 32))
    d = rng.normal(0, 0.05, 3)
    mn = rng.normal(0, 0.05, 3)
    got = decode([pack_q4_0(d[i], L[i]) for i in range(3)], R.Q4_0)
    want = np.concatenate([h(d[i]) * (L[i] - 8).astype(F32) for i in range(3)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got = decode([pack_q4_1(d[i], mn[i], L[i]) for i in range(3)], R.Q4_1)
    want = np.concatenate([h(d[i]) * L[i].astype(F32) + h(mn[i]) for i in range(3)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(4))
def test_q5_0_q5_1_round_trip(seed):
    rng = np.random.default_rng(10 + seed)
    L = rng.integers(0, 32, (3, 32))
    d = rng.normal(0, 0.05, 3)
    mn = rng.normal(0, 0.05, 3)
    got = decode([pack_q5(d[i], None, L[i]) for i in range(3)], R.Q5_0)
    want = np.concatenate([h(d[i]) * (L[i] - 16).astype(F32) + F32(0.0) for i in range(3)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got = decode([pack_q5(d[i], mn[i], L[i]) for i in range(3)], R.Q5_1)
    want = np.concatenate([h(d[i]) * L[i].astype(F32) + h(mn[i]) for i in range(3)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5_0_zero_value_is_positive_zero():
    """Q5_0 adds a 0.0 minimum (moelan/kernels.py:297): d < 0 times q = 0 gives +0.0."""
    L = np.full(32, 16)
    got = decode([pack_q5(-0.5, None, L)], R.Q5_0)
    assert np.all(got == 0) and not np.signbit(got).any()
    got = decode([pack_q4_0(-0.5, np.full(32, 8))], R.Q4_0)
    assert np.signbit(got).all()          # Q4_0 has no minimum: -0.0 stays


@pytest.mark.parametrize("seed", range(3))
def test_q2_k_round_trip(seed):
    rng = np.random.default_rng(20 + seed)
    blocks, want = [], []
    for _ in range(2):
        L = rng.integers(0, 4, 256)
        sc, m = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
        d, dmin = rng.uniform(0.001, 0.1), rng.uniform(0.001, 0.1)
        blocks.append(pack_q2_k(d, dmin, sc, m, L))
        v = np.arange(256)
        want.append((h(d) * sc[v // 16].astype(F32)) * L.astype(F32) - h(dmin) * m[v // 16].astype(F32))
    got = decode(blocks, R.Q2_K)
    assert np.array_equal(got.view(np.uint32), np.concatenate(want).astype(F32).view(np.uint32))


@pytest.mark.parametrize("seed", range(3))
def test_q3_k_round_trip(seed):
    rng = np.random.default_rng(30 + seed)
    blocks, want = [], []
    for _ in range(2):
        q = rng.integers(-4, 4, 256)
        s = rng.integers(-32, 32, 16)
        d = rng.uniform(0.001, 0.1)
        blocks.append(pack_q3_k(d, s, q))
        v = np.arange(256)
        want.append((h(d) * s[v // 16].astype(F32)) * q.astype(F32))
    got = decode(blocks, R.Q3_K)
    assert np.array_equal(got.view(np.uint32), np.concatenate(want).astype(F32).view(np.uint32))


def test_q3_k_scale_rule_matches_the_reference_words_form():
    """The two ways the reference unpacks Q3_K scales (moelan/kernels.py:418-431
    through 32-bit words and masks; :634-641 per scale) agree with the packer."""
    rng = np.random.default_rng(33)
    for _ in range(20):
        s = rng.integers(-32, 32, 16)
        raw = pack_q3_k(0.5, s, np.zeros(256, np.int64))[96:108]
        assert np.array_equal(R.q3_k_scales(raw), s)
        a0, a1, t = (int(np.frombuffer(raw[i:i + 4].tobytes(), np.uint32)[0]) for i in (0, 4, 8))
        km1, km2 = 0x03030303, 0x0F0F0F0F
        words = ((a0 & km2) | (((t >> 0) & km1) << 4), (a1 & km2) | (((t >> 2) & km1) << 4),
                 ((a0 >> 4) & km2) | (((t >> 4) & km1) << 4), ((a1 >> 4) & km2) | (((t >> 6) & km1) << 4))
        via_words = [((words[w] >> (8 * k)) & 0xFF) - 32 for w in range(4) for k in range(4)]
        assert via_words == list(s)


@pytest.mark.parametrize("seed", range(3))
def test_q5_k_round_trip(seed):
    rng = np.random.default_rng(40 + seed)
    blocks, want = [], []
    for _ in range(2):
        L = rng.integers(0, 32, 256)
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        d, dmin = rng.uniform(0.001, 0.1), rng.uniform(0.001, 0.1)
        blocks.append(pack_q5_k(d, dmin, sc, m, L))
        v = np.arange(256)
        want.append((h(d) * sc[v // 32].astype(F32)) * L.astype(F32) - h(dmin) * m[v // 32].astype(F32))
    got = decode(blocks, R.Q5_K)
    assert np.array_equal(got.view(np.uint32), np.concatenate(want).astype(F32).view(np.uint32))


@pytest.mark.parametrize("seed", range(3))
def test_q6_k_round_trip(seed):
    rng = np.random.default_rng(50 + seed)
    blocks, want = [], []
    for _ in range(2):
        q = rng.integers(-32, 32, 256)
        sc = rng.integers(-128, 128, 16)
        d = rng.uniform(0.0001, 0.01)
        blocks.append(pack_q6_k(d, sc, q))
        v = np.arange(256)
        want.append(h(d) * (sc[v // 16] * q).astype(F32))
    got = decode(blocks, R.Q6_K)
    assert np.array_equal(got.view(np.uint32), np.concatenate(want).astype(F32).view(np.uint32))


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
@pytest.mark.parametrize("qtype", [R.Q4_0, R.Q4_1, R.Q5_0, R.Q5_1, R.Q2_K, R.Q3_K, R.Q5_K, R.Q6_K])
def test_infinite_scale_fields_read_as_infinity(qtype):
    """Exponent-31 f16 fields (Inf and NaN) decode to a signed infinity
    (moelan/kernels.py:244-255): every value of such a block is non-finite or
    NaN, never a finite number made from a NaN's payload."""
    _, per, size = R.QTYPES[qtype]
    rng = np.random.default_rng(qtype)
    raw = R.random_blocks(1, per, qtype, rng)
    off = R.SCALE_FIELDS[qtype][0]
    raw[0, off:off + 2] = [0x01, 0x7E]       # a NaN pattern
    w = R.gguf_dequant(raw, qtype, per)
    assert not np.isfinite(w).any()
