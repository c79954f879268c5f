"""The C/OpenMP restatement of the reference's numba kernels (oracle/cpuref.c,
the CPU baseline bench.py times) against the numpy restatement
(oracle/restate.py) on the CPU: every function it exports, at small shapes,
within 1e-5 relative of the float64 product (it is built with -ffast-math, as
numba's fastmath=True, so its sums are reassociated f32)."""

import ctypes

import numpy as np
import pytest

from oracle import build_cpuref
from oracle import restate as R

RTOL = 1e-5


@pytest.fixture(scope="module")
def L():
    build_cpuref.build(verbose=False)
    return build_cpuref.load()


def ptr(a):
    return a.ctypes.data


def rel(got, want):
    return np.linalg.norm(np.asarray(got, np.float64) - want) / np.linalg.norm(want)


def int4(rng, O, I, gs):
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 8).astype(np.float32)
    return raw, s


@pytest.mark.parametrize("n", [1, 3, 8])
@pytest.mark.parametrize("offset", [False, True])
def test_ref_q4_matmul_t(L, n, offset):
    rng = np.random.default_rng(n + 10 * offset)
    O, I, gs = 96, 256, 32
    raw, s = int4(rng, O, I, gs)
    x = rng.standard_normal((n, I)).astype(np.float32)
    y = np.zeros((n, O), np.float32)
    L.ref_q4_matmul_t(ptr(x), n, ptr(raw), ptr(s), O, I, gs, 0 if offset else 0x88, ptr(y))
    assert rel(y, R.q4_matmul_t(x, raw, s, gs, offset)) < RTOL


def test_ref_q8_matmul_t(L):
    rng = np.random.default_rng(2)
    O, I, gs, n = 64, 256, 32, 5
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 127).astype(np.float32)
    x = rng.standard_normal((n, I)).astype(np.float32)
    y = np.zeros((n, O), np.float32)
    L.ref_q8_matmul_t(ptr(x), n, ptr(q), ptr(s), O, I, gs, ptr(y))
    assert rel(y, R.q8_matmul_t(x, q, s, gs)) < RTOL


def test_ref_moe_q4_matches_the_layer_semantics(L):
    """_moe_q4's contract (moelan/kernels.py:712-782): out[r] += sum of w *
    expert(x[r]) over the row's pairs, out accumulated in place."""
    rng = np.random.default_rng(3)
    H, I, gs, k, n = 128, 64, 32, 5, 3
    mats = [(int4(rng, 2 * I, H, gs), int4(rng, H, I, gs)) for _ in range(k)]
    ptrs = np.array([[ptr(g[0]), ptr(g[1]), ptr(d[0]), ptr(d[1])] for g, d in mats], np.uint64).reshape(-1)
    xors = np.full(k, 0x88, np.uint8)
    rows = [np.array([0]), np.array([0, 2]), np.array([1]), np.array([0, 1, 2]), np.array([2])]
    poff = np.zeros(k + 1, np.int64)
    np.cumsum([len(r) for r in rows], out=poff[1:])
    prow = np.concatenate(rows).astype(np.int64)
    pw = rng.random(len(prow)).astype(np.float32)
    x = rng.standard_normal((n, H)).astype(np.float32)
    items = []
    for e, ((gr, gsc), (dr, dsc)) in enumerate(mats):
        Wgu, Wdn = R.q4_dequant64(gr, gsc, gs, False), R.q4_dequant64(dr, dsc, gs, False)
        items.append((lambda xr, a=Wgu, b=Wdn: R.expert_exact(xr, a, b, I), rows[e],
                      pw[poff[e]:poff[e + 1]]))
    delta = R.moe_q4(x, items, np.zeros((n, H)))
    out = np.zeros((n, H), np.float32)
    L.ref_moe_q4(ptr(x), n, ptr(ptrs), ptr(xors), ptr(poff), ptr(prow), ptr(pw), k, len(prow), H, I, gs, ptr(out))
    assert rel(out, delta) < RTOL
    # accumulated in place: a second call adds the same again onto what is there
    base = (rng.standard_normal((n, H)) * delta.std()).astype(np.float32)
    out = base.copy()
    L.ref_moe_q4(ptr(x), n, ptr(ptrs), ptr(xors), ptr(poff), ptr(prow), ptr(pw), k, len(prow), H, I, gs, ptr(out))
    assert rel(out, base + delta) < RTOL


@pytest.mark.parametrize("qtype", [8, 12])
@pytest.mark.parametrize("n", [1, 2])
def test_ref_gguf_matvec(L, qtype, n):
    rng = np.random.default_rng(qtype + n)
    O, cols = 48, 512
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    y = np.zeros((n, O), np.float32)
    fn = L.ref_mv_q8_0 if qtype == 8 else L.ref_mv_q4_k
    fn(ptr(x), n, ptr(np.ascontiguousarray(raw)), O, cols, ptr(y))
    assert rel(y, R.gguf_matmul_t(x, raw, qtype, cols)) < RTOL


def test_ref_threads(L):
    assert L.ref_threads() >= 1
