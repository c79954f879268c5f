"""Sizes past the common ones, which the reference's functions take as they
come: routing over many experts and many picks (moelan/model.py:154-167),
grouping over more than 1024 experts (:226-236), a prompt layer over 512
experts and over 80 picks a token, and GGUF rows longer than 8192 values
(moelan/kernels.py:981-998)."""

import numpy as np
import pytest

from distributedmoellm_amd import experts as X
from oracle import restate as R

from test_layer_gpu import oracle_expert
from test_matvec_gpu import close
from test_prefill_gpu import assert_tie_swaps_only, close_rows, weights_of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k", [(512, 8), (1000, 16), (2000, 8), (300, 100), (1500, 200), (130, 130)])
def test_route_many_experts_and_picks(kernels, E, k):
    """Registers hold the probabilities up to 1024 experts, beyond that they
    are recomputed each round; more than 64 picks are written one at a time.
    Picks match the oracle's up to near-ties; the normalised weights are the
    device's own probabilities divided by their numpy sum, bit for bit (the
    pairwise summation order, also past 128 picks)."""
    rng = np.random.default_rng(E * 7 + k)
    logits = (rng.standard_normal((96, E)) * 3).astype(np.float32)
    logits[2] = 0.5                                   # all tied: ids 0..k-1
    idx, w = kernels.route(logits, k, True)
    idx_raw, p = kernels.route(logits, k, False)
    assert np.array_equal(idx, idx_raw)
    ridx, _ = R.route(logits, k, True)
    diff = assert_tie_swaps_only(logits, idx, ridx, k)
    assert len(diff) <= 3
    assert idx[2].tolist() == list(range(k))
    assert all(len(set(r.tolist())) == k for r in idx)
    want = (p / p.sum(-1, keepdims=True)).astype(np.float32)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))
    np.testing.assert_allclose(w, weights_of(logits, idx, True), rtol=3e-6, atol=1e-8)
    np.testing.assert_allclose(p, weights_of(logits, idx, False), rtol=3e-6, atol=1e-9)


def test_route_nan_logits_sort_last(kernels):
    """A NaN logit makes a token's probabilities NaN (as numpy's softmax):
    numpy's argsort puts NaN last, so the picks are ids 0..k-1 with NaN
    weights; other tokens are untouched."""
    rng = np.random.default_rng(5)
    for E, k in ((64, 4), (700, 8), (1100, 70)):
        logits = rng.standard_normal((8, E)).astype(np.float32)
        logits[1, E // 2] = np.nan
        idx, w = kernels.route(logits, k, True)
        assert idx[1].tolist() == list(range(k)) and np.all(np.isnan(w[1]))
        rest = np.delete(logits, 1, 0)
        ridx, _ = R.route(rest, k, True)
        assert len(assert_tie_swaps_only(rest, np.delete(idx, 1, 0), ridx, k)) <= 1
        assert np.all(np.isfinite(np.delete(w, 1, 0)))


@pytest.mark.parametrize("T,k,E", [(300, 8, 3000), (40, 3, 5000)])
def test_group_by_expert_beyond_1024_experts(kernels, T, k, E):
    import torch
    rng = np.random.default_rng(T + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    idx[0, 0] = E - 1                                 # the last id is used
    w = rng.random((T, k)).astype(np.float32)
    got = kernels.group_by_expert(torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), E, with_pos=True)
    experts, offsets, rows, weights = (t.cpu().numpy() for t in got[:4])
    re, ro, rr, rwt = R.group_by_expert(idx, w)
    assert np.array_equal(experts, re) and np.array_equal(offsets, ro)
    assert np.array_equal(rows, rr) and np.array_equal(weights, rwt)


def oracle_layer(kernels, x, Rw, ex, k):
    """The layer on the oracle, routed on the device's logits; tokens whose
    picks differ only inside a near-tie take the device's picks."""
    logits = kernels.router_logits(x, Rw)
    ridx, _ = R.route(logits, k, True)
    gidx, _ = kernels.route(logits, k, True)
    diff = assert_tie_swaps_only(logits, gidx, ridx, k)
    assert len(diff) <= 2
    ridx[diff] = gidx[diff]
    rw = weights_of(logits, ridx, True)
    ref = np.zeros((x.shape[0], x.shape[1]))
    for e in np.unique(ridx):
        sel = np.nonzero((ridx == e).any(1))[0]
        we = rw[sel, np.argmax(ridx[sel] == e, axis=1)].astype(np.float64)
        ref[sel] += R.expert_exact(x[sel], *oracle_expert(ex[e])) * we[:, None]
    return ref


@pytest.mark.parametrize("T,E,k", [(96, 512, 8), (48, 96, 80), (40, 1100, 4)])
def test_prefill_layer_many_experts_and_picks(kernels, T, E, k):
    """The prompt layer over 512 and 1100 experts (the router's top-k past one
    register set, the used-expert scan past 1024) and over 80 picks a token
    (the combine's ordering in LDS)."""
    rng = np.random.default_rng(T + E + k)
    H, I = 256, 128
    ex = [X.synthetic_expert(H, I, "int4", 32, rng) for _ in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    Rw = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    out = kernels.prefill_layer(x, Rw, kernels.expert_table(ex), k, True, H, I, 32)
    close_rows(out, oracle_layer(kernels, x, Rw, ex, k))


@pytest.mark.parametrize("qtype,cols", [(R.Q8_0, 8192 + 32 * 5), (R.Q4_K, 256 * 40), (R.Q6_K, 256 * 33),
                                        (R.Q4_0, 32 * 600), (R.Q2_K, 256 * 70)])
@pytest.mark.parametrize("rows", [1, 3])
def test_gguf_matmul_long_rows(kernels, qtype, cols, rows):
    """Rows past 8192 values: one launch per 8192-value segment, the later
    ones adding to the first's output."""
    rng = np.random.default_rng(qtype * 10 + rows)
    O = 96
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("T,E,k,H,I,gs", [
    (64, 8, 2, 256, 128, 32),       # few rows an expert, one column tile a product
    (700, 32, 4, 512, 256, 32),     # ~87 rows an expert: two passes of its weight tiles
    (300, 256, 4, 1024, 256, 64),   # group 64; down tiles chained 4 a workgroup
    (2100, 64, 2, 256, 128, 32),    # past 2048 tokens: two passes over the prompt
])
def test_prefill_layer_dispatch(kernels, T, E, k, H, I, gs):
    """The prompt layer over shapes that pick its different paths (passes of
    48 rows, chained down tiles, token passes), against the oracle on the
    device's routing at the MFMA tolerance (2e-3)."""
    rng = np.random.default_rng(T + E + k + H + I + gs)
    ex = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(E)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    Rw = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    out = kernels.prefill_layer(x, Rw, kernels.expert_table(ex), k, True, H, I, gs)
    close_rows(out, oracle_layer(kernels, x, Rw, ex, k))
