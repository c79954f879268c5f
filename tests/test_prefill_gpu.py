"""Prompt reading on the GPU against the oracle: router product, routing and
grouping (indices bit-exact), the grouped f16-MFMA expert FFN and a whole
Qwen3-30B-A3B-shaped MoE layer (T=512, 128 experts, top-8) within 2e-3
relative (norm-wise per token; TOL below)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from distributedmoellm_amd import experts as X
from distributedmoellm_amd import model as M
from oracle import restate as R

from test_layer_gpu import oracle_expert

pytestmark = pytest.mark.gpu
TOL = 2e-3
GOLDEN = Path(__file__).parent / "golden"


def close_rows(got, ref, tol=TOL, rows=None):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    sel = range(ref.shape[0]) if rows is None else rows
    worst = 0.0
    for r in sel:
        e = np.linalg.norm(got[r] - ref[r]) / max(np.linalg.norm(ref[r]), 1e-30)
        worst = max(worst, e)
    assert worst <= tol, f"worst per-row relative error {worst:.3e} > {tol}"
    return worst


# ---------------------------------------------------------------- router

def test_router_logits(kernels):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((512, 2048)).astype(np.float32)
    Rw = (rng.standard_normal((128, 2048)) * 0.02).astype(np.float32)
    got = kernels.router_logits(x, Rw)
    ref = x.astype(np.float64) @ Rw.T.astype(np.float64)
    assert np.linalg.norm(got - ref) <= 1e-6 * np.linalg.norm(ref)


def test_route_literal(kernels):
    """The reference's known answer (tests/test_moelan.py:64-72), on the device."""
    g = json.loads((GOLDEN / "route_literal.json").read_text())
    idx, w = kernels.route(np.array(g["logits"], np.float32), g["top_k"], True)
    assert idx.tolist() == g["idx"]
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    experts, offsets, rows, weights = kernels.group_by_expert(idx, w, 4)
    assert experts.tolist() == g["experts"]
    assert rows[offsets[2]:offsets[3]].tolist() == g["rows_of_expert_3"]


def near_tie_rows(logits, k, rel=4e-7):
    """Rows whose k-th and (k+1)-th probabilities are within a few ulps (f32
    softmax rounding may order them either way)."""
    p = np.sort(R.softmax(logits.astype(np.float32)), axis=1)[:, ::-1]
    gap = (p[:, k - 1] - p[:, k]) / np.maximum(p[:, k - 1], 1e-30)
    return set(np.nonzero(gap < rel)[0].tolist())


def assert_tie_swaps_only(logits, gidx, ridx, k, rel=4e-7):
    """Where the device's picks differ from the oracle's, they differ only
    inside a near-tie: the picks outside the experts whose probability is
    within `rel` of the k-th one agree, every device pick outside that group is
    an oracle pick, and the device's picks come in descending probability
    order (up to `rel`). Returns the rows that differ."""
    p = R.softmax(np.asarray(logits, np.float32)).astype(np.float64)
    diff = [r for r in range(len(logits)) if not np.array_equal(gidx[r], ridx[r])]
    for r in diff:
        pk = np.sort(p[r])[::-1][k - 1]
        group = set(np.nonzero(np.abs(p[r] - pk) <= rel * pk)[0].tolist())
        assert len(group) >= 2, f"row {r}: picks {gidx[r]} vs {ridx[r]} without a near-tie"
        g, o = set(gidx[r].tolist()), set(ridx[r].tolist())
        assert g - group == o - group, f"row {r}: {sorted(g)} vs {sorted(o)} beyond the tie {sorted(group)}"
        assert len(g) == k and g <= o | group
        pg = p[r][gidx[r]]
        assert np.all(pg[1:] <= pg[:-1] * (1 + rel)), f"row {r}: picks not in descending order"
    return diff


def weights_of(logits, idx, normalize):
    """The oracle's f32 route weights for the given picks (moelan/model.py:160-167)."""
    p = R.softmax(np.asarray(logits, np.float32))
    w = np.take_along_axis(p, np.asarray(idx, np.int64), 1)
    return (w / w.sum(1, keepdims=True)).astype(np.float32) if normalize else w


@pytest.mark.parametrize("E,k", [(128, 8), (64, 4), (256, 8), (8, 2), (60, 6)])
def test_route_matches_oracle_on_identical_logits(kernels, E, k):
    """Picks bit-exact with the oracle's, except inside near-ties (f32 softmax
    rounding may order those either way), where only the tied experts may
    trade places; weights then match the oracle's for the device's picks."""
    rng = np.random.default_rng(E + k)
    logits = rng.standard_normal((700, E)).astype(np.float32) * 2
    logits[3] = 0.25                        # all tied: lowest ids win
    logits[7, : min(E, 12)] = 3.0           # ties among the winners
    for normalize in (True, False):
        idx, w = kernels.route(logits, k, normalize)
        ridx, rw = R.route(logits, k, normalize)
        ties = near_tie_rows(logits, k)
        diff = assert_tie_swaps_only(logits, idx, ridx, k)
        assert set(diff) <= ties and len(ties) <= 2
        assert idx[3].tolist() == list(range(k))
        np.testing.assert_allclose(w, weights_of(logits, idx, normalize), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("T,k,E", [(512, 8, 128), (1792, 8, 128), (4000, 8, 128), (37, 4, 16), (1, 2, 8),
                                   (300, 6, 61), (64, 8, 1024)])
def test_group_by_expert_bit_exact(kernels, T, k, E):
    rng = np.random.default_rng(T)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    got = kernels.group_by_expert(torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), E, with_pos=True)
    experts, offsets, rows, weights = (t.cpu().numpy() for t in got[:4])
    eoff, pos = (t.cpu().numpy() for t in got[4])
    re, ro, rr, rwt = R.group_by_expert(idx, w)
    assert np.array_equal(experts, re) and np.array_equal(offsets, ro)
    assert np.array_equal(rows, rr) and np.array_equal(weights, rwt)
    assert eoff[-1] == T * k
    flat = idx.reshape(-1)
    assert np.array_equal(rows[pos], np.arange(T * k) // k)
    assert np.array_equal(weights[pos], w.reshape(-1))
    assert np.all(np.diff(eoff) >= 0) and np.array_equal(np.diff(eoff)[re], np.diff(ro))
    assert np.array_equal(np.bincount(flat, minlength=E), np.diff(eoff))


def test_group_drops_invalid_ids_and_keeps_pick_order(kernels):
    """Ids outside 0..E-1 are dropped (pos -1); a token naming one expert twice
    keeps both picks in pick order (stable argsort of the flat ids)."""
    rng = np.random.default_rng(5)
    T, k, E = 200, 4, 32
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    idx[3, 1] = -1
    idx[10, 0] = E
    idx[11, 2] = 1000
    idx[20] = [7, 7, 2, 7]
    w = rng.random((T, k)).astype(np.float32)
    got = kernels.group_by_expert(torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda(), E, with_pos=True)
    experts, offsets, rows, weights = (t.cpu().numpy() for t in got[:4])
    eoff, pos = (t.cpu().numpy() for t in got[4])
    flat = idx.reshape(-1)
    ok = (flat >= 0) & (flat < E)
    assert np.array_equal(pos[~ok], np.full((~ok).sum(), -1))
    order = np.argsort(np.where(ok, flat, E + 1), kind="stable")[: ok.sum()]
    assert np.array_equal(rows, order // k) and np.array_equal(weights, w.reshape(-1)[order])
    assert np.array_equal(pos[order], np.arange(ok.sum()))
    assert np.array_equal(experts, np.unique(flat[ok]))
    assert eoff[-1] == ok.sum() and offsets[-1] == ok.sum()


# ---------------------------------------------------------------- grouped expert FFN

@pytest.fixture(scope="module")
def c4_experts():
    """128 Qwen3-30B-A3B-shaped int4 experts (H=2048, I=768, gs=32, f16 scales)."""
    rng = np.random.default_rng(42)
    return [X.synthetic_expert(2048, 768, "int4", 32, rng) for _ in range(128)]


def test_grouped_ffn_matches_oracle(kernels, c4_experts):
    rng = np.random.default_rng(1)
    sizes = [1, 5, 16, 33, 64, 100, 0, 7]
    ex = c4_experts[:len(sizes)]
    x = rng.standard_normal((120, 2048)).astype(np.float32)
    rows = [np.sort(rng.choice(120, n, replace=False)).astype(np.int32) for n in sizes]
    eoff = np.zeros(len(sizes) + 1, np.int32)
    np.cumsum(sizes, out=eoff[1:])
    table = kernels.expert_table(ex)
    y = kernels.grouped_ffn(x, table, eoff, np.concatenate(rows), 2048, 768, 32).cpu().numpy()
    for i, e in enumerate(ex):
        if sizes[i] == 0:
            continue
        ref = R.expert_exact(x[rows[i]], *oracle_expert(e))
        close_rows(y[eoff[i]:eoff[i + 1]], ref)


@pytest.mark.parametrize("O,I,n", [(1536, 2048, 64), (2048, 768, 40), (256, 128, 17)])
def test_q4_gemm_mfma(kernels, O, I, n):
    rng = np.random.default_rng(O + n)
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // 32))) / 8).astype(np.float16)
    x = rng.standard_normal((n, I)).astype(np.float32)
    close_rows(kernels.q4_matmul_t_mfma(x, raw, s, 32, False), R.q4_matmul_t(x, raw, s, 32, False))


# ---------------------------------------------------------------- range of the f16 operands

def scaled_experts(rng, n, H, I, smag):
    """int4 experts with f32 scales of magnitude ``smag``."""
    out = []
    for _ in range(n):
        e = X.synthetic_expert(H, I, "int4", 32, rng, scale_dtype=np.float32)
        e.gu.s = (rng.random(e.gu.s.shape) * smag).astype(np.float32)
        e.down.s = (rng.random(e.down.s.shape) * smag).astype(np.float32)
        out.append(e)
    return out


@pytest.mark.parametrize("xmag,smag", [(1e5, 2.5e-3), (1e3, 2.5e-3), (3e4, 2e-4), (1e-4, 2.5e-3)])
def test_grouped_ffn_beyond_f16_range(kernels, xmag, smag):
    """Rows far beyond f16's range (|x| ~ 1e5, with an outlier channel 40x
    that), silu(gate) * up beyond it (|x| ~ 1e3 gives |gate|, |up| ~ 500), and
    rows far below it (|x| ~ 1e-4): the gathered rows are scaled by a power of
    two per row, silu(gate) * up per row and 16 columns, so every f16 operand
    stays in range and the results within the tolerance of the f64 oracle."""
    rng = np.random.default_rng(int(np.log10(xmag) * 10 + np.log10(smag)) % 1000)
    H, I = 1024, 512
    sizes = [3, 17, 40, 1]
    ex = scaled_experts(rng, len(sizes), H, I, smag)
    x = (rng.standard_normal((64, H)) * xmag).astype(np.float32)
    x[5, 7] = 40 * xmag                      # an outlier channel
    rows = [np.sort(rng.choice(64, n, replace=False)).astype(np.int32) for n in sizes]
    eoff = np.zeros(len(sizes) + 1, np.int32)
    np.cumsum(sizes, out=eoff[1:])
    y = kernels.grouped_ffn(x, kernels.expert_table(ex), eoff, np.concatenate(rows), H, I, 32).cpu().numpy()
    big = 0.0
    for i, e in enumerate(ex):
        Wgu, Wdn, inter = oracle_expert(e)
        h = R.matmul_t_exact(x[rows[i]], Wgu)
        big = max(big, np.abs(R.silu(h[:, :inter]) * h[:, inter:]).max())
        close_rows(y[eoff[i]:eoff[i + 1]], R.expert_exact(x[rows[i]], Wgu, Wdn, inter))
    if xmag >= 1e3 and smag > 1e-3:
        assert big > 65504      # silu(gate) * up itself is beyond f16's range


def test_q4_gemm_mfma_beyond_f16_range(kernels):
    """The single-matrix MFMA product on f32 rows of ~1e5 with an outlier of
    4e6, and on rows of ~1e-6: each 128-column piece of a row is scaled into
    f16's range while it is staged."""
    rng = np.random.default_rng(3)
    O, I, n = 512, 1024, 24
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // 32))) / 8).astype(np.float32)
    x = rng.standard_normal((n, I)).astype(np.float32)
    x[:12] *= 1e5
    x[3, 100] = 4e6
    x[12:] *= 1e-6
    close_rows(kernels.q4_matmul_t_mfma(x, raw, s, 32, False), R.q4_matmul_t(x, raw, s, 32, False))


# ---------------------------------------------------------------- whole layer

def test_qwen3_30b_prefill_layer(kernels, c4_experts):
    """One Qwen3-30B-A3B-shaped MoE layer, T=512 prompt tokens, 128 experts, top-8."""
    rng = np.random.default_rng(7)
    T, H, I, E, k = 512, 2048, 768, 128, 8
    x = rng.standard_normal((T, H)).astype(np.float32)
    Rw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    table = kernels.expert_table(c4_experts)
    out = kernels.prefill_layer(x, Rw, table, k, True, H, I, 32)
    # the oracle routes on the device's logits (routing is checked separately);
    # tokens whose picks differ from the oracle's only inside a near-tie are
    # compared with the device's picks and the oracle's weights for them
    logits = kernels.router_logits(x, Rw)
    ridx, _ = R.route(logits, k, True)
    gidx, _ = kernels.route(logits, k, True)
    diff = assert_tie_swaps_only(logits, gidx, ridx, k)
    assert len(diff) <= 2
    ridx[diff] = gidx[diff]
    rw = weights_of(logits, ridx, True)
    ok = None   # every token
    ref = np.zeros((T, H))
    for e in range(E):
        sel = np.nonzero((ridx == e).any(1))[0]
        if len(sel) == 0:
            continue
        we = rw[sel, np.argmax(ridx[sel] == e, axis=1)].astype(np.float64)
        ref[sel] += R.expert_exact(x[sel], *oracle_expert(c4_experts[e])) * we[:, None]
    worst = close_rows(out, ref, rows=ok)
    print(f"prefill layer worst per-token relative error {worst:.2e}")


def test_store_and_backend_prefill(kernels):
    """ExpertStore.compute with big groups (MFMA) and small ones (fused f32), via LocalBackend."""
    rng = np.random.default_rng(9)
    H, I, E, k, T = 256, 128, 16, 4, 96
    ex = {(0, e): X.synthetic_expert(H, I, "int4", 32, rng) for e in range(E)}
    store = X.ExpertStore(ex)
    backend = M.LocalBackend(store)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[:, 0] += 3.0     # expert 0 gets most tokens (MFMA path), others few
    idx, w = R.route(logits, k, True)
    got = backend.moe(0, x, idx, w)
    want = R.store_compute(x, R.groups_of(idx, w), lambda e, xr: R.expert_exact(xr, *oracle_expert(ex[(0, e)])))
    close_rows(got, want)
    assert backend.heat[(0, 0)] == int((idx == 0).sum())


def test_prefill_layer_matches_its_steps(kernels):
    """The prompt layer call, whose routing kernel also writes each token's
    f16 row and whose gate|up GEMM reads grouped rows through the row index
    (and whose down GEMM chains column tiles), against the same steps called
    one by one: router logits, routing, grouping, the grouped FFN on rows
    gathered per pick, and the weighted sum in ascending expert order on the
    host in float64. The f16 operands are the same values either way, so the
    two agree to f32 summation (1e-6), far inside the f16 tolerance."""
    rng = np.random.default_rng(31)
    T, H, I, E, k = 300, 512, 256, 128, 8
    ex = [X.synthetic_expert(H, I, "int4", 32, rng) for _ in range(E)]
    table = kernels.expert_table(ex)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[7] *= 3e4                     # a row scaled far from the rest
    Rw = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    out = kernels.prefill_layer(x, Rw, table, k, True, H, I, 32)
    logits = kernels.router_logits(x, Rw)
    idx, w = kernels.route(logits, k, True)
    dev = torch.device("cuda")
    _, _, rows, wts, (eoff, pos) = kernels.group_by_expert(torch.from_numpy(idx).to(dev),
                                                            torch.from_numpy(w).to(dev), E, with_pos=True)
    y = kernels.grouped_ffn(torch.from_numpy(x).to(dev), table, eoff, rows, H, I, 32).cpu().numpy()
    pos = pos.cpu().numpy().reshape(T, k)
    wts = wts.cpu().numpy()
    want = np.zeros((T, H))
    for t in range(T):
        for p in np.sort(pos[t]):
            want[t] += wts[p] * y[p].astype(np.float64)
    close_rows(out, want, tol=1e-6)
