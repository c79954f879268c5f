"""The layer call at the Qwen3-235B-A22B expert shape (H=4096, I=1536, int4
group 32, f16 scales) with a continuous-batching decode step's routing:
top-8 per token from a seeded Zipf(1.1) expert popularity over 128 experts,
at B = 1, 8 and 32 tokens, so hot experts carry up to ~30 rows in one call.

Reference: moe_q4 / _moe_q4 (moelan/kernels.py:942-968, 712-782) and the
row-decoding path _q4_rows (:108-131) that many rows per expert take. Bar:
1e-5 relative to the float64 oracle, norm-wise and per row, for the layer
call's output and for each sweep (gate|up, then down) of
moe_q4_experts_matvec on its own.
"""

import numpy as np
import pytest
import torch

from distributedmoellm_amd import experts as X
from oracle import restate as R

from test_matvec_gpu import close

pytestmark = pytest.mark.gpu

H, I, GS, E, K = 4096, 1536, 32, 128, 8


def zipf_layer(rng, B: int, E: int = E, k: int = K, s: float = 1.1):
    """One layer's routing for B tokens: each token picks k distinct experts
    with probability proportional to r^-s over a seeded permutation of the ids
    (its popularity rank r), with weights softmax(N(0,1)). Returns
    {expert: (rows int32 ascending, weights f32)}."""
    perm = rng.permutation(E)
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    picks: dict = {}
    for t in range(B):
        ex = perm[rng.choice(E, size=k, replace=False, p=p)]
        w = np.exp(rng.standard_normal(k))
        w /= w.sum()
        for e, wt in zip(ex, w):
            picks.setdefault(int(e), []).append((t, wt))
    return {e: (np.array([t for t, _ in v], np.int32), np.array([w for _, w in v], np.float32))
            for e, v in sorted(picks.items())}


class Layer:
    """A layer's routed experts (only those picked), its input rows and the
    float64 oracle of every pair: h (gate|up), y (down of SiLU(gate)*up) and
    the weighted sum."""

    def __init__(self, B: int, seed: int):
        rng = np.random.default_rng(seed)
        self.B = B
        self.picks = zipf_layer(rng, B)
        self.experts = {e: X.synthetic_expert(H, I, "int4", GS, rng) for e in self.picks}
        self.x = rng.standard_normal((B, H)).astype(np.float32)
        h, y = [], []
        out = np.zeros((B, H))
        for e, (rows, w) in self.picks.items():
            m = self.experts[e]
            Wgu = R.q4_dequant64(m.gu.raw, m.gu.s, GS, False)
            hp = R.matmul_t_exact(self.x[rows], Wgu)
            del Wgu
            a = R.silu(hp[:, :I]) * hp[:, I:]
            yp = R.matmul_t_exact(a, R.q4_dequant64(m.down.raw, m.down.s, GS, False))
            out[rows] += yp * w.astype(np.float64)[:, None]
            h.append(hp)
            y.append(yp)
        self.h = np.concatenate(h, 0)
        self.y = np.concatenate(y, 0)
        self.out = out
        self.max_rows = max(len(r) for r, _ in self.picks.values())

    def items(self, kernels):
        return [(kernels.q4_expert_ptrs(self.experts[e]), rows, w) for e, (rows, w) in self.picks.items()]


_LAYERS: dict = {}


def layer(B: int) -> Layer:
    if B not in _LAYERS:
        _LAYERS[B] = Layer(B, 2350 + B)
    return _LAYERS[B]


@pytest.mark.parametrize("B", [1, 8, 32])
def test_qwen3_235b_layer_call_zipf(kernels, B):
    """moe_q4 over one layer's routed experts: out += sum_e w * expert_e(x[rows])."""
    L = layer(B)
    print(f"B={B}: {len(L.picks)} experts, {sum(len(r) for r, _ in L.picks.values())} pairs, "
          f"hottest expert {L.max_rows} rows", flush=True)
    if B == 32:
        assert L.max_rows >= 16   # the case of experts with many rows is exercised
    base = np.random.default_rng(B).standard_normal((B, H)).astype(np.float32) * float(L.out.std())
    out = base.copy()
    kernels.moe_q4(L.x, L.items(kernels), H, I, GS, out)
    close(out, base + L.out)
    close(out - base, L.out, rtol=1e-4)


@pytest.mark.parametrize("B", [8, 32])
def test_qwen3_235b_experts_matvec_sweeps(kernels, B):
    """moe_q4_experts_matvec on its own: the gate|up sweep (input rows through
    xrow) and the down sweep (SiLU(gate)*up on load), each against float64."""
    from distributedmoellm_amd import _lib
    L = layer(B)
    meta = kernels.LayerMeta([p for p, _, _ in L.items(kernels)], [r for r, _ in L.picks.values()],
                             [w for _, w in L.picks.values()])
    dev = torch.device("cuda")
    xd = torch.from_numpy(L.x).to(dev)
    h = torch.empty((meta.P, 2 * I), dtype=torch.float32, device=dev)
    y = torch.empty((meta.P, H), dtype=torch.float32, device=dev)
    st = kernels.stream_handle()
    _lib.call("moe_q4_experts_matvec", xd.data_ptr(), H, meta.prow, meta.table, None, meta.k, meta.poff, 0,
              H, I, GS, meta.max_rows, h.data_ptr(), 2 * I, st)
    close(h.cpu().numpy(), L.h)
    # the down sweep reads the exact gate|up values, so its own error is measured
    hx = torch.from_numpy(L.h.astype(np.float32)).to(dev)
    _lib.call("moe_q4_experts_matvec", hx.data_ptr(), 2 * I, None, meta.table, None, meta.k, meta.poff, 1,
              H, I, GS, meta.max_rows, y.data_ptr(), H, st)
    h32 = L.h.astype(np.float32).astype(np.float64)
    a = R.silu(h32[:, :I]) * h32[:, I:]
    yw, p0 = [], 0   # pairs are in expert order
    for e, (rows, _) in L.picks.items():
        m = L.experts[e]
        yw.append(R.matmul_t_exact(a[p0:p0 + len(rows)], R.q4_dequant64(m.down.raw, m.down.s, GS, False)))
        p0 += len(rows)
    close(y.cpu().numpy(), np.concatenate(yw, 0))
