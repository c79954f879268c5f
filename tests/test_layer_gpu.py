"""The fused per-layer int4 call and the store on the GPU, mirroring moelan's
tests/test_fused.py: the layer call must give what one call per expert gives,
resident (XOR-ed) and stored copies mix in one call, and everything matches
the float64 oracle within 1e-5 (norm-wise and per row)."""

import numpy as np
import pytest
import torch

from distributedmoellm_amd import experts as X
from distributedmoellm_amd import gguf as G
from oracle import restate as R

from test_matvec_gpu import close

pytestmark = pytest.mark.gpu


def oracle_expert(e):
    """(Wgu, Wdn, inter) decoded exactly (float64) from an expert's host arrays."""
    def dec(m):
        if isinstance(m, X.Packed4):
            raw = m.raw.cpu().numpy() if isinstance(m.raw, torch.Tensor) else m.raw
            s = m.s.cpu().numpy() if isinstance(m.s, torch.Tensor) else m.s
            return R.q4_dequant64(raw, s, m.gs, m.offset)
        if isinstance(m, X.GroupQuant):
            return R.q8_dequant64(m.q, m.s, m.gs)
        if isinstance(m, G.Stacked):
            return np.concatenate([dec(p) for p in m.parts], 0)
        if isinstance(m, G.QuantMatrix):
            return R.gguf_dequant(m.raw, m.qtype, m.shape[1]).astype(np.float64)
        raise TypeError(m)
    return dec(e.gu), dec(e.down), e.inter


def groups_for(rng, picks):
    return [(e, np.array(rows), rng.random(len(rows)).astype(np.float32)) for e, rows in picks]


@pytest.fixture(scope="module")
def small_experts():
    rng = np.random.default_rng(0)
    return {(1, e): X.synthetic_expert(64, 96, "int4", 32, rng) for e in range(8)}


def test_layer_call_matches_one_call_per_expert(kernels, small_experts, monkeypatch):
    """moelan tests/test_fused.py:37-53 on the device."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    groups = groups_for(rng, [(0, [0]), (2, [0, 3]), (4, [1, 2, 3]), (5, [0, 1, 2, 4, 5]), (7, [5])])
    got = {}
    for flag in (False, True):
        monkeypatch.setattr(kernels, "FUSED", flag)
        for e in small_experts.values():
            e.fused = None
        store = X.ExpertStore(small_experts, fmt="int4")
        got[flag] = store.compute(1, x, groups)
    want = R.store_compute(x, groups, lambda e, xr: R.expert_exact(xr, *oracle_expert(small_experts[(1, e)])))
    close(got[True], want)
    close(got[False], want)
    assert np.abs(got[False]).max() > 1e-3


def test_layer_call_reads_resident_copies_too(kernels, small_experts):
    """moelan tests/test_fused.py:57-74: a stored (XOR 0x88) and a resident (offset) expert in one call."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    mapped = small_experts[(1, 3)]
    copy = small_experts[(1, 6)]
    copy = X.Expert(copy.gu.resident(), copy.down.resident(), copy.inter)
    assert copy.gu.offset and not mapped.gu.offset
    w = np.array([0.25, 0.75], np.float32)
    out = np.zeros_like(x)
    items = [(kernels.q4_expert_ptrs(mapped), np.array([0, 1]), w),
             (kernels.q4_expert_ptrs(copy), np.array([1]), w[:1])]
    kernels.moe_q4(x, items, 64, 96, 32, out)
    want = np.zeros(x.shape)
    want[[0, 1]] += R.expert_exact(x[[0, 1]], *oracle_expert(mapped)) * w[:, None]
    want[[1]] += R.expert_exact(x[[1]], *oracle_expert(copy)) * w[:1, None]
    close(out, want)


def test_layer_call_adds_into_out(kernels, small_experts):
    """moe_q4 accumulates: out[uniq] += part (moelan/kernels.py:968)."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    base = rng.standard_normal((4, 64)).astype(np.float32)
    e = small_experts[(1, 2)]
    out = base.copy()
    kernels.moe_q4(x, [(kernels.q4_expert_ptrs(e), np.array([1, 3]), np.array([0.5, 2.0], np.float32))],
                   64, 96, 32, out)
    want = base.astype(np.float64)
    want[[1, 3]] += R.expert_exact(x[[1, 3]], *oracle_expert(e)) * np.array([[0.5], [2.0]])
    close(out, want)
    assert np.array_equal(out[[0, 2]], base[[0, 2]])


@pytest.mark.parametrize("rows_per_token,k", [(1, 8), (8, 8), (3, 24)])
def test_qwen3_30b_layer_decode(kernels, rows_per_token, k):
    """A layer's picks at the Qwen3-30B-A3B expert shape (H=2048, I=768, gs=32, f16 scales)."""
    rng = np.random.default_rng(rows_per_token * 10 + k)
    experts = [X.synthetic_expert(2048, 768, "int4", 32, rng) for _ in range(k)]
    T = rows_per_token
    x = rng.standard_normal((T, 2048)).astype(np.float32)
    items, oitems = [], []
    for i, e in enumerate(experts):
        rows = np.sort(rng.choice(T, size=min(T, 1 + i % 3), replace=False)).astype(np.int32)
        w = rng.random(len(rows)).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(e), rows, w))
        oitems.append((lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)), rows, w))
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, 2048, 768, 32, out)
    close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))


def test_decode_step_384_experts_full_shape(kernels):
    """The decode benchmark's workload at full size: one token's 384 expert
    evaluations (48 layers x top-8) in one layer call at the Qwen3-30B-A3B
    expert shape (H=2048, I=768, gs=32, f16 scales), so gate|up on the
    integer dot, down on the LDS ring and the tree combine over 384 pairs;
    48 distinct experts, each evaluated 8 times, against float64."""
    rng = np.random.default_rng(384)
    H, I, gs = 2048, 768, 32
    pool = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(48)]
    mats = [oracle_expert(e) for e in pool]
    x = rng.standard_normal((1, H)).astype(np.float32)
    items, oitems = [], []
    for j in rng.permutation(np.repeat(np.arange(48), 8)):
        rows = np.zeros(1, np.int32)
        w = rng.random(1).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(pool[j]), rows, w))
        oitems.append((lambda xr, m=mats[j]: R.expert_exact(xr, *m), rows, w))
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, gs, out)
    close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))


@pytest.mark.parametrize("k,counts", [(384, (384,)), (100, (100, 21, 8, 9, 1))])
def test_rows_with_many_pairs(kernels, k, counts):
    """A row in many experts' pair lists (one token's 48 layers x top-8 in one
    call): the weighted sum over runs of pairs, added into a non-zero out."""
    rng = np.random.default_rng(k)
    H, I = 256, 128
    experts = [X.synthetic_expert(H, I, "int4", 32, rng) for _ in range(k)]
    T = len(counts)
    x = rng.standard_normal((T, H)).astype(np.float32)
    member = np.zeros((k, T), bool)
    for t, c in enumerate(counts):
        member[rng.choice(k, size=c, replace=False), t] = True
    items, oitems = [], []
    for i, e in enumerate(experts):
        rows = np.nonzero(member[i])[0].astype(np.int32)
        if len(rows) == 0:
            continue
        w = rng.random(len(rows)).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(e), rows, w))
        oitems.append((lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)), rows, w))
    delta = R.moe_q4(x, oitems, np.zeros((T, H)))
    # out starts at values of the size of what is added, so 1e-5 measures the sum
    base = (rng.standard_normal((T, H)) * delta.std()).astype(np.float32)
    out = base.copy()
    kernels.moe_q4(x, items, H, I, 32, out)
    close(out, base + delta)
    close(out - base, delta, rtol=1e-4)


def test_expert_call_int4_int8_gguf(kernels):
    """Expert.__call__ for each format against the oracle's SwiGLU."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    for e in (X.synthetic_expert(512, 256, "int4", 32, rng),
              X.synthetic_expert(512, 256, "int8", 32, rng),
              G.synthetic_expert(512, 256, ["Q4_K", "Q4_K", "Q8_0"], rng),
              G.synthetic_expert(512, 256, ["Q8_0", "Q8_0", "Q8_0"], rng)):
        close(e(x), R.expert_exact(x, *oracle_expert(e)))


def test_store_mixes_formats(kernels):
    rng = np.random.default_rng(4)
    ex = {(0, 0): X.synthetic_expert(256, 256, "int4", 32, rng),
          (0, 1): X.synthetic_expert(256, 256, "int8", 32, rng),
          (0, 2): X.synthetic_expert(256, 256, "int4", 32, rng)}
    store = X.ExpertStore(ex)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    groups = groups_for(rng, [(0, [0, 1, 4]), (1, [1, 2]), (2, [0, 3, 4])])
    got = store.compute(0, x, groups)
    want = R.store_compute(x, groups, lambda e, xr: R.expert_exact(xr, *oracle_expert(ex[(0, e)])))
    close(got, want)


class _MappedSource:
    """A zero-copy source (as a memory-mapped container): each load() builds a
    new Expert, so an expert dropped from the store's bounded map tier takes
    its device copy with it."""
    zero_copy = True

    def __init__(self, H, I, n, seed=0):
        self.H, self.I, self.n, self.seed = H, I, n, seed

    def has(self, key):
        return key[0] == 0 and 0 <= key[1] < self.n

    def load(self, key):
        return X.synthetic_expert(self.H, self.I, "int4", 32, np.random.default_rng(self.seed + key[1]))


@pytest.mark.parametrize("map_size", [1, 2])
def test_store_keeps_fused_experts_alive_until_the_call(kernels, map_size):
    """With a map tier smaller than a layer's experts, each get() drops an
    earlier expert (and its device copy) while the next one uploads; the layer
    call must still read every expert's own weights (the store holds them
    until the call is enqueued, as moelan/experts.py:732-735)."""
    H, I, n = 512, 256, 6
    src = _MappedSource(H, I, n, seed=40)
    store = X.ExpertStore([src], fmt="int4", map_size=map_size)
    rng = np.random.default_rng(41)
    x = rng.standard_normal((3, H)).astype(np.float32)
    groups = groups_for(rng, [(e, [e % 3] if e % 2 else [0, 2]) for e in range(n)])
    got = store.compute(0, x, groups)
    assert len(store.mapped) == map_size
    want = R.store_compute(x, groups, lambda e, xr: R.expert_exact(xr, *oracle_expert(src.load((0, e)))))
    close(got, want)


@pytest.mark.parametrize("H,I", [(2048, 768), (4096, 1536), (1024, 384)])
def test_decode_call_against_its_steps(kernels, H, I):
    """Experts with one row each and rows with 1 to 16 pairs (a decode
    step's top-k), f16 and f32 scales mixed in one call, experts taken
    through an index table, rows already holding values: the layer call
    against its steps called one by one (moe_q4_experts_matvec twice, then
    moe_combine) to 1e-6, and against float64 to 1e-5."""
    from distributedmoellm_amd import _lib
    rng = np.random.default_rng(H + I)
    npairs = [1, 8, 16, 3]                         # pairs of rows 0..3
    T = len(npairs)
    k = sum(npairs)
    experts = [X.synthetic_expert(H, I, "int4", 32, rng, scale_dtype=np.float32 if e % 5 == 2 else np.float16)
               for e in range(k)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    rows = [np.array([t], np.int32) for t in range(T) for _ in range(npairs[t])]
    ws = [rng.random(1).astype(np.float32) for _ in range(k)]
    perm = rng.permutation(k)                      # the table holds the experts in another order
    table = kernels.expert_table([experts[j] for j in perm])
    eidx = torch.from_numpy(np.argsort(perm).astype(np.int32)).cuda()
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e) for e in experts], rows, ws)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    base = rng.standard_normal((T, H)).astype(np.float32)
    out = torch.from_numpy(base).to(dev)
    ws_t = torch.empty(_lib.lib().moe_q4_layer_workspace(meta.P, H, I), dtype=torch.uint8, device=dev)
    st = kernels.stream_handle()
    _lib.call("moe_q4_layer", xd.data_ptr(), H, table.data_ptr(), eidx.data_ptr(), meta.k, meta.poff, meta.prow,
              meta.pw, meta.P, meta.rrow, meta.rptr, meta.rpair, meta.nr, out.data_ptr(), H, H, I, 32, 1,
              ws_t.data_ptr(), ws_t.numel(), st)
    h = torch.empty((meta.P, 2 * I), dtype=torch.float32, device=dev)
    y = torch.empty((meta.P, H), dtype=torch.float32, device=dev)
    two = torch.from_numpy(base).to(dev)
    _lib.call("moe_q4_experts_matvec", xd.data_ptr(), H, meta.prow, table.data_ptr(), eidx.data_ptr(), meta.k,
              meta.poff, 0, H, I, 32, 1, h.data_ptr(), 2 * I, st)
    _lib.call("moe_q4_experts_matvec", h.data_ptr(), 2 * I, None, table.data_ptr(), eidx.data_ptr(), meta.k,
              meta.poff, 1, H, I, 32, 1, y.data_ptr(), H, st)
    _lib.call("moe_combine", y.data_ptr(), H, meta.pw, meta.rrow, meta.rptr, meta.rpair, meta.nr, 16,
              two.data_ptr(), H, H, st)
    got, steps = out.cpu().numpy(), two.cpu().numpy()
    close(got - base, steps - base, rtol=1e-6)
    oitems = [(lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)), r, w) for e, r, w in zip(experts, rows, ws)]
    close(got, R.moe_q4(x, oitems, base.astype(np.float64)))


@pytest.mark.parametrize("H,I,gs,B,k,E", [
    (512, 256, 32, 1, 4, 16), (512, 256, 32, 6, 4, 16),      # mat-vec / rows GEMM
    (768, 384, 64, 3, 2, 8), (1024, 1536, 32, 5, 8, 32),     # 24-byte chunks; rows GEMM at I = 1536
    (2048, 768, 64, 2, 8, 64), (1024, 512, 128, 4, 4, 24),   # group 64 and 128 (int8 activations)
    (384, 640, 32, 3, 3, 12), (2048, 768, 32, 1, 8, 400),    # rows not a multiple of 256; many experts
])
def test_layer_call_dispatch_matrix(kernels, H, I, gs, B, k, E):
    """The layer call over the shapes that pick its different paths (the
    mat-vec with 1-4 rows a pass, the 24-byte chunks with and without the LDS
    ring, the rows GEMM, int8 activations at group 64 and 128), with random
    top-k routing of B tokens over E experts, against the float64 oracle
    (moe_q4 / moe_q4i, moelan/kernels.py:942-968, 854-917) at 1e-5."""
    rng = np.random.default_rng(H * 7 + I + gs + B * 13 + k + E)
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(E)]
    x = rng.standard_normal((B, H)).astype(np.float32)
    picks = {}
    for t in range(B):
        for e in rng.choice(E, size=k, replace=False):
            picks.setdefault(int(e), []).append(t)
    items, oitems, iitems = [], [], []
    for e, rows in sorted(picks.items()):
        r = np.array(rows, np.int32)
        w = rng.random(len(r)).astype(np.float32)
        m = experts[e]
        items.append((kernels.q4_expert_ptrs(m), r, w))
        oitems.append((lambda xr, m=m: R.expert_exact(xr, *oracle_expert(m)), r, w))
        iitems.append((m.gu.raw, m.gu.s, m.down.raw, m.down.s, m.gu.offset, r, w))
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, gs, out)
    if kernels.int8_act_for(H, I, gs):
        close(out, R.moe_q4i(x, iitems, np.zeros_like(x), H, I, gs))
    else:
        close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))
