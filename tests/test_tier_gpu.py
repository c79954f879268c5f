"""moelan's own call shapes through the drop-in, with moelan-shaped stand-ins
(objects with exactly the fields moelan's classes have, host numpy arrays
only, no device side):

- the fused layer call as moelan's ExpertStore._compute_fused makes it
  (moelan/experts.py:729-753): ``kernels.q4_expert_ptrs(e)`` on an expert
  whose int4 matrices are moelan ``Packed4``s (``raw`` uint8, ``s`` f32,
  ``gs``, ``shape``, ``offset``), then ``kernels.moe_q4(x, items, H, I, gs,
  out)`` on numpy ``x`` / ``out``; the weights are copied to HBM once, not
  per call, also when the store reads the same mapped bytes again as new
  views;
- the device-tier hook of moelan's ExpertStore.compute (``store.gpu``,
  moelan/experts.py:641-670 and accel.py:75-188) served by ``HipTier``.
Every result is checked against the float64 oracle at 1e-5."""

import numpy as np
import pytest

from distributedmoellm_amd import experts as X
from distributedmoellm_amd import sources as S
from distributedmoellm_amd.tier import HipTier
from oracle import restate as R

from test_matvec_gpu import close
from test_sources import write_colibri

pytestmark = pytest.mark.gpu


class MoelanPacked4:
    """The fields of moelan's Packed4 (moelan/experts.py:170-186)."""
    __slots__ = ("raw", "s", "gs", "shape", "offset")

    def __init__(self, raw, s, gs, shape, offset=False):
        self.raw, self.s, self.gs, self.shape, self.offset = raw, s, gs, tuple(shape), offset


class MoelanExpert:
    """The fields of moelan's Expert (moelan/experts.py:247-263)."""
    __slots__ = ("gu", "down", "inter", "fused")

    def __init__(self, gu, down, inter):
        self.gu, self.down, self.inter, self.fused = gu, down, inter, None


def moelan_expert(H, I, gs, rng):
    """Host-only int4 expert with f32 scales, as moelan's CheckpointSource makes."""
    def mat(o, i):
        return MoelanPacked4(rng.integers(0, 256, (o, i // 2), dtype=np.uint8),
                             (np.abs(rng.normal(0, 0.02, (o, i // gs))) / 8).astype(np.float32), gs, (o, i))
    return MoelanExpert(mat(2 * I, H), mat(H, I), I)


def exact_of(e):
    def dec(m):
        return R.q4_dequant64(np.asarray(m.raw), np.asarray(m.s), m.gs, m.offset)
    return lambda xr: R.expert_exact(xr, dec(e.gu), dec(e.down), e.inter)


def compute_fused(kernels, experts, x, groups, out):
    """moelan's ExpertStore._compute_fused, minus its store (experts.py:729-753)."""
    items, shape = [], None
    for expert, rows, weights in groups:
        e = experts[expert]
        if e.fused is None:
            e.fused = kernels.q4_expert_ptrs(e) or False
        assert e.fused, "a moelan Packed4 expert must qualify"
        shape = (e.gu.shape[1], e.inter, e.gu.gs)
        items.append((e.fused, rows, weights))
    kernels.moe_q4(x, items, *shape, out)


def routed(rng, T, E, k):
    picks = np.argsort(rng.random((T, E)), axis=1)[:, :k]
    return [(e, np.flatnonzero((picks == e).any(1)).astype(np.int32)) for e in range(E)
            if (picks == e).any()]


def test_moelan_packed4_through_the_layer_call_uploads_once(kernels):
    rng = np.random.default_rng(3)
    H, I, gs, E = 1024, 512, 32, 6
    experts = [moelan_expert(H, I, gs, rng) for _ in range(E)]
    before = kernels.HOST_COPIES.uploads
    used = set()
    for step in range(4):
        T = (1, 4, 7, 2)[step]
        x = rng.standard_normal((T, H)).astype(np.float32)
        groups = [(e, r, rng.random(len(r)).astype(np.float32)) for e, r in routed(rng, T, E, 2)]
        out = np.zeros_like(x)
        compute_fused(kernels, experts, x, groups, out)
        want = R.moe_q4(x, [(exact_of(experts[e]), r, w) for e, r, w in groups], np.zeros(x.shape))
        close(out, want)
        used |= {e for e, _, _ in groups}
        # four arrays an expert (gate|up and down bytes and scales), each copied once, on first use
        assert kernels.HOST_COPIES.uploads - before == 4 * len(used)
    for e in experts:
        e.fused = e.fused or kernels.q4_expert_ptrs(e)
    first = kernels.HOST_COPIES.uploads
    assert first - before == 4 * E
    # the store reads an expert again: new objects, new views of the same bytes -> no upload
    again = [MoelanExpert(MoelanPacked4(e.gu.raw[:], e.gu.s[:], gs, e.gu.shape),
                          MoelanPacked4(e.down.raw[:], e.down.s[:], gs, e.down.shape), I) for e in experts]
    x = rng.standard_normal((3, H)).astype(np.float32)
    groups = [(e, np.arange(3, dtype=np.int32), np.full(3, 0.5, np.float32)) for e in range(E)]
    out = np.zeros_like(x)
    compute_fused(kernels, again, x, groups, out)
    assert kernels.HOST_COPIES.uploads == first
    close(out, R.moe_q4(x, [(exact_of(again[e]), r, w) for e, r, w in groups], np.zeros(x.shape)))


def test_moelan_mapped_experts_and_copies_freed_with_the_host_arrays(kernels, tmp_path):
    """Experts as views of a memory-mapped colibri container (read-only
    arrays, as moelan's CheckpointSource gives them); their device copies go
    when the last host view does."""
    import gc
    H, I, gs = 512, 256, 32
    write_colibri(tmp_path / "c", H=H, I=I, gs=gs, layers=1, experts=3)
    src = S.CheckpointSource(tmp_path / "c")
    n0 = len(kernels.HOST_COPIES)

    def as_moelan(e):
        return MoelanExpert(MoelanPacked4(e.gu.raw, e.gu.s, gs, e.gu.shape),
                            MoelanPacked4(e.down.raw, e.down.s, gs, e.down.shape), e.inter)
    experts = [as_moelan(src.load((0, i))) for i in range(3)]
    assert not experts[0].gu.raw.flags.writeable
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, H)).astype(np.float32)
    groups = [(0, np.array([0, 3], np.int32), np.array([0.25, 1.0], np.float32)),
              (1, np.array([1, 2, 3, 4], np.int32), rng.random(4).astype(np.float32)),
              (2, np.array([4], np.int32), np.array([2.0], np.float32))]
    out = np.ones_like(x)                                   # the call adds into out
    compute_fused(kernels, experts, x, groups, out)
    close(out, R.moe_q4(x, [(exact_of(experts[e]), r, w) for e, r, w in groups], np.ones(x.shape)))
    assert len(kernels.HOST_COPIES) == n0 + 12
    del experts, src
    gc.collect()
    assert len(kernels.HOST_COPIES) == n0


def store_compute(tier, layer, x, groups, host_expert):
    """The GPU part of moelan's ExpertStore.compute (experts.py:641-670): the
    tier's share is launched first, the host computes the rest meanwhile (here
    the oracle stands in for moelan's CPU kernels), then the tier's sum is
    collected."""
    out = np.zeros_like(x, dtype=np.float32)
    handle, rest = tier.launch_held(layer, x, groups)
    for expert, rows, w in rest:
        out[rows] += (host_expert(expert)(x[rows]) * w[:, None]).astype(np.float32)
    if handle is not None:
        tier.collect(handle, out)
    return out


def test_hip_tier_serves_the_store_protocol(kernels):
    rng = np.random.default_rng(5)
    H, I, gs, E = 1024, 512, 32, 8
    experts = {e: moelan_expert(H, I, gs, rng) for e in range(E)}
    tier = HipTier("hip", budget_bytes=5 * tier_bytes(H, I, gs))
    placed = [e for e in range(E) if tier.add((2, e), experts[e])]
    assert placed == [0, 1, 2, 3, 4]                            # the budget holds five
    assert (2, 3) in tier and (2, 6) not in tier and (1, 0) not in tier
    before = kernels.HOST_COPIES.uploads
    for T in (1, 6, 16):
        x = rng.standard_normal((T, H)).astype(np.float32)
        groups = [(e, r, rng.random(len(r)).astype(np.float32)) for e, r in routed(rng, T, E, 3)]
        got = store_compute(tier, 2, x, groups, lambda e: exact_of(experts[e]))
        want = R.moe_q4(x, [(exact_of(experts[e]), r, w) for e, r, w in groups], np.zeros(x.shape))
        close(got, want)
    assert kernels.HOST_COPIES.uploads == before                # the tier's experts are its own HBM copies
    st = tier.stats()
    assert st["experts"] == 5 and st["calls"] == 3 and st["used_bytes"] == 5 * tier_bytes(H, I, gs)
    share = tier.calibrate(experts[7], lambda xx: exact_of(experts[7])(xx), hidden=H, repeats=2)
    assert 0.0 < share < 1.0 and (-1, 0) not in tier and tier.stats()["used_bytes"] == 5 * tier_bytes(H, I, gs)
    tier.release()
    assert not tier.experts and tier.used == 0
    h, rest = tier.launch_held(2, np.zeros((1, H), np.float32), [(0, np.array([0]), np.ones(1, np.float32))])
    assert h is None and len(rest) == 1


def tier_bytes(H, I, gs):
    return 3 * H * I // 2 + 3 * H * I // gs * 4


def test_hip_tier_other_formats(kernels):
    """int8 (moelan GroupQuant fields) and f32 experts in the tier, next to int4."""
    rng = np.random.default_rng(6)
    H, I, gs = 256, 128, 32
    e4 = moelan_expert(H, I, gs, rng)
    e8 = X.synthetic_expert(H, I, "int8", 64, rng, scale_dtype=np.float32)
    w_gu = rng.standard_normal((2 * I, H)).astype(np.float32) * 0.05
    w_dn = rng.standard_normal((H, I)).astype(np.float32) * 0.05

    class MoelanF32:
        __slots__ = ("w",)

        def __init__(self, w):
            self.w = w
    ef = MoelanExpert(MoelanF32(w_gu), MoelanF32(w_dn), I)
    tier = HipTier()
    for k, e in enumerate((e4, e8, ef)):
        assert tier.add((0, k), e)
    x = rng.standard_normal((4, H)).astype(np.float32)
    groups = [(0, np.array([0, 1], np.int32), np.array([1.0, 0.5], np.float32)),
              (1, np.array([1, 2, 3], np.int32), np.array([0.25, 0.5, 0.75], np.float32)),
              (2, np.array([0, 3], np.int32), np.array([2.0, 1.0], np.float32))]
    got = store_compute(tier, 0, x, groups, None)
    q8 = lambda m: R.q8_dequant64(m.q, m.s, m.gs)  # noqa: E731
    fns = [exact_of(e4), lambda xr: R.expert_exact(xr, q8(e8.gu), q8(e8.down), I),
           lambda xr: R.expert_exact(xr, w_gu.astype(np.float64), w_dn.astype(np.float64), I)]
    want = R.moe_q4(x, [(fns[e], r, w) for e, r, w in groups], np.zeros(x.shape))
    close(got, want)


def test_store_f32_format_with_threads(kernels):
    """ExpertStore(sources, fmt="f32", threads=4, gs=32): int4 experts read by
    four loader threads and widened to f32 on the device; the layer's sum
    matches the oracle of the int4 experts (the widening is exact)."""
    rng = np.random.default_rng(9)
    H, I, gs = 256, 128, 32
    experts = {e: X.synthetic_expert(H, I, "int4", gs, rng) for e in range(4)}

    class Source:
        zero_copy = False

        def has(self, key):
            return key[0] == 0 and key[1] in experts

        def load(self, key):
            return experts[key[1]]
    store = X.ExpertStore([Source()], fmt="f32", lru_size=0, threads=4, gs=gs, map_size=16)
    store.pin([(0, e) for e in range(4)])
    assert all(isinstance(store.pinned[(0, e)].gu, X.F32Matrix) for e in range(4))
    x = rng.standard_normal((6, H)).astype(np.float32)
    groups = [(e, np.sort(rng.choice(6, 3, replace=False)).astype(np.int32), rng.random(3).astype(np.float32))
              for e in range(4)]
    got = store.compute(0, x, groups)

    def exact(e):
        m = experts[e]
        d = lambda p: R.q4_dequant64(p.raw, p.s, p.gs, p.offset)  # noqa: E731
        return lambda xr: R.expert_exact(xr, d(m.gu), d(m.down), I)
    close(got, R.moe_q4(x, [(exact(e), r, w) for e, r, w in groups], np.zeros(x.shape)))
