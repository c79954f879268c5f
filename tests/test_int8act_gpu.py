"""The layer call with int8 activations on the GPU (moelan/kernels.py:784-917,
chosen by int8_act_for :920-922), mirroring moelan tests/test_fused.py:89-192.

- The rounding is bit-exact to the oracle's _round_q8 (ties, zero groups, every
  group size).
- The layer call matches the oracle's _moe_q4i within RTOL_I8. Its integer group
  sums are exact; what differs is the f32 order in which the group terms are
  added (a lane tree here, groups in order there), a few 1e-7 of a row, and
  SiLU's last bit, which could move an activation onto the next int8 step (about
  1e-4 of its row); on these seeded inputs no step moves.
- It stays within the reference's own bounds of the float layer.
- With MOELAN_INT8_ACT off it is the exact float call.
"""

import numpy as np
import pytest
import torch

from distributedmoellm_amd import experts as X
from oracle import restate as R

from test_layer_gpu import oracle_expert
from test_matvec_gpu import close

pytestmark = pytest.mark.gpu

# the layer call against the oracle's _moe_q4i, norm-wise and per row
RTOL_I8 = 1e-5


def host(a):
    return a.cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)


def oracle_item(e, rows, w):
    return (host(e.gu.raw), host(e.gu.s), host(e.down.raw), host(e.down.s), e.gu.offset, rows, w)


def assert_close_to_float(want, got):
    """The reference's bounds (moelan tests/test_fused.py:104-111)."""
    assert np.linalg.norm(got - want) < 3e-2 * np.linalg.norm(want)
    assert float((want * got).sum() / np.sqrt((want * want).sum() * (got * got).sum())) > 0.999
    for r in range(want.shape[0]):
        if np.abs(want[r]).max() > 0:
            assert np.linalg.norm(got[r] - want[r]) < 5e-2 * np.linalg.norm(want[r])


@pytest.fixture
def int8_on(kernels, monkeypatch):
    monkeypatch.setattr(kernels, "INT8_ACT", True)
    return kernels


@pytest.mark.parametrize("gs", [64, 128, 192, 256, 512])
def test_rounding_is_bit_exact(kernels, gs):
    rng = np.random.default_rng(gs)
    K = 1536 if gs in (192, 512) else 2048
    K = K // gs * gs
    x = (rng.standard_normal((7, K)) * rng.choice([1e-3, 1.0, 40.0], (7, 1))).astype(np.float32)
    x[1, :gs] = 0.0                                   # a zero group: scale 1, q 0
    ties = rng.integers(-127, 127, gs).astype(np.float32) + 0.5
    ties[0] = 127.0                                   # scale exactly 1: every other value a tie
    x[2, gs:2 * gs] = ties
    x[3, :gs] = -x[3, :gs]
    q, d, s8 = kernels.round_q8(x, gs)
    for r in range(x.shape[0]):
        wq, wd, ws8 = R.round_q8(x[r], gs)
        assert np.array_equal(q[r].astype(np.int32), wq), f"row {r}"
        assert np.array_equal(d[r].view(np.uint32), wd.view(np.uint32)), f"row {r}"
        assert np.array_equal(s8[r], ws8), f"row {r}"
    # the tie group rounds half up, as floor(v + 0.5)
    assert np.array_equal(q[2, gs + 1:2 * gs], np.floor(ties[1:] + 0.5).astype(np.int8))


def run_layer(kernels, experts, picks, x, H, I, gs, base=None):
    items, oitems = [], []
    for e, rows in zip(experts, picks):
        w = np.random.default_rng(len(items) + 7).random(len(rows)).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(e), rows, w))
        oitems.append(oracle_item(e, rows, w))
    out = np.zeros_like(x) if base is None else base.copy()
    kernels.moe_q4(x, items, H, I, gs, out)
    torch.cuda.synchronize()
    want = R.moe_q4i(x, oitems, np.zeros_like(x) if base is None else base, H, I, gs)
    return out, want, items


@pytest.mark.parametrize("H,I,gs,T,k", [
    (128, 128, 64, 6, 8),        # the reference's group-64 fixture shape (general kernel)
    (2048, 768, 64, 1, 8),       # Qwen3-30B-A3B shape, one token (two lanes a group)
    (2048, 768, 64, 4, 8),
    (2048, 768, 128, 3, 8),      # four lanes a group
    (1536, 384, 192, 2, 6),      # a group size that is not a power of two (general kernel)
    (2048, 768, 256, 2, 4),
])
def test_layer_matches_the_oracle(int8_on, H, I, gs, T, k):
    kernels = int8_on
    assert kernels.int8_act_for(H, I, gs)
    rng = np.random.default_rng(H + I + gs + T)
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(k)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    picks = [np.sort(rng.choice(T, size=min(T, 1 + i % 3), replace=False)).astype(np.int32) for i in range(k)]
    out, want, _ = run_layer(kernels, experts, picks, x, H, I, gs)
    err = np.linalg.norm(out - want) / np.linalg.norm(want)
    print(f"int8 layer H={H} I={I} gs={gs} T={T} k={k}: rel err vs oracle {err:.2e}")
    close(out, want, rtol=RTOL_I8)


def test_resident_and_stored_copies_in_one_call(int8_on):
    """moelan tests/test_fused.py:146-163 with a resident (offset) and a stored copy."""
    kernels = int8_on
    H, I, gs = 2048, 768, 64
    rng = np.random.default_rng(11)
    a, b = (X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(2))
    b = X.Expert(b.gu.resident(), b.down.resident(), b.inter)
    assert b.gu.offset and not a.gu.offset
    x = rng.standard_normal((2, H)).astype(np.float32)
    out, want, _ = run_layer(kernels, [a, b], [np.array([0, 1], np.int32), np.array([1], np.int32)], x, H, I, gs)
    close(out, want, rtol=RTOL_I8)


@pytest.mark.parametrize("H,I,gs", [(128, 128, 64), (2048, 768, 64)])
def test_close_to_float_activations(kernels, monkeypatch, H, I, gs):
    """moelan tests/test_fused.py:114-143: eight rows, each with its own experts;
    int8 against float activations within the reference's bounds."""
    rng = np.random.default_rng(6)
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(8)]
    x = rng.standard_normal((8, H)).astype(np.float32)
    items = [(kernels.q4_expert_ptrs(experts[i]), np.array(sorted({i, (i + 3) % 8}), np.int32),
              rng.random(2).astype(np.float32)) for i in range(8)]
    got = {}
    for flag in (False, True):
        monkeypatch.setattr(kernels, "INT8_ACT", flag)
        got[flag] = np.zeros_like(x)
        kernels.moe_q4(x, items, H, I, gs, got[flag])
    torch.cuda.synchronize()
    assert_close_to_float(got[False], got[True])
    assert not np.array_equal(got[False], got[True])    # the int8 call did run


def test_int8_off_is_the_exact_float_call(kernels, monkeypatch):
    """moelan tests/test_fused.py:166-178: MOELAN_INT8_ACT=0 at groups of 64."""
    monkeypatch.setattr(kernels, "INT8_ACT", False)
    H, I, gs = 2048, 768, 64
    rng = np.random.default_rng(5)
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(3)]
    x = rng.standard_normal((3, H)).astype(np.float32)
    want = np.zeros(x.shape)
    items = []
    for i, e in enumerate(experts):
        rows = np.array([0, i], np.int32) if i else np.array([0], np.int32)
        w = rng.random(len(rows)).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(e), rows, w))
        want[rows] += R.expert_exact(x[rows], *oracle_expert(e)) * w[:, None].astype(np.float64)
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, gs, out)
    close(out, want)


def test_rows_with_many_pairs(int8_on):
    """One row in 96 experts' lists and another in 17, added into a non-zero out."""
    kernels = int8_on
    H, I, gs, k = 256, 128, 64, 96
    rng = np.random.default_rng(96)
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(k)]
    x = rng.standard_normal((2, H)).astype(np.float32)
    picks = [np.array([0, 1], np.int32) if i < 17 else np.array([0], np.int32) for i in range(k)]
    base = rng.standard_normal((2, H)).astype(np.float32) * 0.05
    out, want, _ = run_layer(kernels, experts, picks, x, H, I, gs, base=base)
    close(out, want, rtol=RTOL_I8)
    close(out - base, want - base, rtol=1e-3)
