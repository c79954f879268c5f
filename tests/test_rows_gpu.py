"""The layer call for experts with several rows each (the integer-MFMA rows
GEMM of csrc/rows.hip, taken when some expert has 2 or more rows, H and I are
multiples of 256 and the group size is 32) against the float64 oracle at
1e-5: row counts 1..13 per expert (quads of 4 rows, partial quads), f16 and
f32 scales, stored and XOR-ed (offset) copies, experts with no rows, rows
shared between experts, outlier and non-finite activations. Reference:
moe_q4 / _moe_q4 (moelan/kernels.py:942-968, 712-782) and _q4_rows (:108-131)."""

import numpy as np
import pytest
import torch

from distributedmoellm_amd import experts as X
from oracle import restate as R

from test_layer_gpu import oracle_expert
from test_matvec_gpu import close

pytestmark = pytest.mark.gpu


def layer_case(kernels, rng, H, I, counts, T, scale_dtype=np.float16, offset=False, x=None):
    experts = []
    for c in counts:
        e = X.synthetic_expert(H, I, "int4", 32, rng, scale_dtype=scale_dtype)
        if scale_dtype == np.float32:   # full 24-bit scales
            e.gu.s = (rng.random(e.gu.s.shape) * 1e-3).astype(np.float32)
            e.down.s = (rng.random(e.down.s.shape) * 1e-3).astype(np.float32)
        if offset:
            e = X.Expert(e.gu.resident(), e.down.resident(), e.inter)
        experts.append(e)
    if x is None:
        x = rng.standard_normal((T, H)).astype(np.float32)
    items, oitems = [], []
    for e, c in zip(experts, counts):
        rows = np.sort(rng.choice(T, size=c, replace=False)).astype(np.int32)
        w = rng.random(c).astype(np.float32)
        items.append((kernels.q4_expert_ptrs(e), rows, w))
        oitems.append((lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)), rows, w))
    return experts, x, items, oitems


@pytest.mark.parametrize("counts", [(2,), (3, 1, 4), (5, 2, 9, 1, 13), (8, 8, 8, 8), (1, 1, 6)])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_rows_layer_row_counts(kernels, counts, sdt):
    rng = np.random.default_rng(sum(counts) * 7 + (sdt == np.float32))
    H, I, T = 512, 256, 16
    _, x, items, oitems = layer_case(kernels, rng, H, I, counts, T, sdt)
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, out)
    close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))


def test_rows_layer_offset_copies_and_shapes(kernels):
    """XOR-ed resident copies, the Qwen3-30B-A3B expert shape (H=2048, I=768:
    3-stage down rows) and the Qwen3-235B-A22B one (H=4096, I=1536)."""
    for H, I, offset in ((2048, 768, True), (2048, 768, False), (4096, 1536, True)):
        rng = np.random.default_rng(H + offset)
        _, x, items, oitems = layer_case(kernels, rng, H, I, (3, 6, 1), 8, offset=offset)
        out = np.zeros_like(x)
        kernels.moe_q4(x, items, H, I, 32, out)
        close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))


def test_rows_layer_empty_expert_and_eidx(kernels):
    """An expert with no rows in the pair lists (through the C ABI with an
    expert index list), next to experts with several."""
    from distributedmoellm_amd import _lib
    rng = np.random.default_rng(5)
    H, I, T = 512, 256, 6
    experts = [X.synthetic_expert(H, I, "int4", 32, rng) for _ in range(4)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    rows = [np.array([0, 2, 5], np.int32), np.zeros(0, np.int32), np.array([1, 2, 3, 4, 5], np.int32),
            np.array([3], np.int32)]
    ws = [rng.random(len(r)).astype(np.float32) for r in rows]
    order = [2, 0, 3, 1]   # table entries used through eidx
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e) for e in experts], [rows[o] for o in order],
                             [ws[o] for o in order])
    eidx = torch.tensor(order, dtype=torch.int32, device="cuda")
    xd = torch.from_numpy(x).cuda()
    out = torch.zeros_like(xd)
    need = _lib.lib().moe_q4_layer_workspace(meta.P, H, I)
    wsp = torch.empty(need, dtype=torch.uint8, device="cuda")
    _lib.call("moe_q4_layer", xd.data_ptr(), H, meta.table, eidx.data_ptr(), meta.k, meta.poff, meta.prow, meta.pw,
              meta.P, meta.rrow, meta.rptr, meta.rpair, meta.nr, out.data_ptr(), H, H, I, 32, meta.max_rows,
              wsp.data_ptr(), wsp.numel(), kernels.stream_handle())
    want = R.moe_q4(x, [(lambda xr, e=experts[o]: R.expert_exact(xr, *oracle_expert(e)), rows[o], ws[o])
                        for o in order], np.zeros(x.shape))
    close(out.cpu().numpy(), want)


def test_rows_layer_outliers_keep_precision(kernels):
    """Rows with outlier channels 1e4 times the rest: the rows GEMM takes each
    input row as 30-bit fixed point, so the other values keep ~17 bits and every
    output stays within 1e-5 of float64, element by element relative to the
    row's norm."""
    rng = np.random.default_rng(9)
    H, I, T = 2048, 768, 8
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[:, 100] = 1e4
    x[3, 1500] = -3e4
    _, x, items, oitems = layer_case(kernels, rng, H, I, (4, 7, 2), T, x=x)
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, out)
    want = R.moe_q4(x, oitems, np.zeros(x.shape))
    close(out, want)


@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_rows_layer_non_finite_row(kernels, bad):
    """A non-finite value in one input row makes that row's outputs NaN; the
    other rows stay exact."""
    rng = np.random.default_rng(10)
    H, I, T = 512, 256, 5
    x = rng.standard_normal((T, H)).astype(np.float32)
    x[2, 77] = bad
    experts = [X.synthetic_expert(H, I, "int4", 32, rng) for _ in range(2)]
    rows = [np.arange(5, dtype=np.int32), np.array([0, 1, 3], np.int32)]
    w = [rng.random(len(r)).astype(np.float32) for r in rows]
    items = [(kernels.q4_expert_ptrs(e), r, ww) for e, r, ww in zip(experts, rows, w)]
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, out)
    assert np.isnan(out[2]).all()
    ok = [0, 1, 3, 4]
    want = R.moe_q4(x[ok], [(lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)),
                             np.searchsorted(ok, r[np.isin(r, ok)]), ww[np.isin(r, ok)])
                            for e, r, ww in zip(experts, rows, w)], np.zeros((4, H)))
    close(out[ok], want)


def test_rows_layer_matches_row_by_row_calls(kernels):
    """The same experts and rows through the rows GEMM (several rows an
    expert) and one row a call (the mat-vec path): within 1e-5 of each other
    and of float64."""
    rng = np.random.default_rng(11)
    H, I, T = 1024, 512, 12
    experts, x, items, oitems = layer_case(kernels, rng, H, I, (12, 5, 3), T)
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, out)
    one = np.zeros_like(x)
    for p, rows, w in items:
        for r, ww in zip(rows, w):
            kernels.moe_q4(x, [(p, np.array([r], np.int32), np.array([ww], np.float32))], H, I, 32, one)
    want = R.moe_q4(x, oitems, np.zeros(x.shape))
    close(out, want)
    close(one, want)


@pytest.mark.parametrize("H", [8192, 16384])
def test_rows_layer_long_rows(kernels, H):
    """Input rows of 8192 and 16384 values: the limb kernel holds 4 and 8
    chunks of 8 values a thread."""
    rng = np.random.default_rng(H)
    I, T = 256, 6
    _, x, items, oitems = layer_case(kernels, rng, H, I, (3, 5, 2), T)
    x[1, H - 7] = 40.0      # the row's largest value in its last chunk
    out = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, out)
    close(out, R.moe_q4(x, oitems, np.zeros(x.shape)))


def test_rows_layer_unaligned_input_rows(kernels):
    """Input rows 4 bytes apart from 16-byte alignment (ldx = H + 1): the limb
    kernel's scalar loads, the same results as aligned rows."""
    from distributedmoellm_amd import _lib
    rng = np.random.default_rng(5)
    H, I, T = 1024, 512, 8
    _, x, items, oitems = layer_case(kernels, rng, H, I, (4, 7, 2), T)
    meta = kernels.LayerMeta([p for p, _, _ in items], [r for _, r, _ in items], [w for _, _, w in items])
    dev = torch.device("cuda")
    buf = torch.zeros((T, H + 1), dtype=torch.float32, device=dev)
    buf[:, 1:] = torch.from_numpy(x).to(dev)
    out = torch.zeros((T, H), dtype=torch.float32, device=dev)
    ws = torch.empty(_lib.lib().moe_q4_layer_workspace(meta.P, H, I), dtype=torch.uint8, device=dev)
    _lib.call("moe_q4_layer", buf.data_ptr() + 4, H + 1, meta.table, None, meta.k, meta.poff, meta.prow, meta.pw,
              meta.P, meta.rrow, meta.rptr, meta.rpair, meta.nr, out.data_ptr(), H, H, I, 32, meta.max_rows,
              ws.data_ptr(), ws.numel(), kernels.stream_handle())
    got = out.cpu().numpy()
    close(got, R.moe_q4(x, oitems, np.zeros(x.shape)))
    aligned = np.zeros_like(x)
    kernels.moe_q4(x, items, H, I, 32, aligned)
    assert np.array_equal(got, aligned)
