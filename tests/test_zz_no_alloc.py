"""moe_q4_layer_noalloc: the layer call with its scratch in library-held device
memory (no workspace argument, no allocation) against moe_q4_layer with a
caller workspace, through the C ABI: bit-identical outputs (the same kernels
in the same order) on two calls in a row, the second one smaller, and both
within 1e-5 of the float64 oracle; a call needing more than the held scratch
is refused with a message."""

import numpy as np
import pytest
import torch

from distributedmoellm_amd import _lib
from distributedmoellm_amd import experts as X
from oracle import restate as R

from test_layer_gpu import oracle_expert
from test_matvec_gpu import close

pytestmark = pytest.mark.gpu


def noalloc():
    return _lib.lib().moe_q4_layer_noalloc


def case(kernels, rng, H, I, gs, T, k):
    experts = [X.synthetic_expert(H, I, "int4", gs, rng) for _ in range(k)]
    x = rng.standard_normal((T, H)).astype(np.float32)
    rows = [np.sort(rng.choice(T, size=1 + i % min(T, 3), replace=False)).astype(np.int32) for i in range(k)]
    ws = [rng.random(len(r)).astype(np.float32) for r in rows]
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e) for e in experts], rows, ws)
    want = R.moe_q4(x, [(lambda xr, e=e: R.expert_exact(xr, *oracle_expert(e)), r, w)
                        for e, r, w in zip(experts, rows, ws)], np.zeros(x.shape))
    return experts, torch.from_numpy(x).cuda(), meta, want


def run_with_workspace(kernels, xd, meta, H, I, gs):
    out = torch.zeros_like(xd)
    kernels.moe_q4_run(xd, meta, H, I, gs, out, int8=False)
    return out


def run_noalloc(kernels, xd, meta, H, I, gs):
    out = torch.zeros_like(xd)
    rc = noalloc()(xd.data_ptr(), H, meta.table, None, meta.k, meta.poff, meta.prow, meta.pw, meta.P, meta.rrow,
                   meta.rptr, meta.rpair, meta.nr, out.data_ptr(), H, H, I, gs, meta.max_rows,
                   kernels.stream_handle())
    _lib.check(rc)
    return out


def test_noalloc_layer_matches_workspace_call_twice(kernels):
    rng = np.random.default_rng(77)
    H, I, gs = 2048, 768, 32
    big = case(kernels, rng, H, I, gs, T=4, k=24)
    small = case(kernels, rng, H, I, gs, T=2, k=5)
    for experts, xd, meta, want in (big, small):
        a = run_noalloc(kernels, xd, meta, H, I, gs)
        b = run_with_workspace(kernels, xd, meta, H, I, gs)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        close(a.cpu().numpy(), want)


def test_noalloc_layer_refuses_more_than_its_scratch(kernels):
    rng = np.random.default_rng(78)
    H, I, gs = 4096, 1536, 32
    e = X.synthetic_expert(H, I, "int4", gs, rng)
    # 1200 pairs x (2I + H) x 4 bytes = 34.4 MB > 32 MiB held
    T = 1200
    rows = [np.arange(T, dtype=np.int32)]
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e)], rows, [np.ones(T, np.float32)])
    xd = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    out = torch.zeros_like(xd)
    rc = noalloc()(xd.data_ptr(), H, meta.table, None, meta.k, meta.poff, meta.prow, meta.pw, meta.P, meta.rrow,
                   meta.rptr, meta.rpair, meta.nr, out.data_ptr(), H, H, I, gs, meta.max_rows,
                   kernels.stream_handle())
    assert rc == _lib.MOE_EWORKSPACE
    assert "scratch" in _lib.last_error()
