"""Experts read from checkpoint files run on the GPU: a colibri int4 container
and a Q4_K / Q5_K / Q6_K GGUF file through ExpertStore (pinned, mapped and
on-demand) and the worker's moe step, against the float64 oracle on the bytes
the files hold."""

import numpy as np
import pytest

from distributedmoellm_amd import experts as X
from distributedmoellm_amd import sources as S
from distributedmoellm_amd import wire as W
from oracle import restate as R

from test_matvec_gpu import close
from test_sources import gguf_moe, write_colibri

pytestmark = pytest.mark.gpu


def groups_for(rng, T, picks):
    return [(e, np.array(rows, np.int32), rng.random(len(rows)).astype(np.float32)) for e, rows in picks]


def test_colibri_store_layer_call(kernels, tmp_path, monkeypatch):
    H, I, gs = 256, 128, 64
    written = write_colibri(tmp_path / "c", H=H, I=I, gs=gs)
    store = X.ExpertStore([S.CheckpointSource(tmp_path / "c")], fmt="int4")
    store.pin([(1, 0), (1, 2)])
    assert all(e.gu._dev is not None for e in store.pinned.values())     # uploaded at pin
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, H)).astype(np.float32)
    groups = groups_for(rng, 5, [(0, [0, 2]), (1, [1, 2, 3]), (2, [4]), (3, [0, 1, 2, 3, 4])])

    def exact(e, xr):
        w, s = written[(1, e)]
        ngu = I * H
        Wgu = R.q4_dequant64(w[:ngu].reshape(2 * I, H // 2), s[:2 * I * H // gs].reshape(2 * I, H // gs), gs, False)
        Wdn = R.q4_dequant64(w[ngu:].reshape(H, I // 2), s[2 * I * H // gs:].reshape(H, I // gs), gs, False)
        return R.expert_exact(xr, Wgu, Wdn, I)
    monkeypatch.setattr(kernels, "INT8_ACT", False)      # float activations: the exact layer
    close(store.compute(1, x, groups), R.store_compute(x, groups, exact))
    assert store.hits == 2 and store.misses == 2 and len(store.mapped) == 2


def test_gguf_store_layer_call_and_worker_step(kernels, tmp_path):
    path = tmp_path / "m.gguf"
    H = I = 256
    stacks = gguf_moe(path, H=H, I=I)
    store = X.ExpertStore([S.GGUFSource(path)], fmt="native")
    store.pin([(0, 1)])
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, H)).astype(np.float32)
    groups = groups_for(rng, 4, [(1, [0, 3]), (2, [1]), (3, [0, 1, 2])])

    def exact(e, xr):
        Wg = R.gguf_dequant(stacks[(0, "gate")][e], R.Q4_K, H)
        Wu = R.gguf_dequant(stacks[(0, "up")][e], R.Q5_K, H)
        Wd = R.gguf_dequant(stacks[(0, "down")][e], R.Q6_K, I)
        return R.expert_exact(xr, np.concatenate([Wg, Wu], 0).astype(np.float64), Wd.astype(np.float64), I)
    want = R.store_compute(x, groups, exact)
    close(store.compute(0, x, groups), want)
    # the same layer through the worker's moe op, y back in f32 on the wire
    ex = np.array([e for e, _, _ in groups], np.int32)
    rows = np.concatenate([r for _, r, _ in groups])
    off = np.concatenate([[0], np.cumsum([len(r) for _, r, _ in groups])]).astype(np.int32)
    w = np.concatenate([wt for _, _, wt in groups])
    reply = W.worker_moe(store, 0, dict(x=x, experts=ex, offsets=off, rows=rows, weights=w), "f32")
    assert reply["rows"].tolist() == [0, 1, 2, 3]
    close(reply["y"].cpu().numpy(), want[[0, 1, 2, 3]])


def test_staged_upload_matches_per_array_upload(kernels, tmp_path):
    """ExpertStore.pin's staged copies (pinned buffers, one device allocation
    per matrix) hold the same bytes as device_arrays(), for int4, int8 and GGUF
    matrices, across several staging-buffer switches."""
    from distributedmoellm_amd import gguf as G
    rng = np.random.default_rng(4)
    ex = [X.synthetic_expert(512, 256, "int4", 32, rng) for _ in range(5)]
    ex += [X.synthetic_expert(512, 256, "int8", 64, rng, scale_dtype=np.float32) for _ in range(3)]
    ex += [G.synthetic_expert(512, 256, ["Q4_K", "Q5_0", "Q6_K"], rng) for _ in range(3)]
    X.upload_experts(ex, stage_bytes=200_000)
    for e in ex:
        for part in X._matrices(e):
            staged = [t.cpu().numpy() for t in part._dev]
            part._dev = None
            direct = [t.cpu().numpy() for t in part.device_arrays()]
            assert len(staged) == len(direct)
            for a, b in zip(staged, direct):
                assert a.dtype == b.dtype and a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))
