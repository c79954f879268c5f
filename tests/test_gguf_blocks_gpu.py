"""The GGUF block types besides Q8_0 / Q4_K on the GPU (moelan/kernels.py:
270-453 decoders, 499-676 fused mat-vecs), as moelan tests/test_gguf.py:25-39
checks them against gguf-py: dequant bit-exact on random bytes (Inf/NaN
scale fields included, +0.0 and -0.0 told apart), the mat-vec within 1e-5 of
the float64 product of the decoded weights, rows of every alignment, and a
Q4_K / Q5_K / Q6_K expert (the mix of a Q4_K_M file) through the expert call."""

import numpy as np
import pytest

from distributedmoellm_amd import gguf as G
from oracle import restate as R

from test_matvec_gpu import close

pytestmark = pytest.mark.gpu

TYPES = [R.Q4_0, R.Q4_1, R.Q5_0, R.Q5_1, R.Q2_K, R.Q3_K, R.Q5_K, R.Q6_K]
IDS = [R.QTYPES[q][0] for q in TYPES]


@pytest.mark.parametrize("qtype", TYPES, ids=IDS)
def test_dequant_bit_exact_on_random_bytes(kernels, qtype):
    rng = np.random.default_rng(qtype)
    cols = 512
    raw = rng.integers(0, 256, (64, cols // R.QTYPES[qtype][1] * R.QTYPES[qtype][2]), dtype=np.uint8)
    out = np.empty((64, cols), np.float32)
    kernels.gguf_dequant(raw, qtype, out)
    with np.errstate(invalid="ignore", over="ignore"):
        want = R.gguf_dequant(raw, qtype, cols)
    ok = np.isfinite(want)
    assert np.array_equal(np.isfinite(out), ok)
    assert np.array_equal(out[ok].view(np.uint32), want[ok].view(np.uint32))
    assert np.array_equal(np.isnan(out), np.isnan(want))


@pytest.mark.parametrize("qtype", TYPES, ids=IDS)
def test_dequant_well_behaved_blocks(kernels, qtype):
    rng = np.random.default_rng(100 + qtype)
    raw = R.random_blocks(48, 768, qtype, rng)
    out = np.empty((48, 768), np.float32)
    kernels.gguf_dequant(raw, qtype, out)
    want = R.gguf_dequant(raw, qtype, 768)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", TYPES, ids=IDS)
@pytest.mark.parametrize("rows", [1, 2, 5])
@pytest.mark.parametrize("O,cols", [(768, 2048), (2048, 768)])
def test_matmul(kernels, qtype, rows, O, cols):
    """The Qwen3-30B-A3B expert shapes: gate / up [768, 2048], down [2048, 768]
    (rows of 768 values are 2-byte aligned for Q3_K and Q6_K)."""
    rng = np.random.default_rng(qtype * 100 + rows + O)
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("qtype", TYPES, ids=IDS)
@pytest.mark.parametrize("nblk", [1, 3, 5, 7])
def test_matmul_every_row_alignment(kernels, qtype, nblk):
    """Odd block counts: rows start at every byte offset the block size allows;
    few chunks a row leave most lanes of a row group idle."""
    per = R.QTYPES[qtype][1]
    cols = per * nblk
    rng = np.random.default_rng(qtype + 17 * nblk)
    raw = R.random_blocks(37, cols, qtype, rng)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("qtype", [R.Q4_0, R.Q6_K], ids=["Q4_0", "Q6_K"])
def test_matmul_wide_rows(kernels, qtype):
    """Rows of 4096 and 8192 values: two and four chunks a lane."""
    rng = np.random.default_rng(qtype + 5)
    for cols in (4096, 8192):
        raw = R.random_blocks(300, cols, qtype, rng)
        x = rng.standard_normal((2, cols)).astype(np.float32)
        close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("qtype", [R.Q4_0, R.Q4_1, R.Q5_0, R.Q5_1, R.Q8_0, R.Q4_K, R.Q5_K],
                         ids=["Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "Q4_K", "Q5_K"])
@pytest.mark.parametrize("O,cols", [(37, 2048), (300, 16384)])
def test_matmul_one_row_shared_setup(kernels, qtype, O, cols):
    """One input row, 32-value kinds: the workgroup builds the row's chunks
    once in LDS. 37 rows leave waves past the matrix's end; rows of 16384
    values take two launches of 256 chunks, the second adding to the first."""
    rng = np.random.default_rng(qtype + O)
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


def test_q4_k_m_style_expert(kernels):
    """gate Q4_K, up Q5_K, down Q6_K (moelan tests/test_gguf.py:46 expert types)
    through Expert.__call__: SwiGLU on the device against float64."""
    rng = np.random.default_rng(3)
    H, I = 2048, 768
    e = G.synthetic_expert(H, I, ["Q4_K", "Q5_K", "Q6_K"], rng)
    x = rng.standard_normal((3, H)).astype(np.float32)
    Wg = R.gguf_dequant(e.gu.parts[0].raw, R.Q4_K, H)
    Wu = R.gguf_dequant(e.gu.parts[1].raw, R.Q5_K, H)
    Wd = R.gguf_dequant(e.down.raw, R.Q6_K, I)
    want = R.expert_exact(x, np.concatenate([Wg, Wu], 0).astype(np.float64), Wd.astype(np.float64), I)
    close(e(x), want)


@pytest.mark.parametrize("qtype", [R.Q8_0, R.Q4_K], ids=["Q8_0", "Q4_K"])
@pytest.mark.parametrize("rows", [16, 32, 50])
@pytest.mark.parametrize("O,cols", [(768, 2048), (2048, 768), (37, 256)])
def test_many_rows_mfma(kernels, qtype, rows, O, cols):
    """From 16 rows a Q8_0 / Q4_K product widens each block in registers with
    the dequant's own f32 operations and runs f32 MFMA: within 1e-5 of the
    float64 product of the decoded weights."""
    rng = np.random.default_rng(rows + O + qtype)
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("qtype", [R.Q8_0, R.Q4_K], ids=["Q8_0", "Q4_K"])
def test_many_rows_mfma_one_hot_exact(kernels, qtype):
    """Row i of x = e_c: column c of the decoded matrix bit for bit."""
    rng = np.random.default_rng(40 + qtype)
    O, cols = 64, 512
    raw = R.random_blocks(O, cols, qtype, rng)
    W = R.gguf_dequant(raw, qtype, cols)
    cs = [0, 1, 31, 32, 33, 63, 64, 127, 128, 200, 255, 256, 300, 383, 384, 511]
    x = np.zeros((len(cs), cols), np.float32)
    x[np.arange(len(cs)), cs] = 1.0
    assert np.array_equal(kernels.gguf_matmul_t(x, raw, qtype, cols), W[:, cs].T)
