"""Decode mat-vec and dequant on the GPU against the oracle, through the C ABI.

Bars: unpacking bit-exact (dequant, one-hot columns); the f32 FMA mat-vec
within 1e-5 relative to the float64 oracle, norm-wise over the output and per
output row (tolerance RTOL below). Shapes: the reference test's 96x128, the
Qwen3-30B-A3B expert (gate|up 1536x2048, down 2048x768), the Qwen3-235B-A22B
expert (gate|up 3072x4096, down 4096x1536), tiny and odd shapes that take the
LDS-reduction and generic kernels.
"""

import numpy as np
import pytest
import torch

from oracle import restate as R

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def close(got, ref, rtol=RTOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    assert np.all(np.isfinite(got))
    err = np.linalg.norm(got - ref)
    assert err <= rtol * np.linalg.norm(ref), f"relative error {err / np.linalg.norm(ref):.3e}"
    for r in range(ref.shape[0]):
        e = np.linalg.norm(got[r] - ref[r])
        assert e <= rtol * max(np.linalg.norm(ref[r]), 1e-30), f"row {r}: {e / np.linalg.norm(ref[r]):.3e}"


def int4_matrix(rng, O, I, gs, sdt=np.float16):
    raw = rng.integers(0, 256, (O, I // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 8).astype(sdt)
    return raw, s


SHAPES = [(96, 128, 32), (1536, 2048, 32), (2048, 768, 32), (64, 64, 32), (2048, 64, 32), (64, 96, 32),
          (128, 128, 64), (3072, 4096, 32), (4096, 1536, 32), (40, 8192, 32)]


@pytest.mark.parametrize("O,I,gs", SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 17])
def test_q4_matmul(kernels, O, I, gs, rows):
    rng = np.random.default_rng(O * 7 + I + rows)
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, gs, False), R.q4_matmul_t(x, raw, s, gs, False))


@pytest.mark.parametrize("offset", [False, True])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_q4_offset_and_scale_types(kernels, offset, sdt):
    rng = np.random.default_rng(1)
    raw, s = int4_matrix(rng, 1536, 2048, 32, sdt)
    if sdt == np.float32:
        s = rng.random(s.shape).astype(np.float32) * 1e-3      # full 24-bit scales
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, 32, offset), R.q4_matmul_t(x, raw, s, 32, offset))


@pytest.mark.parametrize("O,I,gs", [(96, 128, 32), (2048, 768, 32), (64, 96, 32)])
def test_q4_one_hot_columns_are_exact(kernels, O, I, gs):
    """x = e_c: the kernel returns column c of W bit-exactly (nibble order, sign, scale index)."""
    rng = np.random.default_rng(2)
    raw, s = int4_matrix(rng, O, I, gs)
    W = R.q4_dequant(raw, s, gs, False)
    cols = [0, 1, 2, 31, 32, 33, I - 2, I - 1]
    x = np.zeros((len(cols), I), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = kernels.q4_matmul_t(x, raw, s, gs, False)
    for i, c in enumerate(cols):
        assert np.array_equal(y[i], W[:, c]), f"column {c}"


@pytest.mark.parametrize("spread", [0.0, 3.0, 6.0])
def test_q4_activation_dynamic_range(kernels, spread):
    """The 32-value chunks are multiplied as exact fixed point scaled from each
    chunk's largest |x| (integer dot8 on 4-bit limbs): values spread over
    `spread` decades inside a chunk, all-zero chunks, and overall scales of
    1e20 and 1e-20 stay within 1e-5 of the float64 product (four input rows)."""
    rng = np.random.default_rng(int(spread * 10) + 5)
    O, I, gs = 1536, 2048, 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((4, I)) * 10.0 ** rng.uniform(-spread, 0, (4, I))
    x[1, 64:128] = 0.0
    x[2] *= 1e20
    x[3] *= 1e-20
    x = x.astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, gs, False), R.q4_matmul_t(x, raw, s, gs, False))


@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_q4_non_finite_activation_is_not_hidden(kernels, bad):
    """An inf or a NaN in the input row makes every output of the row NaN, as
    in the float product (where inf * 0 and inf - inf give NaN); the other
    input rows stay finite."""
    rng = np.random.default_rng(8)
    O, I, gs = 256, 2048, 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((2, I)).astype(np.float32)
    x[0, 100] = bad
    y = kernels.q4_matmul_t(x, raw, s, gs, False)
    assert np.isnan(y[0]).all()
    close(y[1:], R.q4_matmul_t(x[1:], raw, s, gs, False))


@pytest.mark.parametrize("O,I", [(1536, 2048), (2048, 768)])
@pytest.mark.parametrize("ratio", [1e3, 1e4])
def test_q4_outlier_channels(kernels, O, I, ratio):
    """Activations with one or two outlier channels per row, 1e3-1e4 times the
    rest (as LLM hidden states have), at the Qwen3-30B-A3B expert shapes.
    Norm-wise per input row the product stays within 1e-5 of float64; element
    by element the error stays within the integer dot's bound (each product
    term off by at most 8 * 2^-22 of its run's largest |x|, times the group
    scale), plus f32 rounding of the sums. The largest element-wise relative
    error is reported (it is large only where an output row gives the outlier
    a zero nibble and the rest of its sum is small)."""
    rng = np.random.default_rng(int(ratio) + O)
    gs = 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((3, I)).astype(np.float32)
    x[0, 77] = ratio
    x[1, [5, I - 300]] = [-ratio, 0.5 * ratio]
    x[2, 33] = ratio * 3.0
    got = kernels.q4_matmul_t(x, raw, s, gs, False)
    want = R.q4_matmul_t(x, raw, s, gs, False)
    close(got, want)
    # the bound, per output: sum over the row's runs of 8 * 2^-22 * max|x in run| * sum |s| over the run
    W_abs_s = np.repeat(np.abs(s.astype(np.float64)), gs, axis=1)          # |s| per column
    run = 32                                                              # three input rows: 32-value chunks
    xm = np.abs(x.astype(np.float64)).reshape(3, I // run, run).max(2)
    term = np.repeat(xm, run, axis=1) * 8 * 2.0 ** -22                     # per column, per input row
    bound = term @ W_abs_s.T
    f32_slack = 64 * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ (W_abs_s * 8).T)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound + f32_slack), f"max excess {(err - bound - f32_slack).max():.3e}"
    rel = err / np.maximum(np.abs(want), 1e-30)
    print(f"outlier x{ratio:g} [{O}x{I}]: max element-wise relative error {rel.max():.2e}, "
          f"norm-wise {np.linalg.norm(err) / np.linalg.norm(want):.2e}")


def test_q4_generic_shapes(kernels):
    """Group sizes that split a 32-column chunk and widths not divisible by 32 take the generic kernel."""
    rng = np.random.default_rng(3)
    for O, I, gs in ((24, 64, 16), (10, 48, 16), (7, 20, 10)):
        raw, s = int4_matrix(rng, O, I, gs, np.float32)
        x = rng.standard_normal((3, I)).astype(np.float32)
        close(kernels.q4_matmul_t(x, raw, s, gs, False), R.q4_matmul_t(x, raw, s, gs, False))


def test_q4_unaligned_device_buffers(kernels):
    """Weights at an odd byte offset in HBM: the kernel reads bytes instead of 16-byte words."""
    rng = np.random.default_rng(4)
    O, I, gs = 256, 2048, 32
    raw, s = int4_matrix(rng, O, I, gs)
    big = torch.zeros(raw.size + 1, dtype=torch.uint8, device="cuda")
    big[1:] = torch.from_numpy(raw.reshape(-1)).cuda()
    raw_d = big[1:].view(O, I // 2)
    x = rng.standard_normal((2, I)).astype(np.float32)
    got = kernels.q4_matmul_t(torch.from_numpy(x).cuda(), raw_d, torch.from_numpy(s).cuda(), gs, False)
    close(got.cpu().numpy(), R.q4_matmul_t(x, raw, s, gs, False))


def test_q4_device_tensors_stay_on_device(kernels):
    rng = np.random.default_rng(5)
    raw, s = int4_matrix(rng, 256, 512, 32)
    x = torch.from_numpy(rng.standard_normal((2, 512)).astype(np.float32)).cuda()
    y = kernels.q4_matmul_t(x, torch.from_numpy(raw).cuda(), torch.from_numpy(s).cuda(), 32, False)
    assert isinstance(y, torch.Tensor) and y.is_cuda and y.shape == (2, 256)


def test_zero_rows(kernels):
    raw, s = int4_matrix(np.random.default_rng(0), 64, 64, 32)
    assert kernels.q4_matmul_t(np.zeros((0, 64), np.float32), raw, s, 32, False).shape == (0, 64)


# ---------------------------------------------------------------- int8

@pytest.mark.parametrize("rows", [1, 4, 16, 64])
@pytest.mark.parametrize("O,I,gs", [(1536, 2048, 32), (2048, 768, 32), (96, 128, 32), (64, 96, 16)])
def test_q8_matmul(kernels, rows, O, I, gs):
    rng = np.random.default_rng(rows + O)
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 127).astype(np.float16)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    close(kernels.q8_matmul_t(x, q, s, gs), R.q8_matmul_t(x, q, s, gs))


def test_q8_one_hot_exact(kernels):
    rng = np.random.default_rng(6)
    O, I, gs = 2048, 768, 32
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = rng.random((O, I // gs)).astype(np.float32)
    W = R.q8_dequant(q, s, gs)
    cols = [0, 15, 16, 767]
    x = np.zeros((4, I), np.float32)
    x[np.arange(4), cols] = 1.0
    y = kernels.q8_matmul_t(x, q, s, gs)
    for i, c in enumerate(cols):
        assert np.array_equal(y[i], W[:, c])


# ---------------------------------------------------------------- GGUF

@pytest.mark.parametrize("qtype", [8, 12])
@pytest.mark.parametrize("rows", [1, 2, 5, 32])
@pytest.mark.parametrize("O,cols", [(768, 2048), (2048, 768)])
def test_gguf_matmul(kernels, qtype, rows, O, cols):
    rng = np.random.default_rng(qtype * 100 + rows + O)
    raw = R.random_blocks(O, cols, qtype, rng)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


@pytest.mark.parametrize("qtype", [8, 12])
def test_gguf_odd_block_counts(kernels, qtype):
    """Q8_0 rows of an odd number of blocks start 2-byte aligned: the byte path."""
    rng = np.random.default_rng(7)
    cols = 32 * 5 if qtype == 8 else 256 * 3
    raw = R.random_blocks(9, cols, qtype, rng)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    close(kernels.gguf_matmul_t(x, raw, qtype, cols), R.gguf_matmul_t(x, raw, qtype, cols))


# ---------------------------------------------------------------- dequant (bit-exact)

@pytest.mark.parametrize("offset", [False, True])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_q4_dequant_bit_exact(kernels, offset, sdt):
    rng = np.random.default_rng(8)
    raw, s = int4_matrix(rng, 1536, 2048, 32, sdt)
    if sdt == np.float32:
        s = rng.random(s.shape).astype(np.float32)
    out = np.empty((1536, 2048), np.float32)
    kernels.q4_dequant(raw, s, 32, offset, out)
    assert np.array_equal(out, R.q4_dequant(raw, s, 32, offset))


def test_q8_dequant_bit_exact(kernels):
    rng = np.random.default_rng(9)
    q = rng.integers(-127, 128, (2048, 768), dtype=np.int8)
    s = rng.random((2048, 24)).astype(np.float32)
    out = np.empty((2048, 768), np.float32)
    kernels.q8_dequant(q, s, 32, out)
    assert np.array_equal(out, R.q8_dequant(q, s, 32))


@pytest.mark.parametrize("qtype", [8, 12])
def test_gguf_dequant_bit_exact_on_random_bytes(kernels, qtype):
    """Every byte random, Inf/NaN scale fields included (moelan tests/test_gguf.py:25-33 style):
    finite values equal bit for bit, non-finite ones in the same places."""
    rng = np.random.default_rng(qtype)
    cols = 512
    raw = rng.integers(0, 256, (64, cols // R.QTYPES[qtype][1] * R.QTYPES[qtype][2]), dtype=np.uint8)
    out = np.empty((64, cols), np.float32)
    kernels.gguf_dequant(raw, qtype, out)
    want = R.gguf_dequant(raw, qtype, cols)
    ok = np.isfinite(want)
    assert np.array_equal(np.isfinite(out), ok)
    assert np.array_equal(out[ok], want[ok])
    assert np.array_equal(np.isnan(out), np.isnan(want))


# ---------------------------------------------------------------- 24-byte chunks (one input row)

# (1001, 768, 64) and (1002, 768, 128) with f16 scales: the matrix's scale bytes
# do not end on a 16-byte boundary (24 and 12 bytes a row), which the LDS ring
# does not take; those matrices run the register path.
W24_SHAPES = [(200, 384, 32), (2048, 768, 32), (2048, 768, 16), (1000, 768, 48), (2048, 768, 64),
              (4096, 1536, 32), (96, 3072, 64), (1001, 768, 64), (1002, 768, 128), (1003, 384, 64)]


@pytest.mark.parametrize("O,I,gs", W24_SHAPES)
@pytest.mark.parametrize("offset", [False, True])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_q4_w24_single_row(kernels, O, I, gs, offset, sdt):
    """Rows whose 16-byte chunks leave lanes idle but whose 24-byte chunks fill
    8, 16, 32 or 64 lanes (I = 384, 768, 1536, 3072), one input row."""
    rng = np.random.default_rng(O + I + gs)
    raw, s = int4_matrix(rng, O, I, gs, sdt)
    if sdt == np.float32:
        s = rng.random(s.shape).astype(np.float32) * 1e-3
    x = rng.standard_normal((1, I)).astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, gs, offset), R.q4_matmul_t(x, raw, s, gs, offset))


@pytest.mark.parametrize("sdt", [np.float16, np.float32])
@pytest.mark.parametrize("shift", [4, 8])
def test_q4_w24_unaligned_operands(kernels, sdt, shift):
    """Weights and scales `shift` bytes past a 16-byte boundary (the LDS ring
    takes 16-byte aligned operands only; these rows take the register path):
    the same results as aligned operands."""
    from distributedmoellm_amd import _lib
    rng = np.random.default_rng(11 + shift)
    O, I, gs = 2048, 768, 32
    raw, s = int4_matrix(rng, O, I, gs, sdt)
    x = rng.standard_normal((1, I)).astype(np.float32)
    dev = torch.device("cuda")
    rb = torch.zeros(raw.nbytes + 16, dtype=torch.uint8, device=dev)
    rb[shift:shift + raw.nbytes].copy_(torch.from_numpy(raw.reshape(-1)))
    sb = torch.zeros(s.nbytes + 16, dtype=torch.uint8, device=dev)
    sb[shift:shift + s.nbytes].copy_(torch.from_numpy(np.ascontiguousarray(s).view(np.uint8).reshape(-1)))
    xd = torch.from_numpy(x).to(dev)
    y = torch.empty((1, O), dtype=torch.float32, device=dev)
    _lib.call("moe_q4_matmul_t", xd.data_ptr(), 1, rb.data_ptr() + shift, sb.data_ptr() + shift,
              1 if sdt == np.float16 else 0, O, I, gs, 0, y.data_ptr(), kernels.stream_handle())
    got = y.cpu().numpy()
    close(got, R.q4_matmul_t(x, raw, s, gs, False))
    assert np.array_equal(got, kernels.q4_matmul_t(x, raw, s, gs, False))


@pytest.mark.parametrize("scale", [1.0, 1e20, 1e-20])
def test_q4_w24_activation_dynamic_range(kernels, scale):
    """768-value rows (24-byte chunks, integer dot per 16-value sub-chunk):
    values spread over 6 decades, all-zero sub-chunks and overall scales of
    1e20 / 1e-20 stay within 1e-5 of the float64 product."""
    rng = np.random.default_rng(21)
    O, I, gs = 2048, 768, 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((1, I)) * 10.0 ** rng.uniform(-6, 0, (1, I)) * scale
    x[0, 16:48] = 0.0
    x = x.astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, gs, False), R.q4_matmul_t(x, raw, s, gs, False))


@pytest.mark.parametrize("bad", [-np.inf, np.nan])
def test_q4_w24_non_finite_activation_is_not_hidden(kernels, bad):
    rng = np.random.default_rng(22)
    O, I, gs = 512, 768, 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((1, I)).astype(np.float32)
    x[0, 700] = bad
    assert np.isnan(kernels.q4_matmul_t(x, raw, s, gs, False)).all()


def test_q4_w24_one_hot_columns_are_exact(kernels):
    """x = e_c, one row at a time: column c of W bit-exactly, across sub-chunk and group edges."""
    rng = np.random.default_rng(3)
    O, I, gs = 256, 768, 32
    raw, s = int4_matrix(rng, O, I, gs)
    W = R.q4_dequant(raw, s, gs, False)
    for c in [0, 1, 15, 16, 31, 32, 47, 48, 63, 64, 95, 96, 767]:
        x = np.zeros((1, I), np.float32)
        x[0, c] = 1.0
        y = kernels.q4_matmul_t(x, raw, s, gs, False)
        assert np.array_equal(y[0], W[:, c]), f"column {c}"


@pytest.mark.parametrize("H,I,gs,sdt,n", [(4096, 1536, 32, np.float16, 64), (2048, 768, 16, np.float32, 256),
                                          (960, 768, 64, np.float16, 256), (2048, 384, 32, np.float16, 384)])
def test_q4_w24_ring_many_experts(kernels, H, I, gs, sdt, n):
    """The down sweep of moe_q4_experts_matvec over n experts, one row each
    (SiLU(gate) * up on load): with this many matrices every resident wave
    streams 8 or more stages, which takes the LDS ring (a single matrix or a
    few take the register path, covered above). One expert's row holds a NaN
    and gives NaN outputs; the rest are within 1e-5 of float64."""
    from distributedmoellm_amd import _lib
    from distributedmoellm_amd import experts as X
    rng = np.random.default_rng(H + I + gs + n)
    ex = [X.synthetic_expert(H, I, "int4", gs, rng, scale_dtype=sdt) for _ in range(n)]
    h = rng.standard_normal((n, 2 * I)).astype(np.float32)
    h[n // 2, 5] = np.nan
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e) for e in ex], [np.array([i], np.int32) for i in range(n)],
                             [np.ones(1, np.float32)] * n)
    dev = torch.device("cuda")
    hd = torch.from_numpy(h).to(dev)
    y = torch.empty((n, H), dtype=torch.float32, device=dev)
    _lib.call("moe_q4_experts_matvec", hd.data_ptr(), 2 * I, None, meta.table, None, meta.k, meta.poff, 1,
              H, I, gs, 1, y.data_ptr(), H, kernels.stream_handle())
    got = y.cpu().numpy()
    h64 = h.astype(np.float64)
    a = R.silu(h64[:, :I]) * h64[:, I:]
    want = np.stack([R.matmul_t_exact(a[i:i + 1], R.q4_dequant64(e.down.raw, e.down.s, gs, False))[0]
                     for i, e in enumerate(ex)])
    assert np.isnan(got[n // 2]).all()
    keep = np.arange(n) != n // 2
    close(got[keep], want[keep])


@pytest.mark.parametrize("which,H,I,gs,sdt,n", [
    (0, 4096, 1536, 32, np.float16, 8),     # 128 chunks a row: 2 a lane
    (0, 2048, 768, 32, np.float32, 40),     # 64 chunks a row
    (0, 1792, 96, 32, np.float16, 5),       # 56 chunks on 64 lanes, 192 rows a matrix
    (0, 2048, 768, 32, np.float16, 300),    # a large launch: runs of 16 groups a wave
    (0, 8192, 64, 32, np.float32, 3),       # 256 chunks a row, 4 a lane (25.6 KB of LDS)
    (1, 768, 1024, 32, np.float16, 16),     # down sweep, SiLU(gate) * up built once a workgroup
    (1, 1008, 768, 16, np.float16, 5),      # down sweep in 24-byte chunks, 126 waves a matrix
    (1, 4096, 1536, 32, np.float16, 8),     # the same, one token on the Qwen3-235B-A22B expert
    (1, 2048, 768, 32, np.float32, 200),    # the same through the LDS ring
])
def test_q4_one_row_a_matrix_shared_setup(kernels, which, H, I, gs, sdt, n):
    """One input row a matrix: the workgroup's 4 waves build the row's
    activation chunks once, in LDS; waves past a matrix's last output row
    still take part (16- and 24-byte chunks, register path and LDS ring).
    Input rows are shared between matrices through xrow, one
    matrix reads a row holding an infinity (non-finite outputs, nothing else
    touched). Within 1e-5 of float64."""
    from distributedmoellm_amd import _lib
    from distributedmoellm_amd import experts as X
    rng = np.random.default_rng(which + H + I + n)
    ex = [X.synthetic_expert(H, I, "int4", gs, rng, scale_dtype=sdt) for _ in range(n)]
    cols = 2 * I if which else H
    nx = max(2, n // 2)
    x = rng.standard_normal((nx, cols)).astype(np.float32)
    xrow = rng.integers(0, nx - 1, n).astype(np.int32)   # the last input row only where set below
    xrow[n // 2] = nx - 1
    x[nx - 1, 3] = np.inf
    meta = kernels.LayerMeta([kernels.q4_expert_ptrs(e) for e in ex], [np.array([i], np.int32) for i in range(n)],
                             [np.ones(1, np.float32)] * n)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xr = torch.from_numpy(xrow).to(dev)
    O = H if which else 2 * I
    y = torch.empty((n, O), dtype=torch.float32, device=dev)
    _lib.call("moe_q4_experts_matvec", xd.data_ptr(), cols, xr.data_ptr(), meta.table, None, meta.k, meta.poff, which,
              H, I, gs, 1, y.data_ptr(), O, kernels.stream_handle())
    got = y.cpu().numpy()
    x64 = x.astype(np.float64)[xrow]
    if which:
        x64 = R.silu(x64[:, :I]) * x64[:, I:]
    mats = [e.down if which else e.gu for e in ex]
    keep = np.arange(n) != n // 2
    want = np.stack([R.matmul_t_exact(x64[i:i + 1], R.q4_dequant64(m.raw, m.s, gs, False))[0]
                     for i, m in enumerate(mats) if keep[i]])
    assert not np.isfinite(got[n // 2]).all()
    close(got[keep], want)


# ---------------------------------------------------------------- many rows: f32 MFMA product

@pytest.mark.parametrize("rows", [16, 33, 64])
@pytest.mark.parametrize("O,I,gs", [(1536, 2048, 32), (2048, 768, 32), (100, 256, 64), (37, 512, 128)])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_q8_matmul_many_rows(kernels, rows, O, I, gs, sdt):
    """From 16 rows the int8 product widens q * s in registers and runs f32
    MFMA (exact weights, f32 sums): within 1e-5 of float64, rows and weight
    rows past a 16-tile edge included."""
    rng = np.random.default_rng(rows * 3 + O + I)
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 127).astype(sdt)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    close(kernels.q8_matmul_t(x, q, s, gs), R.q8_matmul_t(x, q, s, gs))


@pytest.mark.parametrize("rows", [16, 40])
@pytest.mark.parametrize("offset", [False, True])
@pytest.mark.parametrize("O,I,gs,sdt", [(1536, 2048, 32, np.float16), (4096, 1536, 32, np.float16),
                                        (70, 512, 64, np.float32), (48, 320, 32, np.float32)])
def test_q4_matmul_many_rows(kernels, rows, offset, O, I, gs, sdt):
    rng = np.random.default_rng(rows + O * 5 + int(offset))
    raw, s = int4_matrix(rng, O, I, gs, sdt)
    x = rng.standard_normal((rows, I)).astype(np.float32)
    close(kernels.q4_matmul_t(x, raw, s, gs, offset), R.q4_matmul_t(x, raw, s, gs, offset))


def test_many_rows_one_hot_columns_are_exact(kernels):
    """Row c of x = e_c: the f32 MFMA product returns column c of the widened
    matrix bit for bit (int4 and int8), across chunk and group edges."""
    rng = np.random.default_rng(9)
    O, I, gs = 80, 256, 32
    cols = [0, 1, 15, 16, 31, 32, 63, 64, 100, 127, 128, 200, 255, 3, 77, 190, 250]
    x = np.zeros((len(cols), I), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    raw, s = int4_matrix(rng, O, I, gs)
    W = R.q4_dequant(raw, s, gs, False)
    assert np.array_equal(kernels.q4_matmul_t(x, raw, s, gs, False), W[:, cols].T)
    q = rng.integers(-127, 128, (O, I), dtype=np.int8)
    s8 = (np.abs(rng.normal(0, 0.02, (O, I // gs))) / 127).astype(np.float16)
    W8 = R.q8_dequant(q, s8, gs)
    assert np.array_equal(kernels.q8_matmul_t(x, q, s8, gs), W8[:, cols].T)


def test_many_rows_dynamic_range_and_non_finite(kernels):
    """Rows scaled by 1e20 and 1e-20 stay within 1e-5 (f32 products and sums);
    a NaN in a row makes that row's outputs NaN and leaves the others."""
    rng = np.random.default_rng(10)
    O, I, gs = 256, 512, 32
    raw, s = int4_matrix(rng, O, I, gs)
    x = rng.standard_normal((32, I)).astype(np.float32)
    x[:8] *= 1e20
    x[8:16] *= 1e-20
    close(kernels.q4_matmul_t(x, raw, s, gs, False), R.q4_matmul_t(x, raw, s, gs, False))
    x[20, 100] = np.nan
    y = kernels.q4_matmul_t(x, raw, s, gs, False)
    assert np.isnan(y[20]).all()
    assert np.isfinite(np.delete(y, 20, 0)).all()
