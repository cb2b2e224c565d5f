"""QTensor::matmul / dequantize on the GPU vs the CPU oracle.

Bars:
  - dequantized weights bit-exact: fl(scale * q) (qtensor.rs:265-272);
  - int formats: bit-exact against the closed form of the GPU arithmetic
    (tests/qgen.py) -- this pins the digitisation and the dot8/dot4 lanes;
  - all formats: within the reference's own SIMD-vs-scalar bound,
    1e-4 * max(|oracle|, 1) (undertow-quant/src/avx512.rs:335-366), of the
    scalar oracle (kernels.rs:21-81);
  - a row's value does not depend on seq (qtensor.rs:274-280): bitwise equal
    for M = 1..5.
Shapes: the reference's odd SIMD test shapes, BASELINE config-2 expert
shapes, and the dense projection shapes of configs 1 and 4.
"""
import numpy as np
import pytest

from conftest import dev, host
from oracle import oracle as O
from qgen import F32, INT4, INT8, codes, gemv_closed_form, rand_qtensor

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 16), (5, 17), (8, 64), (7, 130), (16, 256), (2, 31),  # avx512.rs:335-366
          (96, 256), (256, 512), (64, 128), (2048, 7168), (7168, 2048), (192, 96), (1536, 7168),
          (256, 7168), (576, 7168), (96, 16384),  # split-K shapes: router, kv_a, o_proj-like
          (65600, 256)]  # >= 65,536 rows: int8 at 3-4 rows takes two tiles per wave, ragged last tile
FMTS = [INT4, INT8, F32]


def upload(ctx, fmt, payload, scales, o, i):
    import undertow_amd as U
    return U.QTensor(ctx, fmt, payload, scales, o, i)


def run_matmul(ctx, qt, x):
    import torch
    seq, i = x.shape
    out = torch.full((seq, qt.out_dim), float("nan"), device="cuda:0")
    xd = dev(x)
    qt.matmul(out, xd, seq)
    return host(out)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("o,i", SHAPES)
def test_matmul_matches_oracle(ctx, fmt, o, i):
    rng = np.random.default_rng(o * 1000 + i + fmt)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    qt = upload(ctx, fmt, payload, scales, o, i)
    x = rng.standard_normal((3, i)).astype(np.float32)
    got = run_matmul(ctx, qt, x)
    want = O.matmul(fmt, payload, scales, o, i, x)
    assert np.isfinite(got).all()
    tol = 1e-4 * np.maximum(np.abs(want), 1.0)
    assert (np.abs(got - want) <= tol).all(), np.abs(got - want).max()
    if fmt != F32:
        exact = gemv_closed_form(fmt, payload, scales, o, i, x)
        assert np.array_equal(got, exact)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("o,i", [(2048, 7168), (7168, 2048), (130, 64), (5, 17), (256, 7168),
                                 (7168, 16384), (1000, 192), (65600, 256)])
def test_rows_do_not_depend_on_seq(ctx, fmt, o, i):
    rng = np.random.default_rng(7)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    qt = upload(ctx, fmt, payload, scales, o, i)
    x = rng.standard_normal((5, i)).astype(np.float32)
    full = run_matmul(ctx, qt, x)
    for m in range(1, 6):
        part = run_matmul(ctx, qt, x[:m])
        assert np.array_equal(part, full[:m]), m
    for s in range(5):
        assert np.array_equal(run_matmul(ctx, qt, x[s:s + 1])[0], full[s])


@pytest.mark.parametrize("fmt", [INT4, INT8, F32])
@pytest.mark.parametrize("o,i", [(5, 17), (2048, 7168), (33, 96)])
def test_dequantize_bit_exact(ctx, fmt, o, i):
    rng = np.random.default_rng(11)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    qt = upload(ctx, fmt, payload, scales, o, i)
    got = host(qt.dequantize())
    want = O.dequantize(fmt, payload, scales, o, i)
    assert np.array_equal(got, want)
    if fmt != F32:
        closed = (scales[:, None] * codes(fmt, payload, o, i).astype(np.float32)).astype(np.float32)
        assert np.array_equal(got, closed)


def test_oracle_quantized_checkpoint_tensors(ctx):
    """Weights produced by the restated quantizer (qtensor.rs:142-213)."""
    rng = np.random.default_rng(3)
    w = rng.standard_normal((96, 256)).astype(np.float32) * 0.05
    x = rng.standard_normal((2, 256)).astype(np.float32)
    for fmt in (INT8, INT4):
        q, s = O.quantize(w, fmt)
        qt = upload(ctx, fmt, q, s, 96, 256)
        got = run_matmul(ctx, qt, x)
        want = O.matmul(fmt, q, s, 96, 256, x)
        assert np.abs(got - want).max() <= 1e-5


def test_zero_and_extreme_rows(ctx):
    o, i = 64, 256
    rng = np.random.default_rng(5)
    payload, scales = rand_qtensor(rng, INT4, o, i)
    qt = upload(ctx, INT4, payload, scales, o, i)
    x = np.zeros((4, i), np.float32)
    x[1, 3] = 1e-30                      # a tiny row
    x[2] = rng.standard_normal(i) * 3e4  # a large row
    x[3, :] = rng.standard_normal(i)
    x[3, 0] = 1e6                        # one dominant element
    got = run_matmul(ctx, qt, x)
    assert (got[0] == 0).all()
    want = O.matmul(INT4, payload, scales, o, i, x)
    assert np.array_equal(got, gemv_closed_form(INT4, payload, scales, o, i, x))
    # f32 rounding (the oracle's and ours) is relative to the row's magnitude
    row_mag = np.abs(want).max(axis=1, keepdims=True)
    assert (np.abs(got - want) <= 1e-5 * row_mag).all()


def test_non_finite_activation_gives_nan(ctx):
    o, i = 16, 64
    rng = np.random.default_rng(6)
    payload, scales = rand_qtensor(rng, INT8, o, i)
    qt = upload(ctx, INT8, payload, scales, o, i)
    x = rng.standard_normal((2, i)).astype(np.float32)
    x[1, 5] = np.inf
    got = run_matmul(ctx, qt, x)
    assert np.isfinite(got[0]).all() and np.isnan(got[1]).all()


def test_shape_mismatch_raises(ctx):
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(1)
    payload, scales = rand_qtensor(rng, INT4, 8, 64)
    qt = upload(ctx, INT4, payload, scales, 8, 64)
    x = torch.zeros(2 * 63, device="cuda:0")
    out = torch.zeros(2 * 8, device="cuda:0")
    with pytest.raises(U.ShapeError):
        qt.matmul(out, x, 2)
    with pytest.raises(U.UtError):
        U.QTensor(ctx, INT4, payload[:, :-1], scales, 8, 64)  # payload size mismatch
    q = U.QTensor(ctx, U.INFER, payload, scales, 8, 64)
    assert q.format == INT4


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("o,i,row0,nrows", [(16, 256, 3, 9), (7, 130, 0, 7), (32768, 512, 128, 128),
                                            (32768, 512, 32640, 128), (2048, 7168, 1000, 37)])
def test_matvec_rows_matches_oracle(ctx, fmt, o, i, row0, nrows):
    """QTensor::matvec_rows (qtensor.rs:548-586), e.g. one head's V block of
    kv_b at DeepSeek-V3 shape (128 heads x (128 + 128) rows x 512)."""
    import torch
    rng = np.random.default_rng(o + i + row0 + fmt)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    qt = upload(ctx, fmt, payload, scales, o, i)
    x = rng.standard_normal(i).astype(np.float32)
    out = torch.full((nrows,), float("nan"), device="cuda:0")
    qt.matvec_rows(row0, nrows, dev(x), out)
    got = host(out)
    want = O.matvec_rows(fmt, payload, scales, o, i, row0, nrows, x)
    tol = 1e-4 * np.maximum(np.abs(want), 1.0)
    assert (np.abs(got - want) <= tol).all(), np.abs(got - want).max()
    if fmt != F32:
        # the same rows of the whole-matrix GEMV, bit for bit
        full = run_matmul(ctx, qt, x[None, :])[0]
        assert np.array_equal(got, full[row0:row0 + nrows])


def test_matvec_rows_shape_errors(ctx):
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(1)
    payload, scales = rand_qtensor(rng, INT8, 16, 32)
    qt = upload(ctx, INT8, payload, scales, 16, 32)
    x = dev(rng.standard_normal(32).astype(np.float32))
    with pytest.raises(U.ShapeError):
        qt.matvec_rows(10, 7, x, torch.empty(7, device="cuda:0"))
    with pytest.raises(U.ShapeError):
        qt.matvec_rows(0, 4, x, torch.empty(5, device="cuda:0"))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("o,i,row,factor", [(16, 256, 5, 0.75), (7, 131, 6, -1.5), (512, 7168, 300, 3.0)])
def test_add_scaled_row_matches_oracle(ctx, fmt, o, i, row, factor):
    """QTensor::add_scaled_row (qtensor.rs:516-543): acc += (factor*scale)*q,
    bit-exact (one rounding per element, as the reference)."""
    rng = np.random.default_rng(o + i + row + fmt)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    qt = upload(ctx, fmt, payload, scales, o, i)
    acc0 = rng.standard_normal(i).astype(np.float32)
    acc = dev(acc0)
    qt.add_scaled_row(row, factor, acc)
    got = host(acc)
    want = O.add_scaled_row(fmt, payload, scales, o, i, row, factor, acc0)
    assert np.array_equal(got, want), np.abs(got - want).max()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("o,i", [(1, 1), (5, 17), (7, 130), (64, 129), (2048, 7168), (300, 1000)])
def test_quantize_bit_exact(ctx, fmt, o, i):
    """QTensor::quantize (qtensor.rs:142-213) on the device: codes and scales
    bit-identical to the oracle, including rows of zeros, rows whose ratios
    land on .5 (round half away from zero) and the odd-column nibble."""
    import undertow_amd as U
    rng = np.random.default_rng(o * 31 + i + fmt)
    w = (rng.standard_normal((o, i)) * rng.uniform(0.01, 3.0, (o, 1))).astype(np.float32)
    if o > 2:
        w[1] = 0.0
        # exact half-way ratios: max 7 (or 127) -> s = 1, entries k + 0.5
        qmax = 7.0 if fmt == INT4 else 127.0
        w[2] = np.float32(0.5) + np.arange(i, dtype=np.float32) % 5 - 2
        w[2, 0] = qmax
    qt = U.QTensor.quantize(ctx, dev(w), fmt)
    payload, scales = qt.download()
    want_p, want_s = O.quantize(w, fmt)
    assert np.array_equal(payload, np.ascontiguousarray(want_p).view(np.uint8).reshape(-1))
    if fmt != F32:
        assert np.array_equal(scales, want_s)
    # and it feeds the GEMV like an uploaded tensor
    x = rng.standard_normal((2, i)).astype(np.float32)
    assert np.array_equal(run_matmul(ctx, qt, x),
                          run_matmul(ctx, upload(ctx, fmt, want_p, want_s, o, i), x))


def test_quantize_rejects_non_finite(ctx):
    import undertow_amd as U
    w = np.ones((4, 10), np.float32)
    w[2, 7] = np.inf
    w[3, 1] = np.nan
    for fmt in (INT4, INT8, F32):
        with pytest.raises(U.UtError) as ei:
            U.QTensor.quantize(ctx, dev(w), fmt)
        assert ei.value.code == U.runtime.UT_ERR_FORMAT
        assert "flat index 27 (row 2, col 7)" in str(ei.value)


# ------------------------------------------------------------ fast int8
@pytest.mark.parametrize("o,i,seq", [(4, 64, 2), (7, 130, 2), (3, 16, 2), (512, 7168, 3),
                                     (129, 1000, 1), (2048, 2048, 4)])
def test_fast_int8_matches_oracle(ctx, o, i, seq):
    """set_fast_int8 (lib.rs:31-59, avx512.rs:221-242): bit for bit the
    oracle's restatement, within the reference's 3 % of the row magnitude of
    the exact path (neon.rs:257-278), and off again restores the exact
    path."""
    import torch
    rng = np.random.default_rng(900 + o + i)
    w = rng.uniform(-1.0, 1.0, (o, i)).astype(np.float32)
    q, s = O.quantize(w, INT8)
    qt = upload(ctx, INT8, q, s, o, i)
    x = rng.uniform(-1.0, 1.0, (seq, i)).astype(np.float32)
    exact = run_matmul(ctx, qt, x)
    assert not ctx.fast_int8_enabled()
    ctx.set_fast_int8(True)
    try:
        assert ctx.fast_int8_enabled()
        got = run_matmul(ctx, qt, x)
        # matvec_rows takes the same path
        out = torch.full((o // 2 + 1,), float("nan"), device="cuda:0")
        qt.matvec_rows(o // 3, o // 2 + 1, dev(x[0]), out)
        rows = host(out)
    finally:
        ctx.set_fast_int8(False)
    want = O.matmul_fast_i8(q, s, o, i, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(rows.view(np.uint32), want[0, o // 3:o // 3 + o // 2 + 1].view(np.uint32))
    mag = np.maximum(np.abs(exact).max(axis=1, keepdims=True), 1e-3)
    assert (np.abs(got - exact) <= 0.03 * mag).all()
    assert np.array_equal(run_matmul(ctx, qt, x), exact)


def test_fast_int8_edges_and_other_formats(ctx):
    """Zero, NaN and infinite activation rows as the oracle has them; int4
    and f32 tensors keep the exact path while the switch is on."""
    rng = np.random.default_rng(44)
    o, i = 8, 64
    q = rng.integers(-127, 128, (o, i)).astype(np.int8).view(np.uint8)
    s = (rng.random(o) * 0.1 + 0.01).astype(np.float32)
    qt = upload(ctx, INT8, q, s, o, i)
    x = rng.standard_normal((4, i)).astype(np.float32)
    x[0] = 0.0
    x[1, 5] = np.nan
    x[2, 7] = np.inf
    p4, s4 = rand_qtensor(rng, INT4, o, i)
    qt4 = upload(ctx, INT4, p4, s4, o, i)
    exact4 = run_matmul(ctx, qt4, x[3:])
    ctx.set_fast_int8(True)
    try:
        got = run_matmul(ctx, qt, x)
        got4 = run_matmul(ctx, qt4, x[3:])
    finally:
        ctx.set_fast_int8(False)
    want = O.matmul_fast_i8(q, s, o, i, x)
    assert np.array_equal(got[0], np.zeros(o, np.float32))
    assert np.array_equal(got[[0, 1, 3]].view(np.uint32), want[[0, 1, 3]].view(np.uint32))
    assert np.isnan(got[2]).all() and np.isnan(want[2]).all()
    assert np.array_equal(got4, exact4)
