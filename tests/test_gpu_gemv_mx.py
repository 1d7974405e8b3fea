"""1-4-row products on the scaled matrix cores over operand-order weights
(gemv_mx.hip): Dense layers with at least 4081 output rows and 16-128 K
chunks of 128 (FP8: up to 64; four rows: up to 96), and the 1-4-row SwiGLU,
whose gate+up launch writes the three-term split of h that the down
projection reads.

Parity reference: the oracle's contract (dequantize, f64 serial sums, bias in
f64, activation; src/cuda/kernels.cu:130-161; SwiGLU swiglu.cpp:87-136,
kernels.cu:296-304). Tolerances:
  * rel-L2 <= 5e-5 per product, as on the batched matrix-core paths (three
    E4M3 terms of x per 16 elements, matrix-core accumulation);
  * bit-exact where x and the weights are small integers (every partial sum
    is exact in the matrix core and in f32);
  * non-finite inputs: the oracle's IEEE values (NaN where the oracle has
    NaN, the same infinities, finite values within the bound), because a
    wave whose inputs are not finite sums on the VALU.
"""
import numpy as np
import pytest

from test_gpu_dense import TOL_MFMA, rel_l2

pytestmark = pytest.mark.gpu


def dequant(oracle, dt, scheme, W):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    return oracle.dequant(dt, scheme, rows, cols, native, rs, blk)


def run_dense(gpu, dt, scheme, W, x, act=-1, bias=None):
    s = gpu.DenseSession(x.shape[0], W.shape[1], W.shape[0], act, dt, scheme, W, bias)
    try:
        return s.execute(x)
    finally:
        s.close()


def assert_ieee_match(got, want, tol):
    """Same NaN positions, same infinities, finite values within tol."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf)
    assert np.array_equal(got[inf], want[inf])
    fin = np.isfinite(want)
    if fin.any():
        assert rel_l2(got[fin], want[fin]) <= tol


@pytest.mark.parametrize("dt,scheme,rows,cols,act,with_bias", [
    (4, 2, 4096, 4096, -1, False),    # the headline GEMV: 32 chunks, 8 waves
    (5, 1, 4100, 3000, 1, True),      # ragged rows (257 row blocks) and K; bias + SiLU
    (16, 3, 4096, 11008, -1, False),  # SwiGLU down shape: 86 chunks, 16 waves of <= 8
    (16, 0, 4200, 2048, 0, False),    # 16 chunks (the fewest), ReLU
    (4, 3, 4096, 8192, -1, False),    # E4M3 with E8M0 blocks, 64 chunks
    (16, 3, 4096, 16384, -1, False),  # 128 chunks (the most)
    (16, 3, 4096, 13000, -1, False),  # 102 chunks: 16 waves of 6 or 7 in ranges of 8
    (5, 3, 4096, 5000, 2, True),      # E5M2 with E8M0 blocks, 40 chunks; bias + GELU
    (5, 2, 4096, 2050, 3, False),     # cols % 4 != 0: stays on the VALU GEMV (x read as vectors); tanh
])
def test_dense_batch1_matches_oracle(gpu, oracle, dt, scheme, rows, cols, act, with_bias):
    rng = np.random.default_rng(rows + cols + dt + scheme)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1 if with_bias else None
    pre, post = run_dense(gpu, dt, scheme, W, x, act, bias)
    o_pre, o_post = oracle.dense(dequant(oracle, dt, scheme, W), x, act, bias, threads=8)
    assert rel_l2(pre, o_pre) <= TOL_MFMA, rel_l2(pre, o_pre)
    assert rel_l2(post, o_post) <= TOL_MFMA


@pytest.mark.parametrize("dt,values,rows,cols", [
    (4, [-8, -6, -3, -1, 0, 1, 2, 5, 7, 8], 4096, 4096),
    (16, [-6, -4, -3, -1.5, -0.5, 0, 0.5, 1, 2, 6], 4100, 3000),
    (5, [-8, -4, -3, -1.5, 0, 1, 2, 3, 6, 8], 4096, 8192),
])
def test_dense_batch1_integer_exact(gpu, oracle, dt, values, rows, cols):
    rng = np.random.default_rng(dt + cols)
    W = rng.choice(np.array(values, np.float32), (rows, cols))
    x = rng.integers(-4, 5, (1, cols)).astype(np.float32)
    pre, post = run_dense(gpu, dt, 0, W, x)
    o_pre, _ = oracle.dense(dequant(oracle, dt, 0, W), x)
    assert np.array_equal(pre, o_pre)
    assert np.array_equal(post, o_pre)


@pytest.mark.parametrize("dt,scheme,cols", [(4, 2, 4096), (16, 3, 11008), (5, 3, 6000)])
def test_dense_batch1_nonfinite_x(gpu, oracle, dt, scheme, cols):
    """inf in one wave's K range, -inf in another's, NaN in a third call:
    those waves sum on the VALU, the others on the matrix cores."""
    rows = 4096
    rng = np.random.default_rng(cols + dt)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    Wd = dequant(oracle, dt, scheme, W)
    for marks in ([(7, np.inf)], [(cols // 3, np.inf), (cols - 5, -np.inf)], [(cols // 2, np.nan)]):
        x = rng.standard_normal((1, cols)).astype(np.float32)
        for k, v in marks:
            x[0, k] = v
        pre, _ = run_dense(gpu, dt, scheme, W, x)
        o_pre, _ = oracle.dense(Wd, x)
        assert_ieee_match(pre, o_pre, TOL_MFMA)


def oracle_swiglu(oracle, dt, scheme, G, U, D, x):
    g, _ = oracle.dense(dequant(oracle, dt, scheme, G), x, threads=8)
    u, _ = oracle.dense(dequant(oracle, dt, scheme, U), x, threads=8)
    h = oracle.swiglu_product(g, u)
    Dd = dequant(oracle, dt, scheme, D)
    y, _ = oracle.dense(Dd, h, threads=8)
    return h, y, Dd


@pytest.mark.parametrize("dt,scheme,d,inter", [
    (16, 3, 2048, 4100),  # gate+up on the matrix cores, down (2048 rows) on the VALU GEMV
    (4, 2, 4096, 4196),   # FP8 pair; the down reads the pair's split, last piece ragged
    (5, 1, 4096, 8192),   # E5M2 per-tensor, split read over 64 chunks
    (16, 0, 4096, 6000),  # FP4 without scales, 48 chunks
])
def test_swiglu_batch1_matrix_core(gpu, oracle, dt, scheme, d, inter):
    rng = np.random.default_rng(d + inter + dt)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    s = gpu.SwiGLUSession(1, 1, d, inter, dt, scheme, G, U, D)
    try:
        # two calls on one session: the split buffer is rewritten each time
        for rep in range(2):
            x = rng.standard_normal((1, d)).astype(np.float32)
            h, y = s.execute(x)
            oh, oy, Dd = oracle_swiglu(oracle, dt, scheme, G, U, D, x)
            assert rel_l2(h, oh) <= TOL_MFMA, (rep, rel_l2(h, oh))
            oy_own, _ = oracle.dense(Dd, h, threads=8)
            assert rel_l2(y, oy_own) <= TOL_MFMA, (rep, rel_l2(y, oy_own))
            assert rel_l2(y, oy) <= 2 * TOL_MFMA
    finally:
        s.close()


def test_swiglu_batch1_nonfinite_x(gpu, oracle):
    """inf in x: the gate+up waves that see it sum on the VALU, the pieces of
    h that are not finite carry the non-finite mark, and the down waves that
    read them sum on the VALU over h."""
    d, inter = 4096, 4196
    rng = np.random.default_rng(11)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((1, d)).astype(np.float32)
    x[0, 1000] = np.inf
    s = gpu.SwiGLUSession(1, 1, d, inter, 4, 2, G, U, D)
    try:
        h, y = s.execute(x)
    finally:
        s.close()
    oh, _, Dd = oracle_swiglu(oracle, 4, 2, G, U, D, x)
    assert_ieee_match(h, oh, TOL_MFMA)
    oy_own, _ = oracle.dense(Dd, h)
    assert_ieee_match(y, oy_own, TOL_MFMA)


# 2-4 batch rows: six A rows per batch row (two halves x three terms), one
# MFMA per weight fragment for 2 rows, two for 3-4
@pytest.mark.parametrize("batch", [2, 3, 4])
@pytest.mark.parametrize("dt,scheme,rows,cols,act,with_bias", [
    (4, 2, 4096, 4096, -1, False),    # 32 chunks, 8 waves of 4
    (5, 1, 4100, 3000, 1, True),      # ragged rows and K; bias + SiLU
    (16, 3, 4096, 11008, -1, False),  # SwiGLU down shape: 16 waves of <= 6
    (4, 3, 4096, 8192, -1, False),    # E4M3 with E8M0 blocks, 16 waves of 4
    (16, 3, 4096, 16384, 0, False),   # 128 chunks: 16 waves of 8 (4 rows: stays on the VALU kernel); ReLU
])
def test_dense_rows_matches_oracle(gpu, oracle, batch, dt, scheme, rows, cols, act, with_bias):
    rng = np.random.default_rng(rows + cols + dt + scheme + batch)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    x[-1] *= 1e3  # batch rows of different magnitudes
    bias = rng.standard_normal(rows) * 0.1 if with_bias else None
    pre, post = run_dense(gpu, dt, scheme, W, x, act, bias)
    o_pre, o_post = oracle.dense(dequant(oracle, dt, scheme, W), x, act, bias, threads=8)
    for b in range(batch):
        assert rel_l2(pre[b], o_pre[b]) <= TOL_MFMA, (b, rel_l2(pre[b], o_pre[b]))
        assert rel_l2(post[b], o_post[b]) <= TOL_MFMA, b


@pytest.mark.parametrize("batch", [2, 3, 4])
def test_dense_rows_integer_exact(gpu, oracle, batch):
    rng = np.random.default_rng(batch)
    rows, cols = 4100, 3000
    W = rng.choice(np.array([-6, -4, -3, -1.5, -0.5, 0, 0.5, 1, 2, 6], np.float32), (rows, cols))
    x = rng.integers(-4, 5, (batch, cols)).astype(np.float32)
    pre, _ = run_dense(gpu, 16, 0, W, x)
    o_pre, _ = oracle.dense(dequant(oracle, 16, 0, W), x)
    assert np.array_equal(pre, o_pre)


@pytest.mark.parametrize("batch", [2, 4])
def test_dense_rows_nonfinite_x(gpu, oracle, batch):
    """inf in one batch row only: the waves whose K range holds it sum all
    batch rows on the VALU, the other batch rows keep finite results."""
    rows, cols = 4096, 4096
    rng = np.random.default_rng(batch + 100)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    Wd = dequant(oracle, 4, 2, W)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    x[1, 700] = np.inf
    x[batch - 1, 3000] = np.nan
    pre, _ = run_dense(gpu, 4, 2, W, x)
    o_pre, _ = oracle.dense(Wd, x)
    for b in range(batch):
        assert_ieee_match(pre[b], o_pre[b], TOL_MFMA)


@pytest.mark.parametrize("rows", [2, 3, 4])
@pytest.mark.parametrize("dt,scheme,d,inter", [
    (16, 3, 4096, 11008),  # the C3 shapes: the down reads the pair's split over 86 chunks
    (4, 2, 4096, 4196),    # FP8 pair; last piece ragged
])
def test_swiglu_rows_matrix_core(gpu, oracle, rows, dt, scheme, d, inter):
    rng = np.random.default_rng(d + inter + dt + rows)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    s = gpu.SwiGLUSession(rows, 1, d, inter, dt, scheme, G, U, D)
    try:
        for rep in range(2):
            x = rng.standard_normal((rows, d)).astype(np.float32)
            x[0] *= 1e-3
            h, y = s.execute(x)
            oh, oy, Dd = oracle_swiglu(oracle, dt, scheme, G, U, D, x)
            oy_own, _ = oracle.dense(Dd, h, threads=8)
            for b in range(rows):
                assert rel_l2(h[b], oh[b]) <= TOL_MFMA, (rep, b, rel_l2(h[b], oh[b]))
                assert rel_l2(y[b], oy_own[b]) <= TOL_MFMA, (rep, b, rel_l2(y[b], oy_own[b]))
                assert rel_l2(y[b], oy[b]) <= 2 * TOL_MFMA
    finally:
        s.close()


def test_swiglu_rows_nonfinite_x(gpu, oracle):
    """inf in the second of three batch rows: its pieces of h carry the
    non-finite mark, the other rows' pieces are split as usual."""
    d, inter, rows = 4096, 4196, 3
    rng = np.random.default_rng(12)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    x[1, 1000] = np.inf
    s = gpu.SwiGLUSession(rows, 1, d, inter, 4, 2, G, U, D)
    try:
        h, y = s.execute(x)
    finally:
        s.close()
    oh, _, Dd = oracle_swiglu(oracle, 4, 2, G, U, D, x)
    oy_own, _ = oracle.dense(Dd, h)
    for b in range(rows):
        assert_ieee_match(h[b], oh[b], TOL_MFMA)
        assert_ieee_match(y[b], oy_own[b], TOL_MFMA)


def _sweep_cases():
    """Seeded shapes across the launch shapes' boundaries (16/32/33/64/65/96/97/128
    chunks of 128), every dtype and scale scheme, 1-4 batch rows."""
    rng = np.random.default_rng(20261202)
    cases = []
    chunks = [16, 32, 33, 64, 65, 96, 97, 128]
    for i, s in enumerate(chunks):
        dt = [4, 5, 16][i % 3]
        scheme = int(rng.integers(0, 4))
        cols = 128 * (s - 1) + 4 * int(rng.integers(1, 32))  # s chunks, the last ragged
        rows = int(rng.integers(4081, 4700))
        batch = 1 + i % 4
        cases.append((dt, scheme, rows, cols, batch))
    return cases


@pytest.mark.parametrize("dt,scheme,rows,cols,batch", _sweep_cases())
def test_dense_rows_shape_sweep(gpu, oracle, dt, scheme, rows, cols, batch):
    rng = np.random.default_rng(rows * 7 + cols)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    pre, _ = run_dense(gpu, dt, scheme, W, x)
    o_pre, _ = oracle.dense(dequant(oracle, dt, scheme, W), x, threads=8)
    for b in range(batch):
        assert rel_l2(pre[b], o_pre[b]) <= TOL_MFMA, (b, rel_l2(pre[b], o_pre[b]))
