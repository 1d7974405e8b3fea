"""FP6 (E2M3) activation terms: every three-term split (the default), on the
large tiles (above 32 rows: Dense, SwiGLU and MHA projections) and in the
prologue of the 5-32-row kernel.

Each 32-element block of x is split into three E2M3 terms: per term, the
block exponent e is the smallest with amax <= 7.5 * 2^e (at least -126), the
term is RNE_E2M3(v / 2^e) * 2^e, and v keeps the residual. The f8f6f4 matrix
cores multiply the stored FP8/FP4 weight codes by the three terms; FP4
weights times FP6 terms run at the FP4/FP6 rate. Two-term and one-term
splits keep E4M3 terms.

Pinned by a numpy model of the three-term product (the block rule restated,
E2M3 rounding to nearest-even on the grid 0.125 * {0..15}, 0.25 * {8..15},
0.5 * {8..15}, f64 products) at the matrix cores' accumulation floor: a
dropped or repeated term, a wrong block exponent or a misplaced element moves
the result by at least the size of the third term (~1e-3 relative), far
above that floor. The layer result is also checked against the exact oracle
product at the matrix-core tolerance.
"""
import numpy as np
import pytest

from test_gpu_dense import rel_l2, TOL_MFMA

pytestmark = pytest.mark.gpu

FLOOR = 5e-5  # matrix-core accumulation floor


def e2m3_rne(u):
    """Nearest E2M3 value (ties to the even code), saturating at +-7.5."""
    a = np.minimum(np.abs(u), 7.5)
    step = np.where(a < 2.0, 0.125, np.where(a < 4.0, 0.25, 0.5))
    q = np.round(a / step) * step
    # rounding up across a binade edge stays on the grid (2.0, 4.0, 8.0 -> 7.5)
    return np.sign(u) * np.minimum(q, 7.5)


def block_exp(amax):
    """Smallest e with amax <= 7.5 * 2^e, clamped to [-126, 127]; 0 for 0."""
    m, ex = np.frexp(amax.astype(np.float64))
    a = 2.0 * m
    e = (ex - 1) - 2 + (a > 1.875)
    e = np.clip(e, -126, 127)
    return np.where(amax > 0, e, 0)


def fp6_terms(x, terms=3):
    """The sum of the FP6 terms of x [rows][K] (f64), blocks of 32 along K."""
    rows, K = x.shape
    kp = (K + 31) // 32 * 32
    v = np.zeros((rows, kp // 32, 32), np.float64)
    v.reshape(rows, kp)[:, :K] = x
    out = np.zeros_like(v)
    for _ in range(terms):
        e = block_exp(np.abs(v).max(axis=2))[:, :, None]
        sc = np.ldexp(1.0, e)
        t = e2m3_rne(v / sc) * sc
        out += t
        v = v - t
    return out.reshape(rows, kp)[:, :K]


def dequant(oracle, dt, scheme, W):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    return oracle.dequant(dt, scheme, rows, cols, native, rs, blk).astype(np.float64)


def test_fp6_model_known_values():
    # the E2M3 grid itself, and its ties
    grid = np.array([0.125 * i for i in range(16)] + [2 + 0.25 * i for i in range(8)]
                    + [4 + 0.5 * i for i in range(8)])
    assert np.array_equal(e2m3_rne(grid), grid)
    assert np.array_equal(e2m3_rne(-grid), -grid)
    assert e2m3_rne(np.array([0.0625]))[0] == 0.0     # tie -> code 0
    assert e2m3_rne(np.array([0.1875]))[0] == 0.25    # tie -> code 2
    assert e2m3_rne(np.array([2.125]))[0] == 2.0      # tie -> code 16
    assert e2m3_rne(np.array([2.375]))[0] == 2.5      # tie -> code 18
    assert e2m3_rne(np.array([7.75, 100.0]))[1] == 7.5
    # block exponents: 7.5 fits e = 0, 7.6 needs e = 1, 3.75 fits e = -1
    assert list(block_exp(np.array([7.5, 7.6, 3.75, 3.76, 0.0]))) == [0, 1, -1, 0, 0]
    # a block of grid values is one exact term; the residual terms are zero
    x = grid[None, :]
    assert np.array_equal(fp6_terms(x, 1), x)
    # three terms leave a small residual on random data
    r = np.random.default_rng(1).standard_normal((64, 1024))
    err = np.linalg.norm(fp6_terms(r) - r) / np.linalg.norm(r)
    assert 1e-7 < err < 1e-4, err


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3), (5, 1)])
@pytest.mark.parametrize("rows,K,N", [(4096, 1024, 1024), (64, 1024, 1024), (300, 700, 513),
                                      (1024, 4096, 1024), (2048, 256, 4096), (16, 4096, 2048),
                                      (5, 700, 513), (32, 11008, 512)])
def test_three_term_dense_matches_fp6_model(gpu, oracle, dt, scheme, rows, K, N):
    rng = np.random.default_rng(rows * 3 + K + N + dt)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    s = gpu.DenseSession(rows, K, N, -1, dt, scheme, W)
    y, _ = s.execute(x)
    s.close()
    Wd = dequant(oracle, dt, scheme, W)
    x64 = x.astype(np.float64)
    model = fp6_terms(x64) @ Wd.T
    exact = x64 @ Wd.T
    e_model, e_exact = rel_l2(y, model), rel_l2(y, exact)
    # the same product with the third term left out: what a dropped term costs
    two = rel_l2(fp6_terms(x64, 2) @ Wd.T, model)
    print(f"FP6 three terms: rel-L2 {e_exact:.2e} against the exact Dense, {e_model:.1e} against "
          f"the model (the third term alone {two:.1e}; {rows}x{K}x{N} dtype {dt})")
    assert e_model <= FLOOR
    assert two > 10 * FLOOR
    assert e_exact <= TOL_MFMA
