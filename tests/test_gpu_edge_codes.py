"""Stored payloads holding every code byte, through every product path.

A WMN1 model (one Dense child, scheme 0) is mounted from a FormatNone
payload written byte by byte, so the codes the encoder never produces reach
the kernels: E4M3 0x78-0x7F / 0xF8-0xFF (0x7F decodes to 448,
float_codecs.cpp:112-113) and the exponent-0 codes that decode to signed
zero (:110); E5M2 0x7C-0x7F / 0xFC-0xFF, which decode to +-inf and NaN
(:171-181); all 16 FP4 nibbles (:184-200). The oracle dequantizes the same
bytes with the reference's weight_at (native_codec.cpp:534-549) and runs the
f64 Dense contract (kernels.cu:130-161).

Batch 1 runs the VALU GEMV, 3 the small-batch matrix-core GEMV, 16 the
5..32-row GEMM and 64 the large-tile GEMM. Rows holding inf / NaN codes: the
output is non-finite and equal to the oracle's as IEEE values (same
infinity, or NaN for NaN). Finite outputs: rel-L2 <= 1e-5 on the VALU GEMV
(exact decode, fp32 accumulation) and <= 2e-4 on the matrix-core paths.
Uniformly random code bytes give log-uniform weight magnitudes (E4M3 2^-6 to
448, E5M2 2^-14 to 57344), so each output is dominated by a few products and
the activation-split and accumulation errors (~1.5e-5 and ~1.1e-5 relative
per product) do not average down over K as they do for Gaussian weights
(5e-5 there); measured 5.8e-5 for E4M3 at 16 rows. The contract bound is
1e-3.
"""
import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import rel_l2

pytestmark = pytest.mark.gpu

E5M2_SPECIAL = [0x7C, 0x7D, 0x7E, 0x7F, 0xFC, 0xFD, 0xFE, 0xFF]


def one_dense_model(dt, rows, cols, native, act=-1, bias=None):
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(0, 1, 1, 1, 1, 1)
    w.i32(19, 1)
    pw.dense_child(w, cols, rows, act, dt, np.zeros((rows, cols), np.float32), bias)
    pw.empty_controls(w)
    pw.empty_controls(w)
    pw.empty_controls(w)
    w.i32(1)
    pw.store_payload(w, dt, rows, cols, native, bias=bias)
    return w.bytes()


def payload(dt, rows, cols, rng):
    """Bytes covering every code of the format; for E5M2 the non-finite codes
    sit only in rows 3, 7, 11, 19 and 30 (one row each pattern)."""
    n = rows * cols
    if dt == 16:
        nib = rng.integers(0, 16, n).astype(np.uint8)
        nib[:16] = np.arange(16)
        if n % 2:
            nib = np.append(nib, 0)
        return (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    if dt == 4:
        b = rng.integers(0, 256, n).astype(np.uint8)
        b[:256] = np.arange(256)
        return b
    finite = np.array([c for c in range(256) if c not in E5M2_SPECIAL], np.uint8)
    b = finite[rng.integers(0, finite.size, n)]
    b[:finite.size] = finite
    M = b.reshape(rows, cols)
    M[3, 5] = 0x7C                   # one +inf: sign of x[5]
    M[7, 9] = 0x7E                   # NaN
    M[11, 2], M[11, 40] = 0x7C, 0xFC  # +inf and -inf
    M[19, [0, 8, 70]] = 0xFC         # several -inf
    M[30, 1], M[30, 77] = 0xFF, 0x7D  # NaN codes of both signs
    return M.ravel()


def tol_codes(batch):
    return 1e-5 if batch == 1 else 2e-4


def check(got, want, batch):
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf])
    assert np.all(np.isfinite(got[fin]))
    assert rel_l2(got[fin], want[fin]) <= tol_codes(batch)


@pytest.mark.parametrize("batch", [1, 3, 16, 64])
@pytest.mark.parametrize("dt", [4, 5, 16])
def test_stored_codes_every_byte(gpu, oracle, dt, batch):
    rows, cols = 40, 300
    rng = np.random.default_rng(1000 * dt + batch)
    native = payload(dt, rows, cols, rng)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    if dt == 5:
        x[:, 5] = np.where(np.arange(batch) % 2 == 0, 1.5, -0.75)  # both signs of +inf
        x[:, 2] = 1.0
        x[:, 40] = 1.0  # +inf - inf -> NaN
    m = pw.ModelSession(one_dense_model(dt, rows, cols, native))
    y = m.forward(x)
    m.close()
    ones = np.ones(rows, np.float32)
    Wd = oracle.dequant(dt, 0, rows, cols, native, ones, np.zeros(1, np.uint8))
    with np.errstate(invalid="ignore", over="ignore"):
        _, want = oracle.dense(Wd, x)
    if dt == 5:
        assert not np.isfinite(want[:, [3, 7, 11, 19, 30]]).any()
        assert np.isfinite(np.delete(want, [3, 7, 11, 19, 30], axis=1)).all()
    check(y, want, batch)


@pytest.mark.parametrize("batch", [3, 16, 64])
def test_stored_e5m2_nonfinite_rows_epilogue(gpu, oracle, batch):
    """Rows with inf / NaN codes through the bias + activation epilogue
    (ReLU: -inf -> 0, +inf stays, NaN stays)."""
    rows, cols = 40, 300
    rng = np.random.default_rng(50 + batch)
    native = payload(5, rows, cols, rng)
    bias = rng.standard_normal(rows)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    m = pw.ModelSession(one_dense_model(5, rows, cols, native, act=0, bias=bias))
    y = m.forward(x)
    m.close()
    Wd = oracle.dequant(5, 0, rows, cols, native, np.ones(rows, np.float32), np.zeros(1, np.uint8))
    with np.errstate(invalid="ignore", over="ignore"):
        _, want = oracle.dense(Wd, x, 0, bias)
    check(y, want, batch)


def test_e5m2_overflow_from_fp32_weights(gpu, oracle):
    """Scheme 0 encodes |w| above the E5M2 range to inf (float_codecs.cpp:
    119-158): the mounted codes hold inf and the matrix-core paths must keep
    it (not turn inf * 0 terms into NaN)."""
    rng = np.random.default_rng(9)
    W = rng.standard_normal((64, 256)).astype(np.float32)
    W[5, 17] = 1e6
    W[9, 3] = -7e4
    for batch in (1, 4, 20, 48):
        x = rng.standard_normal((batch, 256)).astype(np.float32)
        s = gpu.DenseSession(batch, 256, 64, -1, 5, 0, W)
        pre, _ = s.execute(x)
        s.close()
        native, rs, blk = oracle.quantize(5, 0, 64, 256, W)
        Wd = oracle.dequant(5, 0, 64, 256, native, rs, blk)
        with np.errstate(invalid="ignore", over="ignore"):
            want, _ = oracle.dense(Wd, x)
        assert np.isinf(want[:, 5]).all() and np.isinf(want[:, 9]).all()
        check(pre, want, batch)
