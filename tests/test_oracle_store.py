"""FormatNone payload layout and the scale extension of the oracle.

Payloads are pinned by WeightStore::make / export_f32 of the compiled
reference (tests/golden/store_cases.npz): FP8 one byte per element; FP4 two
codes per byte over the flattened matrix, even index in the low nibble, so
rows of odd width straddle bytes (native_codec.cpp:193-211, :534-549).
The scale schemes are not in the reference; they are pinned by what the
mathematics fixes: E8M0 scales are the least power of two that brings the
block maximum within maxrep, dequantization by a power of two is exact, and
scaled codes never saturate.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def store_cases():
    z = np.load(os.path.join(GOLD, "store_cases.npz"))
    for i in range(int(z["count"][0])):
        dt, rows, cols = z[f"c{i}_meta"].tolist()
        yield (dt, rows, cols, z[f"c{i}_W"], z[f"c{i}_native"], float(z[f"c{i}_scale"][0]),
               z[f"c{i}_export"])


def test_pack_matches_reference_store(oracle):
    n = 0
    for dt, rows, cols, W, native, scale, exp in store_cases():
        assert np.array_equal(oracle.pack(dt, W), native), (dt, rows, cols)
        assert scale == 1.0  # FP types carry no scale in the reference
        got = np.array([oracle.weight_at(dt, native, i) for i in range(rows * cols)], np.float32)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (dt, rows, cols)
        n += 1
    assert n == 18


def test_fp4_nibble_order_straddles_rows(oracle):
    W = np.array([[0.5, 1.0, 1.5], [2.0, 3.0, 4.0]], np.float32)  # codes 1 2 3 / 4 5 6
    assert oracle.pack(16, W).tolist() == [0x21, 0x43, 0x65]


@pytest.mark.parametrize("dt,maxrep", [(4, 240.0), (5, 57344.0), (16, 6.0)])
def test_e8m0_exponent_is_least_power_of_two(oracle, dt, maxrep):
    assert oracle.L.or_e8m0_exponent(0.0, maxrep) == 0
    for e in range(-120, 100, 7):
        a = np.float32(np.ldexp(np.float32(maxrep), e))
        if not np.isfinite(a):
            continue
        assert oracle.L.or_e8m0_exponent(float(a), maxrep) == e
        up = np.nextafter(a, np.float32(np.inf))
        assert oracle.L.or_e8m0_exponent(float(up), maxrep) == e + 1
        dn = np.nextafter(a, np.float32(0))
        assert oracle.L.or_e8m0_exponent(float(dn), maxrep) == e
    assert oracle.L.or_e8m0_exponent(1e-45, maxrep) == -127


@pytest.mark.parametrize("dt", [4, 5, 16])
@pytest.mark.parametrize("scheme", [0, 1, 2, 3])
def test_quantize_dequant_properties(oracle, dt, scheme):
    rng = np.random.default_rng(dt * 10 + scheme)
    rows, cols = 9, 70
    W = (rng.standard_normal((rows, cols)) * np.exp(rng.uniform(-3, 3, (rows, 1)))).astype(np.float32)
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    Wd = oracle.dequant(dt, scheme, rows, cols, native, rs, blk)
    maxrep = oracle.L.or_maxrep(dt)
    codes = np.array([oracle.weight_at(dt, native, i) for i in range(rows * cols)],
                     np.float32).reshape(rows, cols)
    if scheme == 0:
        assert np.all(rs == 1) and np.array_equal(Wd, codes)
    if scheme == 1:
        s = np.float32(np.abs(W).max()) / np.float32(maxrep)
        assert np.all(rs == s)
    if scheme == 2:
        s = (np.abs(W).max(axis=1).astype(np.float32) / np.float32(maxrep)).astype(np.float32)
        assert np.array_equal(rs, s)
    if scheme in (1, 2):
        assert np.abs(codes).max() <= maxrep  # never saturates
        assert np.array_equal(Wd, (codes * rs[:, None]).astype(np.float32))
    if scheme == 3:
        e = blk.reshape(rows, -1).astype(np.int32) - 127
        for r in range(rows):
            for b in range(e.shape[1]):
                seg = W[r, 32 * b:32 * b + 32]
                a = np.abs(seg).max()
                assert a <= np.ldexp(maxrep, e[r, b]) and a > np.ldexp(maxrep, e[r, b] - 1)
        scale = np.ldexp(1.0, np.repeat(e, 32, axis=1)[:, :cols]).astype(np.float32)
        assert np.array_equal(Wd, codes * scale)  # power-of-two dequant is exact
        assert np.abs(codes).max() <= maxrep
    if scheme != 0:
        # the scaled grid resolves each scale group: the error is at most half
        # the top code step relative to the group maximum, which the scale maps
        # into (maxrep/2, maxrep]: E4M3 8/120, E5M2 4096/28672, FP4 1/3
        bound = {4: 1.0 / 15.0, 5: 1.0 / 7.0, 16: 1.0 / 3.0}[dt]
        err = np.abs(Wd - W)
        if scheme == 1:
            assert err.max() <= bound * np.abs(W).max() * 1.0001
        elif scheme == 2:
            assert np.all(err.max(axis=1) <= bound * np.abs(W).max(axis=1) * 1.0001)
        else:
            for b in range(0, cols, 32):
                g = np.abs(W[:, b:b + 32]).max(axis=1)
                assert np.all(err[:, b:b + 32].max(axis=1) <= bound * g * 1.0001)


def test_quantize_tiny_negative_keeps_sign(oracle):
    # 1e-40 / (1/240) stays a subnormal f32: E4M3 keeps the sign (0x80)
    W = np.array([[1.0, -1e-40, 1e-40, -0.0]], np.float32)
    native, rs, blk = oracle.quantize(4, 2, 1, 4, W)
    assert native.tolist() == [0x77, 0x80, 0x00, 0x00]
