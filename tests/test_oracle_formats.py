"""The oracle's packed block formats (oracle/formats.c), pinned without the
library: IEEE half conversions against numpy, closed-form blocks whose codes,
scales and dequantized values are known exactly, the packing positions of
single codes, and the quantizers' error bounds.

The reference reserves these formats (include/welvet/weights.hpp:12-15,
README.md:361-383) but implements none; the rules are ggml's published block
formats. No ggml output is in the image, so parity against ggml itself is
unpinned: what is pinned is that the oracle implements the layouts stated in
its header."""
import numpy as np
import pytest

from format_blocks import GEOM, IQ, IQ4_NL, IQ4_XS, IQ4NL_TABLE, KQUANT, LEGACY, Q2_K, Q3_K, Q4_0, \
    Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, random_blocks
from oracle_lib import Oracle


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def test_half_to_float_every_pattern(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_rne(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=60000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the half range, its subnormals, overflow and exact ties
    e = rng.integers(100, 145, size=bits.size).astype(np.uint32)
    bits = (bits & 0x807FFFFF) | (e << 23)
    ties = []
    for hb in (0x0001, 0x0002, 0x03FF, 0x0400, 0x3C00, 0x3C01, 0x7BFE, 0x7BFF):
        lo = np.array([hb], np.uint16).view(np.float16).astype(np.float32)[0]
        hi = np.array([hb + 1], np.uint16).view(np.float16).astype(np.float32)[0]
        ties += [(np.float64(lo) + np.float64(hi)) / 2]
    x = np.concatenate([bits.view(np.float32), np.array(ties, np.float32),
                        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2**-25, 2**-26,
                                  3 * 2**-26, np.inf, -np.inf], np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    got = orc.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_q8_0_closed_form(orc):
    x = np.arange(-127, 129, dtype=np.float32)[:256].copy()
    x[x > 127] = 5.0
    x.reshape(8, 32)[:, 0] = -127.0  # amax 127 in every block -> d = 1
    b = orc.fmt_quantize(Q8_0, x).reshape(8, 34)
    assert np.all(b[:, :2].copy().view(np.float16).astype(np.float32) == 1.0)
    assert np.array_equal(b[:, 2:].view(np.int8).ravel().astype(np.float32), x)
    assert np.array_equal(orc.fmt_dequant(Q8_0, b, x.shape), x)


def _levels_block(offset, levels, step, rng):
    """32 values offset + k * step with k covering 0 and levels - 1."""
    k = rng.integers(0, levels, 32)
    k[rng.integers(0, 32)] = 0
    k[rng.integers(0, 32)] = levels - 1
    return k, (offset + k * step).astype(np.float32)


@pytest.mark.parametrize("fmt,levels", [(Q4_0, 16), (Q5_0, 32)])
def test_symmetric_formats_closed_form(orc, fmt, levels):
    """max = -levels/2 * d is the signed extreme, so d = 0.25 exactly and every
    value is on the grid: q = k, dequant = x exactly. Element j sits in the low
    nibble of qs[j], j + 16 in the high one; bit 4 in bit j of qh."""
    rng = np.random.default_rng(levels)
    half = levels // 2
    for _ in range(20):
        k, x = _levels_block(-half * 0.25, levels, 0.25, rng)
        k[0], x[0] = 0, -half * 0.25  # the first extreme is the negative one
        b = orc.fmt_quantize(fmt, x)
        assert b[:2].view(np.float16)[0] == 0.25
        qs = b[-16:]
        assert np.array_equal(qs & 15, k[:16] & 15) and np.array_equal(qs >> 4, k[16:] & 15)
        if fmt == Q5_0:
            qh = int(b[2:6].view(np.uint32)[0])
            assert all(((qh >> j) & 1) == (k[j] >> 4) for j in range(32))
        assert np.array_equal(orc.fmt_dequant(fmt, b, x.shape), x)


@pytest.mark.parametrize("fmt,levels", [(Q4_1, 16), (Q5_1, 32)])
def test_affine_formats_closed_form(orc, fmt, levels):
    """min = -1, d = 1/8 exactly: q = k, m = -1, dequant = x exactly."""
    rng = np.random.default_rng(100 + levels)
    for _ in range(20):
        k, x = _levels_block(-1.0, levels, 0.125, rng)
        b = orc.fmt_quantize(fmt, x)
        d, m = b[:4].view(np.float16).astype(np.float32)
        assert d == 0.125 and m == -1.0
        qs = b[-16:]
        assert np.array_equal(qs & 15, k[:16] & 15) and np.array_equal(qs >> 4, k[16:] & 15)
        if fmt == Q5_1:
            qh = int(b[4:8].view(np.uint32)[0])
            assert all(((qh >> j) & 1) == (k[j] >> 4) for j in range(32))
        assert np.array_equal(orc.fmt_dequant(fmt, b, x.shape), x)


@pytest.mark.parametrize("fmt", LEGACY)
def test_quantizer_error_bound(orc, fmt):
    """Random rows: each element is within one grid step (half a step where no
    clipping applies) plus the fp16 rounding of the scale and the minimum."""
    rng = np.random.default_rng(fmt)
    x = (rng.standard_normal((64, 256)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    b = orc.fmt_quantize(fmt, x)
    y = orc.fmt_dequant(fmt, b, x.shape).astype(np.float64)
    bb = GEOM[fmt][1]
    blocks = b.reshape(-1, bb)
    xb = x.reshape(-1, 32).astype(np.float64)
    yb = y.reshape(-1, 32)
    amax = np.abs(xb).max(1)
    lo, hi = xb.min(1), xb.max(1)
    d16 = blocks[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    if fmt == Q8_0:
        d = amax / 127
        bound = 0.5 * d + 127 * np.abs(d - d16)
    elif fmt in (Q4_0, Q5_0):
        n = 8 if fmt == Q4_0 else 16
        d = amax / n
        bound = d + n * np.abs(d - np.abs(d16))
    else:
        n = 15 if fmt == Q4_1 else 31
        d = (hi - lo) / n
        m16 = blocks[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
        bound = 0.5 * d + n * np.abs(d - d16) + np.abs(lo - m16)
    err = np.abs(xb - yb).max(1)
    assert np.all(err <= bound * (1 + 1e-5) + 1e-6 * amax)


def _pack_scale_min_k4(sc, m):
    """The 12 scale bytes of a Q4_K/Q5_K super-block holding 6-bit sc[j], m[j]
    (j < 4 in the low 6 bits of bytes j and j + 4; j >= 4 split into a low
    nibble in byte j + 4 and the top two bits of bytes j - 4 and j)."""
    q = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            q[j] |= sc[j] & 63
            q[j + 4] |= m[j] & 63
        else:
            q[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            q[j - 4] |= (sc[j] >> 4) << 6
            q[j] |= (m[j] >> 4) << 6
    return q


@pytest.mark.parametrize("fmt", [Q4_K, Q5_K])
def test_k4_scales_and_positions(orc, fmt):
    """d = 1, dmin = 1, sub-block scales sc[j] and mins m[j] chosen: element
    (sub-block 2i + h, l) = sc * (nibble h of qs[32 i + l] + 16 * bit (2i + h)
    of qh[l]) - m."""
    rng = np.random.default_rng(fmt)
    for _ in range(10):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        blk = np.zeros(GEOM[fmt][1], np.uint8)
        blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
        blk[2:4] = np.array([1.0], np.float16).view(np.uint8)
        blk[4:16] = _pack_scale_min_k4(sc, m)
        qs_off = 48 if fmt == Q5_K else 16
        qs = rng.integers(0, 256, 128, dtype=np.uint8)
        blk[qs_off:qs_off + 128] = qs
        qh = rng.integers(0, 256, 32, dtype=np.uint8) if fmt == Q5_K else np.zeros(32, np.uint8)
        if fmt == Q5_K:
            blk[16:48] = qh
        want = np.zeros(256)
        for s in range(8):
            i, h = divmod(s, 2)
            for l in range(32):
                code = (int(qs[32 * i + l]) >> (4 * h)) & 15
                code += 16 * ((int(qh[l]) >> s) & 1)
                want[32 * s + l] = sc[s] * code - m[s]
        got = orc.fmt_dequant(fmt, blk, (256,))
        assert np.array_equal(got, want.astype(np.float32))


def test_q6_k_scales_and_positions(orc):
    """d = 0.5, int8 scales sc[16]: element 128 n + 32 t + l = d * sc[8 n + 2 t
    + l // 16] * (q - 32), q = nibble (t >> 1) of ql[64 n + 32 (t & 1) + l]
    plus 16 * bits 2t..2t+1 of qh[32 n + l]."""
    rng = np.random.default_rng(6)
    for _ in range(10):
        blk = rng.integers(0, 256, 210, dtype=np.uint8)
        sc = rng.integers(-128, 128, 16).astype(np.int8)
        blk[192:208] = sc.view(np.uint8)
        blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
        ql, qh = blk[:128], blk[128:192]
        want = np.zeros(256)
        for n in range(2):
            for t in range(4):
                for l in range(32):
                    lo = (int(ql[64 * n + 32 * (t & 1) + l]) >> (4 * (t >> 1))) & 15
                    hi = (int(qh[32 * n + l]) >> (2 * t)) & 3
                    want[128 * n + 32 * t + l] = 0.5 * sc[8 * n + 2 * t + l // 16] * ((lo | hi << 4) - 32)
        got = orc.fmt_dequant(Q6_K, blk, (256,))
        assert np.array_equal(got, want.astype(np.float32))


def test_q2_k_scales_and_positions(orc):
    """d = 0.5, dmin = 0.25, scale bytes sc[16] (scale in the low nibble, min
    in the high one): element 128 n + 32 j + l = (d * (sc & 15)) * q -
    (dmin * (sc >> 4)), q = bits 2j, 2j+1 of qs[32 n + l], sc = sc[8 n + 2 j +
    l // 16]."""
    rng = np.random.default_rng(2)
    for _ in range(10):
        blk = np.zeros(84, np.uint8)
        sc = rng.integers(0, 256, 16, dtype=np.uint8)
        qs = rng.integers(0, 256, 64, dtype=np.uint8)
        blk[:16], blk[16:80] = sc, qs
        blk[80:82] = np.array([0.5], np.float16).view(np.uint8)
        blk[82:84] = np.array([0.25], np.float16).view(np.uint8)
        want = np.zeros(256)
        for n in range(2):
            for j in range(4):
                for l in range(32):
                    s_ = int(sc[8 * n + 2 * j + l // 16])
                    q = (int(qs[32 * n + l]) >> (2 * j)) & 3
                    want[128 * n + 32 * j + l] = 0.5 * (s_ & 15) * q - 0.25 * (s_ >> 4)
        assert np.array_equal(orc.fmt_dequant(Q2_K, blk, (256,)), want.astype(np.float32))


def _pack_q3k_scales(sc):
    """The 12 scale bytes of a Q3_K super-block holding 6-bit sc[0..15]
    (stored as scale + 32): scale 4g + i keeps its low nibble in the low (g =
    0, 1) or high (g = 2, 3) half of byte i (g even) or 4 + i (g odd), and its
    top two bits in bits 2g, 2g + 1 of byte 8 + i."""
    q = np.zeros(12, np.uint8)
    for s_ in range(16):
        g, i = divmod(s_, 4)
        v = int(sc[s_])
        q[(g & 1) * 4 + i] |= (v & 15) << (4 * (g >> 1))
        q[8 + i] |= (v >> 4) << (2 * g)
    return q


def test_q3_k_scales_and_positions(orc):
    """d = 0.25, scales (6-bit, minus 32) chosen: element 128 n + 32 j + l =
    (d * (sc - 32)) * (q - 4 unless bit 4n + j of hmask[l] is set), q = bits
    2j, 2j+1 of qs[32 n + l], scale 8 n + 2 j + l // 16."""
    rng = np.random.default_rng(3)
    for _ in range(10):
        sc = rng.integers(0, 64, 16)
        blk = np.zeros(110, np.uint8)
        hm = rng.integers(0, 256, 32, dtype=np.uint8)
        qs = rng.integers(0, 256, 64, dtype=np.uint8)
        blk[:32], blk[32:96] = hm, qs
        blk[96:108] = _pack_q3k_scales(sc)
        blk[108:110] = np.array([0.25], np.float16).view(np.uint8)
        want = np.zeros(256)
        for n in range(2):
            for j in range(4):
                for l in range(32):
                    q = (int(qs[32 * n + l]) >> (2 * j)) & 3
                    q -= 0 if (int(hm[l]) >> (4 * n + j)) & 1 else 4
                    want[128 * n + 32 * j + l] = 0.25 * (int(sc[8 * n + 2 * j + l // 16]) - 32) * q
        assert np.array_equal(orc.fmt_dequant(Q3_K, blk, (256,)), want.astype(np.float32))


def test_iq4_nl_codebook_and_positions(orc):
    """d = 1: element j takes the table value of the low nibble of qs[j],
    element j + 16 that of its high nibble; every code appears."""
    table = np.array(IQ4NL_TABLE, np.float32)
    rng = np.random.default_rng(16)
    for _ in range(5):
        blk = np.zeros(18, np.uint8)
        blk[:2] = np.array([1.0], np.float16).view(np.uint8)
        lo, hi = rng.permutation(16), rng.integers(0, 16, 16)
        blk[2:] = lo | (hi << 4)
        want = np.concatenate([table[lo], table[hi]])
        assert np.array_equal(orc.fmt_dequant(IQ4_NL, blk, (32,)), want)


def test_iq4_xs_scales_and_positions(orc):
    """d = 0.5, 6-bit scales ls[8] chosen (low nibble of sub-block ib in nibble
    ib & 1 of scales_l[ib / 2], top two bits in bits 2ib, 2ib + 1 of
    scales_h): element 32 ib + e = (d * (ls - 32)) * table[code]."""
    table = np.array(IQ4NL_TABLE, np.float64)
    rng = np.random.default_rng(17)
    for _ in range(10):
        ls = rng.integers(0, 64, 8)
        blk = np.zeros(136, np.uint8)
        blk[:2] = np.array([0.5], np.float16).view(np.uint8)
        sh = 0
        for ib in range(8):
            blk[4 + ib // 2] |= (int(ls[ib]) & 15) << (4 * (ib & 1))
            sh |= (int(ls[ib]) >> 4) << (2 * ib)
        blk[2:4] = np.array([sh], np.uint16).view(np.uint8)
        qs = rng.integers(0, 256, 128, dtype=np.uint8)
        blk[8:] = qs
        want = np.zeros(256)
        for ib in range(8):
            for e in range(32):
                byte = int(qs[16 * ib + (e % 16)])
                code = byte & 15 if e < 16 else byte >> 4
                want[32 * ib + e] = 0.5 * (int(ls[ib]) - 32) * table[code]
        assert np.array_equal(orc.fmt_dequant(IQ4_XS, blk, (256,)), want.astype(np.float32))


@pytest.mark.parametrize("fmt", KQUANT + IQ)
def test_k_formats_have_no_quantizer(orc, fmt):
    x = np.zeros(256, np.float32)
    out = np.zeros(GEOM[fmt][1], np.uint8)
    from oracle_lib import _f, _u8
    assert orc.L.or_fmt_quantize(fmt, 256, _f(x), _u8(out)) == -1


@pytest.mark.parametrize("fmt", KQUANT + LEGACY + IQ)
def test_random_blocks_decode_finite(orc, fmt):
    rng = np.random.default_rng(fmt + 50)
    b = random_blocks(fmt, 8, 512, rng)
    y = orc.fmt_dequant(fmt, b, (8, 512))
    assert np.all(np.isfinite(y)) and np.abs(y).max() > 0
