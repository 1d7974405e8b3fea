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


# ---- the library's quantizers of the K and IQ4 formats (one pass: scales
# from each sub-block's range or extreme element, integer super-block scales,
# codes for the f16-rounded scales). Pinned by closed-form blocks that must
# come back exactly (grid values with power-of-two scales) and by per-element
# error bounds computed from the block's own stored scales.

def _closed_form_affine(fmt, rng):
    """x on the grid of an affine K format: y = d*ls*q - dmin*lm, with d and
    dmin powers of two, one sub-block at ls = lm = lmax, every sub-block
    holding the codes 0 and qmax."""
    nsub, sub, qmax, lmax = {Q4_K: (8, 32, 15, 63), Q5_K: (8, 32, 31, 63),
                             Q2_K: (16, 16, 3, 15)}[fmt]
    d, dmin = 2.0 ** -6, 2.0 ** -7
    ls = rng.integers(1, lmax + 1, nsub)
    lm = rng.integers(0, lmax + 1, nsub)
    j = rng.integers(0, nsub)
    ls[j] = lm[rng.integers(0, nsub)] = lmax
    q = rng.integers(0, qmax + 1, (nsub, sub))
    q[:, 0], q[:, 1] = 0, qmax
    for r in range(nsub):
        rng.shuffle(q[r])
    x = (d * ls[:, None] * q - dmin * lm[:, None]).astype(np.float32).ravel()
    return x


def _closed_form_signed(fmt, rng):
    """x on the grid of Q3_K / Q6_K: y = d*l*q, d a power of two, one
    sub-block at l = lmin, no l = 0, every sub-block holding the code qlo."""
    qlo, qhi, lmin, lmax = {Q3_K: (-4, 3, -32, 31), Q6_K: (-32, 31, -128, 127)}[fmt]
    d = 2.0 ** -9
    l = rng.integers(lmin + 1, lmax + 1, 16)
    l[l == 0] = 1
    l[rng.integers(0, 16)] = lmin
    q = rng.integers(qlo + 1, qhi + 1, (16, 16))
    q[:, 0] = qlo
    for r in range(16):
        rng.shuffle(q[r])
    return (d * l[:, None] * q).astype(np.float32).ravel()


def _closed_form_iq4(fmt, rng):
    table = np.array(IQ4NL_TABLE, np.float64)
    d = 2.0 ** -10
    if fmt == IQ4_NL:
        idx = rng.integers(0, 16, 32)
        idx[rng.integers(0, 32)] = 0
        return (d * table[idx]).astype(np.float32)
    l = rng.integers(-31, 32, 8)
    l[l == 0] = 1
    l[rng.integers(0, 8)] = -32
    idx = rng.integers(0, 16, (8, 32))
    idx[:, 0] = 0
    for r in range(8):
        rng.shuffle(idx[r])
    return (d * l[:, None] * table[idx]).astype(np.float32).ravel()


@pytest.mark.parametrize("fmt", KQUANT + IQ)
def test_k_quantizers_closed_form(orc, fmt):
    """Values on a format's grid come back exactly, and quantizing the
    decoded block again gives the same bytes."""
    rng = np.random.default_rng(fmt + 900)
    for _ in range(20):
        if fmt in (Q2_K, Q4_K, Q5_K):
            x = _closed_form_affine(fmt, rng)
        elif fmt in (Q3_K, Q6_K):
            x = _closed_form_signed(fmt, rng)
        else:
            x = _closed_form_iq4(fmt, rng)
        b = orc.fmt_quantize(fmt, x)
        y = orc.fmt_dequant(fmt, b, x.shape)
        assert np.array_equal(y, x)
        assert np.array_equal(orc.fmt_quantize(fmt, y), b)


def _k_bound(fmt, x, b):
    """Per-element error bound of one block from its stored scales: half a
    step of the sub-block's scale (a full step on the short side of the
    signed formats' code range), plus what the integer super-block scales
    lose against the sub-block's exact range (the codes that clip)."""
    f16 = lambda v: float(np.array([v], np.uint16).view(np.float16)[0])
    g16 = lambda off: f16(int(b[off]) | (int(b[off + 1]) << 8))
    table = np.array(IQ4NL_TABLE, np.float64)
    x = x.astype(np.float64)
    if fmt in (Q4_K, Q5_K, Q2_K):
        if fmt == Q2_K:
            nsub, sub, qmax = 16, 16, 3
            d, dm = g16(80), g16(82)
            ls = [int(b[j]) & 15 for j in range(16)]
            lm = [int(b[j]) >> 4 for j in range(16)]
        else:
            nsub, sub, qmax = 8, 32, 15 if fmt == Q4_K else 31
            d, dm = g16(0), g16(2)
            sc = b[4:16]
            ls, lm = [], []
            for j in range(8):
                if j < 4:
                    ls.append(int(sc[j]) & 63), lm.append(int(sc[j + 4]) & 63)
                else:
                    ls.append((int(sc[j + 4]) & 15) | ((int(sc[j - 4]) >> 6) << 4))
                    lm.append((int(sc[j + 4]) >> 4) | ((int(sc[j]) >> 6) << 4))
        out = np.zeros(x.size)
        for j in range(nsub):
            v = x[sub * j:sub * (j + 1)]
            mn = min(0.0, float(v.min()))
            scale, off = (float(v.max()) - mn) / qmax, -mn
            ds, dmn = d * ls[j], dm * lm[j]
            out[sub * j:sub * (j + 1)] = 0.5 * ds + qmax * abs(scale - ds) + abs(off - dmn)
        return out
    if fmt in (Q3_K, Q6_K):
        qdiv = 4.0 if fmt == Q3_K else 32.0
        if fmt == Q3_K:
            d = g16(108)
            sc = b[96:108]
            l = []
            for s in range(16):
                g, i = s >> 2, s & 3
                lo = (int(sc[(g & 1) * 4 + i]) >> ((g >> 1) * 4)) & 15
                hi = (int(sc[8 + i]) >> (2 * g)) & 3
                l.append((lo | (hi << 4)) - 32)
        else:
            d = g16(208)
            l = [int(np.int8(b[192 + s])) for s in range(16)]
        out = np.zeros(x.size)
        for j in range(16):
            v = x[16 * j:16 * (j + 1)]
            m = float(v[np.argmax(np.abs(v))])
            s, ds = m / qdiv, d * l[j]
            # the code range is one step shorter on the side opposite the
            # extreme element (Q3_K: -4..3): values there may lose a full step
            out[16 * j:16 * (j + 1)] = abs(ds) + qdiv * abs(abs(s) - abs(ds))
        return out
    # IQ4: the code book's largest half gap is 12 steps of the scale, and its
    # top entry (113) is 14 steps short of the extreme (-127) on the other side
    if fmt == IQ4_NL:
        d = g16(0)
        m = float(x[np.argmax(np.abs(x))])
        return np.full(x.size, 14 * abs(d) + 127 * abs(abs(m) / 127 - abs(d)))
    d, sh = g16(0), int(b[2]) | (int(b[3]) << 8)
    out = np.zeros(x.size)
    for ib in range(8):
        ls = ((int(b[4 + ib // 2]) >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
        dl = d * (ls - 32)
        v = x[32 * ib:32 * (ib + 1)]
        m = float(v[np.argmax(np.abs(v))])
        out[32 * ib:32 * (ib + 1)] = 14 * abs(dl) + 127 * abs(abs(m) / 127 - abs(dl))
    return out


@pytest.mark.parametrize("fmt", [Q2_K, Q4_K, Q5_K])
def test_affine_zero_and_constant_blocks(orc, fmt):
    """An all-zero super-block is all zero bytes (d = dmin = +0, not -0: the
    sign bit of a stored zero is not left to how fmax orders signed zeros);
    a constant positive block has dmin = +0 and decodes to within d of x."""
    qk, bb = GEOM[fmt]
    zero = np.zeros(qk, np.float32)
    b = orc.fmt_quantize(fmt, zero)
    assert not b.any()
    assert not orc.fmt_dequant(fmt, b, zero.shape).view(np.uint32).any()
    const = np.full(qk, 0.37, np.float32)
    b = orc.fmt_quantize(fmt, const)
    dmin = b[bb - 2:bb] if fmt == Q2_K else b[2:4]
    assert not dmin.any()
    y = orc.fmt_dequant(fmt, b, const.shape)
    assert np.all(np.abs(y - const) <= 0.37 / 15)


@pytest.mark.parametrize("fmt", KQUANT + IQ)
def test_k_quantizer_error_bound(orc, fmt):
    """Random rows over six orders of magnitude, constant and all-zero blocks:
    every element within the bound of its block's stored scales."""
    rng = np.random.default_rng(fmt + 400)
    x = (rng.standard_normal((16, 512)) * rng.uniform(1e-3, 1e3, (16, 1))).astype(np.float32)
    x[3] = 0.0
    x[4] = -0.75
    x[5, :256] = 2.5
    x[6] = np.abs(x[6])
    x[7] = -np.abs(x[7])
    b = orc.fmt_quantize(fmt, x)
    y = orc.fmt_dequant(fmt, b, x.shape).astype(np.float64)
    qk, bb = GEOM[fmt][0], GEOM[fmt][1]
    xb, yb, bl = x.reshape(-1, qk), y.reshape(-1, qk), b.reshape(-1, bb)
    for i in range(xb.shape[0]):
        bound = _k_bound(fmt, xb[i], bl[i])
        err = np.abs(xb[i].astype(np.float64) - yb[i])
        tol = bound * (1 + 1e-6) + 1e-30 + np.abs(xb[i]) * 2e-7
        bad = np.flatnonzero(err > tol)
        assert bad.size == 0, (i, bad[:4], err[bad[:4]], bound[bad[:4]])
    # the rows' overall error stays small against their size
    rel = np.linalg.norm(x - y) / np.linalg.norm(x)
    assert rel < {Q2_K: 0.4, Q3_K: 0.2, Q4_K: 0.1, Q5_K: 0.05, Q6_K: 0.025, IQ4_NL: 0.1,
                  IQ4_XS: 0.1}[fmt], rel


@pytest.mark.parametrize("fmt", KQUANT + LEGACY + IQ)
def test_random_blocks_decode_finite(orc, fmt):
    rng = np.random.default_rng(fmt + 50)
    b = random_blocks(fmt, 8, 512, rng)
    y = orc.fmt_dequant(fmt, b, (8, 512))
    assert np.all(np.isfinite(y)) and np.abs(y).max() > 0
