"""One activation term on the matrix-core paths (backend bit 32): the
throughput mode, outside the contract.

With one E4M3 term per 32-element block, x is replaced by
x1 = 2^e * RNE_E4M3(x / 2^e), e the block's E8M0 exponent (the smallest e
with amax <= 448 * 2^e), and the product is W_deq x1: about 2.7e-2 relative
L2 against the oracle's exact Dense, far outside the 1e-3 bound. The mode
exists to report the matrix-core rate at one term beside the contract modes.

Pinned two ways: (1) against a numpy model of that single-term product (the
block rule restated from the split's definition, RNE to 3 mantissa bits,
E4M3 subnormals below 2^-6, f64 products), at the matrix cores' own
accumulation floor; a dropped or extra term, a wrong block exponent or a
transposed operand moves the result by the size of the split residual
(~1e-2), far above that floor; (2) the error against the exact oracle lies
in the range the E4M3 grid implies. Covered: 128-row tiles over 8 K steps
(the two-steps-ahead loop), the generic loop (ragged K), the K split, wide
tiles, and a grouped chain whose epilogue writes the next layer's one-term
split. 5..32-row batches refuse the option at mount.
"""
import numpy as np
import pytest

from test_gpu_dense import rel_l2

pytestmark = pytest.mark.gpu

ONE = 32
FLOOR = 5e-5  # matrix-core accumulation floor (as for the three-term paths)


def e8m0_exp(amax):
    """Smallest e with amax <= 448 * 2^e (amax > 0), clamped to [-127, 127]."""
    m, ex = np.frexp(amax.astype(np.float64))  # amax = m * 2^ex, m in [0.5, 1)
    a = 2.0 * m  # [1, 2)
    e = (ex - 1) - 8 + (a > 1.75)
    e = np.clip(e, -127, 127)
    return np.where(amax > 0, e, 0)


def e4m3_rne(v):
    a = np.abs(v)
    ex = np.floor(np.log2(np.maximum(a, 2.0 ** -6)))
    step = 2.0 ** (ex - 3)
    return np.sign(v) * np.round(a / step) * step


def one_term(x):
    """The single-term approximation of x [rows][K] (f64), blocks of 32 along K."""
    rows, K = x.shape
    kp = (K + 31) // 32 * 32
    xp = np.zeros((rows, kp), np.float64)
    xp[:, :K] = x
    b = xp.reshape(rows, kp // 32, 32)
    e = e8m0_exp(np.abs(b).max(axis=2))[:, :, None]
    sc = np.ldexp(1.0, e)
    return (e4m3_rne(b / sc) * sc).reshape(rows, kp)[:, :K]


def dequant(oracle, dt, scheme, W):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    return oracle.dequant(dt, scheme, rows, cols, native, rs, blk).astype(np.float64)


def test_one_term_model_on_known_values():
    # blocks whose terms are exact: the model returns them unchanged
    x = np.array([[448.0, -3.5, 0.0, 2.0 ** -9] + [1.0] * 28], np.float64)
    assert np.array_equal(one_term(x), x)
    # 448 * 2^1 needs e = 1: 1.0 then sits on the grid, 0.3 rounds to 0.3125
    x = np.array([[896.0, 1.0, 0.3] + [0.0] * 29])
    got = one_term(x)
    assert got[0, 0] == 896.0 and got[0, 1] == 1.0 and got[0, 2] == 0.3125
    # ties go to even: 1.0625 lies halfway between 1.0 and 1.125
    x = np.array([[448.0, 1.0625, 1.1875] + [0.0] * 29])
    got = one_term(x)
    assert got[0, 1] == 1.0 and got[0, 2] == 1.25


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3), (5, 1)])
@pytest.mark.parametrize("rows,K,N", [(4096, 1024, 1024), (64, 1024, 1024), (300, 700, 513),
                                      (1024, 4096, 1024), (2048, 256, 4096)])
def test_one_term_dense(gpu, oracle, dt, scheme, rows, K, N):
    rng = np.random.default_rng(rows + K + N + dt + 1)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    s = gpu.DenseSession(rows, K, N, -1, dt, scheme | ONE, W)
    y, _ = s.execute(x)
    s.close()
    Wd = dequant(oracle, dt, scheme, W)
    model = one_term(x.astype(np.float64)) @ Wd.T
    exact = x.astype(np.float64) @ Wd.T  # the oracle's Dense, summed by BLAS in f64
    e_model, e_exact = rel_l2(y, model), rel_l2(y, exact)
    print(f"one term: rel-L2 {e_exact:.2e} against the exact Dense, {e_model:.1e} against "
          f"the one-term model ({rows}x{K}x{N} dtype {dt})")
    assert e_model <= FLOOR
    assert 5e-3 <= e_exact <= 6e-2


def test_one_term_refused_for_5_to_32_rows(gpu):
    W = np.zeros((64, 64), np.float32)
    for rows in (5, 16, 32):
        with pytest.raises(gpu.WelvetError) as e:
            gpu.DenseSession(rows, 64, 64, -1, 4, 2 | ONE, W)
        assert e.value.code == 2
    for rows in (1, 4, 33):
        gpu.DenseSession(rows, 64, 64, -1, 4, 2 | ONE, W).close()


def test_one_and_two_term_bits_together_invalid(gpu):
    W = np.zeros((64, 64), np.float32)
    with pytest.raises(gpu.WelvetError) as e:
        gpu.DenseSession(64, 64, 64, -1, 4, 2 | ONE | 16, W)
    assert e.value.code == 1


def test_one_term_grouped_chain(gpu, oracle):
    """8 cells x 3 layers (E4M3 row, FP4 E8M0, E4M3 row) at 256 rows, wide
    tiles, chained: every layer against the one-term model of its own input
    as the GPU computed it."""
    cells, d, batch = 8, 1024, 256
    kinds = [(4, 2), (16, 3), (4, 2)]
    hip = gpu.Hip()
    sessions, bufs, Ws, xs = [], [], [], []
    try:
        for c in range(cells):
            rng = np.random.default_rng(900 + c)
            row, wrow = [], []
            for dt, sc in kinds:
                W = (rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32)
                row.append(gpu.DenseSession(batch, d, d, -1, dt, sc | ONE, W))
                wrow.append(W)
            sessions.append(row)
            Ws.append(wrow)
            x = rng.standard_normal((batch, d)).astype(np.float32)
            xs.append(x)
            bufs.append([hip.upload(x)] + [hip.malloc(batch * d * 4) for _ in kinds])
        groups = [gpu.DenseGroup([sessions[c][li] for c in range(cells)],
                                 [bufs[c][li] for c in range(cells)],
                                 [bufs[c][li + 1] for c in range(cells)],
                                 [bufs[c][li + 1] for c in range(cells)])
                  for li in range(len(kinds))]
        chain = gpu.DenseChain(groups)
        chain.execute()
        hip.sync()
        outs = [[hip.download(bufs[c][li + 1], (batch, d)) for li in range(len(kinds))]
                for c in range(cells)]
        chain.close()
        for g in groups:
            g.close()
    finally:
        for row in sessions:
            for s in row:
                s.close()
        for b in bufs:
            for p in b:
                hip.free(p)
    for c in range(cells):
        cur = xs[c]
        for li, (dt, sc) in enumerate(kinds):
            model = one_term(cur.astype(np.float64)) @ dequant(oracle, dt, sc, Ws[c][li]).T
            assert rel_l2(outs[c][li], model) <= FLOOR, (c, li)
            cur = outs[c][li]
