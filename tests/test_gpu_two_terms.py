"""Two activation terms on the matrix-core paths (backend bit 16).

The matrix cores take FP8/FP4 on both operands, so fp32 activations are split
into E4M3 terms with per-32 E8M0 scales. Three terms (the default) leave a
~2^-12 relative residual per element and ~2e-5 rel-L2 per product; two terms
leave ~2^-8 and cost two thirds of the matrix-core work and activation
bytes. The bound here is the contract's, rel-L2 <= 1e-3 per product against
the oracle's dequantize-then-f64 Dense (kernels.cu:130-161); the measured
value is printed (~6.3e-4). Also checked: the paths that take the option
(5..32-row GEMM, large tiles, the K-split large tiles, grouped and chained
launches) and the layers that refuse it (SwiGLU and MHA, whose chained
products and softmax take the error past the bound).
"""
import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import oracle_dense, rel_l2, tol

pytestmark = pytest.mark.gpu

TWO = 16
TOL_TWO = 1e-3


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3), (5, 1)])
@pytest.mark.parametrize("rows,K,N", [(20, 1024, 2048), (64, 1024, 1024), (300, 700, 513),
                                      (1024, 4096, 1024), (2048, 256, 4096)])
def test_two_terms_dense_within_contract(gpu, oracle, dt, scheme, rows, K, N):
    rng = np.random.default_rng(rows + K + N + dt)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    s2 = gpu.DenseSession(rows, K, N, -1, dt, scheme | TWO, W)
    y2, _ = s2.execute(x)
    s2.close()
    s3 = gpu.DenseSession(rows, K, N, -1, dt, scheme, W)
    y3, _ = s3.execute(x)
    s3.close()
    want, _ = oracle_dense(oracle, dt, scheme, W, x)
    e2, e3 = rel_l2(y2, want), rel_l2(y3, want)
    print(f"two terms rel-L2 {e2:.2e}, three terms {e3:.2e} ({rows}x{K}x{N} dtype {dt})")
    assert e2 <= TOL_TWO
    assert e3 <= tol(rows)
    assert e2 > e3  # the option takes effect


def test_two_terms_batch_up_to_four_and_one_unchanged(gpu):
    """Batches of 1-4 rows run the GEMV paths, which do not split into E4M3
    terms the same way: the option leaves them bit for bit as they are."""
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((300, 512)) / 22).astype(np.float32)
    for rows in (1, 3):
        x = rng.standard_normal((rows, 512)).astype(np.float32)
        a = gpu.DenseSession(rows, 512, 300, -1, 4, 2 | TWO, W)
        b = gpu.DenseSession(rows, 512, 300, -1, 4, 2, W)
        assert np.array_equal(a.execute(x)[0], b.execute(x)[0])
        a.close()
        b.close()


@pytest.mark.parametrize("batch", [256, 512])
def test_two_terms_grouped_chain(gpu, oracle, batch):
    """16 cells x 3 layers (E4M3 row, FP4 E8M0, E4M3 row) at 256 and 512
    rows (128-row and 256-row tiles), grouped and chained through the epilogue
    split, every layer within the bound on the GPU's own input."""
    cells, d = 16, 1024
    kinds = [(4, 2), (16, 3), (4, 2)]
    hip = gpu.Hip()
    sessions, bufs, Ws, xs = [], [], [], []
    try:
        for c in range(cells):
            rng = np.random.default_rng(700 + c)
            row, wrow = [], []
            for dt, sc in kinds:
                W = (rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32)
                row.append(gpu.DenseSession(batch, d, d, -1, dt, sc | TWO, W))
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
    worst = 0.0
    for c in range(cells):
        cur = xs[c]
        for li, (dt, sc) in enumerate(kinds):
            want, _ = oracle_dense(oracle, dt, sc, Ws[c][li], cur)
            err = rel_l2(outs[c][li], want)
            worst = max(worst, err)
            assert err <= TOL_TWO, (c, li, err)
            cur = outs[c][li]
    print(f"two-term chain: worst per-layer rel-L2 {worst:.2e}")


def test_two_terms_refused_for_mha(gpu):
    """Two-term Q/K/V/O projections gave attention rel-L2 1.0e-3 and output
    1.16e-3 (B=2, S=128, d=256): the softmax amplifies the score error past
    the layer bound, so MHA layers refuse the option."""
    W = np.zeros((64, 64), np.float32)
    with pytest.raises(gpu.WelvetError) as e:
        gpu.MHASession(1, 8, 64, 4, 4, 0, 8, 1, 0, 5, 2 | TWO, W, W, W, W)
    assert e.value.code == 2


def test_two_terms_refused_for_swiglu(gpu):
    W = np.zeros((64, 32), np.float32)
    with pytest.raises(gpu.WelvetError) as e:
        gpu.SwiGLUSession(1, 8, 32, 64, 16, 3 | TWO, W, W, W.T.copy())
    assert e.value.code == 2
