"""Small-batch GEMMs split along K (partial sums per split, then the reduce
that adds them in split order and applies the epilogue). One session is
executed several times with alternating inputs, so the partial buffer is
reused: every result against the oracle (tolerances of test_gpu_dense),
repeated inputs bit for bit, and a fresh session bit for bit. The SwiGLU
gate+up product (two matrices) likewise."""
import numpy as np
import pytest

from test_gpu_dense import oracle_dense, rel_l2, run, tol

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt,scheme,K,N,batch", [
    (16, 3, 4096, 3000, 16),   # 12 tiles of 256 columns, K split 21 ways
    (4, 2, 11008, 4096, 9),    # 16 tiles, K split 16 ways (the SwiGLU down shape)
    (5, 1, 1000, 700, 32),     # two row blocks, ragged K and N, K split 8 ways
    (4, 3, 2048, 100, 5),      # one tile, K split 16 ways
])
def test_dense_split_reduce_repeated(gpu, oracle, dt, scheme, K, N, batch):
    rng = np.random.default_rng(K + N + batch + dt)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    xs = [rng.standard_normal((batch, K)).astype(np.float32) for _ in range(2)]
    s = gpu.DenseSession(batch, K, N, -1, dt, scheme, W)
    try:
        outs = [s.execute(x)[0] for x in (xs[0], xs[1], xs[0], xs[1])]
    finally:
        s.close()
    for i, x in enumerate(xs):
        o_pre, _ = oracle_dense(oracle, dt, scheme, W, x, threads=16)
        assert rel_l2(outs[i], o_pre) <= tol(batch), (K, N, batch, i)
    assert np.array_equal(outs[0], outs[2])
    assert np.array_equal(outs[1], outs[3])
    fresh, _ = run(gpu, dt, scheme, W, xs[1])
    assert np.array_equal(fresh, outs[3])


def test_swiglu_split_reduce_repeated(gpu, oracle):
    d, f, batch = 1024, 2816, 16
    rng = np.random.default_rng(2816)
    G = (rng.standard_normal((f, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((f, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, f)) / np.sqrt(f)).astype(np.float32)
    xs = [rng.standard_normal((batch, d)).astype(np.float32) for _ in range(2)]
    s = gpu.SwiGLUSession(batch, 1, d, f, 16, 3, G, U, D)
    try:
        outs = [s.execute(x) for x in (xs[0], xs[1], xs[0])]
    finally:
        s.close()

    def deq(W):
        native, rs, blk = oracle.quantize(16, 3, W.shape[0], W.shape[1], W)
        return oracle.dequant(16, 3, W.shape[0], W.shape[1], native, rs, blk)

    Gd, Ud, Dd = deq(G), deq(U), deq(D)
    for i, x in enumerate(xs):
        g, _ = oracle.dense(Gd, x, threads=16)
        u, _ = oracle.dense(Ud, x, threads=16)
        oh = oracle.swiglu_product(g, u)
        h, y = outs[i]
        assert rel_l2(h, oh) <= tol(batch), i
        oy, _ = oracle.dense(Dd, h, threads=16)
        assert rel_l2(y, oy) <= tol(batch), i
    assert np.array_equal(outs[0][0], outs[2][0])
    assert np.array_equal(outs[0][1], outs[2][1])
