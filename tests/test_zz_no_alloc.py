"""welvet_dense_execute_noalloc (no counterpart in the reference): the Dense
execute for callers that cannot allocate, its scratch memory a fixed device
array of the library. Checked through the C ABI against
welvet_dense_execute_device on sessions mounted at the same row counts, two
calls in a row with the second smaller, bit for bit (same kernels, same
arithmetic), and against the oracle within the path's tolerance."""
import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import oracle_dense, rel_l2, tol

pytestmark = pytest.mark.gpu


def existing(gpu, hip, rows, K, N, dt, scheme, W, x, act=-1, bias=None):
    s = gpu.DenseSession(rows, K, N, act, dt, scheme, W, bias)
    dx = hip.upload(x[:rows])
    pre, post = hip.malloc(rows * N * 4), hip.malloc(rows * N * 4)
    s.execute_device(dx, pre, post)
    hip.sync()
    out = hip.download(pre, (rows, N)), hip.download(post, (rows, N))
    for p in (dx, pre, post):
        hip.free(p)
    s.close()
    return out


@pytest.mark.parametrize("dt,scheme,K,N,act,rows_seq", [
    (4, 2, 1024, 2048, -1, (256, 48)),   # large tiles, then the K-split large-tile path
    (16, 3, 4096, 1024, 1, (64, 20)),    # large tiles then the 5..32-row GEMM, SiLU
    (5, 1, 700, 300, 0, (40, 3)),        # ragged K, bias + ReLU, then the 2..4-row path
])
def test_noalloc_matches_execute_device(gpu, oracle, dt, scheme, K, N, act, rows_seq):
    hip = gpu.Hip()
    rng = np.random.default_rng(K + N + dt)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    bias = rng.standard_normal(N) if act != -1 else None
    big = max(rows_seq)
    x = rng.standard_normal((big, K)).astype(np.float32)
    s = gpu.DenseSession(big, K, N, act, dt, scheme, W, bias)
    dx = hip.upload(x)
    pre, post = hip.malloc(big * N * 4), hip.malloc(big * N * 4)
    try:
        for rows in rows_seq:  # two calls in a row on the shared scratch, the second smaller
            s.execute_noalloc(rows, dx, pre, post)
            hip.sync()
            got_pre = hip.download(pre, (rows, N))
            got_post = hip.download(post, (rows, N))
            want_pre, want_post = existing(gpu, hip, rows, K, N, dt, scheme, W, x, act, bias)
            assert np.array_equal(got_pre, want_pre)
            assert np.array_equal(got_post, want_post)
            o_pre, o_post = oracle_dense(oracle, dt, scheme, W, x[:rows], act, bias)
            assert rel_l2(got_pre, o_pre) <= tol(rows)
            assert rel_l2(got_post, o_post) <= tol(rows)
    finally:
        for p in (dx, pre, post):
            hip.free(p)
        s.close()


def test_noalloc_rejects_oversized_rows(gpu):
    """Rows whose activation split exceeds the fixed 64 MiB scratch: code 1,
    nothing queued."""
    hip = gpu.Hip()
    K, N = 16384, 256
    W = np.zeros((N, K), np.float32)
    s = gpu.DenseSession(8, K, N, -1, 4, 0, W)
    rows = 2048  # 3 terms x 2048 x 16384 bytes = 96 MiB of split
    dx, dy = hip.malloc(16), hip.malloc(16)
    try:
        with pytest.raises(gpu.WelvetError) as e:
            s.execute_noalloc(rows, dx, dy, dy)
        assert e.value.code == 1 and b"scratch" in str(e.value).encode()
        with pytest.raises(gpu.WelvetError) as e:
            s.execute_noalloc(0, dx, dy, dy)
        assert e.value.code == 1
    finally:
        hip.free(dx)
        hip.free(dy)
        s.close()
