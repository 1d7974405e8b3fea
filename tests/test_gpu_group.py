"""Grouped Dense execution (independent cells of one shape, one launch).

Each member must equal its own session's device execute bit for bit (same
kernels and arithmetic) and the oracle within the matrix-core bound.
"""
import numpy as np
import pytest

from test_gpu_dense import TOL_MFMA, oracle_dense, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt,scheme,batch,act,bias,n,K,N", [
    (4, 2, 40, -1, False, 5, 96, 160), (16, 3, 130, 1, True, 5, 96, 160),
    (5, 1, 8, 3, True, 5, 96, 160),
    (4, 2, 256, -1, False, 16, 128, 2048),   # wide tiles: 16 x 2 x 8 workgroups
    (16, 3, 256, 2, True, 16, 128, 2048)])
def test_group_matches_members_and_oracle(gpu, oracle, dt, scheme, batch, act, bias, n, K, N):
    import pywelvet as pw
    hip = pw.Hip()
    rng = np.random.default_rng(batch + dt)
    Ws = [(rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32) for _ in range(n)]
    bs = [rng.standard_normal(N) if bias else None for _ in range(n)]
    xs = [rng.standard_normal((batch, K)).astype(np.float32) for _ in range(n)]
    sessions = [pw.DenseSession(batch, K, N, act, dt, scheme, W, b) for W, b in zip(Ws, bs)]
    dx = [hip.upload(x) for x in xs]
    dpre = [hip.malloc(batch * N * 4) for _ in range(n)]
    dpost = [hip.malloc(batch * N * 4) for _ in range(n)]
    grp = pw.DenseGroup(sessions, dx, dpre, dpost)
    for _ in range(2):  # a second run over the same buffers gives the same result
        grp.execute()
        hip.sync()
    for i in range(n):
        pre = hip.download(dpre[i], (batch, N))
        post = hip.download(dpost[i], (batch, N))
        ref_pre, ref_post = sessions[i].execute(xs[i])
        assert np.array_equal(pre, ref_pre) and np.array_equal(post, ref_post), i
        o_pre, o_post = oracle_dense(oracle, dt, scheme, Ws[i], xs[i], act, bs[i])
        assert rel_l2(pre, o_pre) <= TOL_MFMA and rel_l2(post, o_post) <= TOL_MFMA
    grp.close()
    for p in dx + dpre + dpost:
        hip.free(p)
    for s in sessions:
        s.close()


def test_group_rejects_mixed_shapes(gpu):
    import pywelvet as pw
    hip = pw.Hip()
    a = pw.DenseSession(64, 32, 48, -1, 4, 2, np.ones((48, 32), np.float32))
    b = pw.DenseSession(64, 32, 40, -1, 4, 2, np.ones((40, 32), np.float32))
    bufs = [hip.malloc(64 * 48 * 4) for _ in range(6)]
    with pytest.raises(pw.WelvetError) as e:
        pw.DenseGroup([a, b], bufs[:2], bufs[2:4], bufs[4:])
    assert e.value.code == 1
    for p in bufs:
        hip.free(p)
    a.close()
    b.close()
