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


def _chain_setup(hip, pw, rng, batch, n, widths, layers):
    """n cells, each a Stack of Dense layers widths[k] -> widths[k + 1];
    layers[k] = (dtype, scheme, act, bias). Linear layers without bias get one
    buffer for pre and post (as a volume keeps it); the others two."""
    Ws, bs, sessions, bufs, groups = [], [], [], [], []
    x0 = [hip.malloc(batch * widths[0] * 4) for _ in range(n)]
    cur = x0
    for k, (dt, sc, act, bias) in enumerate(layers):
        K, N = widths[k], widths[k + 1]
        Wk = [(rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32) for _ in range(n)]
        bk = [rng.standard_normal(N) if bias else None for _ in range(n)]
        sk = [pw.DenseSession(batch, K, N, act, dt, sc, W, b) for W, b in zip(Wk, bk)]
        pre = [hip.malloc(batch * N * 4) for _ in range(n)]
        post = pre if (act == -1 and not bias) else [hip.malloc(batch * N * 4) for _ in range(n)]
        groups.append(pw.DenseGroup(sk, cur, pre, post))
        Ws.append(Wk), bs.append(bk), sessions.append(sk), bufs.append((pre, post))
        cur = post
    return Ws, bs, sessions, x0, bufs, groups


@pytest.mark.parametrize("batch,n,widths,layers", [
    # volume cells: E4M3 per-row -> FP4 E8M0/32 -> E4M3 per-row (wide tiles)
    (256, 16, [1024, 1024, 1024, 1024], [(4, 2, -1, False), (16, 3, -1, False), (4, 2, -1, False)]),
    # ragged rows (200 of 256 padded), an activation + bias producer, 128-wide tiles
    (200, 3, [256, 512, 256, 384], [(5, 1, -1, False), (4, 3, 1, True), (16, 3, 2, True)]),
    # a link whose width is not a multiple of 256 runs its own split
    (130, 2, [128, 384, 256, 128], [(4, 2, 0, False), (16, 3, -1, False), (4, 2, -1, True)]),
    # 16 rows: the groups run member by member
    (16, 3, [256, 256, 256], [(4, 2, -1, False), (16, 3, 3, True)]),
])
def test_chain_matches_groups(gpu, oracle, batch, n, widths, layers):
    import pywelvet as pw
    hip = pw.Hip()
    rng = np.random.default_rng(batch * 7 + n)
    Ws, bs, sessions, x0, bufs, groups = _chain_setup(hip, pw, rng, batch, n, widths, layers)
    chain = pw.DenseChain(groups)
    xa = [rng.standard_normal((batch, widths[0])).astype(np.float32) for _ in range(n)]
    xb = [rng.standard_normal((batch, widths[0])).astype(np.float32) for _ in range(n)]
    # a first input, then a second: a consumer that skipped reading its own
    # split would still hold the first input's terms
    for i in range(n):
        hip.copy_in(x0[i], xa[i])
    chain.execute()
    hip.sync()
    for i in range(n):
        hip.copy_in(x0[i], xb[i])
    chain.execute()
    hip.sync()
    L = len(layers)
    got = [[(hip.download(bufs[k][0][i], (batch, widths[k + 1])),
             hip.download(bufs[k][1][i], (batch, widths[k + 1]))) for i in range(n)] for k in range(L)]
    for g in groups:  # the same layers one group at a time
        g.execute()
    hip.sync()
    for k in range(L):
        for i in range(n):
            pre = hip.download(bufs[k][0][i], (batch, widths[k + 1]))
            post = hip.download(bufs[k][1][i], (batch, widths[k + 1]))
            assert np.array_equal(got[k][i][0], pre) and np.array_equal(got[k][i][1], post), (k, i)
            # each layer against the oracle on the GPU's own input to it
            xin = xb[i] if k == 0 else hip.download(bufs[k - 1][1][i], (batch, widths[k]))
            dt, sc, act, _ = layers[k]
            o_pre, o_post = oracle_dense(oracle, dt, sc, Ws[k][i], xin, act, bs[k][i])
            tol = TOL_MFMA if batch > 4 else 1e-5
            assert rel_l2(pre, o_pre) <= tol and rel_l2(post, o_post) <= tol, (k, i)
    chain.close()
    for g in groups:
        g.close()
    seen = set()
    for p in x0 + [q for pre, post in bufs for q in pre + post]:
        if p not in seen:
            seen.add(p)
            hip.free(p)
    for sk in sessions:
        for s in sk:
            s.close()


def test_chain_rejects_unlinked_groups(gpu):
    import pywelvet as pw
    hip = pw.Hip()
    W = np.ones((256, 256), np.float32) / 256
    a = pw.DenseSession(64, 256, 256, -1, 4, 2, W)
    b = pw.DenseSession(64, 256, 256, -1, 4, 2, W)
    bufs = [hip.malloc(64 * 256 * 4) for _ in range(3)]
    g1 = pw.DenseGroup([a], [bufs[0]], [bufs[1]], [bufs[1]])
    g2 = pw.DenseGroup([b], [bufs[0]], [bufs[2]], [bufs[2]])  # reads x, not g1's output
    with pytest.raises(pw.WelvetError) as e:
        pw.DenseChain([g1, g2])
    assert e.value.code == 1
    for g in (g1, g2):
        g.close()
    for p in bufs:
        hip.free(p)
    a.close()
    b.close()


@pytest.mark.parametrize("batch,n,widths,layers", [
    (256, 16, [1024, 1024, 1024, 1024], [(4, 2, -1, False), (16, 3, -1, False), (4, 2, -1, False)]),
    (200, 3, [256, 512, 256, 384], [(5, 1, -1, False), (4, 3, 1, True), (16, 3, 2, True)]),
    (130, 2, [128, 384, 256, 128], [(4, 2, 0, False), (16, 3, -1, False), (4, 2, -1, True)]),
])
def test_chain_inner_not_kept(gpu, batch, n, widths, layers):
    """WELVET_CHAIN_INNER_NOT_KEPT: the last group's outputs equal those of the
    chain that keeps every output, bit for bit; a group whose epilogue writes
    the next split leaves its own pre / post untouched; a group that the next
    one reads from memory (width not a multiple of 256) still writes them."""
    import pywelvet as pw
    hip = pw.Hip()
    rng = np.random.default_rng(batch * 11 + n)
    Ws, bs, sessions, x0, bufs, groups = _chain_setup(hip, pw, rng, batch, n, widths, layers)
    full = pw.DenseChain(groups)
    lean = pw.DenseChain(groups, keep_inner=False)
    L = len(layers)
    xa = [rng.standard_normal((batch, widths[0])).astype(np.float32) for _ in range(n)]
    for i in range(n):
        hip.copy_in(x0[i], xa[i])
    full.execute()
    hip.sync()
    want = [(hip.download(bufs[L - 1][0][i], (batch, widths[L])),
             hip.download(bufs[L - 1][1][i], (batch, widths[L]))) for i in range(n)]
    kept = [[hip.download(bufs[k][1][i], (batch, widths[k + 1])) for i in range(n)] for k in range(L)]
    for k in range(L):  # poison every output buffer (0xFF bytes: NaN)
        for i in range(n):
            for p in {bufs[k][0][i], bufs[k][1][i]}:
                hip.memset(p, 0xFF, batch * widths[k + 1] * 4)
    hip.sync()
    for _ in range(2):  # twice: the second run starts from the first's state
        lean.execute()
    hip.sync()
    for i in range(n):
        pre = hip.download(bufs[L - 1][0][i], (batch, widths[L]))
        post = hip.download(bufs[L - 1][1][i], (batch, widths[L]))
        assert np.array_equal(pre, want[i][0]) and np.array_equal(post, want[i][1]), i
    for k in range(L - 1):
        fused = batch > 32 and widths[k + 1] % 256 == 0
        for i in range(n):
            post = hip.download(bufs[k][1][i], (batch, widths[k + 1]))
            if fused:
                assert np.isnan(post).all(), (k, i)
            else:
                assert np.array_equal(post, kept[k][i]), (k, i)
    lean.close()
    full.close()
    for g in groups:
        g.close()
    seen = set()
    for p in x0 + [q for pre, post in bufs for q in pre + post]:
        if p not in seen:
            seen.add(p)
            hip.free(p)
    for sk in sessions:
        for s in sk:
            s.close()


def test_chain_inner_not_kept_nonfinite_consumer(gpu):
    """A consumer whose E5M2 codes hold inf and NaN (scheme 0: weights past
    the E5M2 range encode to 0x7C / 0xFC, NaN to 0x7E) recomputes those rows
    from its fp32 input after its product. In a chain that leaves out the
    inner outputs, the producer feeding such a consumer still writes that
    input, so the lean chain's last outputs equal the kept chain's bit for
    bit."""
    import pywelvet as pw
    hip = pw.Hip()
    rng = np.random.default_rng(77)
    batch, n, d = 64, 3, 256
    W0 = [(rng.standard_normal((d, d)) / 16).astype(np.float32) for _ in range(n)]
    W1 = [(rng.standard_normal((d, d)) / 16).astype(np.float32) for _ in range(n)]
    for i, W in enumerate(W1):
        W[3 + i, 5] = 7.0e4     # -> 0x7C (+inf)
        W[40, 7 + i] = -7.0e4   # -> 0xFC (-inf)
        W[100 + i, 0] = np.nan  # -> 0x7E (NaN)
    s0 = [pw.DenseSession(batch, d, d, -1, 4, 2, W) for W in W0]
    s1 = [pw.DenseSession(batch, d, d, -1, 5, 0, W) for W in W1]
    x0 = [hip.malloc(batch * d * 4) for _ in range(n)]
    y0 = [hip.malloc(batch * d * 4) for _ in range(n)]
    y1 = [hip.malloc(batch * d * 4) for _ in range(n)]
    g0 = pw.DenseGroup(s0, x0, y0, y0)
    g1 = pw.DenseGroup(s1, y0, y1, y1)
    full = pw.DenseChain([g0, g1])
    lean = pw.DenseChain([g0, g1], keep_inner=False)
    for i in range(n):
        hip.copy_in(x0[i], rng.standard_normal((batch, d)).astype(np.float32))
    full.execute()
    hip.sync()
    want = [hip.download(y1[i], (batch, d)) for i in range(n)]
    for i in range(n):
        assert np.isposinf(want[i][:, 3 + i]).any() or np.isneginf(want[i][:, 3 + i]).any()
        assert np.isnan(want[i][:, 100 + i]).all()
        for p in (y0[i], y1[i]):
            hip.memset(p, 0xFF, batch * d * 4)
    hip.sync()
    lean.execute()
    hip.sync()
    for i in range(n):
        got = hip.download(y1[i], (batch, d))
        assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), i
    for c in (lean, full, g1, g0):
        c.close()
    for p in x0 + y0 + y1:
        hip.free(p)
    for s in s0 + s1:
        s.close()
