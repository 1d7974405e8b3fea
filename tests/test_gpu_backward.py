"""Dense backward and SGD on the GPU (welvet_dense_normalbp_f32) against the
oracle.

The backward is checked on the GPU's own forward outputs (pre, post), so each
stage is compared with exactly the inputs it received:
  * d_pre and dW (kernels.cu:83-127): bit-exact for the piecewise-polynomial
    activations (Linear, ReLU, LeakyReLU, ReLU2): the f64 product of two
    floats is exact and the f32 roundings happen at the same points. With
    exp/tanh in act' the device and host math libraries may differ in the
    last f64 bit: relative L2 <= 1e-6;
  * dX = W^T d_pre (kernels.cu:92-107): f64 accumulation of exact terms in a
    different order than the reference's serial sum: relative L2 <= 1e-6;
  * the MSE loss (training.cpp:44-56): relative difference <= 1e-12;
  * W_after: the oracle's SGD element rule (native_codec.cpp:1112-1128) on the
    GPU's dW, re-quantized with the layer's scheme, then dequantized:
    bit-exact (scheme 0 re-encodes every element with the reference codec).
The forward outputs themselves are checked against the oracle with the
Dense tolerances.
"""
import numpy as np
import pytest

from test_gpu_dense import rel_l2, tol

pytestmark = pytest.mark.gpu

EXACT_ACTS = (-1, 0, 5, 6)


def check_normalbp(gpu, oracle, dt, scheme, batch, inn, out, act, use_target, lr, bias, seed):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((out, inn)) / np.sqrt(inn)).astype(np.float32)
    if scheme == 0:
        W *= 8.0
    x = rng.standard_normal((batch, inn)).astype(np.float32)
    g = rng.standard_normal((batch, out)).astype(np.float32)
    b = rng.standard_normal(out) * 0.1 if bias else None
    pre, post, dx, dw, wa, loss = gpu.dense_normalbp(batch, inn, out, act, dt, scheme, W, x, g,
                                                     use_target, lr, b)
    native, rs, blk = oracle.quantize(dt, scheme, out, inn, W)
    Wd = oracle.dequant(dt, scheme, out, inn, native, rs, blk)
    o_pre, o_post = oracle.dense(Wd, x, act, b)
    assert rel_l2(pre, o_pre) <= tol(batch) and rel_l2(post, o_post) <= tol(batch)

    gy = oracle.mse_grad(post, g) if use_target else g
    dpre_o, dx_o, dw_o = oracle.backward(Wd, gy, pre, x, act)
    if act in EXACT_ACTS:
        assert np.array_equal(dw, dw_o)
    else:
        assert rel_l2(dw, dw_o) <= 1e-6
    assert rel_l2(dx, dx_o) <= 1e-6
    if use_target:
        lo = oracle.mse(post, g)
        assert abs(loss - lo) <= 1e-12 * lo
    else:
        assert loss == 0.0
    if lr == 0.0:
        assert np.array_equal(wa, Wd)
    else:
        nxt = oracle.sgd(Wd, dw, lr)
        n2, rs2, blk2 = oracle.quantize(dt, scheme, out, inn, nxt)
        assert np.array_equal(wa, oracle.dequant(dt, scheme, out, inn, n2, rs2, blk2))
    return dx, dw


@pytest.mark.parametrize("dt,scheme", [(4, 0), (5, 0), (16, 0), (4, 2), (16, 3), (5, 1)])
@pytest.mark.parametrize("batch,inn,out,act,use_target,lr,bias", [
    (1, 300, 70, -1, False, 0.0, False),     # ragged, one partial band
    (3, 1000, 33, 0, True, 0.05, True),      # MSE target, ReLU, bias, SGD
    (5, 513, 129, 1, False, 0.5, False),     # SiLU, odd widths (FP4 nibbles straddle rows)
    (40, 256, 512, 2, True, 0.01, False),    # matrix-core forward, GELU
    (9, 1536, 1100, 5, False, 1.0, True),    # two d_pre chunks + one, LeakyReLU
])
def test_normalbp_matches_oracle(gpu, oracle, dt, scheme, batch, inn, out, act, use_target, lr,
                                 bias):
    check_normalbp(gpu, oracle, dt, scheme, batch, inn, out, act, use_target, lr, bias,
                   seed=batch * 131 + inn + out + dt + scheme)


def test_normalbp_c2_shape(gpu, oracle):
    """GEMV 4096 x 4096, E4M3 per-row scales, batch 1 (the headline GEMV shape)."""
    check_normalbp(gpu, oracle, 4, 2, 1, 4096, 4096, -1, True, 0.1, False, seed=2)


@pytest.mark.parametrize("dt", [4, 5, 16])
def test_normalbp_integer_exact(gpu, oracle, dt):
    """Integer weights that every format holds, integer inputs and gradients:
    every term and sum is exact, so dX is the integer product bit for bit."""
    rng = np.random.default_rng(dt)
    vals = np.array([-4, -2, -1, 0, 1, 2, 4], np.float32)
    W = rng.choice(vals, (70, 300))
    x = rng.integers(-4, 5, (3, 300)).astype(np.float32)
    g = rng.integers(-4, 5, (3, 70)).astype(np.float32)
    _, _, dx, dw, _, _ = gpu.dense_normalbp(3, 300, 70, -1, dt, 0, W, x, g)
    assert np.array_equal(dx, (g.astype(np.int64) @ W.astype(np.int64)).astype(np.float32))
    assert np.array_equal(dw, (g.T.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))


def test_normalbp_sgd_descends(gpu, oracle):
    """A few SGD steps on an MSE target lower the loss (E4M3 per-row, the
    weights re-quantized after every step)."""
    rng = np.random.default_rng(8)
    W = (rng.standard_normal((32, 64)) / 8).astype(np.float32)
    x = rng.standard_normal((16, 64)).astype(np.float32)
    t = (x @ (rng.standard_normal((32, 64)).astype(np.float32) / 8).T).astype(np.float32)
    losses = []
    for _ in range(4):
        _, _, _, _, W, loss = gpu.dense_normalbp(16, 64, 32, -1, 4, 2, W, x, t, True, 0.5)
        losses.append(loss)
    assert all(b < a for a, b in zip(losses, losses[1:])), losses


def test_normalbp_rejects_bad_arguments(gpu):
    W = np.ones((4, 4), np.float32)
    x = np.ones((1, 4), np.float32)
    with pytest.raises(gpu.WelvetError) as e:
        gpu.dense_normalbp(0, 4, 4, -1, 4, 0, W, x, np.ones((1, 4), np.float32))
    assert e.value.code == 1
    with pytest.raises(gpu.WelvetError) as e:
        gpu.dense_normalbp(1, 4, 4, -1, 1, 0, W, x, np.ones((1, 4), np.float32))
    assert e.value.code == 2


@pytest.mark.parametrize("dt,scheme,batch,act,use_target,nonfinite", [
    (4, 2, 1, -1, True, False), (16, 3, 6, 1, False, False), (5, 0, 40, 5, True, False),
    (4, 2, 5, -1, False, False),   # Linear, no target: d_pre = gy from the products' launch
    (16, 3, 1, -1, False, True),   # the same with inf and NaN in gy
])
def test_backward_device_matches_normalbp(gpu, oracle, dt, scheme, batch, act, use_target,
                                          nonfinite):
    """welvet_dense_backward_device on a mounted session (device buffers, the
    session stream) gives the bits of welvet_dense_normalbp_f32, twice in a
    row over the same buffers (the second call reuses the dX partials), and
    its d_pre output is the oracle's (kernels.cu:83-90)."""
    rng = np.random.default_rng(batch + dt)
    inn, out = 700, 300
    W = (rng.standard_normal((out, inn)) / np.sqrt(inn)).astype(np.float32)
    x = rng.standard_normal((batch, inn)).astype(np.float32)
    g = rng.standard_normal((batch, out)).astype(np.float32)
    if nonfinite:
        g[0, 3], g[0, 77], g[-1, -1] = np.inf, -np.inf, np.nan
    pre, post, dx, dw, _, loss = gpu.dense_normalbp(batch, inn, out, act, dt, scheme, W, x, g,
                                                    use_target)
    hip = gpu.Hip()
    s = gpu.DenseSession(batch, inn, out, act, dt, scheme, W)
    bufs = {k: hip.malloc(n * 4) for k, n in [("x", batch * inn), ("pre", batch * out),
                                              ("post", batch * out), ("g", batch * out),
                                              ("d", batch * out), ("dx", batch * inn),
                                              ("dw", out * inn)]}
    nparts = (batch * out + 255) // 256
    lp = hip.malloc(nparts * 8)
    hip.copy_in(bufs["x"], x)
    hip.copy_in(bufs["g"], g)
    s.execute_device(bufs["x"], bufs["pre"], bufs["post"])
    for _ in range(2):
        s.backward_device(bufs["x"], bufs["pre"], bufs["post"], bufs["g"], use_target, bufs["d"],
                          bufs["dx"], bufs["dw"], lp)
        hip.sync()
        assert np.array_equal(hip.download(bufs["pre"], (batch, out)), pre)
        assert np.array_equal(hip.download(bufs["dx"], (batch, inn)), dx, equal_nan=True)
        assert np.array_equal(hip.download(bufs["dw"], (out, inn)), dw, equal_nan=True)
        gy = oracle.mse_grad(post, g) if use_target else g
        dpre_o = oracle.backward(W, gy, pre, x, act)[0]  # d_pre does not depend on W
        d = hip.download(bufs["d"], (batch, out))
        if act in EXACT_ACTS:
            assert np.array_equal(d, dpre_o, equal_nan=True)
        else:
            assert rel_l2(d, dpre_o) <= 1e-6
        if use_target:
            total = 0.0
            for v in hip.download(lp, (nparts,), np.float64):  # in order, as the library adds them
                total += float(v)
            assert total / (batch * out) == loss
    for p in list(bufs.values()) + [lp]:
        hip.free(p)
    s.close()


@pytest.mark.parametrize("dt,scheme,batch,seq,d,f,use_target,lr", [
    (16, 3, 1, 1, 256, 704, False, 0.0),   # batch-1 GEMV forward
    (4, 2, 2, 3, 128, 384, True, 0.05),    # 6 rows: small-batch matrix cores
    (5, 0, 5, 8, 128, 256, True, 0.5),     # 40 rows: large tiles
])
def test_swiglu_normalbp_matches_oracle(gpu, oracle, dt, scheme, batch, seq, d, f, use_target, lr):
    """welvet_swiglu_normalbp_f32 (c_abi.cpp:581-652, swiglu.cpp:156-248):
    Down's dW is bit-exact on the GPU's own h and gradient; Gate/Up recompute
    in fp32, so their dW and dX are within 5e-4 of the oracle chain (the
    forward's relative error, carried through SiLU'); W_after bit-exact
    against the oracle's SGD + re-quantization of the GPU's dW."""
    rng = np.random.default_rng(batch * 10 + d + dt)
    G = (rng.standard_normal((f, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((f, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, f)) / np.sqrt(f)).astype(np.float32)
    rows = batch * seq
    x = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.standard_normal((rows, d)).astype(np.float32)
    h, y, dx, dw, wa, loss = gpu.swiglu_normalbp(batch, seq, d, f, dt, scheme, G, U, D, x, g,
                                                 use_target, lr)
    deq = []
    for W in (G, U, D):
        nat, rs, blk = oracle.quantize(dt, scheme, W.shape[0], W.shape[1], W)
        deq.append(oracle.dequant(dt, scheme, W.shape[0], W.shape[1], nat, rs, blk))
    Gd, Ud, Dd = deq
    gp_o, _ = oracle.dense(Gd, x)
    up_o, _ = oracle.dense(Ud, x)
    h_o = oracle.swiglu_product(gp_o, up_o)
    assert rel_l2(h, h_o) <= tol(rows) and rel_l2(y, oracle.dense(Dd, h_o)[0]) <= tol(rows, chain=2)
    gy = oracle.mse_grad(y, g) if use_target else g
    _, gh_o, dwd_o = oracle.backward(Dd, gy, y, h, -1)
    wf = f * d
    assert np.array_equal(dw[2 * wf:].reshape(d, f), dwd_o)
    d_up, d_gate = oracle.swiglu_bwd_product(gp_o, up_o, gh_o)
    _, gxg, dwg = oracle.backward(Gd, d_gate, gp_o, x, -1)
    _, gxu, dwu = oracle.backward(Ud, d_up, up_o, x, -1)
    dx_o = (gxg.astype(np.float64) + gxu.astype(np.float64)).astype(np.float32)
    assert rel_l2(dw[:wf], dwg.ravel()) <= 5e-4 and rel_l2(dw[wf:2 * wf], dwu.ravel()) <= 5e-4
    assert rel_l2(dx, dx_o) <= 5e-4
    if use_target:
        lo = oracle.mse(y, g)
        assert abs(loss - lo) <= 1e-12 * lo
    else:
        assert loss == 0.0
    off = 0
    for W, Wq in zip((G, U, D), deq):
        n = W.size
        if lr == 0.0:
            assert np.array_equal(wa[off:off + n].reshape(W.shape), Wq)
        else:
            nxt = oracle.sgd(Wq, dw[off:off + n].reshape(W.shape), lr)
            n2, rs2, blk2 = oracle.quantize(dt, scheme, W.shape[0], W.shape[1], nxt)
            want = oracle.dequant(dt, scheme, W.shape[0], W.shape[1], n2, rs2, blk2)
            assert np.array_equal(wa[off:off + n].reshape(W.shape), want)
        off += n


@pytest.mark.parametrize("dt", [4, 5])
def test_release_smoke_normalbp_known_answer(gpu, oracle, dt):
    """The reference's packaged check (scripts/release_smoke.py:55-70): 2x2
    identity, x = (0.5, -0.25), MSE target 0, lr 0.1. The reference runs it
    with FP32 weights; the identity and x are exact in FP8, so the forward,
    the loss 0.15625 and dW hold as they are, and the updated weights
    (0.975, 0.0125, 0.0125, 0.99375) are those values re-encoded in the
    FP8 format (the store re-quantizes after SGD, native_codec.cpp:1080-1133)."""
    W = np.eye(2, dtype=np.float32)
    x = np.array([[0.5, -0.25]], np.float32)
    t = np.zeros((1, 2), np.float32)
    pre, post, dx, dw, wa, loss = gpu.dense_normalbp(1, 2, 2, -1, dt, 0, W, x, t, True, 0.1)
    assert post.tolist() == [[0.5, -0.25]] and pre.tolist() == [[0.5, -0.25]]
    assert abs(loss - 0.15625) < 1e-6
    assert dw.tolist() == [[0.25, -0.125], [-0.125, 0.0625]]
    assert dx.tolist() == [[0.5, -0.25]]
    expected = np.array([0.975, 0.0125, 0.0125, 0.99375], np.float32)
    requant = np.array([oracle.decode(dt, oracle.encode(dt, v)) for v in expected], np.float32)
    assert np.array_equal(wa.ravel(), requant)
