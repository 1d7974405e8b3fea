"""Dense backward / SGD contract of the oracle (the NormalBP leaf).

act' (src/cuda/kernels.cu:48-81) is pinned by the compiled reference
activate_deriv_f64 (src/core/activate.cpp:31-63, golden vectors in
tests/golden/backward_cases.npz) and by central differences of the forward
activation. The SGD element rule (native_codec.cpp:1080-1133) is pinned by
WeightStore::apply_sgd of the compiled reference on FormatNone payloads.
dX = W^T d_pre and the per-batch f32 outer product dW (kernels.cu:92-127) are
pinned by numpy f64 formulations, exact-integer cases and central differences
of an f64 forward. The MSE loss and gradient (src/runtime/training.cpp:44-69)
are pinned by their closed forms.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden", "backward_cases.npz")
ACTS = [-1, 0, 1, 2, 3, 4, 5, 6]


def np_act(act, v):
    if act == 0:
        return np.maximum(v, 0.0)
    if act == 1:
        return v / (1.0 + np.exp(-v))
    if act == 2:
        k = 0.7978845608028654
        return 0.5 * v * (1.0 + np.tanh(k * (v + 0.044715 * v ** 3)))
    if act == 3:
        return np.tanh(v)
    if act == 4:
        return 1.0 / (1.0 + np.exp(-v))
    if act == 5:
        return np.where(v < 0, 0.01 * v, v)
    if act == 6:
        return np.where(v < 0, 0.0, v * v)
    return v


def test_act_deriv_matches_reference(oracle):
    z = np.load(GOLD)
    xs = z["act_x"]
    for act in ACTS:
        want = z[f"act_{act + 1}"]
        got = np.array([oracle.act_deriv(act, x) for x in xs])
        assert np.array_equal(got, want, equal_nan=True), act


@pytest.mark.parametrize("act", ACTS)
def test_act_deriv_central_differences(oracle, act):
    rng = np.random.default_rng(act + 5)
    xs = rng.standard_normal(200) * 3
    xs = xs[np.abs(xs) > 1e-3]  # away from the kinks of ReLU / Leaky / ReLU2
    h = 1e-6
    fd = np.array([(oracle.L.or_activate(act, x + h) - oracle.L.or_activate(act, x - h)) / (2 * h)
                   for x in xs])
    got = np.array([oracle.act_deriv(act, x) for x in xs])
    assert np.max(np.abs(got - fd)) < 1e-6, act


def test_sgd_matches_reference_store(oracle):
    z = np.load(GOLD)
    n = int(z["sgd_count"][0])
    for i in range(n):
        dt, rows, cols = z[f"sgd{i}_meta"].tolist()
        native = z[f"sgd{i}_native"]
        w = np.array([oracle.weight_at(dt, native, k) for k in range(rows * cols)], np.float32)
        nxt = oracle.sgd(w, z[f"sgd{i}_dW"], float(z[f"sgd{i}_lr"][0]))
        assert np.array_equal(oracle.pack(dt, nxt), z[f"sgd{i}_after"]), (i, dt, rows, cols)
    assert n == 15


def test_mse_closed_form(oracle):
    rng = np.random.default_rng(3)
    p = rng.standard_normal(1000).astype(np.float32)
    t = rng.standard_normal(1000).astype(np.float32)
    d = p.astype(np.float64) - t.astype(np.float64)
    assert abs(oracle.mse(p, t) - np.mean(d * d)) <= 1e-15 * np.mean(d * d)
    assert np.array_equal(oracle.mse_grad(p, t), (2.0 / p.size * d).astype(np.float32))


def test_backward_exact_integer_case(oracle):
    """Every product and partial sum is an integer below 2^24: dX and dW are
    the integer products, bit for bit."""
    rng = np.random.default_rng(4)
    W = rng.integers(-8, 9, (37, 53)).astype(np.float32)
    x = rng.integers(-8, 9, (5, 53)).astype(np.float32)
    gy = rng.integers(-8, 9, (5, 37)).astype(np.float32)
    pre = rng.standard_normal((5, 37)).astype(np.float32)
    dpre, dx, dw = oracle.backward(W, gy, pre, x, act=-1)
    assert np.array_equal(dpre, gy)
    assert np.array_equal(dx, (gy.astype(np.int64) @ W.astype(np.int64)).astype(np.float32))
    assert np.array_equal(dw, (gy.T.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))


def test_backward_matches_numpy_f64(oracle):
    rng = np.random.default_rng(6)
    W = rng.standard_normal((64, 96)).astype(np.float32)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    gy = rng.standard_normal((3, 64)).astype(np.float32)
    pre = rng.standard_normal((3, 64)).astype(np.float32)
    dpre, dx, dw = oracle.backward(W, gy, pre, x, act=1)
    d64 = np.array([[oracle.act_deriv(1, float(v)) for v in row] for row in pre])
    assert np.array_equal(dpre, (gy.astype(np.float64) * d64).astype(np.float32))
    want = dpre.astype(np.float64) @ W.astype(np.float64)
    assert np.max(np.abs(dx - want) / (np.abs(want) + 1e-30)) < 2 ** -23
    # batch 1 row of the outer product: one rounding of an exact f64 product
    _, _, dw1 = oracle.backward(W, gy[:1], pre[:1], x[:1], act=-1)
    assert np.array_equal(dw1, (gy[0].astype(np.float64)[:, None] * x[0].astype(np.float64)[None, :]).astype(np.float32))
    # several rows: f32 rounding after each row's f64 add
    acc = np.zeros((64, 96), np.float32)
    for b in range(3):
        acc = (acc.astype(np.float64) + np.outer(dpre[b].astype(np.float64), x[b].astype(np.float64))).astype(np.float32)
    assert np.array_equal(dw, acc)


@pytest.mark.parametrize("act", [-1, 1, 2, 3])
def test_backward_central_differences(oracle, act):
    """dX and dW against central differences of L = sum(gy * act(x W^T)),
    evaluated in f64 (the backward gets pre from the same f64 forward)."""
    rng = np.random.default_rng(10 + act)
    out, inn, batch = 6, 9, 2
    W = (rng.standard_normal((out, inn)) / 3).astype(np.float32)
    x = rng.standard_normal((batch, inn)).astype(np.float32)
    gy = rng.standard_normal((batch, out)).astype(np.float32)
    W64, x64, g64 = W.astype(np.float64), x.astype(np.float64), gy.astype(np.float64)

    def loss(Wm, xm):
        return float(np.sum(g64 * np_act(act, xm @ Wm.T)))

    pre = (x64 @ W64.T).astype(np.float32)
    _, dx, dw = oracle.backward(W, gy, pre, x, act=act)
    h = 1e-6
    for b in range(batch):
        for i in range(inn):
            e = np.zeros_like(x64)
            e[b, i] = h
            fd = (loss(W64, x64 + e) - loss(W64, x64 - e)) / (2 * h)
            assert abs(dx[b, i] - fd) < 1e-4 * (1 + abs(fd)), (b, i)
    for o in range(out):
        for i in range(inn):
            e = np.zeros_like(W64)
            e[o, i] = h
            fd = (loss(W64 + e, x64) - loss(W64 - e, x64)) / (2 * h)
            assert abs(dw[o, i] - fd) < 1e-4 * (1 + abs(fd)), (o, i)


def test_swiglu_bwd_product_central_differences(oracle):
    """d_up and d_gate against central differences of h = SiLU(g) * u in f64
    (the rounding points of the product rule aside: relative 1e-6)."""
    rng = np.random.default_rng(12)
    g = (rng.standard_normal(300) * 3).astype(np.float32)
    u = rng.standard_normal(300).astype(np.float32)
    gh = rng.standard_normal(300).astype(np.float32)
    d_up, d_gate = oracle.swiglu_bwd_product(g, u, gh)
    g64, u64, h = g.astype(np.float64), u.astype(np.float64), 1e-6

    def silu(v):
        return v / (1.0 + np.exp(-v))

    fd_g = gh * u64 * (silu(g64 + h) - silu(g64 - h)) / (2 * h)
    fd_u = gh * silu(g64)
    assert np.max(np.abs(d_gate - fd_g) / (np.abs(fd_g) + 1e-6)) < 1e-5
    assert np.max(np.abs(d_up - fd_u) / (np.abs(fd_u) + 1e-6)) < 1e-6
