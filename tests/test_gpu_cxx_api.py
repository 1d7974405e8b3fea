"""The C++ layer/weights API (include/welvet/*.hpp) on the GPU, called from
a C++ caller that includes only those headers (tests/cpp/api_probe.cpp),
against the oracle:
  * WeightStore::make / decode_row_f64 / export_f32: the payload equals the
    oracle's quantization byte for byte, the decoded rows its dequantization;
  * dense::new_layer + forward_f32 (reference dense.cpp:10-86), repeated
    forwards reusing the device weights, sessions (session.cpp:12-82),
    backward_f32 + apply_grad_sgd (dense.cpp:88-232);
  * swiglu::forward and mha::forward against the oracle's layer chains.
Tolerances as in test_gpu_dense and test_gpu_swiglu_mha."""
import numpy as np
import pytest

import cxx_probe
from test_gpu_dense import rel_l2, tol
from test_gpu_swiglu_mha import oracle_dequant, oracle_mha, oracle_swiglu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt,scheme", [(4, 0), (5, 2), (16, 3), (4, 1), (16, 0)])
@pytest.mark.parametrize("rows,cols", [(7, 33), (64, 96), (129, 1000)])
def test_store_make_decode_export(gpu, oracle, dt, scheme, rows, cols):
    rng = np.random.default_rng(rows * 3 + cols + dt + scheme)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    native, rs, blk, rows64, exported = cxx_probe.store(rows, cols, dt, scheme, W)
    o_native, o_rs, o_blk = oracle.quantize(dt, scheme, rows, cols, W)
    assert np.array_equal(native, o_native)
    if scheme in (1, 2):
        assert np.array_equal(rs, o_rs)
    if scheme == 3:
        assert np.array_equal(blk, o_blk)
    Wd = oracle.dequant(dt, scheme, rows, cols, o_native, o_rs, o_blk)
    assert np.array_equal(exported, Wd)
    assert np.array_equal(rows64, Wd.astype(np.float64))


@pytest.mark.parametrize("dt,scheme", [(4, 0), (5, 2), (16, 3), (4, 2)])
@pytest.mark.parametrize("batch,in_dim,out_dim,act", [(1, 512, 512, -1), (3, 96, 160, 1),
                                                      (16, 256, 320, 0), (40, 1024, 768, 2)])
def test_new_layer_forward_matches_oracle(gpu, oracle, dt, scheme, batch, in_dim, out_dim, act):
    rng = np.random.default_rng(batch + in_dim + dt * 7 + scheme)
    W = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    pre, post = cxx_probe.dense_forward(in_dim, out_dim, act, dt, scheme, W, x, repeats=2)
    Wd = oracle_dequant(oracle, dt, scheme, W)
    o_pre, o_post = oracle.dense(Wd, x, act)
    assert rel_l2(pre, o_pre) <= tol(batch)
    assert rel_l2(post, o_post) <= tol(batch)


def test_release_smoke_known_answer(gpu):
    """The 2x2 known answer of the reference's release smoke check
    (scripts/release_smoke.py:55-70), through new_layer + forward_f32 with
    E4M3 codes that hold the identity exactly: y = x."""
    W = np.array([[1, 0], [0, 1]], np.float32)
    x = np.array([[3.0, -5.0]], np.float32)
    pre, post = cxx_probe.dense_forward(2, 2, -1, 4, 0, W, x)
    assert np.array_equal(pre, x) and np.array_equal(post, x)


@pytest.mark.parametrize("batch,act,bias", [(1, -1, False), (8, 1, True), (64, 3, True)])
def test_session_matches_oracle(gpu, oracle, batch, act, bias):
    rng = np.random.default_rng(batch + act)
    in_dim, out_dim = 256, 384
    W = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
    b = rng.standard_normal(out_dim) if bias else None
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    pre, post = cxx_probe.session(batch, in_dim, out_dim, act, 4, W, x, b)
    Wd = oracle_dequant(oracle, 4, 0, W)
    o_pre, o_post = oracle.dense(Wd, x, act, b)
    assert rel_l2(pre, o_pre) <= tol(batch)
    assert rel_l2(post, o_post) <= tol(batch)


@pytest.mark.parametrize("dt,scheme,act", [(4, 2, -1), (16, 3, 0), (5, 0, -1)])
def test_backward_and_sgd(gpu, oracle, dt, scheme, act):
    """backward_f32 gives the oracle's dW bit for bit (Linear / ReLU: act' is
    exact) and dX within f64 summation order; apply_grad_sgd then gives the
    oracle's SGD plus re-quantization of the store."""
    rng = np.random.default_rng(dt + scheme + act + 3)
    batch, in_dim, out_dim, lr = 3, 192, 130, 0.05
    W = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    gy = rng.standard_normal((batch, out_dim)).astype(np.float32)
    gi, gw, w_after = cxx_probe.dense_backward(in_dim, out_dim, act, dt, scheme, W, x, gy, lr)
    Wd = oracle_dequant(oracle, dt, scheme, W)
    pre, _ = cxx_probe.dense_forward(in_dim, out_dim, act, dt, scheme, W, x)
    _, o_dx, o_dw = oracle.backward(Wd, gy, pre, x, act)
    assert np.array_equal(gw, o_dw)
    assert rel_l2(gi, o_dx) <= 1e-6
    stepped = (Wd.astype(np.float64) - lr * o_dw.astype(np.float64)).astype(np.float32)
    want = oracle_dequant(oracle, dt, scheme, stepped)
    assert np.array_equal(w_after, want)


@pytest.mark.parametrize("dt", [16, 4])
@pytest.mark.parametrize("rows,d,inter", [(1, 128, 352), (16, 256, 704), (40, 96, 200)])
def test_swiglu_forward_matches_oracle(gpu, oracle, dt, rows, d, inter):
    rng = np.random.default_rng(rows + d + dt)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    h, y = cxx_probe.swiglu(d, inter, dt, G, U, D, x)
    oh, oy = oracle_swiglu(oracle, dt, 0, G, U, D, x)
    assert rel_l2(h, oh) <= tol(rows)
    assert rel_l2(y, oy) <= tol(rows, chain=2)


@pytest.mark.parametrize("B,S,d,H,KVH,msl,mask,pos", [
    (2, 8, 64, 4, 4, 8, 1, 0),
    (2, 64, 256, 4, 2, 64, 1, 0),   # matrix-core attention, GQA
    (1, 24, 64, 4, 2, 24, 2, 2),    # bidirectional, ALiBi
])
def test_mha_forward_matches_oracle(gpu, oracle, B, S, d, H, KVH, msl, mask, pos):
    dt = 5
    hd = d // H
    rng = np.random.default_rng(B * 11 + S + d)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    attn, y = cxx_probe.mha(B, S, d, H, KVH, msl, mask, pos, dt, Q, K, V, O, x)
    oattn, oy = oracle_mha(oracle, dt, 0, Q, K, V, O, x, B, S, H, KVH, hd, msl, mask, pos)
    assert rel_l2(attn, oattn) <= 1e-4
    assert rel_l2(y, oy) <= 1e-4
