"""Dense / SwiGLU / attention contract of the oracle.

Dense (src/cuda/kernels.cu:130-161, :895-906): f64 serial accumulation, one
f32 rounding, then bias in f64 with pre re-rounded, activation on the f64
value. Pinned by exact small-integer cases (every partial sum exact, so the
result is fixed bit-for-bit), the 2x2 identity known answer of
scripts/release_smoke.py:55-70, and brute force against math.fsum.
Attention (kernels.cu:470-631) is checked against a numpy formulation that
indexes the KV ring in closed form (p = last - ((last - k_pos) mod msl))
instead of simulating the ring buffer as the oracle does.
"""
import math

import numpy as np
import pytest


def test_release_smoke_identity_known_answer(oracle):
    W = np.eye(2, dtype=np.float32)
    x = np.array([[0.5, -0.25]], np.float32)
    pre, post = oracle.dense(W, x)
    assert pre.tolist() == [[0.5, -0.25]] and post.tolist() == [[0.5, -0.25]]


def test_dense_exact_integer_case(oracle):
    rng = np.random.default_rng(1)
    W = rng.integers(-8, 9, (37, 53)).astype(np.float32)
    x = rng.integers(-8, 9, (3, 53)).astype(np.float32)
    pre, post = oracle.dense(W, x)
    want = (x.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32)
    assert np.array_equal(pre, want) and np.array_equal(post, want)


def test_dense_brute_force_fsum(oracle):
    rng = np.random.default_rng(2)
    W = rng.standard_normal((11, 29)).astype(np.float32)
    x = rng.standard_normal((2, 29)).astype(np.float32)
    pre, _ = oracle.dense(W, x)
    for b in range(2):
        for o in range(11):
            exact = math.fsum(float(W[o, k]) * float(x[b, k]) for k in range(29))
            assert abs(float(pre[b, o]) - exact) <= 2e-7 * max(1.0, abs(exact))


def test_dense_bias_and_activation_rules(oracle):
    W = np.array([[1.0, 2.0], [-3.0, 0.5], [0.25, 0.25]], np.float32)
    x = np.array([[1.0, -1.0]], np.float32)
    bias = np.array([0.1, -0.2])  # shorter than out: row 2 has no bias
    pre, post = oracle.dense(W, x, act=0, bias=bias)  # ReLU
    y = np.array([-1.0, -3.5, 0.0])
    v = y + np.array([0.1, -0.2, 0.0])
    assert np.array_equal(pre[0], v.astype(np.float32))
    assert np.array_equal(post[0], np.maximum(v, 0).astype(np.float32))
    # SiLU on the f64 value
    pre, post = oracle.dense(W, x, act=1)
    assert np.array_equal(pre[0], y.astype(np.float32))
    assert np.allclose(post[0], y / (1 + np.exp(-y)), rtol=1e-7, atol=1e-30)


def test_activation_ids(oracle):
    xs = [-2.0, -0.5, 0.0, 0.5, 3.0]
    for x in xs:
        assert oracle.activate(-1, x) == x
        assert oracle.activate(0, x) == max(x, 0.0)
        assert oracle.activate(5, x) == (0.01 * x if x < 0 else x)
        assert oracle.activate(6, x) == (0.0 if x < 0 else x * x)
        assert oracle.activate(3, x) == math.tanh(x)
        assert abs(oracle.activate(4, x) - 1 / (1 + math.exp(-x))) < 1e-15
        assert abs(oracle.activate(1, x) - x / (1 + math.exp(-x))) < 1e-15
        k = math.sqrt(2 / math.pi)
        assert abs(oracle.activate(2, x) - 0.5 * x * (1 + math.tanh(k * (x + 0.044715 * x ** 3)))) < 1e-14


def test_swiglu_product(oracle):
    rng = np.random.default_rng(3)
    g = rng.standard_normal(257).astype(np.float32)
    u = rng.standard_normal(257).astype(np.float32)
    h = oracle.swiglu_product(g, u)
    gd = g.astype(np.float64)
    silu = (gd / (1 + np.exp(-gd))).astype(np.float32)
    assert np.array_equal(h, (silu.astype(np.float64) * u.astype(np.float64)).astype(np.float32))


def rope(vec, pos, heads, hd, theta=10000.0):
    out = vec.astype(np.float64).copy()
    half = hd // 2
    for h in range(heads):
        for d in range(half):
            ang = pos / theta ** (2 * d / hd)
            a0, a1 = out[h * hd + d], out[h * hd + d + half]
            out[h * hd + d] = a0 * math.cos(ang) - a1 * math.sin(ang)
            out[h * hd + d + half] = a0 * math.sin(ang) + a1 * math.cos(ang)
    return out


def allow(qp, kp, mask, window, msl, prefix):
    if mask == 2:
        return True
    if mask == 3:
        w = window if window > 0 else msl
        return kp <= qp and kp >= qp - w + 1
    if mask == 4:
        return (qp < prefix and kp < prefix) or kp <= qp
    return kp <= qp


def attention_closed_form(q, k, v, B, S, H, KVH, hd, msl, mask=1, pos=0, softmax=0, window=0,
                          prefix=0):
    T = B * S
    qd, kvd = H * hd, KVH * hd
    rot = pos in (0, 3)
    qr = np.stack([rope(q[t], t, H, hd) if rot else q[t].astype(np.float64) for t in range(T)])
    kr = np.stack([rope(k[t], t, KVH, hd) if rot else k[t].astype(np.float64) for t in range(T)])
    out = np.zeros((T, qd))
    scale = 1 / math.sqrt(hd)
    for b in range(B):
        last = b * S + S - 1
        for s in range(S):
            qp = b * S + s
            for h in range(H):
                kvh = h // (H // KVH)
                sc, ps = [], []
                for kp in range(last + 1):
                    if not allow(qp, kp, mask, window, msl, prefix):
                        continue
                    p = last - ((last - kp) % msl)
                    val = qr[qp, h * hd:(h + 1) * hd] @ kr[p, kvh * hd:(kvh + 1) * hd] * scale
                    if pos in (2, 3):
                        val += -(2.0 ** (-(h + 1) * 8.0 / H)) * abs(qp - kp)
                    sc.append(val)
                    ps.append(p)
                if not sc:
                    continue
                sc = np.array(sc)
                w = 1 / (1 + np.exp(-sc)) if softmax == 1 else np.exp(sc - sc.max()) / np.exp(sc - sc.max()).sum()
                out[qp, h * hd:(h + 1) * hd] = sum(wi * v[p, kvh * hd:(kvh + 1) * hd] for wi, p in zip(w, ps))
    return out.astype(np.float32)


@pytest.mark.parametrize("B,S,msl,mask,pos,softmax,H,KVH", [
    (2, 4, 4, 1, 0, 0, 2, 2),   # ring exactly one sequence long
    (3, 3, 5, 1, 0, 0, 2, 1),   # ring wraps mid-sequence, GQA
    (2, 4, 6, 2, 1, 0, 2, 2),   # bidirectional, no RoPE
    (2, 3, 4, 3, 2, 0, 2, 2),   # sliding window, ALiBi
    (2, 3, 8, 4, 3, 1, 4, 2),   # prefix LM, RoPE+ALiBi, sigmoid
])
def test_attention_matches_closed_form_ring(oracle, B, S, msl, mask, pos, softmax, H, KVH):
    hd = 4
    rng = np.random.default_rng(B * 100 + S * 10 + mask)
    T = B * S
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    k = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    v = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    window, prefix = (2, 0) if mask == 3 else (0, 2 if mask == 4 else 0)
    got = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos, softmax, window, prefix)
    want = attention_closed_form(q, k, v, B, S, H, KVH, hd, msl, mask, pos, softmax, window, prefix)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mask,pos", [(0, 0), (5, 0), (9, 1), (-1, 4), (5, -2)])
def test_attention_out_of_range_kinds(oracle, mask, pos):
    """The reference casts mask and position kinds through unchecked
    (c_abi.cpp:805-806); its kernel treats masks other than 2-4 as causal and
    applies RoPE / ALiBi only for kinds 0, 3 / 2, 3 (kernels.cu:470-485,
    550-551)."""
    B, S, msl, H, KVH, hd = 2, 4, 4, 2, 2, 4
    rng = np.random.default_rng(77 + mask)
    T = B * S
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    k = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    v = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    got = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos)
    want_pos = pos if pos in (0, 1, 2, 3) else 1
    want = attention_closed_form(q, k, v, B, S, H, KVH, hd, msl, 1, want_pos)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_attention_threads_bit_identical(oracle):
    """Heads spread over threads compute the same bits as one thread."""
    B, S, msl, H, KVH, hd = 3, 6, 8, 8, 2, 8
    rng = np.random.default_rng(3)
    T = B * S
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    k = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    v = rng.standard_normal((T, KVH * hd)).astype(np.float32)
    for mask, pos in ((1, 0), (2, 3), (4, 2)):
        one = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos, prefix_len=3)
        for th in (2, 3, 8):
            many = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos, prefix_len=3,
                                        threads=th)
            assert np.array_equal(one, many)
