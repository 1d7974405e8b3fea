"""ctypes binding of the CPU oracle (oracle/liboracle.so) for the tests."""
import ctypes
import os

import numpy as np

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i = ctypes.c_int


def _f(a):
    return None if a is None else a.ctypes.data_as(_fp)


def _u8(a):
    return None if a is None else a.ctypes.data_as(_u8p)


class Oracle:
    def __init__(self, path=None):
        L = ctypes.CDLL(path or os.path.join(ROOT, "oracle", "liboracle.so"))
        L.or_encode.restype = ctypes.c_uint8
        L.or_encode.argtypes = [_i, ctypes.c_float]
        L.or_decode.restype = ctypes.c_float
        L.or_decode.argtypes = [_i, ctypes.c_uint8]
        L.or_sweep_digest.argtypes = [_i, ctypes.c_uint32, ctypes.c_uint32, _i64p, _i]
        L.or_native_bytes.restype = ctypes.c_size_t
        L.or_native_bytes.argtypes = [_i, ctypes.c_int64]
        L.or_pack.argtypes = [_i, _fp, ctypes.c_int64, _u8p]
        L.or_weight_at.restype = ctypes.c_float
        L.or_weight_at.argtypes = [_i, _u8p, ctypes.c_int64]
        L.or_e8m0_exponent.restype = _i
        L.or_e8m0_exponent.argtypes = [ctypes.c_float, ctypes.c_float]
        L.or_maxrep.restype = ctypes.c_float
        L.or_maxrep.argtypes = [_i]
        L.or_quantize.argtypes = [_i, _i, _i, _i, _fp, _u8p, _fp, _u8p]
        L.or_dequant.argtypes = [_i, _i, _i, _i, _u8p, _fp, _u8p, _fp]
        L.or_activate.restype = ctypes.c_double
        L.or_activate.argtypes = [_i, ctypes.c_double]
        L.or_dense_forward.argtypes = [_i, _i, _i, _i, _fp, _dp, _i, _fp, _fp, _fp, _i]
        L.or_swiglu_product.argtypes = [_fp, _fp, _fp, ctypes.c_int64]
        L.or_mha_attention.argtypes = [_fp, _fp, _fp, _fp] + [_i] * 12 + [ctypes.c_double] * 2
        L.or_mha_attention_mt.argtypes = ([_fp, _fp, _fp, _fp] + [_i] * 12
                                          + [ctypes.c_double] * 2 + [_i])
        L.or_act_deriv.restype = ctypes.c_double
        L.or_act_deriv.argtypes = [_i, ctypes.c_double]
        L.or_dense_backward.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _i]
        L.or_mse.restype = ctypes.c_double
        L.or_mse.argtypes = [ctypes.c_int64, _fp, _fp]
        L.or_mse_grad.argtypes = [ctypes.c_int64, _fp, _fp, _fp]
        L.or_sgd.argtypes = [ctypes.c_int64, _fp, _fp, ctypes.c_double, _fp]
        L.or_swiglu_bwd_product.argtypes = [_fp, _fp, _fp, _fp, _fp, ctypes.c_int64]
        L.or_cpu_dense_bench.restype = ctypes.c_double
        L.or_cpu_dense_bench.argtypes = [_i, _i, _i, _i, _i, _u8p, _fp, _u8p, _fp, _fp, _i, _i, _i,
                                         _dp]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_fmt_block_elems.restype = _i
        L.or_fmt_block_elems.argtypes = [_i]
        L.or_fmt_block_bytes.restype = _i
        L.or_fmt_block_bytes.argtypes = [_i]
        L.or_fmt_quantize.restype = _i
        L.or_fmt_quantize.argtypes = [_i, ctypes.c_int64, _fp, _u8p]
        L.or_fmt_dequant.restype = _i
        L.or_fmt_dequant.argtypes = [_i, ctypes.c_int64, _u8p, _fp]
        self.L = L

    def encode(self, dtype, x):
        return self.L.or_encode(dtype, float(x))

    def decode(self, dtype, c):
        return self.L.or_decode(dtype, int(c))

    def encode_array(self, dtype, xs):
        return np.array([self.L.or_encode(dtype, float(x)) for x in np.asarray(xs, np.float32)],
                        dtype=np.uint8)

    def sweep(self, dtype, first=0, n=4096, threads=None):
        out = np.zeros(2 * n, np.int64)
        self.L.or_sweep_digest(dtype, first, n, out.ctypes.data_as(_i64p),
                               threads or min(8, os.cpu_count() or 1))
        return out.reshape(n, 2)

    def pack(self, dtype, W):
        W = np.ascontiguousarray(W, np.float32).ravel()
        out = np.zeros(self.L.or_native_bytes(dtype, W.size), np.uint8)
        self.L.or_pack(dtype, _f(W), W.size, _u8(out))
        return out

    def weight_at(self, dtype, native, i):
        return self.L.or_weight_at(dtype, _u8(native), i)

    def quantize(self, dtype, scheme, rows, cols, W):
        W = np.ascontiguousarray(W, np.float32)
        native = np.zeros(self.L.or_native_bytes(dtype, rows * cols), np.uint8)
        rs = np.zeros(rows, np.float32)
        blk = np.zeros(rows * ((cols + 31) // 32), np.uint8)
        self.L.or_quantize(dtype, scheme, rows, cols, _f(W), _u8(native), _f(rs), _u8(blk))
        return native, rs, blk

    def dequant(self, dtype, scheme, rows, cols, native, rs, blk):
        out = np.zeros((rows, cols), np.float32)
        self.L.or_dequant(dtype, scheme, rows, cols, _u8(native), _f(rs), _u8(blk), _f(out))
        return out

    def dense(self, W, x, act=-1, bias=None, threads=8):
        W = np.ascontiguousarray(W, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        out, in_dim = W.shape
        batch = x.shape[0]
        pre = np.zeros((batch, out), np.float32)
        post = np.zeros((batch, out), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        self.L.or_dense_forward(batch, in_dim, out, act, _f(W),
                                None if b is None else b.ctypes.data_as(_dp),
                                0 if b is None else b.size, _f(x), _f(pre), _f(post), threads)
        return pre, post

    def swiglu_product(self, g, u):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.zeros_like(g)
        self.L.or_swiglu_product(_f(g), _f(u), _f(h), g.size)
        return h

    def mha_attention(self, q, k, v, batch, seq, heads, kv_heads, hd, msl, mask=1, pos=0,
                      softmax=0, window=0, prefix_len=0, window_causal=1, theta=10000.0,
                      scale=0.0, threads=1):
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        out = np.zeros((batch * seq, heads * hd), np.float32)
        self.L.or_mha_attention_mt(_f(q), _f(k), _f(v), _f(out), batch, seq, heads, kv_heads, hd,
                                   msl, mask, pos, softmax, window, prefix_len, window_causal,
                                   theta, scale, threads)
        return out

    def activate(self, act, x):
        return self.L.or_activate(act, float(x))

    def act_deriv(self, act, x):
        return self.L.or_act_deriv(act, float(x))

    def backward(self, W, gy, pre, x, act=-1, threads=8):
        """dpre, dX, dW of the reference NormalBP contract (W dequantized f32)."""
        W = np.ascontiguousarray(W, np.float32)
        gy = np.ascontiguousarray(gy, np.float32)
        pre = np.ascontiguousarray(pre, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        out, in_dim = W.shape
        batch = x.shape[0]
        dpre = np.zeros((batch, out), np.float32)
        dx = np.zeros((batch, in_dim), np.float32)
        dw = np.zeros((out, in_dim), np.float32)
        self.L.or_dense_backward(batch, in_dim, out, act, _f(W), _f(gy), _f(pre), _f(x), _f(dpre),
                                 _f(dx), _f(dw), threads)
        return dpre, dx, dw

    def mse(self, pred, target):
        p = np.ascontiguousarray(pred, np.float32)
        t = np.ascontiguousarray(target, np.float32)
        return self.L.or_mse(p.size, _f(p), _f(t))

    def mse_grad(self, pred, target):
        p = np.ascontiguousarray(pred, np.float32)
        t = np.ascontiguousarray(target, np.float32)
        g = np.zeros_like(p)
        self.L.or_mse_grad(p.size, _f(p), _f(t), _f(g))
        return g

    def sgd(self, w, dw, lr):
        w = np.ascontiguousarray(w, np.float32)
        dw = np.ascontiguousarray(dw, np.float32)
        nxt = np.zeros_like(w)
        self.L.or_sgd(w.size, _f(w), _f(dw), float(lr), _f(nxt))
        return nxt

    def swiglu_bwd_product(self, g, u, gh):
        g, u, gh = (np.ascontiguousarray(a, np.float32) for a in (g, u, gh))
        d_up, d_gate = np.zeros_like(g), np.zeros_like(g)
        self.L.or_swiglu_bwd_product(_f(g), _f(u), _f(gh), _f(d_up), _f(d_gate), g.size)
        return d_up, d_gate

    # --- packed block formats (oracle/formats.c) ---
    def f32_to_f16(self, x):
        return np.array([self.L.or_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()],
                        np.uint16)

    def f16_to_f32(self, h):
        return np.array([self.L.or_f16_to_f32(int(v)) for v in np.asarray(h, np.uint16).ravel()],
                        np.float32)

    def fmt_block(self, fmt):
        return self.L.or_fmt_block_elems(fmt), self.L.or_fmt_block_bytes(fmt)

    def fmt_quantize(self, fmt, W):
        W = np.ascontiguousarray(W, np.float32)
        qk, bb = self.fmt_block(fmt)
        out = np.zeros(W.size // qk * bb, np.uint8)
        assert self.L.or_fmt_quantize(fmt, W.size, _f(W), _u8(out)) == 0
        return out

    def fmt_dequant(self, fmt, blocks, shape):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        out = np.zeros(shape, np.float32)
        assert self.L.or_fmt_dequant(fmt, out.size, _u8(blocks), _f(out)) == 0
        return out
