"""ctypes access to tests/cpp/libapi_probe.so, the C++ caller of the
layer/weights API (include/welvet/*.hpp) built against libwelvet.so."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "cpp", "libapi_probe.so")

_i, _sz, _d = ctypes.c_int, ctypes.c_size_t, ctypes.c_double
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_szp = ctypes.POINTER(ctypes.c_size_t)
_cp = ctypes.c_char_p
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        import pywelvet as pw
        pw.lib()  # libwelvet.so first, from its in-tree path
        if not os.path.exists(PATH):
            raise RuntimeError(f"{PATH} is missing: build it with `make -f tests/cpp/Makefile`")
        L = ctypes.CDLL(PATH)
        L.probe_dense_forward.argtypes = [_i] * 7 + [_fp] * 4 + [_cp, _i]
        L.probe_store.argtypes = [_i] * 4 + [_fp, _u8p, _sz, _szp, _fp, _u8p, _sz, _dp, _fp, _cp, _i]
        L.probe_session.argtypes = [_i] * 5 + [_fp, _dp, _sz, _fp, _fp, _fp, _cp, _i]
        L.probe_dense_backward.argtypes = [_i] * 6 + [_fp] * 5 + [_d, _fp, _cp, _i]
        L.probe_swiglu.argtypes = [_i] * 4 + [_fp] * 6 + [_cp, _i]
        L.probe_mha.argtypes = [_i] * 9 + [_fp] * 7 + [_cp, _i]
        L.probe_dtype.argtypes = [_i, _cp, _i]
        _LIB = L
    return _LIB


def f(a):
    return None if a is None else np.ascontiguousarray(a, np.float32).ctypes.data_as(_fp)


class ProbeError(RuntimeError):
    def __init__(self, code, msg):
        self.code = code
        super().__init__(f"C++ API status {code}: {msg}")


def call(name, *args):
    """Runs probe `name`; returns its status code and message."""
    msg = ctypes.create_string_buffer(256)
    code = getattr(lib(), name)(*args, msg, 256)
    return code, msg.value.decode(errors="replace")


def check(name, *args):
    code, msg = call(name, *args)
    if code != 0:
        raise ProbeError(code, msg)


def dense_forward(in_dim, out_dim, act, dtype, scheme, W, x, repeats=1):
    batch = x.shape[0]
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    pre = np.zeros((batch, out_dim), np.float32)
    post = np.zeros_like(pre)
    check("probe_dense_forward", in_dim, out_dim, act, dtype, scheme, batch, repeats, f(W), f(x),
          f(pre), f(post))
    return pre, post


def store(rows, cols, dtype, scheme, W):
    W = np.ascontiguousarray(W, np.float32)
    n = rows * cols
    native = np.zeros(n, np.uint8)
    nlen = ctypes.c_size_t()
    rs = np.zeros(rows, np.float32)
    nb = (cols + 31) // 32
    blk = np.zeros(rows * nb, np.uint8)
    rows64 = np.zeros((rows, cols), np.float64)
    exported = np.zeros((rows, cols), np.float32)
    check("probe_store", rows, cols, dtype, scheme, f(W), native.ctypes.data_as(_u8p), n,
          ctypes.byref(nlen), f(rs), blk.ctypes.data_as(_u8p), blk.size,
          rows64.ctypes.data_as(_dp), exported.ctypes.data_as(_fp))
    return native[: nlen.value], rs, blk, rows64, exported


def session(batch, in_dim, out_dim, act, dtype, W, x, bias=None):
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float64)
    pre = np.zeros((batch, out_dim), np.float32)
    post = np.zeros_like(pre)
    check("probe_session", batch, in_dim, out_dim, act, dtype, f(W),
          None if b is None else b.ctypes.data_as(_dp), 0 if b is None else b.size, f(x), f(pre),
          f(post))
    return pre, post


def dense_backward(in_dim, out_dim, act, dtype, scheme, W, x, gy, lr=0.0):
    batch = x.shape[0]
    gi = np.zeros((batch, in_dim), np.float32)
    gw = np.zeros((out_dim, in_dim), np.float32)
    wa = np.zeros((out_dim, in_dim), np.float32)
    check("probe_dense_backward", in_dim, out_dim, act, dtype, scheme, batch, f(W), f(x), f(gy),
          f(gi), f(gw), lr, f(wa))
    return gi, gw, wa


def swiglu(in_dim, inter, dtype, G, U, D, x):
    rows = x.shape[0]
    h = np.zeros((rows, inter), np.float32)
    y = np.zeros((rows, in_dim), np.float32)
    check("probe_swiglu", in_dim, inter, dtype, rows, f(G), f(U), f(D), f(x), f(h), f(y))
    return h, y


def mha(B, S, d, H, KVH, msl, mask, pos, dtype, Q, K, V, O, x):
    hd = d // H
    attn = np.zeros((B * S, H * hd), np.float32)
    y = np.zeros((B * S, d), np.float32)
    check("probe_mha", B, S, d, H, KVH, msl, mask, pos, dtype, f(Q), f(K), f(V), f(O), f(x),
          f(attn), f(y))
    return attn, y
