"""Writes the golden vectors for the Dense backward / SGD path.

Run in a container that has the reference tree: it builds oracle/_ref/libref.so
from the reference's own host sources (oracle/Makefile: float_codecs.cpp,
native_codec.cpp, store.cpp, activate.cpp) and records what that compiled code
returns:

  backward_cases.npz
    act_x, act_<id>    activate_deriv_f64 (src/core/activate.cpp:31-63) of each
                       activation id -1..6 at the inputs act_x (f64)
    sgd<i>_meta        (dtype, rows, cols)
    sgd<i>_native      WeightStore::make payload of sgd<i>_W
    sgd<i>_dW, _lr     the f64 gradient and learning rate
    sgd<i>_after       the payload after WeightStore::apply_sgd
                       (native_codec.cpp:1080-1133)

The file is data only (inputs and expected outputs).
"""
import ctypes
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", ".."))
LIB = os.path.join(ROOT, "oracle", "_ref", "libref.so")
_u8p = ctypes.POINTER(ctypes.c_uint8)
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.ref_act_deriv.restype = ctypes.c_double
    lib.ref_act_deriv.argtypes = [ctypes.c_int, ctypes.c_double]
    lib.ref_store_make.restype = ctypes.c_int
    lib.ref_store_make.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _fp, _u8p,
                                   ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                   ctypes.POINTER(ctypes.c_float)]
    lib.ref_store_apply_sgd.restype = ctypes.c_int
    lib.ref_store_apply_sgd.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _u8p,
                                        ctypes.c_size_t, _dp, ctypes.c_double]
    return lib


def act_inputs():
    xs = [0.0, -0.0, 1e-300, -1e-300, 1e-8, -1e-8, 0.5, -0.5, 1.0, -1.0, 3.0, -3.0, 20.0, -20.0,
          40.0, -40.0, 700.0, -700.0, 710.0, -710.0, 1e6, -1e6]
    rng = np.random.default_rng(31)
    xs.extend((rng.standard_normal(200) * 4).tolist())
    return np.array(xs, dtype=np.float64)


def sgd_inputs():
    cases = []
    rng = np.random.default_rng(11)
    for dt in (4, 5, 16):
        for rows, cols, spread, lr in [(3, 5, 1.0, 0.1), (7, 33, 2.0, 1.0), (4, 64, 0.05, 0.01),
                                       (5, 7, 200.0, 3.0), (2, 31, 1.0, -0.25)]:
            W = (rng.standard_normal(rows * cols) * spread).astype(np.float32)
            dW = (rng.standard_normal(rows * cols) * spread * 4).astype(np.float32)
            cases.append((dt, rows, cols, W, dW, lr))
    return cases


def main():
    subprocess.check_call(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile"), "ref"])
    lib = _lib()
    out = {}
    xs = act_inputs()
    out["act_x"] = xs
    for act in range(-1, 7):
        out[f"act_{act + 1}"] = np.array([lib.ref_act_deriv(act, float(x)) for x in xs])
    cases = sgd_inputs()
    for i, (dt, rows, cols, W, dW, lr) in enumerate(cases):
        cap = rows * cols + 8
        native = np.zeros(cap, dtype=np.uint8)
        nlen = ctypes.c_size_t(0)
        scale = ctypes.c_float(0)
        rc = lib.ref_store_make(dt, rows, cols, W.ctypes.data_as(_fp), native.ctypes.data_as(_u8p),
                                cap, ctypes.byref(nlen), ctypes.byref(scale))
        assert rc == 0, rc
        native = native[: nlen.value].copy()
        after = native.copy()
        d64 = dW.astype(np.float64)
        rc = lib.ref_store_apply_sgd(dt, rows, cols, after.ctypes.data_as(_u8p), after.size,
                                     d64.ctypes.data_as(_dp), lr)
        assert rc == 0, rc
        out[f"sgd{i}_meta"] = np.array([dt, rows, cols], dtype=np.int32)
        out[f"sgd{i}_W"] = W
        out[f"sgd{i}_native"] = native
        out[f"sgd{i}_dW"] = dW
        out[f"sgd{i}_lr"] = np.array([lr])
        out[f"sgd{i}_after"] = after
    out["sgd_count"] = np.array([len(cases)], dtype=np.int32)
    np.savez(os.path.join(HERE, "backward_cases.npz"), **out)


if __name__ == "__main__":
    sys.exit(main())
