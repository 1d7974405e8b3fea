"""Writes the golden vectors for the codec / FormatNone-store path.

Run in a container that has the reference tree: it builds oracle/_ref/libref.so
from the reference's own host sources (float_codecs.cpp, native_codec.cpp,
store.cpp — see oracle/Makefile) and records what that compiled code returns:

  codec_tables.npz   decode tables (f32 bits) for E4M3 / E5M2 (256) and FP4 (16)
  codec_sweep.npz    per-format digests of the encoder over all 2^32 f32 inputs,
                     4096 chunks of 2^20 patterns: (sum code, sum code*low20)
  codec_samples.npz  edge-case inputs (f32 bits) and their reference codes
  store_cases.npz    WeightStore::make payloads + export_f32 for odd shapes

The files are data only (inputs and expected outputs).
"""
import ctypes
import os
import subprocess
import sys
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", ".."))
LIB = os.path.join(ROOT, "oracle", "_ref", "libref.so")
DTYPES = {"e4m3": 4, "e5m2": 5, "fp4": 16}
N_CHUNKS = 4096


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.ref_enc.restype = ctypes.c_uint8
    lib.ref_enc.argtypes = [ctypes.c_int, ctypes.c_float]
    lib.ref_dec.restype = ctypes.c_float
    lib.ref_dec.argtypes = [ctypes.c_int, ctypes.c_uint8]
    lib.ref_sweep_digest.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.POINTER(ctypes.c_int64)]
    lib.ref_store_make.restype = ctypes.c_int
    lib.ref_store_make.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8),
                                   ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                   ctypes.POINTER(ctypes.c_float)]
    lib.ref_store_export.restype = ctypes.c_int
    lib.ref_store_export.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_uint8), ctypes.c_size_t,
                                     ctypes.POINTER(ctypes.c_float)]
    return lib


def _sweep_part(args):
    dtype, first, count = args
    lib = _lib()
    out = np.zeros(2 * count, dtype=np.int64)
    lib.ref_sweep_digest(dtype, first, count, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)))
    return first, out


def f32_from_bits(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def sample_inputs():
    """Edge cases of the three encoders plus a deterministic spread."""
    vals = []
    specials = [0.0, -0.0, np.inf, -np.inf, np.nan, 448.0, -448.0, 447.9, 448.0001, 240.0, 247.9,
                248.0, 255.9, 256.0, 57344.0, 61439.0, 61440.0, 65504.0, 2.0 ** -6, 2.0 ** -7,
                2.0 ** -8, 2.0 ** -9, 2.0 ** -10, 2.0 ** -14, 2.0 ** -15, 2.0 ** -16, 0.25, 0.75,
                1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, 1e30, -1e30, 2.0 ** 24, 2.0 ** 25, 2.0 ** 26,
                2.0 ** 27, 1.0 + 2.0 ** -4, 1.0 + 2.0 ** -3, 1.0 + 3 * 2.0 ** -4, 1.5 + 2.0 ** -4]
    for v in specials:
        vals.append(np.float32(v))
        vals.append(np.float32(-v))
    bits = [int(np.array(v, dtype=np.float32).view(np.uint32)) for v in vals]
    # every E4M3/E5M2 rounding boundary neighbourhood: x = code midpoints +- 1 ulp
    for e in range(-10, 17):
        for m in range(16):
            x = np.float32((1.0 + m / 16.0) * 2.0 ** e)
            b = int(x.view(np.uint32))
            bits.extend([b - 1, b, b + 1, b | 0x80000000])
    rng = np.random.default_rng(20261201)
    bits.extend(rng.integers(0, 2 ** 32, size=4096, dtype=np.uint64).astype(np.uint32).tolist())
    bits.extend([0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF, 0x00800000, 0x80800000,
                 0x7F7FFFFF, 0xFF7FFFFF, 0x7FC00000, 0xFFC00000, 0x7F800001])
    return np.array(bits, dtype=np.uint32)


def store_inputs():
    """Odd shapes (odd cols exercise nibbles that straddle rows)."""
    cases = []
    rng = np.random.default_rng(7)
    for dt_name, dt in DTYPES.items():
        for rows, cols, spread in [(1, 1, 1.0), (3, 5, 2.0), (7, 33, 8.0), (4, 64, 0.05),
                                   (5, 7, 600.0), (2, 31, 1e-3)]:
            W = (rng.standard_normal(rows * cols) * spread).astype(np.float32)
            cases.append((dt, rows, cols, W))
    return cases


def main():
    subprocess.check_call(["make", "-s", "-f", os.path.join(ROOT, "oracle", "Makefile"), "ref"])
    lib = _lib()

    tables = {}
    for name, dt in DTYPES.items():
        n = 16 if name == "fp4" else 256
        dec = np.array([lib.ref_dec(dt, c) for c in range(n)], dtype=np.float32)
        tables[name] = dec.view(np.uint32)
    np.savez(os.path.join(HERE, "codec_tables.npz"), **tables)

    bits = sample_inputs()
    samples = {"bits": bits}
    xs = f32_from_bits(bits)
    for name, dt in DTYPES.items():
        samples[name] = np.array([lib.ref_enc(dt, float(x)) for x in xs], dtype=np.uint8)
    np.savez(os.path.join(HERE, "codec_samples.npz"), **samples)

    store = {}
    for idx, (dt, rows, cols, W) in enumerate(store_inputs()):
        cap = rows * cols + 8
        native = np.zeros(cap, dtype=np.uint8)
        nlen = ctypes.c_size_t(0)
        scale = ctypes.c_float(0)
        rc = lib.ref_store_make(dt, rows, cols, W.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                native.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), cap,
                                ctypes.byref(nlen), ctypes.byref(scale))
        assert rc == 0, rc
        native = native[: nlen.value].copy()
        exp = np.zeros(rows * cols, dtype=np.float32)
        rc = lib.ref_store_export(dt, rows, cols,
                                  native.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                  native.size, exp.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        assert rc == 0, rc
        store[f"c{idx}_meta"] = np.array([dt, rows, cols], dtype=np.int32)
        store[f"c{idx}_W"] = W
        store[f"c{idx}_native"] = native
        store[f"c{idx}_scale"] = np.array([scale.value], dtype=np.float32)
        store[f"c{idx}_export"] = exp
    store["count"] = np.array([len(store_inputs())], dtype=np.int32)
    np.savez(os.path.join(HERE, "store_cases.npz"), **store)

    workers = max(1, min(8, os.cpu_count() or 1))
    digests = {}
    for name, dt in DTYPES.items():
        per = N_CHUNKS // (workers * 4)
        jobs = [(dt, s, per) for s in range(0, N_CHUNKS, per)]
        out = np.zeros(2 * N_CHUNKS, dtype=np.int64)
        with ProcessPoolExecutor(workers) as ex:
            for first, part in ex.map(_sweep_part, jobs):
                out[2 * first: 2 * first + part.size] = part
        digests[name] = out.reshape(N_CHUNKS, 2)
        print(f"sweep {name} done", flush=True)
    np.savez(os.path.join(HERE, "codec_sweep.npz"), **digests)


if __name__ == "__main__":
    sys.exit(main())
