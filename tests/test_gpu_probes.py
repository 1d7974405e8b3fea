"""The measurement entry points bench.py uses (no reference counterpart):
welvet_read_probe (the read floor), welvet_fetch_probe (per-CU fetch rate)
and welvet_mfma_probe (scaled matrix-core issue rate).

The read and fetch probes fold every 32-bit word they load into one XOR
digest per workgroup, so their outputs are checked bit for bit against the
XOR of the words each workgroup is documented to read: that pins which bytes
the timed kernels touch. The MFMA probe is checked for finite, repeatable
sums and for its argument errors.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _xor_words(b):
    w = np.frombuffer(b.tobytes(), dtype=np.uint32)
    return int(np.bitwise_xor.reduce(w)) if w.size else 0


@pytest.fixture(scope="module")
def hip(gpu):
    return gpu.Hip()


@pytest.mark.parametrize("nbytes", [16, 4096, 16384, 16384 * 3 + 48])
def test_read_probe_digest(gpu, hip, nbytes):
    """One word per 256-lane workgroup: the XOR of the 16 KiB run it reads
    (the last run ragged)."""
    L = gpu.lib()
    rng = np.random.default_rng(nbytes)
    data = rng.integers(0, 256, nbytes, dtype=np.uint8)
    buf = hip.upload(data)
    words = L.welvet_read_probe_words(nbytes)
    out = hip.malloc(4 * words)
    try:
        gpu.check(L.welvet_read_probe(ctypes.c_void_p(buf), nbytes, ctypes.c_void_p(out), words, None))
        hip.sync()
        got = hip.download(out, (words,), np.uint32)
        want = [_xor_words(data[16384 * i:16384 * (i + 1)]) for i in range(words)]
        assert got.tolist() == want
        st = L.welvet_read_probe(ctypes.c_void_p(buf), nbytes, ctypes.c_void_p(out), words - 1, None)
        assert st.code == 1  # output too small
    finally:
        hip.free(buf)
        hip.free(out)


def test_fetch_probe_digest(gpu, hip):
    """Workgroup w reads regions (7 w + i) mod nreg, i < iters, of 64 KiB."""
    L = gpu.lib()
    nreg, iters, wgs = 5, 3, 4
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, nreg * 65536, dtype=np.uint8)
    buf = hip.upload(data)
    out = hip.malloc(4 * wgs)
    try:
        gpu.check(L.welvet_fetch_probe(ctypes.c_void_p(buf), nreg * 65536, iters, wgs,
                                       ctypes.c_void_p(out), wgs, None))
        hip.sync()
        got = hip.download(out, (wgs,), np.uint32).tolist()
        want = []
        for w in range(wgs):
            x = 0
            for i in range(iters):
                r = (7 * w + i) % nreg
                x ^= _xor_words(data[r * 65536:(r + 1) * 65536])
            want.append(x)
        assert got == want
        for region, it, n, cap in ((65536 + 16, 1, 1, 1), (65536, 0, 1, 1), (65536, 1, 0, 1),
                                   (65536, 1, 2, 1)):
            st = L.welvet_fetch_probe(ctypes.c_void_p(buf), region, it, n, ctypes.c_void_p(out), cap, None)
            assert st.code == 1, (region, it, n, cap)
    finally:
        hip.free(buf)
        hip.free(out)


@pytest.mark.parametrize("fa,fb", [(0, 0), (2, 0), (2, 1), (2, 4), (4, 4)])
@pytest.mark.parametrize("shape", [16, 32])
def test_mfma_probe_runs(gpu, hip, fa, fb, shape):
    L = gpu.lib()
    wgs = 8
    out = hip.malloc(4 * 256 * wgs)
    try:
        res = []
        for _ in range(2):
            gpu.check(L.welvet_mfma_probe(fa, fb, shape, 3, wgs, ctypes.c_void_p(out), 256 * wgs, None))
            hip.sync()
            res.append(hip.download(out, (wgs * 256,), np.float32))
        assert np.all(np.isfinite(res[0]))
        assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))
        assert np.any(res[0] != 0)
    finally:
        hip.free(out)


def test_mfma_probe_errors(gpu, hip):
    L = gpu.lib()
    out = hip.malloc(4 * 256)
    try:
        assert L.welvet_mfma_probe(1, 1, 16, 1, 1, ctypes.c_void_p(out), 256, None).code == 2
        assert L.welvet_mfma_probe(0, 0, 8, 1, 1, ctypes.c_void_p(out), 256, None).code == 1
        assert L.welvet_mfma_probe(0, 0, 16, 0, 1, ctypes.c_void_p(out), 256, None).code == 1
        assert L.welvet_mfma_probe(0, 0, 16, 1, 2, ctypes.c_void_p(out), 256, None).code == 1
    finally:
        hip.free(out)
