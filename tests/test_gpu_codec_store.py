"""Device codecs and mount-time quantization, bit-exact.

* The device encoder (the one mount uses) over all 2^32 f32 inputs, per
  format, against digests of the compiled reference encoder.
* Reference FormatNone payloads (WeightStore::make of the compiled
  reference, tests/golden/store_cases.npz) reproduced by a scheme-0 mount.
* Scaled schemes 1-3: payload, row scales and E8M0 bytes equal the oracle's.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,dt", [("e4m3", 4), ("e5m2", 5), ("fp4", 16)])
def test_device_encoder_all_inputs(gpu, name, dt):
    gold = np.load(os.path.join(GOLD, "codec_sweep.npz"))[name]
    got = gpu.codec_sweep(dt)
    bad = np.nonzero(np.any(got != gold, axis=1))[0]
    assert bad.size == 0, f"{name}: {bad.size} chunks differ, first {bad[:8]}"


def test_mount_reproduces_reference_store(gpu):
    z = np.load(os.path.join(GOLD, "store_cases.npz"))
    for i in range(int(z["count"][0])):
        dt, rows, cols = z[f"c{i}_meta"].tolist()
        s = gpu.DenseSession(1, cols, rows, -1, dt, 0, z[f"c{i}_W"])
        native, rs, _, ts = s.export_store(dt)
        assert np.array_equal(native, z[f"c{i}_native"]), (i, dt, rows, cols)
        assert ts == 1.0 and np.all(rs == 1.0)
        s.close()


def _weights(rng, rows, cols):
    W = rng.standard_normal((rows, cols)) * np.exp(rng.uniform(-4, 4, (rows, 1)))
    W = W.astype(np.float32)
    W[0, :3] = [0.0, -0.0, 1e-40]           # zeros and an f32 subnormal
    W[-1, -1] = -1e-40                      # negative subnormal: sign must survive
    return W


@pytest.mark.parametrize("dt", [4, 5, 16])
@pytest.mark.parametrize("scheme", [0, 1, 2, 3])
@pytest.mark.parametrize("rows,cols", [(7, 33), (130, 257), (64, 1024)])
def test_mount_matches_oracle_quantizer(gpu, oracle, dt, scheme, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols + dt + 10 * scheme)
    W = _weights(rng, rows, cols)
    native_o, rs_o, blk_o = oracle.quantize(dt, scheme, rows, cols, W)
    s = gpu.DenseSession(1, cols, rows, -1, dt, scheme, W)
    native, rs, blk, ts = s.export_store(dt)
    assert np.array_equal(native, native_o)
    assert np.array_equal(rs.view(np.uint32), rs_o.view(np.uint32))
    if scheme == 3:
        assert np.array_equal(blk, blk_o)
    if scheme == 1:
        assert ts == rs_o[0]
    s.close()


def test_block_scale_boundaries(gpu, oracle):
    # block maxima exactly at, just above and just below maxrep * 2^e
    rows, cols = 6, 64
    W = np.full((rows, cols), 0.01, np.float32)
    for r, dt in enumerate([4, 5, 16, 4, 5, 16]):
        m = {4: 240.0, 5: 57344.0, 16: 6.0}[dt]
        a = np.float32(np.ldexp(np.float32(m), -3 + r))
        W[r, 5] = a
        W[r, 40] = -np.nextafter(a, np.float32(np.inf))
    for dt in (4, 5, 16):
        native_o, rs_o, blk_o = oracle.quantize(dt, 3, rows, cols, W)
        s = gpu.DenseSession(1, cols, rows, -1, dt, 3, W)
        native, rs, blk, _ = s.export_store(dt)
        assert np.array_equal(blk, blk_o) and np.array_equal(native, native_o)
        s.close()
