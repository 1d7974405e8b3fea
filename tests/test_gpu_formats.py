"""Packed block formats on the GPU (welvet_dense_mount_format), against the
oracle (oracle/formats.c):
- the device quantizers give the oracle's packed blocks byte for byte (ggml's
  reference quantizers for Q8_0 .. Q5_1, the library's one-pass quantizers
  for the K and IQ4 formats);
- the resident layout dequantizes to the oracle's f32 bit for bit (export);
- the GEMV matches the oracle's dequantize-then-f64 Dense at rel-L2 <= 1e-5
  (f32 accumulation on the VALU, as the FP8/FP4 GEMV);
- mounts from packed blocks export the same blocks;
- the reference's gap convention for the formats not built (code 3), and
  errors for bad shapes and calls a format session does not support.

The reference lists these formats without implementing any (README.md:361-383);
the layouts are ggml's, restated in the oracle."""
import numpy as np
import pytest

import pywelvet as pw
from format_blocks import ALL, GEOM, KQUANT, LEGACY, NAMES, random_blocks

pytestmark = pytest.mark.gpu

TOL = 1e-5


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def want_dense(oracle, Wd, x, act=-1, bias=None):
    return oracle.dense(Wd, x, act, bias)


@pytest.mark.parametrize("fmt", LEGACY, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 64), (300, 1024), (129, 4096)])
def test_quantize_blocks_and_dequant_bit_exact(gpu, oracle, fmt, rows, cols):
    rng = np.random.default_rng(fmt * 1000 + rows + cols)
    W = (rng.standard_normal((rows, cols)) * rng.uniform(1e-3, 10.0, (rows, 1))).astype(np.float32)
    s = gpu.FormatDenseSession(1, cols, rows, -1, fmt, W=W)
    try:
        got = s.export_blocks()
        want = oracle.fmt_quantize(fmt, W)
        assert got.size == want.size
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{NAMES[fmt]}: {bad.size} bytes differ, first at {bad[:4]}"
        Wd = oracle.fmt_dequant(fmt, want, (rows, cols))
        assert np.array_equal(s.export_f32().view(np.uint32), Wd.view(np.uint32))
    finally:
        s.close()


NEW_Q = [f for f in ALL if f not in LEGACY]


@pytest.mark.parametrize("fmt", NEW_Q, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (300, 1024), (129, 4096)])
def test_k_quantize_blocks_and_dequant_bit_exact(gpu, oracle, fmt, rows, cols):
    """The K and IQ4 formats quantized from fp32 on the device (the library's
    one-pass quantizers): the oracle's blocks byte for byte, and the resident
    layout dequantizes to the oracle's f32 bit for bit."""
    rng = np.random.default_rng(fmt * 1000 + rows + cols + 5)
    W = (rng.standard_normal((rows, cols)) * rng.uniform(1e-3, 10.0, (rows, 1))).astype(np.float32)
    s = gpu.FormatDenseSession(1, cols, rows, -1, fmt, W=W)
    try:
        got = s.export_blocks()
        want = oracle.fmt_quantize(fmt, W)
        assert got.size == want.size
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{NAMES[fmt]}: {bad.size} bytes differ, first at {bad[:4]}"
        Wd = oracle.fmt_dequant(fmt, want, (rows, cols))
        assert np.array_equal(s.export_f32().view(np.uint32), Wd.view(np.uint32))
    finally:
        s.close()


@pytest.mark.parametrize("fmt", ALL, ids=lambda f: NAMES[f])
def test_quantize_extreme_blocks(gpu, oracle, fmt):
    """Blocks whose scale is an f16 subnormal or near the f16 maximum, all-zero
    blocks, constant blocks and one-hot blocks."""
    rng = np.random.default_rng(fmt + 77)
    rows, cols = 8, 256
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    W[0] *= 1e-6          # d ~ 1e-8: an f16 subnormal
    W[1] *= 3e-9          # d below half the smallest f16 subnormal for some blocks
    W[2] = 0.0
    W[3] = 0.37
    W[4] = 0.0
    W[4, ::32] = -5.0
    W[5] *= 1000.0        # d ~ 30 (Q8_0) .. 500 (Q4_0)
    W[6, :32] = np.arange(32) - 16.0
    W[7] = -W[7] * 1e-3
    s = gpu.FormatDenseSession(1, cols, rows, -1, fmt, W=W)
    try:
        got = s.export_blocks()
        want = oracle.fmt_quantize(fmt, W)
        qk, bb = GEOM[fmt]
        bad = np.flatnonzero(got != want)
        for i in bad[:8]:
            blk = i // bb
            print(f"block {blk} (row {blk // (cols // qk)}) byte {i % bb}: got {got[i]:#04x} "
                  f"want {want[i]:#04x}; x = {W.reshape(-1, qk)[blk][:4]}")
        assert bad.size == 0
        Wd = oracle.fmt_dequant(fmt, want, (rows, cols))
        assert np.array_equal(s.export_f32().view(np.uint32), Wd.view(np.uint32))
    finally:
        s.close()


@pytest.mark.parametrize("fmt", ALL, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("rows,cols", [(5, 256), (300, 1024), (1024, 2816)])
def test_mount_from_blocks_dequant_and_export(gpu, oracle, fmt, rows, cols):
    rng = np.random.default_rng(fmt * 7 + rows)
    blocks = random_blocks(fmt, rows, cols, rng)
    s = gpu.FormatDenseSession(1, cols, rows, -1, fmt, blocks=blocks)
    try:
        assert np.array_equal(s.export_blocks(), blocks)
        Wd = oracle.fmt_dequant(fmt, blocks, (rows, cols))
        assert np.array_equal(s.export_f32().view(np.uint32), Wd.view(np.uint32))
    finally:
        s.close()


@pytest.mark.parametrize("fmt", ALL, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("batch", [1, 3, 8, 16, 37])
def test_gemv_against_oracle(gpu, oracle, fmt, batch):
    """Batches below 8 run the per-row kernel, from 8 the matrix-core one
    (37: three groups of 16 batch rows, the last ragged)."""
    rng = np.random.default_rng(fmt * 31 + batch)
    rows, cols = 333, 2048
    blocks = random_blocks(fmt, rows, cols, rng)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    s = gpu.FormatDenseSession(batch, cols, rows, -1, fmt, blocks=blocks)
    try:
        pre, post = s.execute(x)
    finally:
        s.close()
    Wd = oracle.fmt_dequant(fmt, blocks, (rows, cols))
    want, _ = want_dense(oracle, Wd, x)
    err = rel_l2(pre, want)
    print(f"{NAMES[fmt]} batch {batch}: rel-L2 {err:.2e}")
    assert err <= TOL
    assert np.array_equal(pre, post)


@pytest.mark.parametrize("fmt,from_fp32", [(2, True), (8, False), (10, False), (8, True),
                                           (17, True)], ids=lambda v: str(v))
def test_gemv_full_size_4096(gpu, oracle, fmt, from_fp32):
    """The benchmark shape: 4096 x 4096 at batch 1, quantized from fp32 on
    the device or mounted from packed blocks."""
    rng = np.random.default_rng(4096 + fmt)
    n = 4096
    x = rng.standard_normal((1, n)).astype(np.float32)
    if from_fp32:
        W = (rng.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
        s = gpu.FormatDenseSession(1, n, n, -1, fmt, W=W)
        blocks = oracle.fmt_quantize(fmt, W)
    else:
        blocks = random_blocks(fmt, n, n, rng)
        s = gpu.FormatDenseSession(1, n, n, -1, fmt, blocks=blocks)
    try:
        assert np.array_equal(s.export_blocks(), blocks)
        pre, _ = s.execute(x)
    finally:
        s.close()
    Wd = oracle.fmt_dequant(fmt, blocks, (n, n))
    want, _ = want_dense(oracle, Wd, x)
    assert rel_l2(pre, want) <= TOL


@pytest.mark.parametrize("act", [-1, 0, 1, 3, 6])
@pytest.mark.parametrize("batch", [2, 9])
def test_epilogue_bias_and_activation(gpu, oracle, act, batch):
    rng = np.random.default_rng(act + 10)
    rows, cols = 100, 512
    W = rng.standard_normal((rows, cols)).astype(np.float32) / 20
    bias = rng.standard_normal(rows)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    s = gpu.FormatDenseSession(batch, cols, rows, act, 3, W=W, bias=bias)
    try:
        pre, post = s.execute(x)
    finally:
        s.close()
    Wd = oracle.fmt_dequant(3, oracle.fmt_quantize(3, W), (rows, cols))
    wpre, wpost = want_dense(oracle, Wd, x, act, bias)
    assert rel_l2(pre, wpre) <= TOL and rel_l2(post, wpost) <= TOL


@pytest.mark.parametrize("fmt", LEGACY, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("batch", [1, 8])
def test_gemv_ragged_columns(gpu, oracle, fmt, batch):
    """45 sub-blocks of 32 columns: the matrix-core kernel's last group of 4
    holds one."""
    rng = np.random.default_rng(fmt * 7 + batch)
    rows, cols = 70, 32 * 45
    blocks = random_blocks(fmt, rows, cols, rng)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    s = gpu.FormatDenseSession(batch, cols, rows, -1, fmt, blocks=blocks)
    try:
        pre, _ = s.execute(x)
    finally:
        s.close()
    want, _ = want_dense(oracle, oracle.fmt_dequant(fmt, blocks, (rows, cols)), x)
    assert rel_l2(pre, want) <= TOL


def test_device_execute_and_noalloc_match_host_execute(gpu):
    hip = gpu.Hip()
    rng = np.random.default_rng(3)
    rows, cols, batch = 256, 1024, 4
    blocks = random_blocks(8, rows, cols, rng)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    s = gpu.FormatDenseSession(batch, cols, rows, -1, 8, blocks=blocks)
    dx = hip.upload(x)
    dp = hip.malloc(batch * rows * 4)
    dq = hip.malloc(batch * rows * 4)
    try:
        host, _ = s.execute(x)
        s.execute_device(dx, dp, dp)
        hip.sync()
        assert np.array_equal(hip.download(dp, (batch, rows)), host)
        s.execute_noalloc(batch, dx, dq, dq)
        hip.sync()
        assert np.array_equal(hip.download(dq, (batch, rows)), host)
    finally:
        s.close()
        for p in (dx, dp, dq):
            hip.free(p)


def test_errors_and_gaps(gpu):
    W = np.zeros((16, 64), np.float32)
    blocks = np.zeros(16 * 2 * 18, np.uint8)

    def mount(**kw):
        args = dict(batch=1, in_dim=64, out_dim=16, act=-1, fmt=2, W=None, blocks=None)
        args.update(kw)
        return gpu.FormatDenseSession(args["batch"], args["in_dim"], args["out_dim"], args["act"],
                                      args["fmt"], W=args["W"], blocks=args["blocks"])

    for fmt in (11, 12, 13, 14, 15, 18, 19, 20):  # listed by the reference, not built here
        with pytest.raises(gpu.WelvetError) as e:
            mount(fmt=fmt, W=W)
        assert e.value.code == 3
    for fmt in (0, 21, -1):
        with pytest.raises(gpu.WelvetError) as e:
            mount(fmt=fmt, W=W)
        assert e.value.code == 1
    with pytest.raises(gpu.WelvetError) as e:  # neither / both inputs
        mount()
    assert e.value.code == 1
    with pytest.raises(gpu.WelvetError) as e:
        mount(W=W, blocks=blocks)
    assert e.value.code == 1
    with pytest.raises(gpu.WelvetError) as e:  # in not a multiple of the block
        mount(in_dim=48, W=np.zeros((16, 48), np.float32))
    assert e.value.code == 1
    with pytest.raises(gpu.WelvetError) as e:  # K formats: in a multiple of 256
        mount(fmt=8, W=np.zeros((16, 128), np.float32), in_dim=128)
    assert e.value.code == 1
    s = mount(fmt=8, W=np.zeros((16, 256), np.float32), in_dim=256)  # quantized from fp32
    s.close()
    with pytest.raises(gpu.WelvetError) as e:  # wrong packed length
        mount(blocks=blocks[:-1])
    assert e.value.code == 1
    s = mount(blocks=blocks)
    try:
        with pytest.raises(gpu.WelvetError) as e:
            s.export_store(4)
        assert e.value.code == 2
    finally:
        s.close()


@pytest.mark.parametrize("dt,scheme", [(4, 0), (4, 2), (5, 1), (16, 3), (16, 2)])
def test_export_f32_of_fp8_fp4_sessions(gpu, oracle, dt, scheme):
    """welvet_dense_export_f32 on an FP8/FP4 session: codes times row scales
    and E8M0 factors, bit for bit the oracle's dequantization."""
    rng = np.random.default_rng(dt * 10 + scheme)
    rows, cols = 77, 300
    W = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    s = gpu.DenseSession(1, cols, rows, -1, dt, scheme, W)
    try:
        got = s.export_f32()
    finally:
        s.close()
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    want = oracle.dequant(dt, scheme, rows, cols, native, rs, blk)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
