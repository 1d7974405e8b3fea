"""Dense forward on the GPU against the oracle.

Parity reference: the oracle quantizes W with the same rules, dequantizes to
f32 and runs the reference Dense contract (f64 serial accumulation, bias in
f64, activation; src/cuda/kernels.cu:130-161). Tolerances, stated per test:
  * contract: relative L2 error <= 1e-3;
  * batch 1, VALU GEMV (fp32 FMA of exactly-decoded codes): <= 1e-5, the only
    difference from the oracle being fp32 accumulation order; batch-1 layers
    of at least 4081 rows and 2048 columns run on the matrix cores instead
    (test_gpu_gemv_mx) and take the matrix-core bound;
  * batches on the scaled matrix cores: <= 5e-5. The activations are split
    into E4M3 terms (residual ~4e-7) and the f8f6f4 MFMA accumulates with
    about 2^-16.5 relative precision (measured ~1.1e-5 at K=4096 even when the
    activations are exact in one term);
  * products chained in sequence (SwiGLU down after gate/up, stacks) add
    their errors: the bound scales with the chain length;
  * integer-exact cases: bit-exact (every partial sum is exact in f32 and in
    the matrix core).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_CONTRACT = 1e-3
TOL_GEMV = 1e-5
TOL_MFMA = 5e-5


def tol(batch, chain=1):
    """Bound for `chain` quantized products applied in sequence to `batch` rows."""
    return (TOL_GEMV if batch == 1 else TOL_MFMA) * chain


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def oracle_dense(oracle, dt, scheme, W, x, act=-1, bias=None, threads=8):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    Wd = oracle.dequant(dt, scheme, rows, cols, native, rs, blk)
    return oracle.dense(Wd, x, act, bias, threads=threads)


def run(gpu, dt, scheme, W, x, act=-1, bias=None):
    s = gpu.DenseSession(x.shape[0], W.shape[1], W.shape[0], act, dt, scheme, W, bias)
    pre, post = s.execute(x)
    s.close()
    return pre, post


def test_release_smoke_known_answer(gpu):
    W = np.eye(2, dtype=np.float32).ravel()
    x = np.array([0.5, -0.25], np.float32)
    pre, post = gpu.dense_forward(1, 2, 2, -1, 4, 0, W, x)
    assert pre.tolist() == [[0.5, -0.25]] and post.tolist() == [[0.5, -0.25]]


@pytest.mark.parametrize("dt,values", [
    (4, [-8, -6, -3, -1, 0, 1, 2, 5, 7, 8]),
    (5, [-8, -4, -3, -1.5, 0, 1, 2, 3, 6, 8]),
    (16, [-6, -4, -3, -1.5, -0.5, 0, 0.5, 1, 2, 6]),
])
def test_integer_exact_bit_for_bit(gpu, oracle, dt, values):
    rng = np.random.default_rng(dt)
    # 12588 and 24876 columns: 25 chunks (512 FP8 or 1024 FP4 elements each)
    # over 4 waves, so every wave takes several and the ragged last chunk is
    # the seventh of wave 0
    for rows, cols, batch in [(129, 1000, 1), (64, 4096, 1), (5, 77, 3), (9, 300, 9), (24, 9300, 1),
                              (40, 301, 9), (130, 4096, 40), (24, 12588, 1), (16, 24876, 2),
                              (8, 16384, 1)]:
        W = rng.choice(np.array(values, np.float32), (rows, cols))
        x = rng.integers(-4, 5, (batch, cols)).astype(np.float32)
        pre, post = run(gpu, dt, 0, W, x)
        o_pre, _ = oracle_dense(oracle, dt, 0, W, x)
        assert np.array_equal(pre, o_pre), (rows, cols, batch)
        assert np.array_equal(post, o_pre)


@pytest.mark.parametrize("dt", [4, 16])
@pytest.mark.parametrize("scheme", [2, 3])
@pytest.mark.parametrize("rows,cols", [(70, 1000), (70, 2000), (70, 3000), (40, 4000),
                                       (40, 5000), (24, 8000), (16, 9300), (24, 12588),
                                       (16, 24876)])
def test_gemv_k_split_over_waves(gpu, oracle, dt, scheme, rows, cols):
    """Batch-1 GEMV whose K axis spans 1-49 chunks of 64 lanes x 8 bytes (FP8:
    2, 4, 6, 8, 10, 16, 19, 25, 49; FP4: 1, 2, 3, 4, 5, 8, 10, 13, 25), so groups
    of 1, 2, 3, 4, 6 and 8 waves split it, and waves of 4-wave groups take
    several chunks, the last one ragged where cols is not a multiple of it."""
    rng = np.random.default_rng(rows * cols + dt + scheme)
    W = rng.standard_normal((rows, cols)).astype(np.float32) / np.sqrt(cols)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    pre, _ = run(gpu, dt, scheme, W, x)
    o_pre, _ = oracle_dense(oracle, dt, scheme, W, x)
    assert rel_l2(pre, o_pre) <= TOL_GEMV, (rows, cols)


@pytest.mark.parametrize("dt,scheme,act", [(4, 2, -1), (16, 3, 1), (5, 1, 3)])
def test_batched_wide_tiles(gpu, oracle, dt, scheme, act):
    """A product large enough for the wide tiles (256 staged weight rows per
    step, 256 workgroups): 1024 rows x 8192 outputs."""
    rng = np.random.default_rng(dt + 7 * scheme)
    rows, cols, batch = 8192, 200, 1024
    W = rng.standard_normal((rows, cols)).astype(np.float32) / np.sqrt(cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1
    pre, post = run(gpu, dt, scheme, W, x, act=act, bias=bias)
    o_pre, o_post = oracle_dense(oracle, dt, scheme, W, x, act=act, bias=bias)
    assert rel_l2(pre, o_pre) <= TOL_MFMA
    assert rel_l2(post, o_post) <= TOL_MFMA


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3), (5, 0)])
@pytest.mark.parametrize("rows,cols,batch", [
    (2176, 1000, 9),    # 2 row blocks per wave, grid past the 128-row padding
    (4096, 3000, 16),   # K split 16 ways
    (300, 4096, 30),    # 2 activation row blocks, 1 row block per wave
    (2100, 3000, 17),   # both, ragged N
    (500, 1001, 7),     # K not a multiple of 4: element loads of the input
])
def test_small_batch_k_split(gpu, oracle, dt, scheme, rows, cols, batch):
    """Batches of 5-32 rows take the weight-streaming GEMM, split along K into
    partial sums that a second kernel adds (bias and activation there)."""
    rng = np.random.default_rng(rows + cols + batch + dt)
    W = rng.standard_normal((rows, cols)).astype(np.float32) / np.sqrt(cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1
    pre, post = run(gpu, dt, scheme, W, x, act=2, bias=bias)
    o_pre, o_post = oracle_dense(oracle, dt, scheme, W, x, act=2, bias=bias)
    assert rel_l2(pre, o_pre) <= TOL_MFMA, (rows, cols, batch)
    assert rel_l2(post, o_post) <= TOL_MFMA, (rows, cols, batch)


@pytest.mark.parametrize("dt,scheme", [(4, 2), (5, 3), (16, 3), (16, 0)])
@pytest.mark.parametrize("rows,cols,batch", [(2176, 1000, 9), (500, 1001, 7), (300, 4096, 30)])
def test_small_batch_operand_order_codes_bit_identical(gpu, dt, scheme, rows, cols, batch):
    """Sessions whose batch runs the 5..32-row GEMM mount an operand-order
    copy of the codes and read it instead of the row-major codes. The NormalBP
    leaf mounts without that copy, so its forward reads the row-major codes:
    both must give the same bits (same bytes, same order of operations)."""
    rng = np.random.default_rng(7 * rows + cols + batch + dt)
    W = rng.standard_normal((rows, cols)).astype(np.float32) / np.sqrt(cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1
    pre, post = gpu.dense_forward(batch, cols, rows, 2, dt, scheme, W, x, bias=bias)
    g = np.zeros((batch, rows), np.float32)
    pre_rm, post_rm, *_ = gpu.dense_normalbp(batch, cols, rows, 2, dt, scheme, W, x, g, bias=bias)
    assert np.array_equal(pre.view(np.uint32), pre_rm.view(np.uint32)), (dt, rows, cols, batch)
    assert np.array_equal(post.view(np.uint32), post_rm.view(np.uint32)), (dt, rows, cols, batch)


def test_small_batch_operand_order_codes_swiglu_bit_identical(gpu):
    """The same for SwiGLU (two matrices in one product): the session reads
    the operand-order copies, the NormalBP leaf the row-major codes."""
    rng = np.random.default_rng(11)
    d, f, rows = 256, 640, 12
    G, U = [(rng.standard_normal((f, d)) / np.sqrt(d)).astype(np.float32) for _ in range(2)]
    D = (rng.standard_normal((d, f)) / np.sqrt(f)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    s = gpu.SwiGLUSession(1, rows, d, f, 16, 3, G, U, D)
    try:
        h, y = s.execute(x)
    finally:
        s.close()
    g = np.zeros((rows, d), np.float32)
    h_rm, y_rm, *_ = gpu.swiglu_normalbp(1, rows, d, f, 16, 3, G, U, D, x, g)
    assert np.array_equal(h.view(np.uint32), h_rm.view(np.uint32))
    assert np.array_equal(y.view(np.uint32), y_rm.view(np.uint32))


@pytest.mark.parametrize("dt", [4, 5, 16])
@pytest.mark.parametrize("scheme", [0, 1, 2, 3])
@pytest.mark.parametrize("rows,cols,batch", [(33, 70, 1), (300, 1024, 2), (7, 33, 3), (1, 1, 1)])
def test_dense_matches_oracle(gpu, oracle, dt, scheme, rows, cols, batch):
    rng = np.random.default_rng(rows + cols + batch + dt + scheme)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    if scheme == 0:
        W *= 8.0  # keep unscaled codes mostly in the normal range
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    pre, post = run(gpu, dt, scheme, W, x)
    o_pre, o_post = oracle_dense(oracle, dt, scheme, W, x)
    e = rel_l2(pre, o_pre)
    assert e <= tol(batch) and e <= TOL_CONTRACT, e
    assert np.array_equal(pre, post)


@pytest.mark.parametrize("act", [-1, 0, 1, 2, 3, 4, 5, 6])
def test_bias_and_activation_epilogue(gpu, oracle, act):
    rng = np.random.default_rng(40 + act)
    rows, cols = 45, 96
    W = (rng.standard_normal((rows, cols)) / 10).astype(np.float32)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    bias = rng.standard_normal(30)  # shorter than out: rows >= 30 get no bias
    pre, post = run(gpu, 4, 2, W, x, act, bias)
    o_pre, o_post = oracle_dense(oracle, 4, 2, W, x, act, bias)
    assert rel_l2(pre, o_pre) <= TOL_MFMA
    assert rel_l2(post, o_post) <= TOL_MFMA


def test_c1_dense_512_e4m3_per_tensor(gpu, oracle):
    """Single Dense 512->512, E4M3 + one fp32 per-tensor scale, batch 1."""
    import pywelvet as pw
    W = pw.normal(pw.seed_for(1), 512 * 512, 1 / np.sqrt(512)).reshape(512, 512)
    x = pw.normal(pw.seed_for(1) + 500, 512).reshape(1, 512)
    pre, _ = run(gpu, 4, 1, W, x)
    o_pre, _ = oracle_dense(oracle, 4, 1, W, x)
    assert rel_l2(pre, o_pre) <= TOL_GEMV


def test_c2_gemv_4096_e4m3_per_row(gpu, oracle):
    """Dense GEMV 4096->4096, E4M3 + per-row fp32 scales, batch 1. A session
    of this size runs the batch-1 product on the matrix cores over the
    operand-order weights (x as three E4M3 terms): the matrix-core bound."""
    import pywelvet as pw
    W = pw.normal(pw.seed_for(2), 4096 * 4096, 1 / 64.0).reshape(4096, 4096)
    x = pw.normal(pw.seed_for(2) + 500, 4096).reshape(1, 4096)
    pre, _ = run(gpu, 4, 2, W, x)
    o_pre, _ = oracle_dense(oracle, 4, 2, W, x)
    e = rel_l2(pre, o_pre)
    assert e <= TOL_MFMA, e
    # the quantized layer itself against the unquantized fp32 layer (what the
    # scale scheme costs): E4M3 with per-row scales keeps ~3-4% error
    full, _ = oracle.dense(W, x)
    assert rel_l2(pre, full) < 0.05


def test_device_resident_execute_matches_host(gpu):
    import pywelvet as pw
    hip = pw.Hip()
    rng = np.random.default_rng(9)
    W = (rng.standard_normal((256, 512)) / 20).astype(np.float32)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    s = pw.DenseSession(2, 512, 256, 1, 16, 3, W, rng.standard_normal(256))
    pre_h, post_h = s.execute(x)
    dx = hip.upload(x)
    dp = hip.malloc(2 * 256 * 4)
    dq = hip.malloc(2 * 256 * 4)
    s.execute_device(dx, dp, dq)
    hip.sync()
    assert np.array_equal(hip.download(dp, (2, 256)), pre_h)
    assert np.array_equal(hip.download(dq, (2, 256)), post_h)
    for p in (dx, dp, dq):
        hip.free(p)
    s.close()


def test_unsupported_dtype_and_scheme(gpu):
    import pywelvet as pw
    W = np.ones((4, 4), np.float32)
    with pytest.raises(pw.WelvetError) as e:
        pw.DenseSession(1, 4, 4, -1, 1, 0, W)  # Float32 storage: not this path
    assert e.value.code == 2
    with pytest.raises(pw.WelvetError) as e:
        pw.DenseSession(1, 4, 4, -1, 4, 7, W)
    assert e.value.code == 1


@pytest.mark.parametrize("dt,scheme", [(4, 2), (5, 2), (16, 3), (4, 3), (16, 1), (5, 0)])
@pytest.mark.parametrize("rows,cols,batch", [(70, 300, 5), (64, 256, 16), (130, 512, 17),
                                              (257, 1024, 64), (96, 160, 257)])
def test_batched_mfma_matches_oracle(gpu, oracle, dt, scheme, rows, cols, batch):
    rng = np.random.default_rng(rows * 7 + cols + batch + dt + scheme)
    W = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    if scheme == 0:
        W *= 8.0
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    pre, post = run(gpu, dt, scheme, W, x)
    o_pre, _ = oracle_dense(oracle, dt, scheme, W, x)
    e = rel_l2(pre, o_pre)
    assert e <= TOL_MFMA, e
    assert np.array_equal(pre, post)


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3), (5, 0), (4, 1)])
@pytest.mark.parametrize("rows,cols,batch", [
    (384, 2000, 200),   # 6 tiles, K split 8 ways, ragged M
    (1000, 4096, 40),   # 8 tiles, 16 splits, ragged N
    (130, 8192, 129),   # 4 tiles, 32 splits: the reduce adds them 16 at a time
    (256, 512, 300),    # 2 splits of one step pair each
])
def test_batched_k_split(gpu, oracle, dt, scheme, rows, cols, batch):
    """Batches above 32 rows with few 128 x 128 tiles split K over the CUs:
    raw partial sums per split, added in split order by a second kernel
    (scale, bias and activation there)."""
    rng = np.random.default_rng(rows + 3 * cols + batch + dt + scheme)
    W = rng.standard_normal((rows, cols)).astype(np.float32) / np.sqrt(cols)
    if scheme == 0:
        W *= 8.0
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = rng.standard_normal(rows) * 0.1
    pre, post = run(gpu, dt, scheme, W, x, act=2, bias=bias)
    o_pre, o_post = oracle_dense(oracle, dt, scheme, W, x, act=2, bias=bias)
    assert rel_l2(pre, o_pre) <= TOL_MFMA, (rows, cols, batch)
    assert rel_l2(post, o_post) <= TOL_MFMA, (rows, cols, batch)
    pre2, _ = run(gpu, dt, scheme, W, x)  # linear, no bias: post is pre
    o_pre2, _ = oracle_dense(oracle, dt, scheme, W, x)
    assert rel_l2(pre2, o_pre2) <= TOL_MFMA


def test_batched_epilogue_bias_act(gpu, oracle):
    rng = np.random.default_rng(77)
    W = (rng.standard_normal((100, 256)) / 16).astype(np.float32)
    x = rng.standard_normal((33, 256)).astype(np.float32)
    bias = rng.standard_normal(64)
    for act in (0, 1, 2):
        pre, post = run(gpu, 16, 3, W, x, act, bias)
        o_pre, o_post = oracle_dense(oracle, 16, 3, W, x, act, bias)
        assert rel_l2(pre, o_pre) <= TOL_MFMA and rel_l2(post, o_post) <= TOL_MFMA


def test_c4_projection_gemm_e5m2(gpu, oracle):
    """MHA projection GEMM 4096 x 1024 -> 1024, E5M2 weights with per-row scales."""
    import pywelvet as pw
    W = pw.normal(pw.seed_for(4), 1024 * 1024, 1 / 32.0).reshape(1024, 1024)
    x = pw.normal(pw.seed_for(4) + 500, 4096 * 1024).reshape(4096, 1024)
    pre, _ = run(gpu, 5, 2, W, x)
    o_pre, _ = oracle_dense(oracle, 5, 2, W, x, threads=16)
    assert rel_l2(pre, o_pre) <= TOL_MFMA


@pytest.mark.parametrize("dt,scheme", [(4, 2), (16, 3)])
def test_c5_cell_layer_batch256(gpu, oracle, dt, scheme):
    """Volume cell layer: Dense 1024 -> 1024, batch 256 (E4M3 per-row / FP4 block-32)."""
    import pywelvet as pw
    W = pw.normal(pw.seed_for(5), 1024 * 1024, 1 / 32.0).reshape(1024, 1024)
    x = pw.normal(pw.seed_for(5) + 500, 256 * 1024).reshape(256, 1024)
    pre, _ = run(gpu, dt, scheme, W, x)
    o_pre, _ = oracle_dense(oracle, dt, scheme, W, x)
    assert rel_l2(pre, o_pre) <= TOL_MFMA
