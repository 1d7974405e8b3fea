"""SwiGLU and MHA layers on the GPU against the oracle chain.

SwiGLU (swiglu.cpp:87-136, kernels.cu:296-304): pre = h = SiLU(Gate x) * Up x
with the reference's f32/f64 rounding; post = Down h.
MHA (mha.cpp:123-183, kernels.cu:470-631): Q/K/V projections, attention core
with the reference's global positions and KV ring, O projection.
Tolerance: relative L2 <= 1e-5 for one row (VALU GEMV, fp32), <= 5e-5 where
rows go through the scaled matrix cores (see test_gpu_dense; batch-1 layers
of 4081 rows and more do too), <= 1e-4 after
the attention core (fp32 exp/sin/cos against f64 libm). The layer contract
bound is 1e-3.
"""
import numpy as np
import pytest

from test_gpu_dense import rel_l2, tol

pytestmark = pytest.mark.gpu


def oracle_dequant(oracle, dt, scheme, W):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    return oracle.dequant(dt, scheme, rows, cols, native, rs, blk)


def oracle_swiglu(oracle, dt, scheme, G, U, D, x):
    g, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, G), x)
    u, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, U), x)
    h = oracle.swiglu_product(g, u)
    y, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, D), h)
    return h, y


@pytest.mark.parametrize("dt,scheme", [(16, 3), (4, 2), (5, 1), (16, 0)])
@pytest.mark.parametrize("batch,seq,d,inter", [(1, 1, 64, 160), (2, 3, 96, 200), (16, 1, 128, 352),
                                               (40, 2, 96, 200),
                                               (8, 128, 128, 4096)])  # gate+up on wide tiles
def test_swiglu_matches_oracle(gpu, oracle, dt, scheme, batch, seq, d, inter):
    rng = np.random.default_rng(d + inter + dt + batch)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((batch * seq, d)).astype(np.float32)
    s = gpu.SwiGLUSession(batch, seq, d, inter, dt, scheme, G, U, D)
    h, y = s.execute(x)
    s.close()
    oh, oy = oracle_swiglu(oracle, dt, scheme, G, U, D, x)
    assert rel_l2(h, oh) <= tol(batch * seq)
    assert rel_l2(y, oy) <= tol(batch * seq, chain=2)


@pytest.mark.parametrize("scheme", [3, 0])
@pytest.mark.parametrize("rows,d,inter", [(5, 700, 8200), (16, 1024, 8300), (12, 4096, 8192),
                                          (17, 700, 8200)])
def test_swiglu_fp4_small_batch_ragged(gpu, oracle, scheme, rows, d, inter):
    """FP4 SwiGLU at 5-17 rows on the K-split matrix-core path (256-row
    workgroups): ragged K, output counts that are no multiple of 256 (the
    grid's last rows clamped), one and two activation row blocks."""
    rng = np.random.default_rng(rows + d + inter + scheme)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    s = gpu.SwiGLUSession(rows, 1, d, inter, 16, scheme, G, U, D)
    h, y = s.execute(x)
    s.close()
    oh, oy = oracle_swiglu(oracle, 16, scheme, G, U, D, x)
    assert rel_l2(h, oh) <= tol(rows)
    assert rel_l2(y, oy) <= tol(rows, chain=2)


@pytest.mark.parametrize("dt,scheme", [(16, 3), (4, 2), (5, 1)])
@pytest.mark.parametrize("rows,d,inter", [(16, 1024, 4100), (24, 1024, 4100), (32, 2000, 8200),
                                          (9, 4096, 4096)])
def test_swiglu_gate_up_whole_k_workgroups(gpu, oracle, dt, scheme, rows, d, inter):
    """The 5-32-row gate+up pair on the path without a K split (16 weight rows
    per workgroup over all of K, at least 256 workgroups: inter > 4080 and
    d >= 1024): one and two activation row blocks, a ragged row count of the
    grid's last block (4100, 8200), ragged K (2000), FP4 and FP8 weights."""
    rng = np.random.default_rng(rows + d + inter + dt)
    G = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    U = (rng.standard_normal((inter, d)) / np.sqrt(d)).astype(np.float32)
    D = (rng.standard_normal((d, inter)) / np.sqrt(inter)).astype(np.float32)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    s = gpu.SwiGLUSession(rows, 1, d, inter, dt, scheme, G, U, D)
    h, y = s.execute(x)
    s.close()
    oh, oy = oracle_swiglu(oracle, dt, scheme, G, U, D, x)
    assert rel_l2(h, oh) <= tol(rows)
    assert rel_l2(y, oy) <= tol(rows, chain=2)


def test_c3_swiglu_fp4_block32_batch1(gpu, oracle):
    """SwiGLU d_model 4096, d_ff 11008, FP4 E2M1 + E8M0 per 32 along K, batch 1:
    both products on the matrix cores over the operand-order weights, the
    down projection on the split of h that the gate+up launch writes."""
    import pywelvet as pw
    d, f = 4096, 11008
    seed = pw.seed_for(3)
    G = pw.normal(seed, f * d, 1 / np.sqrt(d)).reshape(f, d)
    U = pw.normal(seed + 1, f * d, 1 / np.sqrt(d)).reshape(f, d)
    D = pw.normal(seed + 2, d * f, 1 / np.sqrt(f)).reshape(d, f)
    x = pw.normal(seed + 500, d).reshape(1, d)
    s = gpu.SwiGLUSession(1, 1, d, f, 16, 3, G, U, D)
    h, y = s.execute(x)
    s.close()
    oh, oy = oracle_swiglu(oracle, 16, 3, G, U, D, x)
    assert rel_l2(h, oh) <= tol(16)
    oy_own, _ = oracle.dense(oracle_dequant(oracle, 16, 3, D), h)
    assert rel_l2(y, oy_own) <= tol(16)
    assert rel_l2(y, oy) <= tol(16, chain=2)


def oracle_mha(oracle, dt, scheme, Q, K, V, O, x, B, S, H, KVH, hd, msl, mask, pos):
    q, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, Q), x)
    k, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, K), x)
    v, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, V), x)
    attn = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos)
    y, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, O), attn)
    return attn, y


@pytest.mark.parametrize("B,S,d,H,KVH,msl,mask,pos", [
    (2, 8, 64, 4, 4, 8, 1, 0),     # ring = one sequence: batch 1 re-reads batch 1 keys
    (3, 5, 32, 4, 2, 7, 1, 0),     # ring wraps mid-sequence, GQA
    (2, 6, 32, 2, 2, 16, 2, 1),    # bidirectional, no positions
    (2, 6, 48, 3, 3, 6, 3, 2),     # sliding window (msl), ALiBi
    (1, 9, 64, 4, 1, 9, 4, 3),     # prefix LM (prefix 0), RoPE + ALiBi, MQA
    (4, 12, 64, 4, 4, 12, 1, 0),   # 48 tokens: projections on the large-tile GEMM
    (2, 40, 64, 2, 2, 40, 2, 1),   # 80 tokens, no positions, ring below one 64-key tile: VALU attention
])
def test_mha_matches_oracle(gpu, oracle, B, S, d, H, KVH, msl, mask, pos):
    dt, scheme = 5, 2
    hd = d // H
    rng = np.random.default_rng(B * 100 + S + d + mask)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    s = gpu.MHASession(B, S, d, H, KVH, 0, msl, mask, pos, dt, scheme, Q, K, V, O)
    attn, y = s.execute(x)
    s.close()
    oattn, oy = oracle_mha(oracle, dt, scheme, Q, K, V, O, x, B, S, H, KVH, hd, msl, mask, pos)
    assert rel_l2(attn, oattn) <= 1e-4
    assert rel_l2(y, oy) <= 1e-4


@pytest.mark.parametrize("B,S,d,H,KVH,msl,mask", [
    (2, 64, 256, 4, 4, 64, 1),     # hd 64: two heads per 128-column slice
    (2, 48, 256, 8, 2, 64, 2),     # hd 32, GQA, 96 tokens (32 padding rows)
    (1, 96, 256, 2, 2, 96, 1),     # hd 128: one head per slice
    (4, 512, 1024, 16, 16, 512, 1),  # the benchmark layer at half the batch
    (3, 70, 128, 2, 2, 80, 1),     # seq % 16 != 0: the O projection splits its input itself
])
def test_mha_output_split_matches_o_session(gpu, B, S, d, H, KVH, msl, mask):
    """When the matrix-core attention also writes the O projection's FP6
    split of its output (heads * hd % 256 == 0, seq % 16 == 0), the layer's
    output equals an O-projection session run over the returned attention
    output, bit for bit: the split is the one k_split makes from it."""
    dt, scheme = 5, 2
    hd = d // H
    rng = np.random.default_rng(B * 7 + S + d + H)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    s = gpu.MHASession(B, S, d, H, KVH, 0, msl, mask, 0, dt, scheme, Q, K, V, O)
    attn, y = s.execute(x)
    s.close()
    o = gpu.DenseSession(B * S, H * hd, d, -1, dt, scheme, O)
    yo, _ = o.execute(attn.reshape(B * S, H * hd))
    o.close()
    assert np.array_equal(y.reshape(B * S, d), yo)


@pytest.mark.parametrize("B,S,d,H,KVH,msl,mask", [
    (3, 70, 128, 2, 2, 80, 1),     # ring of 80 rows < 210 positions: multiplicities 1..3
    (2, 64, 128, 4, 2, 64, 2),     # bidirectional, GQA, hd 32
    (2, 40, 128, 1, 1, 100, 1),    # hd 128, ragged query block
    (4, 512, 1024, 16, 16, 512, 1),  # the benchmark layer at half the batch
])
def test_mha_matrix_core_attention(gpu, oracle, B, S, d, H, KVH, msl, mask):
    """Causal / bidirectional attention without ALiBi runs on the matrix cores
    over the distinct KV-ring rows with multiplicity weights."""
    dt, scheme, pos = 5, 2, 0
    hd = d // H
    rng = np.random.default_rng(B * 7 + S + d)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    s = gpu.MHASession(B, S, d, H, KVH, 0, msl, mask, pos, dt, scheme, Q, K, V, O)
    attn, y = s.execute(x)
    s.close()
    oattn, oy = oracle_mha(oracle, dt, scheme, Q, K, V, O, x, B, S, H, KVH, hd, msl, mask, pos)
    ea, ey = rel_l2(attn, oattn), rel_l2(y, oy)
    print(f"matrix-core attention B={B} S={S} d={d} H={H}: attention rel-L2 {ea:.2e}, output {ey:.2e}")
    assert ea <= 1e-4
    assert ey <= 1e-4


def test_mha_seq_above_max_is_invalid(gpu):
    import pywelvet as pw
    W = np.zeros((16, 16), np.float32)
    with pytest.raises(pw.WelvetError) as e:
        pw.MHASession(1, 9, 16, 2, 2, 0, 8, 1, 0, 5, 0, W, W, W, W)
    assert e.value.code == 1


@pytest.mark.parametrize("mask,pos", [(0, 0), (5, 0), (7, 1), (-3, 0), (1, 4), (2, -1), (5, 9)])
def test_mha_out_of_range_kinds_match_reference(gpu, oracle, mask, pos):
    """The reference passes mask / position kinds through unchecked
    (c_abi.cpp:805-806): masks other than 2, 3, 4 (Unspecified 0, Custom 5
    and any other value) attend causally, and position kinds outside 0-3
    apply no rotation and no ALiBi (kernels.cu:470-485, 550-551). The oracle
    follows the same reading with the raw values."""
    B, S, d, H, KVH, msl = 2, 24, 64, 4, 2, 24
    dt, scheme = 5, 2
    hd = d // H
    rng = np.random.default_rng(300 + 10 * mask + pos)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    s = gpu.MHASession(B, S, d, H, KVH, 0, msl, mask, pos, dt, scheme, Q, K, V, O)
    attn, y = s.execute(x)
    s.close()
    oattn, oy = oracle_mha(oracle, dt, scheme, Q, K, V, O, x, B, S, H, KVH, hd, msl, mask, pos)
    assert rel_l2(attn, oattn) <= 1e-4
    assert rel_l2(y, oy) <= 1e-4


def test_runtime_identity_names_the_device(gpu):
    """The identity carries a device name (reference device.cpp:57-59:
    "cuda:<name>:idx:..."), here "hip:<name>:idx=0:arch=...": the name field
    is never empty."""
    ident = gpu.lib().welvet_runtime_identity().decode()
    parts = ident.split(":")
    assert parts[0] == "hip" and parts[1] != "" and parts[2] == "idx=0", ident


@pytest.mark.parametrize("score_std", [10.0, 20.0, 30.0])
@pytest.mark.parametrize("pos", [0, 1])
def test_mha_peaked_attention(gpu, oracle, score_std, pos):
    """Peaked softmax: Q and K scaled so the scores have a standard deviation
    of 10-30 (the other tests' scores are about N(0, 1)). exp() turns an
    absolute score error into a relative weight error, so this is where the
    precision of the matrix-core score products shows. The inputs are small
    integers, which the FP6 activation split holds exactly, so the GPU's
    projections differ from the oracle's f64 ones by fp32 summation only and
    the comparison measures the attention core itself (bound 1e-4)."""
    B, S, d, H, KVH, msl, mask = 2, 128, 128, 2, 2, 128, 1
    dt, scheme = 5, 2
    hd = d // H
    rng = np.random.default_rng(int(score_std) * 10 + pos)
    x = rng.integers(-7, 8, size=(B * S, d)).astype(np.float32)
    Q = (rng.standard_normal((H * hd, d)) / np.sqrt(d)).astype(np.float32)
    K = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    V = (rng.standard_normal((KVH * hd, d)) / np.sqrt(d)).astype(np.float32)
    O = (rng.standard_normal((d, H * hd)) / np.sqrt(H * hd)).astype(np.float32)
    # unscaled scores: q, k entries have std ~ 4.3 (x std), q.k / sqrt(hd)
    # std ~ 4.3^2; scale K to reach the target
    xs = float(np.std(x))
    K *= np.float32(score_std / (xs * xs))
    s = gpu.MHASession(B, S, d, H, KVH, 0, msl, mask, pos, dt, scheme, Q, K, V, O)
    attn, y = s.execute(x)
    s.close()
    q, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, Q), x)
    k, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, K), x)
    v, _ = oracle.dense(oracle_dequant(oracle, dt, scheme, V), x)
    scores = np.einsum("thd,thd->th", q.reshape(-1, H, hd)[:S], k.reshape(-1, H, hd)[::-1][:S])
    got_std = float(np.std(scores / np.sqrt(hd)))
    assert 0.5 * score_std <= got_std <= 2.0 * score_std, got_std
    oattn = oracle.mha_attention(q, k, v, B, S, H, KVH, hd, msl, mask, pos)
    err = rel_l2(attn, oattn)
    print(f"peaked attention score std {got_std:.1f} pos {pos}: rel-L2 {err:.2e}")
    assert err <= 1e-4
