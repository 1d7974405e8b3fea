"""The benchmark workloads at their full sizes, against the oracle.

Each test builds the workload the way bench.py measures it (same shapes,
dtypes, scale schemes, seeded inputs and execution path) and compares with
the oracle's reference contract on the same inputs:
  * SwiGLU 4096 / 11008, FP4 E2M1 + E8M0 per 32, 16 rows: the 5..32-row GEMM
    with the operand-order codes, its K split and reduce
    (swiglu.cpp:87-136, kernels.cu:296-304);
  * the MHA layer at batch 8, seq 512, d 1024, 16 heads x 64, E5M2 per-row
    (mha.cpp:123-183, kernels.cu:470-631);
  * 64 cells x 3 Dense 1024^2 (E4M3 per-row, FP4 E8M0/32, E4M3 per-row) at
    256 rows, run as grouped launches chained through the epilogue split:
    every layer of every cell is checked against the oracle on the GPU's own
    input of that layer, and the chain that leaves out the inner outputs (the
    one the benchmark times) gives the same last outputs bit for bit.
Tolerances as in test_gpu_dense (matrix-core products: rel-L2 <= 5e-5 per
product, times the number of chained products; attention core 1e-4).
"""
import os

import numpy as np
import pytest

import pywelvet as pw
from test_gpu_dense import rel_l2, tol

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))


def dequant(oracle, dt, scheme, W):
    rows, cols = W.shape
    native, rs, blk = oracle.quantize(dt, scheme, rows, cols, W)
    return oracle.dequant(dt, scheme, rows, cols, native, rs, blk)


def test_c3_swiglu_fp4_block32_batch16(gpu, oracle):
    d, f, batch = 4096, 11008, 16
    seed = pw.seed_for(3)
    G = pw.normal(seed, f * d, 1 / np.sqrt(d)).reshape(f, d)
    U = pw.normal(seed + 1, f * d, 1 / np.sqrt(d)).reshape(f, d)
    D = pw.normal(seed + 2, d * f, 1 / np.sqrt(f)).reshape(d, f)
    x = pw.normal(seed + 500, batch * d).reshape(batch, d)
    s = gpu.SwiGLUSession(batch, 1, d, f, 16, 3, G, U, D)
    h, y = s.execute(x)
    s.close()
    g, _ = oracle.dense(dequant(oracle, 16, 3, G), x, threads=THREADS)
    u, _ = oracle.dense(dequant(oracle, 16, 3, U), x, threads=THREADS)
    oh = oracle.swiglu_product(g, u)
    assert rel_l2(h, oh) <= tol(batch)
    # down on the GPU's own h isolates the second product; on the oracle's h
    # the two products' errors add
    oy_own, _ = oracle.dense(dequant(oracle, 16, 3, D), h, threads=THREADS)
    oy, _ = oracle.dense(dequant(oracle, 16, 3, D), oh, threads=THREADS)
    assert rel_l2(y, oy_own) <= tol(batch)
    assert rel_l2(y, oy) <= tol(batch, chain=2)


def test_c4_mha_layer_batch8(gpu, oracle):
    B, S, d, H, hd = 8, 512, 1024, 16, 64
    seed = pw.seed_for(4)
    Ws = [pw.normal(seed + i, d * d, 1 / np.sqrt(d)).reshape(d, d) for i in range(4)]
    x = pw.normal(seed + 500, B * S * d).reshape(B * S, d)
    s = gpu.MHASession(B, S, d, H, H, hd, S, 1, 0, 5, 2, *Ws)
    attn, y = s.execute(x)
    s.close()
    Wd = [dequant(oracle, 5, 2, W) for W in Ws]
    q, _ = oracle.dense(Wd[0], x, threads=THREADS)
    k, _ = oracle.dense(Wd[1], x, threads=THREADS)
    v, _ = oracle.dense(Wd[2], x, threads=THREADS)
    oa = oracle.mha_attention(q, k, v, B, S, H, H, hd, S, 1, 0, threads=THREADS)
    assert rel_l2(attn, oa) <= 1e-4
    oy_own, _ = oracle.dense(Wd[3], attn, threads=THREADS)
    assert rel_l2(y, oy_own) <= tol(B * S)
    oy, _ = oracle.dense(Wd[3], oa, threads=THREADS)
    assert rel_l2(y, oy) <= 1e-4 + tol(B * S)


def test_c5_volume_64_cells_grouped_chain(gpu, oracle):
    cells, batch, d = 64, 256, 1024
    kinds = [(4, 2), (16, 3), (4, 2)]
    hip = gpu.Hip()
    sessions, bufs, Ws, xs = [], [], [], []
    try:
        for c in range(cells):
            seed = pw.seed_for(5, c)
            row, wrow = [], []
            for li, (dt, sc) in enumerate(kinds):
                W = pw.normal(seed + 10 * li, d * d, 1 / np.sqrt(d)).reshape(d, d)
                row.append(gpu.DenseSession(batch, d, d, -1, dt, sc, W))
                wrow.append(W)
            sessions.append(row)
            Ws.append(wrow)
            x = pw.normal(seed + 500, batch * d).reshape(batch, d)
            xs.append(x)
            bufs.append([hip.upload(x)] + [hip.malloc(batch * d * 4) for _ in kinds])
        groups = [gpu.DenseGroup([sessions[c][li] for c in range(cells)],
                                 [bufs[c][li] for c in range(cells)],
                                 [bufs[c][li + 1] for c in range(cells)],
                                 [bufs[c][li + 1] for c in range(cells)])
                  for li in range(len(kinds))]
        chain = gpu.DenseChain(groups)
        chain.execute()
        hip.sync()
        outs = [[hip.download(bufs[c][li + 1], (batch, d)) for li in range(len(kinds))]
                for c in range(cells)]
        chain.close()
        # the chain bench.py times: the inner layers write only the next
        # layer's split (WELVET_CHAIN_INNER_NOT_KEPT, 128 x 256 tiles at 64
        # cells). Its last outputs must equal the kept chain's bit for bit.
        last = len(kinds)
        for c in range(cells):
            hip.memset(bufs[c][last], 0xFF, batch * d * 4)  # NaN until written
        lean = gpu.DenseChain(groups, keep_inner=False)
        lean.execute()
        hip.sync()
        lean_out = [hip.download(bufs[c][last], (batch, d)) for c in range(cells)]
        lean.close()
        for g in groups:
            g.close()
    finally:
        for row in sessions:
            for s in row:
                s.close()
        for b in bufs:
            for p in b:
                hip.free(p)
    for c in range(cells):
        assert np.array_equal(lean_out[c].view(np.uint32), outs[c][-1].view(np.uint32)), c
    worst = 0.0
    for c in range(cells):
        cur = xs[c]
        for li, (dt, sc) in enumerate(kinds):
            want, _ = oracle.dense(dequant(oracle, dt, sc, Ws[c][li]), cur, threads=THREADS)
            err = rel_l2(outs[c][li], want)
            worst = max(worst, err)
            assert err <= tol(batch), (c, li, err)
            cur = outs[c][li]  # the next layer is checked on the GPU's own input
    assert np.isfinite(worst)
