"""Throughput of the quantized-weight Dense hot path on one MI355X.

Default workload (c2): Dense GEMV 4096 -> 4096, FP8 E4M3 weights with one fp32
scale per output row, fp32 in/out, batch 1. One step = one GEMV over one
batch. Weights are mounted (quantized on the device) once per copy; 64
distinct copies (1.07 GB, > 4x the 256 MB MALL) are used in a fixed rotation
that continues across the warmup and the timed regions, so every step reads
a copy last read 64 steps (1.07 GB of weight traffic) earlier and streams it
from HBM. Steps are replayed from captured HIP graphs and timed with HIP
events on the launch stream.

Metric: algorithmic bytes / time for the HBM-bound GEMV workloads (bytes =
codes + scales + x + y, 16,826,368 B per c2 step), useful FLOP/s (2*M*N*K)
for the matrix-core GEMM workloads. The CPU baseline is the oracle's
restatement of the reference contract (f64 decode at mount, f64 serial-K
matvec) on this host's cores, timed on a bounded sample of the same workload,
on all the CPU threads this job is given (at most 16) and on one thread, with
mount and execute reported separately.

Other workloads (--config), each its own line:
  c1     Dense 512 -> 512, E4M3, per-tensor scale, batch 1
  c3     SwiGLU 4096 / 11008, FP4 E2M1 + E8M0 per 32, batch 1 (c3b16: batch 16)
  c4     MHA projection GEMM: 4096 tokens x 1024 -> 1024, E5M2 per-row scales
  c4mha  whole MHA layer: B=8, S=512, d=1024, 16 heads x 64, causal, RoPE
  c5     64 cells x (Dense 1024^2 E4M3 row -> FP4 block-32 -> E4M3 row), batch 256
  c5chain  the same cells as the reference's volume: one 192-layer serial chain (model session)
  c2bwd  Dense backward at the GEMV shape: d_pre, dX = W^T d_pre, dW (4096^2 E4M3 per-row, batch 1)
  gemv_<fmt>  the c2 GEMV shape over a packed block format (q8_0, q4_0, q4_1, q5_0, q5_1,
         q2_k, q3_k, q4_k, q5_k, q6_k, iq4_nl, iq4_xs; quantized on the device from the
         same weights; bytes = packed blocks + x + y)
--read-floor BYTES instead times one streaming read of BYTES (default: the c2
step's 16,826,368) over 64 rotated buffers, the same way: the floor for any
kernel that reads those bytes once.
--probe mfma times the scaled matrix-core instruction alone (issue rate per
operand-format pair, 16x16x128 and 32x32x64); --probe fetch the bytes per
cycle one CU takes from L2 (a 2 MiB region) and from HBM (4 GiB).

The default line (c2) also carries "gemm": the c4 and c5 GEMM workloads timed
the same way in the same run (64 steps each, three FP6 activation terms), with
their useful TFLOP/s against the matrix-core peak (--no-gemm leaves them out).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "welvet.cuda_amd"))

HBM_PEAK_GBS = 8000.0
REPEATS = 3  # timed regions per run; the median is reported
WARMUP_S = 0.2  # warmup lasts at least this long (clocks leave their idle level)
# Untimed steps queued right before every timed region, with no host wait in
# between, lasting about this long: the device runs at its sustained-load
# clock when timing starts (a region that starts after an idle gap of even
# tens of microseconds runs ~4% slower at first).
LEAD_S = 0.01
# dense matrix-core peaks of MI355X (TFLOP/s), the published figures: FP8
# weights (any activation terms) and FP4 weights with E4M3 terms (two- and
# one-term modes) are rated against the FP8 peak; FP4 weights with the
# default three FP6 (E2M3) terms against the FP4/FP6 peak. Measured issue
# rates (--probe mfma): the 16x16x128 f8f6f4 form reaches ~4.1 PFLOP/s with
# an FP8 operand and ~4.6 with FP4/FP6 operands only, the 32x32x64 form ~8.5
# with FP4/FP6 operands. The attention core's products run on the bf16
# matrix cores.
MFMA_FP8_PEAK_TFLOPS = 5000.0
MFMA_FP4_PEAK_TFLOPS = 10070.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "FP8/FP4 Dense GEMV GB/s + GEMM TFLOPS (% roofline), 1 MI355X vs host CPU"
# CPU threads for the baseline: the job's CPU share (the affinity mask),
# capped at the 16 threads a one-GPU job is given on the GPU hosts
CPU_THREAD_CAP = 16
C2_BYTES = 16826368

# rocprof summaries (kernel stats + FETCH_SIZE/WRITE_SIZE scaled by a copy of
# known size) per workload; `traffic_bytes:` is the measured HBM bytes per launch.
PROFILES = {"c2": "gemv_fp8e4m3_rowscale_4096x4096_b1.txt",
            "c2_b2": "gemv_fp8e4m3_rowscale_4096x4096_b2.txt",
            "read_floor": "read_floor_16826368B.txt",
            "c2bwd": "dense_backward_4096x4096_fp8e4m3_rowscale_b1.txt",
            "gemv_q4_k": "gemv_q4_k_4096x4096_b1.txt"}


def measured_traffic(config):
    name = PROFILES.get(config)
    path = os.path.join(ROOT, "profiles", name) if name else None
    if not path or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes:"):
                return int(line.split(":")[1])
    return None


def oracle():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib

    return oracle_lib.Oracle()


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(CPU_THREAD_CAP, n))


def cpu_dense_seconds(orc, dtype, scheme, batch, K, N, W, x, threads, budget_s):
    """(seconds per execute, executes timed, mount seconds) of the oracle's
    reference-contract Dense (f64 W, serial K) on `threads` threads: 3 warmup
    executes, then as many as fit the budget (at least 2)."""
    import numpy as np

    native, rs, blk = orc.quantize(dtype, scheme, N, K, W)
    y = np.zeros((batch, N), np.float32)
    mount = ctypes.c_double()
    u8 = ctypes.POINTER(ctypes.c_uint8)
    fp = ctypes.POINTER(ctypes.c_float)
    x = np.ascontiguousarray(x, np.float32)
    args = (dtype, scheme, batch, K, N, native.ctypes.data_as(u8), rs.ctypes.data_as(fp),
            blk.ctypes.data_as(u8), x.ctypes.data_as(fp), y.ctypes.data_as(fp), threads)
    t1 = orc.L.or_cpu_dense_bench(*args, 0, 1, ctypes.byref(mount))
    iters = max(2, int(budget_s / max(t1, 1e-6)))
    per = orc.L.or_cpu_dense_bench(*args, 3, iters, ctypes.byref(mount))
    return per, iters, mount.value


def cpu_layers(layers, budget_s):
    """Times the Dense layers of one step (list of (dtype, scheme, batch, K,
    N, W, x)) on cpu_threads() threads and on one thread. Returns seconds per
    step for both, the mount seconds and a description."""
    orc = oracle()
    th = cpu_threads()
    per_n = per_1 = mount = 0.0
    parts = []
    share = budget_s / (2 * len(layers))
    for (dt, sc, batch, K, N, W, x) in layers:
        pn, itn, mn = cpu_dense_seconds(orc, dt, sc, batch, K, N, W, x, th, share)
        p1, it1, _ = cpu_dense_seconds(orc, dt, sc, batch, K, N, W, x, 1, share)
        per_n += pn
        per_1 += p1
        mount += mn
        parts.append(f"{N}x{K} batch {batch}: {pn * 1e3:.3f} ms ({itn} runs) on {th} threads, "
                     f"{p1 * 1e3:.3f} ms ({it1} runs) on 1")
    return per_n, per_1, mount, th, "; ".join(parts)


def cpu_record(value_n, value_1, unit, th, per_n, per_1, mount, sample):
    return {"value": value_n, "unit": unit, "cores": th, "kind": "port",
            "value_1thread": value_1, "execute_s": round(per_n, 6),
            "execute_s_1thread": round(per_1, 6), "mount_s": round(mount, 4),
            "host_threads_visible": os.cpu_count(), "sample": sample}


def step_peak(parts):
    """Peak for a step made of products at different matrix-core rates:
    parts = [(flops, peak_tflops)]; the step's useful FLOPs over the time
    they take when each product runs at its own peak."""
    total = sum(f for f, _ in parts)
    return total / sum(f / p for f, p in parts)


# --------------------------------------------------------------------------
# workloads: each builds its sessions and returns a dict with
#   desc, enqueue(i, stream), per_graph, bytes, flops, bound, dtype, config,
#   cpu(budget_s) -> cpu_baseline dict, close()


def dense_workload(pw, hip, name, cfg_id, dtype, scheme, batch, K, N, copies, bound):
    import numpy as np

    seed = pw.seed_for(cfg_id)
    W = pw.normal(seed, N * K, 1 / np.sqrt(K)).reshape(N, K)
    x = pw.normal(seed + 500, batch * K).reshape(batch, K)
    sessions = [pw.DenseSession(batch, K, N, -1, dtype, scheme, W) for _ in range(copies)]
    dx = hip.upload(x)
    dy = hip.malloc(batch * N * 4)
    b = 1 if dtype != 16 else 0.5
    sc = scheme & 15  # backend: scale scheme in bits 0-3, bit 4 two activation terms
    scale_bytes = 4 * N if sc in (1, 2) else (N * ((K + 31) // 32) if sc == 3 else 0)
    nbytes = int(N * K * b) + scale_bytes + 4 * batch * K + 4 * batch * N
    flops = 2 * batch * N * K
    dname = {4: "fp8e4m3", 5: "fp8e5m2", 16: "fp4e2m1"}[dtype]
    sname = {0: "none", 1: "per-tensor fp32", 2: "per-row fp32", 3: "e8m0 per 32"}[sc]

    def enqueue(i, stream):
        sessions[i % copies].execute_device(dx, dy, dy, stream)

    def cpu(budget_s):
        rows = min(batch, 256)
        per_n, per_1, mount, th, desc = cpu_layers([(dtype, sc, rows, K, N, W, x[:rows])],
                                                   budget_s)
        f = batch / rows

        def val(per):
            per_step = per * f
            return round(nbytes / per_step / 1e9, 4) if bound == "hbm" else round(
                flops / per_step / 1e12, 5)

        return cpu_record(val(per_n), val(per_1), "GB/s" if bound == "hbm" else "TFLOP/s", th,
                          per_n * f, per_1 * f, mount,
                          "oracle restatement of the reference Dense contract on this host: f64 "
                          f"decode of the codes at mount ({mount * 1e3:.0f} ms), then f64 serial-K "
                          f"executes: {desc}"
                          + (f"; {rows} of the {batch} rows timed, scaled x{f:g}" if rows < batch
                             else ""))

    def close():
        for s in sessions:
            s.close()
        hip.free(dx)
        hip.free(dy)

    fp6_terms = (scheme & 0x30) == 0  # three FP6 terms unless bit 16 or 32 asks for E4M3 ones
    peak = MFMA_FP4_PEAK_TFLOPS if (dtype == 16 and fp6_terms) else MFMA_FP8_PEAK_TFLOPS
    return {"desc": name, "enqueue": enqueue, "per_graph": copies, "bytes": nbytes,
            "flops": flops, "bound": bound, "dtype": dname, "peak_tflops": peak,
            "config": {"workload": name, "in": K, "out": N, "batch": batch, "scale": sname,
                       "weight_copies_rotated": copies},
            "cpu": cpu, "close": close}


FORMATS = {"q8_0": (1, 32, 34), "q4_0": (2, 32, 18), "q4_1": (3, 32, 20), "q5_0": (4, 32, 22),
           "q5_1": (5, 32, 24), "q2_k": (6, 256, 84), "q3_k": (7, 256, 110),
           "q4_k": (8, 256, 144), "q5_k": (9, 256, 176), "q6_k": (10, 256, 210),
           "iq4_nl": (16, 32, 18), "iq4_xs": (17, 256, 136)}


def format_workload(pw, hip, name, fmt_name, batch, K, N, copies):
    """GEMV over a packed block format (welvet_dense_mount_format), every
    format quantized on the device from N(0, 1/sqrt(K)) weights."""
    import numpy as np

    fmt, qk, bb = FORMATS[fmt_name]
    seed = pw.seed_for(2)
    x = pw.normal(seed + 500, batch * K).reshape(batch, K)
    W = pw.normal(seed, N * K, 1 / np.sqrt(K)).reshape(N, K)
    sessions = [pw.FormatDenseSession(batch, K, N, -1, fmt, W=W) for _ in range(copies)]
    dx = hip.upload(x)
    dy = hip.malloc(batch * N * 4)
    nbytes = N * K // qk * bb + 4 * batch * K + 4 * batch * N

    def enqueue(i, stream):
        sessions[i % copies].execute_device(dx, dy, dy, stream)

    def close():
        for s in sessions:
            s.close()
        hip.free(dx)
        hip.free(dy)

    return {"desc": name, "enqueue": enqueue, "per_graph": copies, "bytes": nbytes,
            "flops": 2 * batch * N * K, "bound": "hbm", "dtype": fmt_name,
            "config": {"workload": name, "in": K, "out": N, "batch": batch,
                       "format": fmt_name.upper(), "packed_bytes": N * K // qk * bb,
                       "weight_copies_rotated": copies,
                       "cpu_baseline": "none: the reference has no implementation of this "
                                       "format (README.md:361-383)"},
            "cpu": None, "close": close}


def swiglu_workload(pw, hip, name, batch, copies):
    import numpy as np

    d, f = 4096, 11008
    seed = pw.seed_for(3)
    G = pw.normal(seed, f * d, 1 / np.sqrt(d)).reshape(f, d)
    U = pw.normal(seed + 1, f * d, 1 / np.sqrt(d)).reshape(f, d)
    D = pw.normal(seed + 2, d * f, 1 / np.sqrt(f)).reshape(d, f)
    x = pw.normal(seed + 500, batch * d).reshape(batch, d)
    sessions = [pw.SwiGLUSession(batch, 1, d, f, 16, 3, G, U, D) for _ in range(copies)]
    dx = hip.upload(x)
    dh = hip.malloc(batch * f * 4)
    dy = hip.malloc(batch * d * 4)
    codes = 3 * f * d // 2
    e8m0 = 2 * f * (d // 32) + d * ((f + 31) // 32)
    # h is materialized: written by gate/up, read by down
    nbytes = codes + e8m0 + batch * (4 * d + 4 * d + 2 * 4 * f)
    flops = 2 * batch * 3 * f * d

    def enqueue(i, stream):
        sessions[i % copies].execute_device(dx, dh, dy, stream)

    def cpu(budget_s):
        hx = np.random.default_rng(1).standard_normal((batch, f)).astype(np.float32)
        per_n, per_1, mount, th, desc = cpu_layers(
            [(16, 3, batch, d, f, G, x), (16, 3, batch, d, f, U, x), (16, 3, batch, f, d, D, hx)],
            budget_s)
        return cpu_record(round(nbytes / per_n / 1e9, 4), round(nbytes / per_1 / 1e9, 4), "GB/s",
                          th, per_n, per_1, mount,
                          "oracle restatement of the reference Dense contract (f64 W, serial K) "
                          f"for gate, up and down at batch {batch} (SiLU product not timed): "
                          + desc)

    def close():
        for s in sessions:
            s.close()
        for p in (dx, dh, dy):
            hip.free(p)

    return {"desc": name, "enqueue": enqueue, "per_graph": copies, "bytes": nbytes,
            "flops": flops, "bound": "hbm", "dtype": "fp4e2m1",
            "config": {"workload": name, "d_model": d, "d_ff": f, "batch": batch,
                       "scale": "e8m0 per 32", "weight_copies_rotated": copies,
                       "h_materialized": True},
            "cpu": cpu, "close": close}


def mha_workload(pw, hip, name, two=0):
    import numpy as np

    B, S, d, H, hd = 8, 512, 1024, 16, 64
    seed = pw.seed_for(4)
    Ws = [pw.normal(seed + i, d * d, 1 / np.sqrt(d)).reshape(d, d) for i in range(4)]
    x = pw.normal(seed + 500, B * S * d).reshape(B * S, d)
    s = pw.MHASession(B, S, d, H, H, hd, S, 1, 0, 5, 2 | two, *Ws)
    dx = hip.upload(x)
    da = hip.malloc(B * S * d * 4)
    dy = hip.malloc(B * S * d * 4)
    proj = 4 * 2 * B * S * d * d
    # attention under the reference's semantics: query t sees keys [0, b*S + s]
    pairs = sum(sum(b * S + s_ + 1 for s_ in range(S)) for b in range(B))
    att = pairs * H * hd * 4
    # the kernel folds the repeated KV-ring rows into multiplicity weights:
    # the same result from B * S * min(S, msl) distinct (query, row) pairs
    att_computed = B * S * S * H * hd * 4
    nbytes = 4 * (d * d + 4 * d) + 4 * B * S * d * 3

    def enqueue(i, stream):
        s.execute_device(dx, da, dy, stream)

    def close():
        s.close()
        for p in (dx, da, dy):
            hip.free(p)

    return {"desc": name, "enqueue": enqueue, "per_graph": 4, "bytes": nbytes,
            "flops": proj + att_computed, "bound": "mfma", "dtype": "fp8e5m2",
            "peak_tflops": step_peak([(proj, MFMA_FP8_PEAK_TFLOPS),
                                      (att_computed, MFMA_BF16_PEAK_TFLOPS)]),
            "config": {"workload": name, "batch": B, "seq": S, "d_model": d, "heads": H,
                       "head_dim": hd, "mask": "causal", "pos": "rope",
                       "projection_flops": proj,
                       "attention_flops_computed": att_computed,
                       "attention_flops_reference_semantics": att,
                       "flops_basis": ("value counts the FLOPs computed: the projections plus "
                                       "the attention over distinct KV-ring rows; the "
                                       "reference's per-key-position count is "
                                       "attention_flops_reference_semantics"),
                       "tflops_reference_semantics": None},
            "flops_ref": proj + att,
            "cpu": None, "close": close}


def cells_workload(pw, hip, name, two=0, keep_inner=False):
    import numpy as np

    cells, batch, d = 64, 256, 1024
    kinds = [(4, 2), (16, 3), (4, 2)]
    sessions, bufs = [], []
    for c in range(cells):
        seed = pw.seed_for(5, c)
        row = []
        for li, (dt, sc) in enumerate(kinds):
            W = pw.normal(seed + 10 * li, d * d, 1 / np.sqrt(d)).reshape(d, d)
            row.append(pw.DenseSession(batch, d, d, -1, dt, sc | two, W))
        sessions.append(row)
        x = pw.normal(seed + 500, batch * d).reshape(batch, d)
        bufs.append([hip.upload(x)] + [hip.malloc(batch * d * 4) for _ in kinds])
    flops = cells * len(kinds) * 2 * batch * d * d
    # the 64 cells are independent: layer li of every cell runs as one group
    # (one matrix-core launch per layer position); the groups form a chain,
    # so each layer's epilogue also writes the next layer's activation split
    # and only the first layer runs the split kernel. A cell returns its last
    # layer's output: unless keep_inner, the first two layers write only the
    # next layer's split (WELVET_CHAIN_INNER_NOT_KEPT)
    groups = [pw.DenseGroup([sessions[c][li] for c in range(cells)],
                            [bufs[c][li] for c in range(cells)],
                            [bufs[c][li + 1] for c in range(cells)],
                            [bufs[c][li + 1] for c in range(cells)]) for li in range(len(kinds))]
    chain = pw.DenseChain(groups, keep_inner=keep_inner)

    def enqueue(i, stream):
        chain.execute(stream)

    def cpu(budget_s):
        rng = np.random.default_rng(5)
        layers = [(dt, sc, batch, d, d, rng.standard_normal((d, d)).astype(np.float32) / 32,
                   rng.standard_normal((batch, d)).astype(np.float32)) for dt, sc in kinds]
        per_n, per_1, mount, th, desc = cpu_layers(layers, budget_s)
        return cpu_record(round(flops / (per_n * cells) / 1e12, 5),
                          round(flops / (per_1 * cells) / 1e12, 6), "TFLOP/s", th, per_n * cells,
                          per_1 * cells, mount * cells,
                          "oracle restatement of the reference Dense contract for one cell (3 "
                          f"layers 1024x1024 at batch {batch}): {desc}; scaled x{cells} to the "
                          "64 cells")

    def close():
        chain.close()
        for grp in groups:
            grp.close()
        for row in sessions:
            for s in row:
                s.close()
        for b in bufs:
            for p in b:
                hip.free(p)

    per_layer = flops // len(kinds)
    fp4_peak = MFMA_FP4_PEAK_TFLOPS if two == 0 else MFMA_FP8_PEAK_TFLOPS
    peak = step_peak([(per_layer, fp4_peak if dt == 16 else MFMA_FP8_PEAK_TFLOPS)
                      for dt, _ in kinds])
    return {"desc": name, "enqueue": enqueue, "per_graph": 1, "bytes": None, "flops": flops,
            "bound": "mfma", "dtype": "fp8e4m3+fp4e2m1", "peak_tflops": peak,
            "config": {"workload": name, "cells": cells, "layers_per_cell": 3, "batch": batch,
                       "width": d, "layer_kinds": "E4M3 per-row, FP4 E8M0/32, E4M3 per-row",
                       "execution": ("independent cells, one grouped launch per layer position, "
                                     "chained: each epilogue writes the next layer's split"),
                       "inner_outputs": ("written (fp32 pre/post of layers 1 and 2)" if keep_inner
                                         else "not written: each cell returns its last layer's "
                                         "output; layers 1 and 2 write only the next split")},
            "cpu": cpu, "close": close}


def chain_workload(pw, hip, name, two=0):
    """The reference's volume semantics for the C5 cells: a WMN1 Grid 4x4x4 of
    Stack cells (Dense 1024^2 each: E4M3 per-row, FP4 E8M0/32, E4M3 per-row),
    run as one 192-layer serial chain by welvet_model_forward_device
    (runtime/forward.cpp:98-156). The scaled stores are quantized by the
    library (a Dense session per layer, exported) and carried in the
    descriptor's store payloads; the model mounts them as stored."""
    import numpy as np

    cells, batch, d = 64, 256, 1024
    kinds = [(4, 2), (16, 3), (4, 2)]
    w = pw.Wire()
    w.u32(0x314E4D57)
    w.i32(2, cells, 4, 4, 4, 1)
    stores = []
    for c in range(cells):
        seed = pw.seed_for(5, c)
        w.i32(19, len(kinds))
        for li, (dt, sc) in enumerate(kinds):
            W = pw.normal(seed + 10 * li, d * d, 1 / np.sqrt(d)).reshape(d, d)
            pw.dense_child(w, d, d, -1, dt, W)
            sess = pw.DenseSession(1, d, d, -1, dt, sc, W)
            stores.append((dt, sc) + sess.export_store(dt))
            sess.close()
    pw.empty_controls(w)
    for c in range(cells):
        pw.empty_controls(w)
        for _ in kinds:
            pw.empty_controls(w)
    w.i32(len(stores))
    for dt, sc, native, rs, blk, ts in stores:
        pw.store_payload(w, dt, d, d, native, scale=ts, scheme=sc, row_scale=rs, blk_exp=blk)
    for c in range(cells):
        w.i32(1, 0, 0, 0, 0, 0)
    model = pw.ModelSession(w.bytes(), scheme=two)  # backend 16: stored payloads, two terms
    x = hip.upload(pw.normal(pw.seed_for(5, 0) + 500, batch * d).reshape(batch, d))
    y = hip.malloc(batch * d * 4)
    flops = cells * len(kinds) * 2 * batch * d * d

    def enqueue(i, stream):
        model.forward_device(x, batch, d, y, batch * d, stream)

    def close():
        model.close()
        hip.free(x)
        hip.free(y)

    per_layer = flops // len(kinds)
    fp4_peak = MFMA_FP4_PEAK_TFLOPS if two == 0 else MFMA_FP8_PEAK_TFLOPS
    peak = step_peak([(per_layer, fp4_peak if dt == 16 else MFMA_FP8_PEAK_TFLOPS)
                      for dt, _ in kinds])
    return {"desc": name, "enqueue": enqueue, "per_graph": 1, "bytes": None, "flops": flops,
            "bound": "mfma", "dtype": "fp8e4m3+fp4e2m1", "direct": True, "peak_tflops": peak,
            "config": {"workload": name, "cells": cells, "layers_per_cell": 3, "batch": batch,
                       "width": d, "layer_kinds": "E4M3 per-row, FP4 E8M0/32, E4M3 per-row "
                                               "(scaled WMN1 store payloads)",
                       "execution": ("reference volume semantics: Grid 4x4x4 of Stack cells, a "
                                     "192-layer serial chain, one welvet_model_forward_device "
                                     "per step (synchronous, not graph-captured)")},
            "cpu": None, "close": close}


def backward_workload(pw, hip, name, copies):
    """Dense backward (the NormalBP leaf, kernels.cu:83-127) at the GEMV shape:
    4096 x 4096 E4M3 with per-row scales, batch 1, Linear. A step is one
    welvet_dense_backward_device: d_pre, dX = W^T d_pre from the codes, and
    the f32 dW [4096][4096]. Weight copies and dW buffers rotate (16 each,
    1.3 GB in all, over 4x the MALL)."""
    import numpy as np

    K = N = 4096
    batch = 1
    seed = pw.seed_for(2)
    W = pw.normal(seed, N * K, 1 / np.sqrt(K)).reshape(N, K)
    x = pw.normal(seed + 500, batch * K).reshape(batch, K)
    g = pw.normal(seed + 600, batch * N).reshape(batch, N)
    sessions = [pw.DenseSession(batch, K, N, -1, 4, 2, W) for _ in range(copies)]
    dx_in, dg = hip.upload(x), hip.upload(g)
    dpre_f = hip.malloc(batch * N * 4)
    dd, ddx = hip.malloc(batch * N * 4), hip.malloc(batch * K * 4)
    ddw = [hip.malloc(N * K * 4) for _ in range(copies)]
    sessions[0].execute_device(dx_in, dpre_f, dpre_f)
    for i, s in enumerate(sessions):  # allocates each session's dX partials before capture
        s.backward_device(dx_in, dpre_f, dpre_f, dg, False, dd, ddx, ddw[i])
    hip.sync()
    # codes + row scales + x + pre + g (inputs), d_pre + dX + dW (outputs)
    nbytes = N * K + 4 * N + 4 * K * batch + 8 * N * batch + 4 * N * batch + 4 * K * batch + 4 * N * K
    flops = 2 * N * K * batch * 2

    def enqueue(i, stream):
        sessions[i % copies].backward_device(dx_in, dpre_f, dpre_f, dg, False, dd, ddx,
                                             ddw[i % copies], None, stream)

    def cpu(budget_s):
        orc = oracle()
        t0 = time.perf_counter()
        native, rs, blk = orc.quantize(4, 2, N, K, W)
        Wd = orc.dequant(4, 2, N, K, native, rs, blk)
        mount = time.perf_counter() - t0
        pre = (x.astype(np.float64) @ Wd.T.astype(np.float64)).astype(np.float32)
        th = cpu_threads()

        def timed(threads, budget):
            for _ in range(3):
                orc.backward(Wd, g, pre, x, -1, threads=threads)
            t1, iters = time.perf_counter(), 0
            while time.perf_counter() - t1 < budget or iters < 2:
                orc.backward(Wd, g, pre, x, -1, threads=threads)
                iters += 1
            return (time.perf_counter() - t1) / iters, iters

        per_n, itn = timed(th, budget_s / 2)
        per_1, it1 = timed(1, budget_s / 2)
        return cpu_record(round(nbytes / per_n / 1e9, 4), round(nbytes / per_1 / 1e9, 4), "GB/s",
                          th, per_n, per_1, mount,
                          "oracle restatement of the reference NormalBP backward (act', f64 serial "
                          "MatVec^T, per-batch-row f32 outer product) on the dequantized f32 W: "
                          f"{per_n * 1e3:.2f} ms ({itn} runs) on {th} threads, {per_1 * 1e3:.2f} "
                          f"ms ({it1} runs) on 1")

    def close():
        for s in sessions:
            s.close()
        for p in [dx_in, dg, dpre_f, dd, ddx] + ddw:
            hip.free(p)

    return {"desc": name, "enqueue": enqueue, "per_graph": copies, "bytes": nbytes, "flops": flops,
            "bound": "hbm", "dtype": "fp8e4m3",
            "config": {"workload": name, "in": K, "out": N, "batch": batch, "scale": "per-row fp32",
                       "act": "linear", "weight_copies_rotated": copies,
                       "outputs": "d_pre, dX [1][4096], dW [4096][4096] f32"},
            "cpu": cpu, "close": close}


def make_workload(pw, hip, config, copies, terms=3, batch=1, keep_inner=False):
    two = {1: 32, 2: 16}.get(terms, 0)  # backend bit for two (16) or one (32) activation terms
    tname = {1: "_1term", 2: "_2terms"}.get(terms, "")
    if config == "c2":
        b = max(1, batch)
        return dense_workload(pw, hip, f"dense_gemv_4096x4096_fp8e4m3_rowscale_b{b}", 2, 4, 2, b,
                              4096, 4096, copies, "hbm")
    if config == "c1":
        return dense_workload(pw, hip, "dense_512x512_fp8e4m3_tensorscale_b1", 1, 4, 1, 1,
                              512, 512, copies, "hbm")
    if config == "c3":
        b = max(1, batch)
        return swiglu_workload(pw, hip, f"swiglu_4096x11008_fp4_e8m0_b{b}", b, min(copies, 8))
    if config == "c3b16":
        return swiglu_workload(pw, hip, "swiglu_4096x11008_fp4_e8m0_b16", 16, min(copies, 8))
    if config == "c4":
        return dense_workload(pw, hip, "mha_projection_gemm_4096x1024x1024_fp8e5m2_rowscale"
                              + tname, 4, 5, 2 | two, 4096, 1024, 1024,
                              min(copies, 4), "mfma")
    if config == "c4mha":
        return mha_workload(pw, hip, "mha_layer_b8_s512_d1024_h16_fp8e5m2_rowscale"
                            + tname, two)
    if config == "c2bwd":
        return backward_workload(pw, hip, "dense_backward_4096x4096_fp8e4m3_rowscale_b1", 16)
    if config == "c5chain":
        return chain_workload(pw, hip, "volume_grid_4x4x4_stack3_dense_1024_b256_serial"
                              + tname, two)
    if config.startswith("gemv_"):
        f = config[len("gemv_"):]
        b = max(1, batch)
        return format_workload(pw, hip, f"dense_gemv_4096x4096_{f}_b{b}", f, b, 4096, 4096, copies)
    if config == "c5":
        return cells_workload(pw, hip, "volume_64_cells_3x_dense_1024_b256"
                              + tname + ("_inner_kept" if keep_inner else ""),
                              two, keep_inner)
    raise SystemExit(f"unknown config {config}")


def lib_layout(pw, hip):
    """Prints the executable mappings of this process and the addresses of a
    few runtime entry points after one small Dense mount and execute, so that
    the frames of a native backtrace taken under a profiler can be assigned to
    libraries (libraries loaded at start keep their relative offsets from run
    to run)."""
    import numpy as np

    W = pw.normal(1, 256 * 256, 0.05).reshape(256, 256)
    s = pw.DenseSession(1, 256, 256, -1, 4, 2, W)
    s.execute(np.ones((1, 256), np.float32))

    def addr(lib, name):
        return hex(ctypes.cast(getattr(lib, name), ctypes.c_void_p).value)

    libc = ctypes.CDLL("libc.so.6")
    hl = ctypes.CDLL("libamdhip64.so.7")
    print("libc memcpy", addr(libc, "memcpy"), "sigaction", addr(libc, "sigaction"))
    print("hipMemcpyAsync", addr(hl, "hipMemcpyAsync"), "hipLaunchKernel", addr(hl, "hipLaunchKernel"))
    print("welvet_dense_mount_q", addr(pw.lib(), "welvet_dense_mount_q"))
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and ".so" in parts[5] and "x" in parts[1]:
                print(parts[0], parts[1], os.path.basename(parts[5]))
    s.close()


def copy_calibration(pw, nbytes, steps):
    """Times `steps` device-to-device copies of nbytes (read nbytes, write nbytes)."""
    pw.check(pw.lib().welvet_cuda_init())
    hip = pw.Hip()
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.memset(src, 1, nbytes)
    stream = hip.stream()
    hip.copy_async(dst, src, nbytes, stream)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(steps):
        hip.copy_async(dst, src, nbytes, stream)
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1) / steps
    print(json.dumps({"copy_bytes": nbytes, "steps": steps, "ms_per_copy": round(ms, 6),
                      "GB/s_read_plus_write": round(2 * nbytes / ms / 1e6, 1)}), flush=True)
    hip.free(src)
    hip.free(dst)


MFMA_FORMATS = {0: "E4M3", 1: "E5M2", 2: "FP6 E2M3", 4: "FP4 E2M1"}
CLOCK_GHZ = 2.4  # MI355X peak engine clock: cycles below are at this clock


def best_ms(hip, stream, launch, reps=3):
    """Shortest of `reps` event-timed launches, after one untimed launch."""
    e0, e1 = hip.event(), hip.event()
    launch()
    hip.sync()
    best = None
    for _ in range(reps):
        hip.record(e0, stream)
        launch()
        hip.record(e1, stream)
        ms = hip.elapsed_ms(e0, e1)
        best = ms if best is None else min(best, ms)
    return best


def probe_mfma(pw, hip):
    """Issue rate of the scaled f8f6f4 matrix-core instruction: 2048
    workgroups of 4 waves, each wave 1000 rounds of 8 independent 16x16x128
    MFMAs (or 4 of 32x32x64: the same multiply-adds)."""
    wgs, iters, simds = 2048, 1000, 1024
    out = hip.malloc(4 * 256 * wgs)
    stream = hip.stream()
    rows = []
    for fa, fb in ((0, 0), (2, 0), (2, 1), (2, 4), (4, 4)):
        for shape in (16, 32):
            def launch():
                pw.check(pw.lib().welvet_mfma_probe(fa, fb, shape, iters, wgs, ctypes.c_void_p(out),
                                                    256 * wgs, ctypes.c_void_p(stream)))
            ms = best_ms(hip, stream, launch)
            macs = wgs * 4 * iters * 8 * 32768
            per_simd = wgs * 4 * iters * 8 / simds  # 16x16x128-equivalent MFMAs per SIMD
            rows.append({"a": MFMA_FORMATS[fa], "b": MFMA_FORMATS[fb],
                         "shape": "16x16x128" if shape == 16 else "32x32x64",
                         "ms": round(ms, 4), "tflops": round(2 * macs / ms / 1e9, 1),
                         "cycles_per_16x16x128": round(ms * 1e-3 * CLOCK_GHZ * 1e9 / per_simd, 1)})
    hip.free(out)
    print(json.dumps({"probe": "mfma_issue_rate", "clock_ghz": CLOCK_GHZ, "workgroups": wgs,
                      "waves_per_workgroup": 4, "rows": rows}), flush=True)


def probe_fetch(pw, hip):
    """Bytes per cycle per CU read from an L2-resident region (2 MiB) and
    from HBM (a 4 GiB buffer, every 64 KiB region read once per launch)."""
    big, small, cus = 4 << 30, 2 << 20, 256
    buf = hip.malloc(big)
    hip.memset(buf, 1, big)
    stream = hip.stream()
    rows = []
    for per_cu in (1, 4):
        wgs = cus * per_cu
        out = hip.malloc(4 * wgs)
        for name, region, iters in (("l2", small, 64), ("hbm", big, (big >> 16) // wgs)):
            def launch():
                pw.check(pw.lib().welvet_fetch_probe(ctypes.c_void_p(buf), region, iters, wgs,
                                                     ctypes.c_void_p(out), wgs, ctypes.c_void_p(stream)))
            ms = best_ms(hip, stream, launch)
            nbytes = wgs * iters * 65536
            rows.append({"source": name, "region_bytes": region, "workgroups": wgs,
                         "bytes": nbytes, "ms": round(ms, 4), "GB/s": round(nbytes / ms / 1e6, 1),
                         "bytes_per_cycle_per_cu": round(nbytes / (ms * 1e-3) / cus / (CLOCK_GHZ * 1e9), 2)})
        hip.free(out)
    hip.free(buf)
    print(json.dumps({"probe": "fetch_rate", "clock_ghz": CLOCK_GHZ, "cus": cus,
                      "loads": "16-byte, 4 per lane in flight, 256-lane workgroups", "rows": rows}),
          flush=True)


def read_floor_workload(pw, hip, nbytes, copies):
    """One streaming read of nbytes per step over `copies` rotated buffers."""
    bufs = [hip.malloc(nbytes) for _ in range(copies)]
    for b in bufs:
        hip.memset(b, 0x5A, nbytes)
    words = pw.lib().welvet_read_probe_words(nbytes)
    out = hip.malloc(4 * words)

    def enqueue(i, stream):
        pw.check(pw.lib().welvet_read_probe(ctypes.c_void_p(bufs[i % copies]), nbytes,
                                            ctypes.c_void_p(out), words, ctypes.c_void_p(stream)))

    def close():
        for b in bufs + [out]:
            hip.free(b)

    return {"desc": "read_floor", "enqueue": enqueue, "per_graph": copies, "bytes": nbytes,
            "flops": 0, "bound": "hbm", "dtype": "u8",
            "config": {"workload": f"streaming_read_{nbytes}B", "buffers_rotated": copies,
                       "loads": "16-byte non-temporal, 4 per lane in flight, one XOR digest "
                                "per 256-lane workgroup"},
            "cpu": None, "close": close}


CONFIGS = ["c1", "c2", "c3", "c3b16", "c4", "c4mha", "c5", "c5chain", "c2bwd"] + [
    "gemv_" + f for f in FORMATS]


class Runner:
    """Steps replayed from captured graphs in one rotation over the workload's
    copies (step i uses copy i mod copies) that continues from one call to the
    next, so every step reads the copy least recently used. A graph of n
    steps from rotation offset o is captured once and kept."""

    def __init__(self, pw, hip, wl, stream):
        self.pw, self.hip, self.wl, self.stream = pw, hip, wl, stream
        self.per = max(1, wl["per_graph"])
        self.direct = wl.get("direct", False)  # synchronous calls: no capture
        self.offset = 0
        self.graphs = {}

    def _graph(self, start, count):
        key = (start % self.per, count)
        if key not in self.graphs:
            def go():
                for i in range(start, start + count):
                    self.wl["enqueue"](i, self.stream)
            self.graphs[key] = self.hip.capture(self.stream, go)
        return self.graphs[key]

    def prepare(self, n):
        """Captures the graphs a call of n steps from the current offset uses."""
        if self.direct:
            return
        full, rem = divmod(n, self.per)
        if full:
            self._graph(self.offset, self.per)
        if rem:
            self._graph(self.offset, rem)

    def run(self, n):
        """Queues n steps (call prepare(n) first to keep capture out of timing)."""
        if self.direct:
            for i in range(self.offset, self.offset + n):
                self.wl["enqueue"](i, self.stream)
            self.offset = (self.offset + n) % self.per
            return
        full, rem = divmod(n, self.per)
        for _ in range(full):
            self.hip.launch(self._graph(self.offset, self.per), self.stream)
        if rem:
            self.hip.launch(self._graph(self.offset, rem), self.stream)
            self.offset = (self.offset + rem) % self.per

    def timed(self, steps, stamps):
        """The graph of one timed region: an untimed rotation, a device clock
        stamp into stamps[0], `steps` steps, a stamp into stamps[1], all
        captured as one graph (kept per rotation offset and length). No graph
        launch falls inside the timed steps, whatever `steps` is."""
        key = ("timed", self.offset % self.per, steps)
        if key not in self.graphs:
            start = self.offset
            L = self.pw.lib()

            def go():
                for i in range(start, start + self.per):
                    self.wl["enqueue"](i, self.stream)
                self.pw.check(L.welvet_clock_stamp(ctypes.c_void_p(stamps), ctypes.c_void_p(self.stream)))
                for i in range(start + self.per, start + self.per + steps):
                    self.wl["enqueue"](i, self.stream)
                self.pw.check(L.welvet_clock_stamp(ctypes.c_void_p(stamps + 8),
                                                   ctypes.c_void_p(self.stream)))
            g = self.hip.capture(self.stream, go)
            # one untimed launch: a graph's first launch also uploads its
            # nodes' kernel arguments, which later launches reuse
            self.hip.launch(g, self.stream)
            self.hip.sync()
            self.graphs[key] = g
        return self.graphs[key]

    def close(self):
        for g in self.graphs.values():
            self.hip.graph_free(g)
        self.graphs = {}


def measure(pw, hip, wl, steps, want):
    """Warmup, then REPEATS timed regions of exactly `steps` steps of wl; the
    median region time in ms (less the clock stamps' own cost), all regions,
    the warmup steps run and the Runner (still holding the graphs)."""
    stream = hip.stream()
    runner = Runner(pw, hip, wl, stream)

    # warmup: at least the requested steps and at least WARMUP_S seconds, in
    # whole rotations (the clocks start from their idle level)
    runner.prepare(runner.per)
    warmup, t0 = 0, time.perf_counter()
    while warmup < want or time.perf_counter() - t0 < WARMUP_S:
        runner.run(runner.per)
        hip.sync()
        warmup += runner.per
    # lead-in before each timed region: whole rotations, about LEAD_S long
    per_step_est = (time.perf_counter() - t0) / max(1, warmup)
    lead = runner.per * max(1, int(LEAD_S / (per_step_est * runner.per) + 0.999))
    # The timed region (exactly `steps` steps between device synchronizations)
    # runs REPEATS times; the median is reported, so one disturbed run does not
    # become the result (the three times are in config.ms_runs).
    e0, e1 = hip.event(), hip.event()
    runs = []
    t_wall = 0.0
    # Graph-replayed workloads: each region is one captured graph holding an
    # untimed rotation, a device clock stamp, the `steps` timed steps and a
    # second stamp (Runner.timed), so the steps run back to back with no
    # graph launch among them at any `steps`; the region's time is the
    # difference of the two stamps. Direct workloads (synchronous calls) are
    # timed between events recorded around the calls.
    stamps = hip.malloc(16)
    khz = pw.lib().welvet_clock_rate_khz()

    def stamped(n):
        """ms between the two stamps of one region of n steps."""
        import numpy as np
        g = runner.timed(n, stamps)
        hip.sync()
        runner.run(lead)
        hip.launch(g, stream)
        runner.offset = (runner.offset + n) % runner.per
        hip.sync()
        t = hip.download(stamps, (2,), np.uint64)
        return float(int(t[1]) - int(t[0])) / khz

    # The stamps' own cost (the first stamp's run and the second's dispatch,
    # the same in every region) is the median time of regions with no steps;
    # it is subtracted from every timed region.
    stamp_ms = 0.0 if runner.direct else sorted(stamped(0) for _ in range(5))[2]
    for _ in range(REPEATS):
        if runner.direct:
            hip.sync()
            t1 = time.perf_counter()
            hip.record(e0, stream)
            runner.run(steps)
            hip.record(e1, stream)
        else:
            g = runner.timed(steps, stamps)
            hip.sync()
            t1 = time.perf_counter()
            runner.run(lead)
            hip.launch(g, stream)
            runner.offset = (runner.offset + steps) % runner.per
        hip.sync()
        t_wall += time.perf_counter() - t1
        if runner.direct:
            runs.append(hip.elapsed_ms(e0, e1))
        else:
            import numpy as np
            t = hip.download(stamps, (2,), np.uint64)
            runs.append(float(int(t[1]) - int(t[0])) / khz - stamp_ms)
    hip.free(stamps)
    return {"runner": runner, "warmup": warmup, "runs": runs, "ms": sorted(runs)[len(runs) // 2],
            "stamp_ms": stamp_ms, "lead": lead, "t_wall": t_wall / REPEATS}


# The GEMM half of the metric, measured in the same run as the default GEMV
# line: the MHA projection GEMM and the 64-cell volume, three FP6 activation
# terms (the defaults).
GEMM_LINE = ("c4", "c5")


def gemm_summary(pw, hip, config, copies):
    wl = make_workload(pw, hip, config, copies)
    try:
        steps = 64
        m = measure(pw, hip, wl, steps, 0)
        m["runner"].close()
    finally:
        wl["close"]()
    per_step_s = m["ms"] * 1e-3 / steps
    tflops = wl["flops"] / per_step_s / 1e12
    peak = wl.get("peak_tflops", MFMA_FP8_PEAK_TFLOPS)
    return {"workload": wl["config"]["workload"], "ms_per_step": round(m["ms"] / steps, 6),
            "tflops": round(tflops, 2), "peak_tflops": round(peak, 1),
            "frac": round(tflops / peak, 4), "dtype": wl["dtype"], "activation_terms": 3,
            "steps": steps, "ms_runs": [round(r, 4) for r in m["runs"]]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: 1280 for the GEMV workloads, 64 for the rest)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps; the warmup also lasts at least WARMUP_S seconds")
    ap.add_argument("--config", default="c2", choices=CONFIGS)
    ap.add_argument("--copies", type=int, default=64)
    ap.add_argument("--batch", type=int, default=1,
                    help="batch rows of c2, c3 and of the packed-format GEMV configs (gemv_<fmt>)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--terms", type=int, default=3, choices=(1, 2, 3),
                    help="activation terms of the matrix-core GEMMs (c4, c4mha, c5, c5chain): "
                         "3 (default), 2 (backend bit 16) or 1 (backend bit 32: the throughput mode, "
                         "outside the 1e-3 bound)")
    ap.add_argument("--keep-inner", action="store_true",
                    help="c5: also write the fp32 outputs of each cell's first two layers")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (the known-size copy "
                         "that scales the FETCH_SIZE/WRITE_SIZE counters) and exit")
    ap.add_argument("--read-floor", type=int, nargs="?", const=C2_BYTES, default=0,
                    metavar="BYTES",
                    help="time a plain streaming read of BYTES (default: the c2 step's bytes) "
                         "instead of a workload")
    ap.add_argument("--no-gemm", action="store_true",
                    help="c2: leave out the GEMM workloads (c4, c5) that the default line also times")
    ap.add_argument("--lib-layout", action="store_true",
                    help="only print the process's library mappings after a small mount")
    ap.add_argument("--probe", choices=("mfma", "fetch"), default=None,
                    help="only run a hardware probe: the scaled MFMA issue rate or the per-CU "
                         "fetch rate from L2 and HBM")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: measures one GPU; --gpus above 1 is not part of it",
              file=sys.stderr)
        sys.exit(2)

    import pywelvet as pw

    if args.copy_calibration:
        copy_calibration(pw, args.copy_calibration << 20, args.steps or 10)
        return

    pw.check(pw.lib().welvet_cuda_init())
    hip = pw.Hip()
    if args.probe:
        (probe_mfma if args.probe == "mfma" else probe_fetch)(pw, hip)
        return
    if args.lib_layout:
        lib_layout(pw, hip)
        return
    if args.read_floor:
        wl = read_floor_workload(pw, hip, args.read_floor, max(1, args.copies))
        gemv = True
    else:
        wl = make_workload(pw, hip, args.config, max(1, args.copies), args.terms, args.batch,
                           args.keep_inner)
        gemv = args.config in ("c1", "c2", "c3", "c3b16")
    steps = args.steps if args.steps is not None else (1280 if gemv else 64)
    steps = max(1, steps)
    want = args.warmup if args.warmup is not None else 0
    m = measure(pw, hip, wl, steps, want)
    runner, warmup, runs, ms = m["runner"], m["warmup"], m["runs"], m["ms"]
    stamp_ms, lead, t_wall = m["stamp_ms"], m["lead"], m["t_wall"]
    per_step_s = ms * 1e-3 / steps

    # profiles are per workload: the batch rows of c2 and c3 are part of it
    traffic_key = args.config + (f"_b{args.batch}" if args.batch > 1 and args.config in ("c2", "c3") else "")
    tflops = wl["flops"] / per_step_s / 1e12
    gbs = wl["bytes"] / per_step_s / 1e9 if wl["bytes"] else None
    if wl["bound"] == "hbm":
        value, unit = gbs, "GB/s"
        roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic("read_floor" if args.read_floor else traffic_key)}
    else:
        value, unit = tflops, "TFLOP/s"
        peak = wl.get("peak_tflops", MFMA_FP8_PEAK_TFLOPS)
        roof = {"bound": "mfma", "achieved": round(tflops, 3), "peak": round(peak, 1),
                "unit": "TFLOP/s", "frac": round(tflops / peak, 4),
                "traffic": measured_traffic(traffic_key)}
    cpu = None if (args.no_cpu or wl["cpu"] is None) else wl["cpu"](16.0)
    config = dict(wl["config"])
    rotated = min(runner.per, steps) if runner.direct else runner.per
    config.update({"timer": ("HIP events around the synchronous calls" if runner.direct else
                             "device wall-clock stamps captured in the region's graph, "
                             f"less the stamps' own cost ({stamp_ms * 1e3:.3f} us, the median "
                             "of empty regions)"),
                   "lead_in_steps": 0 if runner.direct else lead})
    config.update({"tflops": round(tflops, 4), "wall_s": round(t_wall, 4),
                   "ms_runs": [round(r, 4) for r in runs], "timed_regions": REPEATS,
                   "copies_rotated": rotated,
                   "rotation": ("one rotation over the copies continuing across warmup and "
                                "timed regions: each step reads the least recently used copy")})
    config.pop("weight_copies_rotated", None)
    if "tflops_reference_semantics" in config:
        config["tflops_reference_semantics"] = round(wl["flops_ref"] / per_step_s / 1e12, 4)
    if wl["bound"] == "mfma":
        config["activation_terms"] = args.terms
    if wl["bytes"]:
        config.update({"algorithmic_bytes_per_step": wl["bytes"], "gbs": round(gbs, 2)})
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms / steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic (seeded splitmix64 normal weights/inputs, random-init)",
        "config": config,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    runner.close()
    wl["close"]()
    if args.config == "c2" and not args.read_floor and not args.no_gemm:
        # the GEMM half of the metric, same process and device (after the
        # GEMV's buffers are freed)
        line["gemm"] = [gemm_summary(pw, hip, c, max(1, args.copies)) for c in GEMM_LINE]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
