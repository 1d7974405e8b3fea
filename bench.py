"""Throughput of the quantized-weight Dense hot path on one MI355X.

Workload (default): Dense GEMV 4096 -> 4096, FP8 E4M3 weights with one fp32
scale per output row, fp32 in/out, batch 1. One step = one GEMV over one
batch. Weights are mounted (quantized on the device) once per copy; 64
distinct copies (1.07 GB, > 4x the 256 MB MALL) are rotated so each step
streams its weights from HBM. The steps are captured in a HIP graph so the
timing measures the GPU, not Python's launch rate.

Metric: algorithmic bytes / time, with bytes = codes + row scales + x + y
= 16,826,368 B per step (TFLOPS reported beside it). The CPU baseline is the
oracle's restatement of the reference contract (f64 decode, f64 serial-K
matvec) on this host's cores, timed on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "welvet.cuda_amd"))

HBM_PEAK_GBS = 8000.0

# rocprof summaries (kernel stats + FETCH_SIZE/WRITE_SIZE scaled by a copy of
# known size) per workload; `traffic_bytes:` is the measured HBM bytes per launch.
PROFILES = {"c2": "gemv_fp8e4m3_rowscale_4096x4096_b1.txt"}


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


def workloads():
    # name: (desc, dtype, scheme, batch, in, out, algorithmic bytes, flops)
    d = {}
    K = N = 4096
    d["c2"] = ("dense_gemv_4096x4096_fp8e4m3_rowscale_b1", 4, 2, 1, K, N,
               N * K + 4 * N + 4 * K + 4 * N, 2 * N * K)
    d["c1"] = ("dense_512x512_fp8e4m3_tensorscale_b1", 4, 1, 1, 512, 512,
               512 * 512 + 4 + 4 * 512 + 4 * 512, 2 * 512 * 512)
    return d


def cpu_baseline(dtype, scheme, batch, K, N, W, x, nbytes, budget_s=10.0):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np

    import oracle_lib

    orc = oracle_lib.Oracle()
    native, rs, blk = orc.quantize(dtype, scheme, N, K, W)
    threads = max(1, min(16, os.cpu_count() or 1))
    y = np.zeros((batch, N), np.float32)
    import ctypes

    mount = ctypes.c_double()
    u8 = ctypes.POINTER(ctypes.c_uint8)
    fp = ctypes.POINTER(ctypes.c_float)
    args = (dtype, scheme, batch, K, N, native.ctypes.data_as(u8), rs.ctypes.data_as(fp),
            blk.ctypes.data_as(u8), x.ctypes.data_as(fp), y.ctypes.data_as(fp), threads)
    t1 = orc.L.or_cpu_dense_bench(*args, 1, 3, ctypes.byref(mount))
    iters = max(3, int(budget_s / max(t1, 1e-6)))
    per = orc.L.or_cpu_dense_bench(*args, 2, iters, ctypes.byref(mount))
    return {
        "value": round(nbytes / per / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle restatement of the reference Dense contract on this host: f64 decode "
                   f"of the codes ({mount.value * 1e3:.0f} ms mount), then {iters} f64 serial-K "
                   f"matvecs {N}x{K} batch {batch} split over {threads} threads, "
                   f"{per * 1e3:.3f} ms each"),
    }


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1280)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--config", default="c2", choices=sorted(workloads()))
    ap.add_argument("--copies", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (the known-size copy "
                         "that scales the FETCH_SIZE/WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus above 1 is not part of it",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import pywelvet as pw

    if args.copy_calibration:
        copy_calibration(pw, args.copy_calibration << 20, args.steps)
        return

    desc, dtype, scheme, batch, K, N, nbytes, flops = workloads()[args.config]
    pw.check(pw.lib().welvet_cuda_init())
    hip = pw.Hip()
    seed = pw.seed_for(2 if args.config == "c2" else 1)
    W = pw.normal(seed, N * K, 1 / np.sqrt(K)).reshape(N, K)
    x = pw.normal(seed + 500, batch * K).reshape(batch, K)
    copies = max(1, args.copies)
    sessions = [pw.DenseSession(batch, K, N, -1, dtype, scheme, W) for _ in range(copies)]
    dx = hip.upload(x)
    dy = hip.malloc(batch * N * 4)
    stream = hip.stream()

    def enqueue(n):
        def go():
            for i in range(n):
                sessions[i % copies].execute_device(dx, dy, dy, stream)
        return go

    full, rem = divmod(args.steps, copies)
    g_full = hip.capture(stream, enqueue(copies))
    g_rem = hip.capture(stream, enqueue(rem)) if rem else None
    for _ in range(max(1, (args.warmup + copies - 1) // copies)):
        hip.launch(g_full, stream)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    t_wall = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(full):
        hip.launch(g_full, stream)
    if g_rem:
        hip.launch(g_rem, stream)
    hip.record(e1, stream)
    hip.sync()
    t_wall = time.perf_counter() - t_wall
    ms = hip.elapsed_ms(e0, e1)
    per_step_s = ms * 1e-3 / args.steps
    gbs = nbytes / per_step_s / 1e9
    y = hip.download(dy, (batch, N))
    assert np.all(np.isfinite(y))

    cpu = None if args.no_cpu else cpu_baseline(dtype, scheme, batch, K, N, W, x, nbytes)
    line = {
        "metric": "FP8/FP4 Dense GEMV GB/s + GEMM TFLOPS (% roofline), 1 MI355X vs host CPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3",
        "data": "synthetic (seeded splitmix64 normal weights/inputs, random-init)",
        "config": {"workload": desc, "in": K, "out": N, "batch": batch,
                   "scale": "per-row fp32" if scheme == 2 else "per-tensor fp32",
                   "weight_copies_rotated": copies, "algorithmic_bytes_per_step": nbytes,
                   "tflops": round(flops / per_step_s / 1e12, 4), "wall_s": round(t_wall, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.config)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    hip.graph_free(g_full)
    if g_rem:
        hip.graph_free(g_rem)
    for s in sessions:
        s.close()


if __name__ == "__main__":
    main()
