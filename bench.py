"""Benchmark of the int8 quantize -> int8 GEMM -> dequantize hot path on one MI355X.

Headline (BASELINE.json metric "int8 GEMM TOPS @8192^3 (% of i8 MFMA peak);
quant/dequant GB/s (% HBM)"): a step is one int8 GEMM of config C3a,
M = N = K = 8192, A/B int8 uniform in [-127, 127], per-tensor scales
0.01 / 0.02, int32 accumulation, fused dequantize to fp32.  `value` is TOPS
(2*M*N*K ops per step) with every operand already resident in HBM.  The
quantize / dequantize half of the metric is measured on config C2 (1 GiB fp32
[16384, 16384], 0.1% +-50 outliers, per-row scales) and reported in
"quant_dequant" with its own roofline; the fp32 matmul of config C3b
(4096^3) is reported in "fp32_matmul".

Timing: HIP events recorded on the library stream around exactly --steps
launches after --warmup untimed ones, device synchronized on both sides.
CPU baseline: the reference's own compiled backend/cpu/src/Ops.cpp matmul
(oracle/_ref) -- what the reference runs for a quantized Linear after
dequantizing the weight (python/kansai/quantize.py:115-122) -- on one core,
over a time-bounded slab of rows of the same workload.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published peaks (dense): int8 5.0 POP/s, fp32 157.3 TFLOP/s, HBM 8 TB/s.
PEAK_INT8_TOPS = 5000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_kernel(fn, steps, warmup):
    """Average ms per call of fn() over `steps` back-to-back calls, HIP events
    on the library stream, synchronized before and after."""
    from kansai_amd import _native as N
    for _ in range(warmup):
        fn()
    N.synchronize()
    e0, e1 = N.Event(), N.Event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    N.synchronize()
    return e0.elapsed_ms(e1) / steps


def measured_traffic(kernel_key):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(kernel_key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def bench_gemm(H, D, steps, warmup):
    M = N = K = 8192
    gen = np.random.Generator(np.random.PCG64(3))
    a = D.from_host(gen.integers(-127, 128, (M, K), dtype=np.int8))
    b = D.from_host(gen.integers(-127, 128, (N, K), dtype=np.int8))
    sa = D.from_host(np.array([0.01]))
    sb = D.from_host(np.array([0.02]))
    from kansai_amd import _native as Nn
    out = D([M, N], "float32")
    args = (a.ptr, b.ptr, M, N, K, sa.ptr, 0, sb.ptr, 0, None, out.ptr, None)
    fn = lambda: Nn.call("kh_gemm_i8", *args)  # noqa: E731
    ms = time_kernel(fn, steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    return ms, tops, (a, b)


def bench_quant_dequant(H, D, steps, warmup):
    rows = cols = 16384
    gen = np.random.Generator(np.random.PCG64(2024))
    x = gen.standard_normal((rows, cols), dtype=np.float32)
    n_out = rows * cols // 1000
    idx = gen.choice(rows * cols, size=n_out, replace=False)
    x.reshape(-1)[idx] = np.where(gen.random(n_out) < 0.5, -50.0, 50.0).astype(np.float32)
    xd = D.from_host(x)
    del x
    from kansai_amd import _native as Nn
    q = D([rows, cols], "int8")
    s = D([rows], "float64")
    out = D([rows, cols], "float32")
    qfn = lambda: Nn.call("kh_quantize_rows", xd.ptr, rows, cols, q.ptr, s.ptr)  # noqa: E731
    dfn = lambda: Nn.call("kh_dequantize_rows", q.ptr, rows, cols, s.ptr, out.ptr)  # noqa: E731
    qms = time_kernel(qfn, steps, warmup)
    dms = time_kernel(dfn, steps, warmup)
    Nn.synchronize()
    nbytes = 5.0 * rows * cols  # quantize: 4 read + 1 written per element; dequantize: 1 read + 4 written
    return qms, dms, nbytes


def bench_f32(H, D, steps, warmup):
    n = 4096
    gen = np.random.Generator(np.random.PCG64(4))
    a = D.from_host(gen.standard_normal((n, n), dtype=np.float32))
    b = D.from_host(gen.standard_normal((n, n), dtype=np.float32))
    out = D([n, n], "float32")
    from kansai_amd import _native as Nn
    fn = lambda: Nn.call("kh_matmul_f32", a.ptr, b.ptr, out.ptr, n, n, n, None)  # noqa: E731
    ms = time_kernel(fn, steps, warmup)
    return ms, 2.0 * n ** 3 / (ms * 1e-3) / 1e12


def cpu_baseline(budget_s=12.0):
    """The reference's compiled fp32 i-k-j matmul (oracle/_ref, built from
    backend/cpu/src/Ops.cpp) on dequantized operands of the C3a workload,
    one core, rows processed in slabs until budget_s elapses."""
    from oracle import oracle as O
    K = N = 8192
    gen = np.random.Generator(np.random.PCG64(3))
    bq = gen.integers(-127, 128, (K, N), dtype=np.int8)
    b = (bq.astype(np.float64) * 0.02).astype(np.float32)  # dequantize(W), quantize.py:76
    del bq
    slab = 4
    a = (gen.integers(-127, 128, (slab, K), dtype=np.int8).astype(np.float64) * 0.01).astype(np.float32)
    use_ref = O.ref_available()
    mm = O.ref_matmul if use_ref else O.ko_matmul_f32
    rows = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and rows < 1024:
        mm(a, b)
        rows += slab
    dt = time.perf_counter() - t0
    tops = 2.0 * rows * N * K / dt / 1e12
    return {
        "value": tops,
        "unit": "TOPS",
        "cores": 1,
        "kind": "reference" if use_ref else "port",
        "sample": (f"{rows} rows x 8192 x 8192 of C3a through the reference's fp32 i-k-j matmul "
                   f"(backend/cpu/src/Ops.cpp:322-339, -O3, 1 thread) on dequantized operands, {dt:.1f} s; "
                   f"host {os.cpu_count()} logical CPUs"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the int8 path has no multi-GPU leg "
                                   "(rows/columns would shard with zero exchange); run with --gpus 1"}))
        sys.exit(2)

    from kansai_amd import _native as Nn
    from kansai_amd import hip as H
    from kansai_amd.device import DeviceTensor as D
    if not H.available():
        raise SystemExit("bench: no gfx950 GPU visible")
    info = Nn.device_info()
    log(f"device {info}")

    log("int8 GEMM 8192^3 ...")
    g_ms, g_tops, keep = bench_gemm(H, D, args.steps, args.warmup)
    log(f"int8 GEMM: {g_ms:.4f} ms/step, {g_tops:.1f} TOPS")
    del keep
    Nn.call("kh_pool_trim")
    log("quantize/dequantize C2 ...")
    q_ms, d_ms, qd_bytes = bench_quant_dequant(H, D, args.steps, args.warmup)
    q_gbs = qd_bytes / (q_ms * 1e-3) / 1e9
    d_gbs = qd_bytes / (d_ms * 1e-3) / 1e9
    log(f"quantize {q_ms:.4f} ms ({q_gbs:.0f} GB/s), dequantize {d_ms:.4f} ms ({d_gbs:.0f} GB/s)")
    Nn.call("kh_pool_trim")
    log("fp32 matmul 4096^3 ...")
    f_ms, f_tflops = bench_f32(H, D, max(5, args.steps // 2), max(2, args.warmup // 2))
    log(f"fp32 matmul: {f_ms:.4f} ms, {f_tflops:.1f} TFLOP/s")
    Nn.call("kh_pool_trim")

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline()
        log(f"CPU baseline {cpu['value']:.6f} TOPS")

    result = {
        "metric": "int8 GEMM TOPS @8192^3 (% of i8 MFMA peak); quant/dequant GB/s (% HBM)",
        "value": round(g_tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "C3a int8 GEMM M=N=K=8192, int32 accumulate, fused dequantize (sa=0.01, sb=0.02) "
                               "to fp32", "M": 8192, "N": 8192, "K": 8192, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(g_tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(g_tops / PEAK_INT8_TOPS, 4), "traffic": measured_traffic("gemm_i8_8192")},
        "quant_dequant": {
            "workload": "C2 per-row quantize and dequantize of fp32 [16384,16384] (1 GiB), 0.1% +-50 outliers",
            "quantize": {"ms": round(q_ms, 5), "GB/s": round(q_gbs, 1),
                         "roofline": {"bound": "hbm", "achieved": round(q_gbs, 1), "peak": PEAK_HBM_GBS,
                                      "unit": "GB/s", "frac": round(q_gbs / PEAK_HBM_GBS, 4),
                                      "traffic": measured_traffic("quant_rows_16384")}},
            "dequantize": {"ms": round(d_ms, 5), "GB/s": round(d_gbs, 1),
                           "roofline": {"bound": "hbm", "achieved": round(d_gbs, 1), "peak": PEAK_HBM_GBS,
                                        "unit": "GB/s", "frac": round(d_gbs / PEAK_HBM_GBS, 4),
                                        "traffic": measured_traffic("dequant_rows_16384")}},
        },
        "fp32_matmul": {"workload": "C3b fp32 matmul 4096^3", "ms": round(f_ms, 5), "TFLOP/s": round(f_tflops, 2),
                        "roofline": {"bound": "mfma", "achieved": round(f_tflops, 2), "peak": PEAK_FP32_TFLOPS,
                                     "unit": "TFLOP/s", "frac": round(f_tflops / PEAK_FP32_TFLOPS, 4),
                                     "traffic": None}},
        "cpu_baseline": cpu,
        "device": info,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
