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

    python bench.py [--gpus 1] [--steps 50] [--warmup 50] [--no-cpu] [--only gemm,probe,quant,f32,c1,skinny,c4,copy,pcie]

Profiling (the summaries under profiles/ are made this way):
    rocprofv3 --kernel-trace --stats -d OUT/trace -o run --output-format csv -- python3 bench.py --no-cpu
    rocprofv3 --pmc FETCH_SIZE -d OUT/fetch -o run --output-format csv -- python3 bench.py --only gemm,quant,copy --steps 3 --warmup 1 --no-cpu
    rocprofv3 --pmc WRITE_SIZE -d OUT/write -o run --output-format csv -- python3 bench.py --only gemm,quant,copy --steps 3 --warmup 1 --no-cpu
    python3 bench.py --summarize OUT
"copy" runs a 1 GiB device-to-device copy: the calibration that turns the
FETCH_SIZE / WRITE_SIZE readings of the other kernels into HBM bytes.
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
    from kansaiml_amd import _native as N
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


def _r(x, nd):
    return None if x != x else round(x, nd)


def bench_gemm(H, D, steps, warmup):
    M = N = K = 8192
    gen = np.random.Generator(np.random.PCG64(3))
    a = D.from_host(gen.integers(-127, 128, (M, K), dtype=np.int8))
    b = D.from_host(gen.integers(-127, 128, (N, K), dtype=np.int8))
    sa = D.from_host(np.array([0.01]))
    sb = D.from_host(np.array([0.02]))
    from kansaiml_amd import _native as Nn
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
    from kansaiml_amd import _native as Nn
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
    from kansaiml_amd import _native as Nn
    fn = lambda: Nn.call("kh_matmul_f32", a.ptr, b.ptr, out.ptr, n, n, n, None)  # noqa: E731
    ms = time_kernel(fn, steps, warmup)
    return ms, 2.0 * n ** 3 / (ms * 1e-3) / 1e12


def bench_skinny(steps, warmup):
    """Config C5: kh_linear_i8 (per-token quantize of fp32 x, int8 GEMM,
    per-output-channel weight scales, fused epilogue) for M in {1, 8, 32},
    (K, N) in {(4096, 4096), (4096, 11008)}.  Weight copies are rotated so
    more than 512 MB of distinct weights pass through HBM (beyond the 256 MB
    Infinity Cache).  `us` is the average over `steps` calls issued back to
    back between one pair of HIP events (a decode loop's dependent layer
    calls); `us_single` brackets each call with its own events (launch
    latency included, host gaps excluded)."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd.device import DeviceTensor as D
    gen = np.random.Generator(np.random.PCG64(5))
    rows = []
    for K, N in ((4096, 4096), (4096, 11008)):
        copies = max(2, -(-(512 << 20) // (N * K)))
        ws = [D([N, K], "int8") for _ in range(copies)]
        w0 = gen.integers(-127, 128, (N, K), dtype=np.int8)
        for w in ws:
            Nn.call("kh_memcpy_h2d", w.ptr, w0.ctypes.data, N * K)
        sw = D.from_host(gen.uniform(1e-3, 1e-2, N))
        bias = D.from_host(np.zeros(N, np.float32))
        for M in (1, 8, 32):
            x = D.from_host(gen.standard_normal((M, K), dtype=np.float32))
            q = D([M, K], "int8")
            sx = D([M], "float64")
            out = D([M, N], "float32")
            # The entry point bound once and each call's arguments built
            # ahead, so the timed loop costs what a native caller's would
            # (Python's per-call overhead otherwise approaches the kernel's
            # few microseconds and leaks into the back-to-back figure).
            fn = getattr(Nn.lib(), "kh_linear_i8")
            argsets = [(x.ptr, M, K, w.ptr, N, sw.ptr, 1, bias.ptr, q.ptr, sx.ptr, out.ptr) for w in ws]

            def call(i):
                rc = fn(*argsets[i % copies])
                if rc:
                    Nn.check(rc, "kh_linear_i8")

            for i in range(max(3, warmup)):
                call(i)
            Nn.synchronize()
            e0, e1 = Nn.Event(), Nn.Event()
            e0.record()
            for i in range(steps):
                call(i)
            e1.record()
            Nn.synchronize()
            us = e0.elapsed_ms(e1) / steps * 1e3
            evs = [(Nn.Event(), Nn.Event()) for _ in range(steps)]
            for i, (a, b) in enumerate(evs):
                a.record()
                call(i)
                b.record()
            Nn.synchronize()
            us_single = sum(a.elapsed_ms(b) for a, b in evs) / steps * 1e3
            nbytes = N * K + 8 * N + 4 * M * K + 2 * M * K + 4 * M * N
            gbs = nbytes / (us * 1e-6) / 1e9
            rows.append({"M": M, "K": K, "N": N, "us": round(us, 2), "us_single": round(us_single, 2),
                         "GB/s": round(gbs, 1), "TOPS": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 2),
                         "path": "fused decode kernel" if M <= 2 else "quantize_rows + skinny GEMM",
                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                      "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}})
            log(f"skinny M={M} K={K} N={N}: {us:.2f} us back-to-back ({gbs:.0f} GB/s), {us_single:.2f} us single")
        # The practical ceiling for these rows: a plain streaming read of the
        # same weight bytes (kh_probe_stream_read), rotated and issued back
        # to back the same way.
        fnr = getattr(Nn.lib(), "kh_probe_stream_read")
        rargs = [(w.ptr, N * K) for w in ws]
        for i in range(max(3, warmup)):
            Nn.check(fnr(*rargs[i % copies]), "kh_probe_stream_read")
        Nn.synchronize()
        e0, e1 = Nn.Event(), Nn.Event()
        e0.record()
        for i in range(steps):
            rc = fnr(*rargs[i % copies])
            if rc:
                Nn.check(rc, "kh_probe_stream_read")
        e1.record()
        Nn.synchronize()
        read_us = e0.elapsed_ms(e1) / steps * 1e3
        read_gbs = N * K / (read_us * 1e-6) / 1e9
        for r in rows:
            if r["K"] == K and r["N"] == N:
                r["roofline"]["attainable"] = {
                    "workload": "plain streaming read of the same weight bytes, back to back",
                    "us": round(read_us, 2), "GB/s": round(read_gbs, 1),
                    "frac_of_published": round(read_gbs / PEAK_HBM_GBS, 4),
                    "frac_achieved_of_attainable": round(r["roofline"]["achieved"] / read_gbs, 4)}
        log(f"skinny K={K} N={N}: plain weight read {read_us:.2f} us ({read_gbs:.0f} GB/s)")
        del ws
        Nn.call("kh_pool_trim")
    return rows


class _Linear:
    """An nn.Linear-like holder (.weight [in, out], .bias [out])."""

    def __init__(self, weight, bias):
        self.weight, self.bias = weight, bias


def _c1_inputs():
    gen = np.random.Generator(np.random.PCG64(0))
    x = gen.standard_normal((64, 512), dtype=np.float32)
    w = gen.standard_normal((512, 512), dtype=np.float32) * np.float32(0.02)
    return x, w, np.zeros(512, np.float32)


def bench_c1(steps, warmup):
    """Config C1, the reference's CPU-runnable case: an int8 quantized Linear,
    x fp32 [64, 512] ~N(0,1), W fp32 [512, 512] ~N(0, 0.02), bias zeros,
    per-tensor scales for x and W (seed 0; W quantized once at construction).
    Latency-bound, so reported as microseconds per call two ways: the two
    kernels back to back (one-launch per-tensor quantize of x; the skinny
    int8 GEMM with the dequantize and bias fused) and the eager QLinear call
    (Python dispatch and output allocation included)."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd.device import DeviceTensor as D
    from kansaiml_amd.quantize import QLinear
    x, w, b = _c1_inputs()
    layer = QLinear(_Linear(w, b), mode="int8", act_granularity="tensor", weight_granularity="tensor")
    xd = D.from_host(x)
    q, s, out = D([64, 512], "int8"), D([1], "float64"), D([64, 512])
    wq, ws, bd = layer.qweight.codes, layer.qweight.scales, layer.bias
    quant = Nn.lib().kh_quantize_tensor
    gemm = Nn.lib().kh_gemm_i8
    qargs = (xd.ptr, 64 * 512, q.ptr, s.ptr)
    gargs = (q.ptr, wq.ptr, 64, 512, 512, s.ptr, 0, ws.ptr, 0, bd.ptr, out.ptr, None)

    def kernels():
        quant(*qargs)
        gemm(*gargs)

    Nn.call("kh_quantize_tensor", *qargs)  # checked once; the timed calls skip the status check
    Nn.call("kh_gemm_i8", *gargs)

    us_kernels = time_kernel(kernels, steps, warmup) * 1e3
    us_eager = time_kernel(lambda: layer(xd), steps, warmup) * 1e3
    ops = 2 * 64 * 512 * 512
    return {"workload": "C1 int8 quantized Linear x[64,512] @ W[512,512] + b, per-tensor scales (seed 0)",
            "us_kernels_back_to_back": round(us_kernels, 2), "us_eager_call": round(us_eager, 2), "ops": ops,
            "TOPS_kernels": round(ops / (us_kernels * 1e-6) / 1e12, 3), "bound": "latency"}


def bench_host_buffers(reps=3):
    """C2 and C3a handed over as host (pageable numpy) buffers: upload, the
    kernel and the download, each between host synchronisations, best of
    `reps`.  Reported beside `value`, never as it: the PCIe-inclusive rate
    a caller holding host arrays sees."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd import hip as H
    from kansaiml_amd.device import DeviceTensor as D

    def timed(fn):
        Nn.synchronize()
        t0 = time.perf_counter()
        r = fn()
        Nn.synchronize()
        return time.perf_counter() - t0, r

    gen = np.random.Generator(np.random.PCG64(0))
    R = 16384
    x = gen.standard_normal((R, R), dtype=np.float32)
    runs = []
    for _ in range(reps):
        tu, xd = timed(lambda: D.from_host(x))
        tk, (q, s) = timed(lambda: H.quantize_rows(xd))
        td, _ = timed(lambda: (q.numpy(), s.numpy()))
        runs.append((tu, tk, td))
        del xd, q, s
    del x
    tu, tk, td = min(runs, key=sum)
    c2 = {"workload": "C2 per-row quantize, fp32 [16384,16384] in, int8 codes + fp64 scales out",
          "upload_ms": round(tu * 1e3, 2), "kernel_ms": round(tk * 1e3, 3), "download_ms": round(td * 1e3, 2),
          "GB/s_pcie_inclusive": round(5.0 * R * R / (tu + tk + td) / 1e9, 2),
          "h2d_GB/s": round(4.0 * R * R / tu / 1e9, 2), "d2h_GB/s": round((R * R + 8 * R) / td / 1e9, 2)}
    M = 8192
    a = gen.integers(-127, 128, (M, M), dtype=np.int8)
    b = gen.integers(-127, 128, (M, M), dtype=np.int8)
    sa, sb = np.array([0.01], np.float64), np.full(M, 0.02, np.float64)
    runs = []
    for _ in range(reps):
        tu, ops = timed(lambda: (D.from_host(a), D.from_host(b), D.from_host(sa), D.from_host(sb)))
        tk, (out, _) = timed(lambda: H.gemm_i8(*ops))
        td, _ = timed(lambda: out.numpy())
        runs.append((tu, tk, td))
        del ops, out
    tu, tk, td = min(runs, key=sum)
    c3a = {"workload": "C3a int8 GEMM 8192^3, int8 operands in, fp32 [8192,8192] out",
           "upload_ms": round(tu * 1e3, 2), "kernel_ms": round(tk * 1e3, 3), "download_ms": round(td * 1e3, 2),
           "TOPS_pcie_inclusive": round(2.0 * M ** 3 / (tu + tk + td) / 1e12, 2)}
    return {"note": "pageable host buffers; timed on the host around synchronised calls", "c2": c2, "c3a": c3a}


def c4_gemm_breakdown(model, ids, ms_forward, steps):
    """The C4 forward's int8 Linear layers one by one, on the activations
    the model itself produces: one unplanned run keeps every node's device
    value, then each int8_linear node is re-executed on its own inputs and
    timed with HIP events.  Returns per-shape microseconds and TOPS and the
    int8 GEMMs' share of the forward's time."""
    from kansaiml_amd import kir
    g, _ = model.graph(*ids.shape)
    vals = {g.inputs[0]: ids}
    out = kir.run_hip(g, ids, to_host=False, observe=lambda n, v: vals.__setitem__(n.id, v))
    del out
    M = ids.shape[0] * ids.shape[1]
    shapes = {}
    for node in g.nodes:
        if node.op != "int8_linear":
            continue
        w = vals[node.inputs[1]]
        N, K = int(node.shape[-1]), int(w.shape[0])
        epi = "+".join(e for e, on in (("bias", node.attrs.get("bias")), (node.attrs.get("act") or "", node.attrs.get("act")),
                                        ("residual", node.attrs.get("residual"))) if on) or "none"
        us = time_kernel(lambda: kir._release(kir._exec(node, vals)), steps, 3) * 1e3
        key = (N, K, epi)
        shapes.setdefault(key, []).append(us)
    rows, total = [], 0.0
    for (N, K, epi), t in sorted(shapes.items(), key=lambda kv: -sum(kv[1])):
        us = float(np.median(t))
        total += us * len(t)
        rows.append({"M": M, "N": N, "K": K, "epilogue": epi, "count": len(t), "us": round(us, 2),
                     "TOPS": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1)})
    vals.clear()
    return {"gemms": rows, "int8_gemm_us_per_forward": round(total, 1),
            "int8_gemm_fraction_of_forward": round(total / (ms_forward * 1e3), 3)}


def bench_c4(steps, warmup):
    """Config C4: the int8 char-LM forward (vocab 65, d 384, 6 heads, 6 layers,
    FFN 1536, seq 256, batch 64; int8 per-channel weights ~N(0, 0.02),
    per-tensor dynamic activation scales, fp32 softmax / LayerNorm / GELU).
    Token ids and weights resident on the device; logits stay on the device.
    Timed two ways: replaying the forward recorded as a HIP graph (one host
    call per forward; the headline figure) and the eager planned run (one
    Python dispatch per graph node)."""
    from kansaiml_amd.charlm import CharLM, CharLMWeights, attention_flops, int8_linear_ops
    from kansaiml_amd.device import DeviceTensor as D
    w = CharLMWeights(seed=0)
    model = CharLM(w)
    ids = D.from_host(np.random.Generator(np.random.PCG64(9)).integers(0, 65, (64, 256)).astype(np.int32))
    eager = time_kernel(lambda: model.forward(ids, to_host=False), steps, warmup)
    g = model.capture(64, 256)
    ms = time_kernel(lambda: g(ids, to_host=False), steps, warmup)
    g.close()
    breakdown = c4_gemm_breakdown(model, ids, ms, steps)
    # the same forward with per-token activation scales (an option beside
    # the reference's per-tensor configuration), replayed as a HIP graph
    gr = CharLM(w, act_granularity="row").capture(64, 256)
    ms_row = time_kernel(lambda: gr(ids, to_host=False), steps, warmup)
    gr.close()
    ops = int8_linear_ops(w, 64, 256)
    return {"workload": "C4 int8 char-LM forward, batch 64 x seq 256 (16384 tokens), 6 layers, d 384",
            "ms_per_forward": round(ms, 4), "tokens_per_s": round(64 * 256 / (ms * 1e-3), 1),
            "ms_per_forward_eager": round(eager, 4), "ms_per_forward_per_token_scales": round(ms_row, 4),
            "int8_linear_ops": ops, "int8_linear_TOPS_over_forward": round(ops / (ms * 1e-3) / 1e12, 2),
            "attention_fp32_flops_full_square": attention_flops(w, 64, 256), **breakdown}


COPY_BYTES = 1 << 30


def bench_mfma_probe():
    """The attainable int8 MFMA rate and the shader clock under that load
    (kh_probe_mfma_i8): random operand bytes, no memory traffic in the loop.
    The published 5.0 POP/s assumes the 2.4 GHz peak clock."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd.device import DeviceTensor as D
    import ctypes
    info = Nn.device_info()
    nbytes = info["cus"] * 64 * 1024
    ops = D.from_host(np.random.Generator(np.random.PCG64(11)).integers(-127, 128, nbytes, dtype=np.int8))
    tops, mhz = ctypes.c_double(), ctypes.c_double()
    Nn.call("kh_probe_mfma_i8", ops.ptr, nbytes, 2000, ctypes.byref(tops), ctypes.byref(mhz))  # warm up
    Nn.call("kh_probe_mfma_i8", ops.ptr, nbytes, 20000, ctypes.byref(tops), ctypes.byref(mhz))
    return {"workload": "v_mfma_i32_32x32x32_i8 only, random int8 operands in registers, 8 waves per CU",
            "TOPS": round(tops.value, 1), "clock_MHz": round(mhz.value), "frac_of_published": round(tops.value / PEAK_INT8_TOPS, 4)}


def bench_copy(steps, warmup):
    """1 GiB device-to-device copy (the library's copy16_kernel): the known-size
    reference for FETCH_SIZE / WRITE_SIZE calibration."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd.device import DeviceTensor as D
    src = D([COPY_BYTES], "int8")
    dst = D([COPY_BYTES], "int8")
    ms = time_kernel(lambda: Nn.call("kh_memcpy_d2d", dst.ptr, src.ptr, COPY_BYTES), steps, warmup)
    return ms, 2.0 * COPY_BYTES / (ms * 1e-3) / 1e9


# Kernel-name fragments (rocprofv3 Kernel_Name) of the kernels each bench line measures.
KERNELS = {
    "gemm_i8_8192": "gemm_i8_pingpong_kernel",
    "quant_rows_16384": "quant_rows_reg_kernel<4, 16>",
    "dequant_rows_16384": "dequant_vec_kernel",
    "fp32_matmul_4096": "gemm_f32_",
    "copy_1GiB": "copy16_kernel",
}
ALGO_BYTES = {"gemm_i8_8192": 2 * 8192 * 8192 + 4 * 8192 * 8192, "quant_rows_16384": 5 * 16384 * 16384,
              "dequant_rows_16384": 5 * 16384 * 16384, "copy_1GiB": 2 * COPY_BYTES,
              "fp32_matmul_4096": 3 * 4 * 4096 * 4096}


def _read_csv(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def _find(root, suffix):
    for dirpath, _, files in os.walk(root):
        for f in files:
            if f.endswith(suffix):
                return os.path.join(dirpath, f)
    return None


def summarize(root):
    """Turns rocprofv3 CSV output under root/{trace,fetch,write} into the
    text summaries in profiles/ and profiles/traffic.json."""
    out_dir = os.path.join(ROOT, "profiles")
    os.makedirs(out_dir, exist_ok=True)
    lines = []
    stats = _find(os.path.join(root, "trace"), "kernel_stats.csv")
    if stats:
        rows = _read_csv(stats)
        lines.append("| kernel | calls | avg us | min us | max us | % time |")
        lines.append("|---|---|---|---|---|---|")
        for r in rows:
            lines.append(f"| {r['Name'][:90]} | {r['Calls']} | {float(r['AverageNs'])/1e3:.2f} | "
                         f"{float(r['MinNs'])/1e3:.2f} | {float(r['MaxNs'])/1e3:.2f} | {float(r['Percentage']):.1f} |")
    traffic = {}
    per = {}
    for which in ("fetch", "write"):
        cc = _find(os.path.join(root, which), "counter_collection.csv")
        if not cc:
            continue
        for r in _read_csv(cc):
            for key, frag in KERNELS.items():
                if frag in r["Kernel_Name"]:
                    per.setdefault(key, {}).setdefault(r["Counter_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
                    per[key][r["Counter_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    def avg(key, ctr):
        d = per.get(key, {}).get(ctr, {})
        return sum(d.values()) / len(d) if d else None
    cf, cw = avg("copy_1GiB", "FETCH_SIZE"), avg("copy_1GiB", "WRITE_SIZE")
    if cf and cw:
        ff, wf = COPY_BYTES / (cf * 1024), COPY_BYTES / (cw * 1024)
        traffic["_calibration"] = {"copy_bytes": COPY_BYTES, "FETCH_SIZE_KiB": cf, "WRITE_SIZE_KiB": cw,
                                   "fetch_factor": ff, "write_factor": wf}
        for key in KERNELS:
            f, w = avg(key, "FETCH_SIZE"), avg(key, "WRITE_SIZE")
            if f is None or w is None or key == "copy_1GiB":
                continue
            b = f * 1024 * ff + w * 1024 * wf
            traffic[key] = {"FETCH_SIZE_KiB": f, "WRITE_SIZE_KiB": w, "bytes_per_launch": b,
                            "algorithmic_bytes": ALGO_BYTES.get(key), "ratio": b / ALGO_BYTES[key]}
    with open(os.path.join(out_dir, "traffic.json"), "w") as fjs:
        json.dump(traffic, fjs, indent=1, sort_keys=True)
    print("\n".join(lines))
    print(json.dumps(traffic, indent=1))
    return lines, traffic


def cpu_c1(reps=200):
    """C1 on the host as the reference runs it (quantize.py:115-122 with the
    weight quantized once): x @ dequantize(W) + b through the reference's
    compiled fp32 i-k-j matmul and bias add (backend/cpu/src/Ops.cpp:322-339,
    34-38; oracle/_ref), one core, microseconds per call."""
    from oracle import oracle as O
    x, w, b = _c1_inputs()
    qw, sw = O.ko_quantize_tensor(w)
    wdeq = O.ko_dequantize_tensor(qw, sw).reshape(w.shape)  # dequantize(W), once
    use_ref = O.ref_available()
    mm = O.ref_matmul if use_ref else O.ko_matmul_f32
    add = O.ref_add_bias if use_ref else (lambda y, bb: (y + bb).astype(np.float32))
    add(mm(x, wdeq), b)
    t0 = time.perf_counter()
    for _ in range(reps):
        add(mm(x, wdeq), b)
    us = (time.perf_counter() - t0) / reps * 1e6
    return {"us_per_call": round(us, 1), "cores": 1, "kind": "reference" if use_ref else "port",
            "sample": f"{reps} calls of x @ dequantize(W) + b on C1's inputs (the reference's weight-only qlinear)"}


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
    ap.add_argument("--steps", type=int, default=50)
    # The shader clock ramps up over the first ~10 ms of load: 50 untimed
    # steps let every leg reach its sustained rate before timing.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="gemm,probe,quant,f32,c1,skinny,c4",
                    help="comma list of gemm,probe,quant,f32,c1,skinny,c4,copy,pcie (pcie: host-buffer rates)")
    ap.add_argument("--summarize", metavar="DIR", help="summarize rocprofv3 CSV output and exit")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    only = set(args.only.split(","))
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the int8 path has no multi-GPU leg "
                                   "(rows/columns would shard with zero exchange); run with --gpus 1"}))
        sys.exit(2)

    from kansaiml_amd import _native as Nn
    from kansaiml_amd import hip as H
    from kansaiml_amd.device import DeviceTensor as D
    if not H.available():
        raise SystemExit("bench: no gfx950 GPU visible")
    info = Nn.device_info()
    log(f"device {info}")

    g_ms = g_tops = q_ms = d_ms = q_gbs = d_gbs = f_ms = f_tflops = float("nan")
    if "gemm" in only:
        log("int8 GEMM 8192^3 ...")
        g_ms, g_tops, keep = bench_gemm(H, D, args.steps, args.warmup)
        log(f"int8 GEMM: {g_ms:.4f} ms/step, {g_tops:.1f} TOPS")
        del keep
        Nn.call("kh_pool_trim")
    probe = None
    if "probe" in only:
        probe = bench_mfma_probe()
        log(f"MFMA-only ceiling: {probe['TOPS']:.0f} TOPS at {probe['clock_MHz']} MHz")
        Nn.call("kh_pool_trim")
    if "quant" in only:
        log("quantize/dequantize C2 ...")
        q_ms, d_ms, qd_bytes = bench_quant_dequant(H, D, args.steps, args.warmup)
        q_gbs = qd_bytes / (q_ms * 1e-3) / 1e9
        d_gbs = qd_bytes / (d_ms * 1e-3) / 1e9
        log(f"quantize {q_ms:.4f} ms ({q_gbs:.0f} GB/s), dequantize {d_ms:.4f} ms ({d_gbs:.0f} GB/s)")
        Nn.call("kh_pool_trim")
    if "f32" in only:
        log("fp32 matmul 4096^3 ...")
        f_ms, f_tflops = bench_f32(H, D, max(5, args.steps // 2), max(2, args.warmup // 2))
        log(f"fp32 matmul: {f_ms:.4f} ms, {f_tflops:.1f} TFLOP/s")
        Nn.call("kh_pool_trim")
    c1 = None
    if "c1" in only:
        log("C1 int8 quantized Linear ...")
        c1 = bench_c1(max(50, args.steps), args.warmup)
        log(f"C1: {c1['us_kernels_back_to_back']:.2f} us per call (kernels back to back), "
            f"{c1['us_eager_call']:.2f} us eager")
    skinny = None
    if "skinny" in only:
        log("skinny decode GEMMs C5 ...")
        skinny = bench_skinny(max(20, args.steps), args.warmup)
    c4 = None
    if "c4" in only:
        log("C4 int8 char-LM forward ...")
        c4 = bench_c4(max(5, args.steps // 4), max(2, args.warmup // 10))
        log(f"C4 forward: {c4['ms_per_forward']:.3f} ms as a HIP graph ({c4['tokens_per_s']:.0f} tokens/s), "
            f"{c4['ms_per_forward_eager']:.3f} ms eager")
        Nn.call("kh_pool_trim")
    host_buffers = None
    if "pcie" in only:
        log("C2 and C3a from host buffers ...")
        host_buffers = bench_host_buffers()
        log(f"host buffers: C2 {host_buffers['c2']['GB/s_pcie_inclusive']} GB/s, "
            f"C3a {host_buffers['c3a']['TOPS_pcie_inclusive']} TOPS")
        Nn.call("kh_pool_trim")
    if "copy" in only:
        c_ms, c_gbs = bench_copy(args.steps, args.warmup)
        log(f"1 GiB d2d copy: {c_ms:.4f} ms, {c_gbs:.0f} GB/s")
        Nn.call("kh_pool_trim")

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline()
        log(f"CPU baseline {cpu['value']:.6f} TOPS")
        if c1 is not None:
            c1["cpu"] = cpu_c1()
            log(f"C1 on the CPU: {c1['cpu']['us_per_call']:.1f} us per call")

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
                     "frac": round(g_tops / PEAK_INT8_TOPS, 4), "traffic": measured_traffic("gemm_i8_8192"),
                     "attainable": probe},
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
        "skinny_decode": {"workload": "C5 kh_linear_i8: per-token quantize + int8 GEMM, per-channel weights",
                          "bytes": "N*K + 8N + 4MK + 2MK + 4MN", "rows": skinny},
        "c1_linear": c1,
        "c4_forward": c4,
        "host_buffers": host_buffers,
        "cpu_baseline": cpu,
        "device": info,
    }
    print(json.dumps(result).replace("NaN", "null"))


if __name__ == "__main__":
    main()
