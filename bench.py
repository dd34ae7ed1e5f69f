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
launches, device synchronized on both sides.  Before its timed launches every
leg runs its own kernel untimed for at least --warmup launches and at least
--warm-ms milliseconds (default 50: the shader clock ramps over the first
~10 ms of load), so each figure is the sustained rate whatever --warmup is;
the milliseconds and launches spent are reported in "warmup_per_leg".
CPU baselines, one host core each (the reference has no threading): the
reference's own compiled backend/cpu/src/Ops.cpp matmul (oracle/_ref) -- what
the reference runs for a quantized Linear after dequantizing the weight
(python/kansai/quantize.py:115-122) -- on a time-bounded slab of C3a rows
("cpu_baseline"), of C3b, of the C4 block and of each C5 row; C2 through the
C restatement of quantize.py:66-76; C1 as the reference's whole call.

    python bench.py [--gpus 1] [--steps 50] [--warmup 50] [--warm-ms 50] [--no-cpu]
                    [--only gemm,probe,quant,f32,c1,skinny,c4,c4row,copy,pcie] [--c5-rows M:K:N,...]

Profiling: `python bench.py --profile-commands OUT` prints the rocprofv3 runs
(kernel traces, FETCH_SIZE / WRITE_SIZE traffic, counter groups for the C3a
GEMM, the C4 forward and each C5 row; one counter group per run);
`python bench.py --summarize OUT` turns their CSV output into every file
under profiles/ (tables with the commands that made them) and
profiles/traffic.json, which the bench line's roofline "traffic" fields read.
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


# Every leg runs its own kernel for at least this long, untimed, before its
# timed calls: the shader clock ramps up over the first ~10 ms of sustained
# load, so a leg timed right after another leg's pause (or after a handful of
# warm-up calls) would measure the ramp.
WARM_MS = 50.0
WARMUP_LOG = {}


def warm_up(fn, calls, min_ms=None, tag=None):
    """At least `calls` untimed calls of fn(), continued in batches (each
    followed by a device synchronization) until min_ms of wall time has
    passed.  Returns the milliseconds spent; recorded under `tag`."""
    from kansaiml_amd import _native as N
    if min_ms is None:
        min_ms = WARM_MS  # read at call time: --warm-ms sets it
    N.synchronize()
    t0 = time.perf_counter()
    n, batch = 0, max(1, calls)
    while True:
        for _ in range(batch):
            fn()
        n += batch
        N.synchronize()
        el = (time.perf_counter() - t0) * 1e3
        if el >= min_ms and n >= calls:
            break
        batch = max(1, min(4 * n, int(n * (min_ms - el) / max(el, 1e-3)) + 1))
    if tag:
        WARMUP_LOG[tag] = {"ms": round(el, 1), "calls": n}
    return el


def time_kernel(fn, steps, warmup, tag=None, min_warm_ms=None):
    """Average ms per call of fn() over `steps` back-to-back calls, HIP events
    on the library stream, synchronized before and after, after warm_up()."""
    from kansaiml_amd import _native as N
    warm_up(fn, warmup, min_warm_ms, tag)
    e0, e1 = N.Event(), N.Event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    N.synchronize()
    return e0.elapsed_ms(e1) / steps


# False (--no-graph-timing, every profiled run): no HIP graph is launched --
# time_graph times a stream of calls instead and the C4 leg times its eager
# forwards (rocprofv3's kernel trace has crashed inside hipGraphLaunch).
GRAPH_TIMING = True


def time_graph(call, steps, reps=15):
    """Microseconds per call of `steps` dependent calls of call() recorded
    once as a HIP graph on the library stream (kh_graph_*), the median over
    `reps` replays, each between its own HIP events.  Unlike a Python loop
    issuing the calls, the replay never waits for the host: for kernels of a
    few microseconds the per-call cost of issuing them from Python (a ctypes
    call and a launch) is as large as the kernel, and a host-side pause
    inside a short timed loop shows up in the average.  call() must have run
    before (scratch sized, pool warm) and must not synchronize.

    With GRAPH_TIMING off (the profiler runs: rocprofv3's kernel trace
    crashed inside hipGraphLaunch on these graphs of short kernels, and the
    profiles read kernel durations, not this figure) it returns the mean
    over `steps` calls issued from Python between HIP events."""
    import ctypes
    from kansaiml_amd import _native as N
    if not GRAPH_TIMING:
        N.synchronize()
        e0, e1 = N.Event(), N.Event()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        N.synchronize()
        return e0.elapsed_ms(e1) / steps * 1e3
    N.synchronize()
    N.call("kh_graph_capture_begin")
    try:
        for _ in range(steps):
            call()
    except BaseException:
        N.lib().kh_graph_capture_end(None)
        raise
    g = ctypes.c_void_p()
    N.call("kh_graph_capture_end", ctypes.byref(g))
    try:
        e0, e1 = N.Event(), N.Event()
        N.call("kh_graph_launch", g)  # first replay: uploads the graph
        N.synchronize()
        times = []
        for _ in range(reps):
            e0.record()
            N.call("kh_graph_launch", g)
            e1.record()
            N.synchronize()
            times.append(e0.elapsed_ms(e1))
    finally:
        N.call("kh_graph_destroy", g)
    return float(np.median(times)) / steps * 1e3


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
    ms = time_kernel(fn, steps, warmup, tag="gemm")
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
    qms = time_kernel(qfn, steps, warmup, tag="quantize")
    dms = time_kernel(dfn, steps, warmup, tag="dequantize")
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
    ms = time_kernel(fn, steps, warmup, tag="fp32_matmul")
    return ms, 2.0 * n ** 3 / (ms * 1e-3) / 1e12


C5_ROWS = [(M, K, N) for K, N in ((4096, 4096), (4096, 11008)) for M in (1, 8, 32)]


def c5_host_weight(K, N, seed=5):
    """Config C5's weight: fp32 [K, N] ([in, out]) ~N(0, 0.02) with 0.5 % of
    its output columns scaled x20 (outlier channels)."""
    gen = np.random.Generator(np.random.PCG64(seed))
    w = gen.standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
    cols = gen.choice(N, size=max(1, N // 200), replace=False)
    w[:, cols] *= np.float32(20.0)
    return w


def c5_weights(K, N):
    """c5_host_weight quantized per output channel on the device
    (kh_quantize_cols_packed): packed codes [N, K], binary64 scales [N]."""
    from kansaiml_amd import hip as H
    from kansaiml_amd.device import DeviceTensor as D
    q, s = H.quantize_cols_packed(D.from_host(c5_host_weight(K, N)))
    return q, s


def bench_skinny(steps, warmup, rows=None):
    """Config C5: kh_linear_i8 (per-token quantize of fp32 x ~N(0,1), int8
    GEMM, per-output-channel weight scales, fused epilogue, zero bias) for M in
    {1, 8, 32}, (K, N) in {(4096, 4096), (4096, 11008)}.  Copies of the
    quantized weight are rotated so more than 512 MB of distinct weights pass
    through HBM (beyond the 256 MB Infinity Cache).  `us` is the average over
    max(steps, copies) dependent calls back to back (a decode loop's layer
    calls), recorded as a HIP graph and replayed (time_graph), so one replay
    walks every copy; `us_stream` is the
    same calls issued one by one from Python between one pair of HIP events;
    `us_single` brackets each call with its own events (launch latency
    included, host gaps excluded)."""
    from kansaiml_amd import _native as Nn
    from kansaiml_amd.device import DeviceTensor as D
    gen = np.random.Generator(np.random.PCG64(6))
    want = set(rows or C5_ROWS)
    out_rows = []
    for K, N in sorted({(k, n) for _, k, n in want}):
        q0, sw = c5_weights(K, N)
        copies = max(2, -(-(512 << 20) // (N * K)))
        ws = [q0] + [D([N, K], "int8") for _ in range(copies - 1)]
        for w in ws[1:]:
            Nn.call("kh_memcpy_d2d", w.ptr, q0.ptr, N * K)
        # A replayed graph holds at least one call per copy, so every replay
        # streams all > 512 MB of distinct weights whatever --steps is.
        gsteps = max(steps, copies)
        bias = D.from_host(np.zeros(N, np.float32))
        for M in (1, 8, 32):
            if (M, K, N) not in want:
                continue
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
            Nn.call("kh_linear_i8", *argsets[0])  # checked once; the timed calls skip the status check
            i_call = [0]

            def call():
                fn(*argsets[i_call[0] % copies])
                i_call[0] += 1

            warm_up(call, max(3, warmup), tag=f"c5_M{M}_N{N}")
            e0, e1 = Nn.Event(), Nn.Event()
            e0.record()
            for _ in range(steps):
                call()
            e1.record()
            Nn.synchronize()
            us_stream = e0.elapsed_ms(e1) / steps * 1e3
            us = time_graph(call, gsteps)
            evs = [(Nn.Event(), Nn.Event()) for _ in range(steps)]
            for a, b in evs:
                a.record()
                call()
                b.record()
            Nn.synchronize()
            us_single = sum(a.elapsed_ms(b) for a, b in evs) / steps * 1e3
            nbytes = N * K + 8 * N + 4 * M * K + 2 * M * K + 4 * M * N
            gbs = nbytes / (us * 1e-6) / 1e9
            key = f"c5_M{M}_K{K}_N{N}"
            out_rows.append({"M": M, "K": K, "N": N, "us": round(us, 2), "us_stream": round(us_stream, 2),
                             "us_single": round(us_single, 2),
                             "GB/s": round(gbs, 1), "TOPS": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 2),
                             "path": "fused decode kernel" if M <= 3 else "quantize_rows + skinny GEMM",
                             "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                          "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                          "traffic": measured_traffic(key), "traffic_key": key}})
            log(f"skinny M={M} K={K} N={N}: {us:.2f} us back-to-back ({gbs:.0f} GB/s; {us_stream:.2f} us issued "
                f"from Python), {us_single:.2f} us single")
        # The practical ceiling for these rows: a plain streaming read of the
        # same weight bytes (kh_probe_stream_read), rotated and issued back
        # to back the same way.
        fnr = getattr(Nn.lib(), "kh_probe_stream_read")
        rargs = [(w.ptr, N * K) for w in ws]
        Nn.call("kh_probe_stream_read", *rargs[0])
        i_read = [0]

        def read():
            fnr(*rargs[i_read[0] % copies])
            i_read[0] += 1

        warm_up(read, max(3, warmup), tag=f"c5_read_N{N}")
        read_us = time_graph(read, gsteps)
        read_gbs = N * K / (read_us * 1e-6) / 1e9
        for r in out_rows:
            if r["K"] == K and r["N"] == N:
                r["roofline"]["attainable"] = {
                    "workload": "plain streaming read of the same weight bytes, back to back",
                    "us": round(read_us, 2), "GB/s": round(read_gbs, 1),
                    "frac_of_published": round(read_gbs / PEAK_HBM_GBS, 4),
                    "frac_achieved_of_attainable": round(r["roofline"]["achieved"] / read_gbs, 4)}
        log(f"skinny K={K} N={N}: plain weight read {read_us:.2f} us ({read_gbs:.0f} GB/s)")
        del ws, q0
        Nn.call("kh_pool_trim")
    return out_rows


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
    Latency-bound, so reported as microseconds per call: kh_linear_i8_tensor
    (one launch: every workgroup quantizes x per tensor and runs its columns
    of the skinny int8 GEMM with the dequantize and bias fused) back to back,
    replayed as a HIP graph (time_graph) and issued from Python
    (`us_kernels_stream`); the same Linear as two launches (kh_quantize_tensor
    then kh_gemm_i8, `us_two_launch`); and the eager QLinear call (Python
    dispatch and output allocation included)."""
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
    lin = Nn.lib().kh_linear_i8_tensor
    qargs = (xd.ptr, 64 * 512, q.ptr, s.ptr)
    gargs = (q.ptr, wq.ptr, 64, 512, 512, s.ptr, 0, ws.ptr, 0, bd.ptr, out.ptr, None)
    largs = (xd.ptr, 64, 512, wq.ptr, 512, ws.ptr, 0, bd.ptr, q.ptr, s.ptr, out.ptr)

    def kernels():
        lin(*largs)

    def two_launch():
        quant(*qargs)
        gemm(*gargs)

    Nn.call("kh_linear_i8_tensor", *largs)  # checked once; the timed calls skip the status check
    Nn.call("kh_quantize_tensor", *qargs)
    Nn.call("kh_gemm_i8", *gargs)

    us_stream = time_kernel(kernels, steps, warmup, tag="c1_kernels") * 1e3
    us_kernels = time_graph(kernels, steps)
    time_kernel(two_launch, steps, warmup, tag="c1_two_launch")
    us_two = time_graph(two_launch, steps)
    us_eager = time_kernel(lambda: layer(xd), steps, warmup, tag="c1_eager") * 1e3
    ops = 2 * 64 * 512 * 512
    return {"workload": "C1 int8 quantized Linear x[64,512] @ W[512,512] + b, per-tensor scales (seed 0)",
            "us_kernels_back_to_back": round(us_kernels, 2), "us_kernels_stream": round(us_stream, 2),
            "us_two_launch": round(us_two, 2), "us_eager_call": round(us_eager, 2), "ops": ops,
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
        us = time_kernel(lambda: kir._release(kir._exec(node, vals)), steps, 3, min_warm_ms=5.0) * 1e3
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
    eager = time_kernel(lambda: model.forward(ids, to_host=False), steps, warmup, tag="c4_eager")
    if GRAPH_TIMING:
        # The token ids go into the graph's own input buffer once: each
        # replay then reads them in place (ids resident in HBM), where
        # passing another buffer adds a device copy per replay.
        g = model.capture(64, 256)
        g(ids, to_host=False)
        ms = time_kernel(lambda: g(g.inputs[0], to_host=False), steps, warmup, tag="c4_graph")
        g.close()
    else:  # a profiled run: the same forward, eager
        ms = eager
    breakdown = c4_gemm_breakdown(model, ids, ms, steps)
    # the same forward with per-token activation scales (an option beside
    # the reference's per-tensor configuration), replayed as a HIP graph:
    # LayerNorms emit per-row codes, the attention output is quantized per
    # row inside the O GEMM (qload, from the attention's per-(row, head)
    # partials), fc1's (-> GELU) rows inside the fc1 GEMM
    # (kh_gemm_i8_quant_rows)
    ms_row = None  # a profiled run traces the configured (per-tensor) forward only
    if GRAPH_TIMING:
        gr = CharLM(w, act_granularity="row").capture(64, 256)
        gr(ids, to_host=False)
        ms_row = time_kernel(lambda: gr(gr.inputs[0], to_host=False), steps, warmup, tag="c4_graph_per_token")
        gr.close()
    ops = int8_linear_ops(w, 64, 256)
    return {"workload": "C4 int8 char-LM forward, batch 64 x seq 256 (16384 tokens), 6 layers, d 384",
            "timing": "HIP graph replay" if GRAPH_TIMING else "eager (profiled run: no graph launches)",
            "ms_per_forward": round(ms, 4), "tokens_per_s": round(64 * 256 / (ms * 1e-3), 1),
            "ms_per_forward_eager": round(eager, 4),
            "ms_per_forward_per_token_scales": round(ms_row, 4) if ms_row is not None else None,
            "int8_linear_ops": ops, "int8_linear_TOPS_over_forward": round(ops / (ms * 1e-3) / 1e12, 2),
            "attention_fp32_flops_full_square": attention_flops(w, 64, 256), **breakdown}


COPY_BYTES = 1 << 30


def bench_c4_per_token(steps, warmup):
    """C4 with per-token activation scales (`CharLM(act_granularity="row")`,
    the option beside the reference's per-tensor configuration): replayed as
    a HIP graph, or run eagerly under --no-graph-timing so that a kernel
    trace sees the same kernels (every per-row quantize inside its producer:
    LayerNorm, the O GEMM, fc1's GEMM)."""
    from kansaiml_amd.charlm import CharLM, CharLMWeights
    from kansaiml_amd.device import DeviceTensor as D
    w = CharLMWeights(seed=0)
    model = CharLM(w, act_granularity="row")
    ids = D.from_host(np.random.Generator(np.random.PCG64(9)).integers(0, 65, (64, 256)).astype(np.int32))
    if GRAPH_TIMING:
        g = model.capture(64, 256)
        g(ids, to_host=False)
        ms = time_kernel(lambda: g(g.inputs[0], to_host=False), steps, warmup, tag="c4_per_token_graph")
        g.close()
    else:
        ms = time_kernel(lambda: model.forward(ids, to_host=False), steps, warmup, tag="c4_per_token_eager")
    return {"workload": "C4 int8 char-LM forward with per-token activation scales, batch 64 x seq 256",
            "timing": "HIP graph replay" if GRAPH_TIMING else "eager (profiled run: no graph launches)",
            "ms_per_forward": round(ms, 4), "tokens_per_s": round(64 * 256 / (ms * 1e-3), 1)}


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

# The profiling runs `--summarize OUT` understands: OUT/<name> made by
#   rocprofv3 <profiler args> -d OUT/<name> -o run --output-format csv -- python3 bench.py <bench args>
# (`bench.py --profile-commands OUT` prints them).  One counter group per run:
# a pass may hold at most 8 SQ_, 4 TCC_, 4 TCP_, 2 TA_, 2 TD_ and 2 GRBM_ counters.
# Every run passes --no-graph-timing: no HIP graph is launched under the profiler.
_GEMM_ARGS = "--only gemm --steps 10 --warmup 1 --no-cpu --warm-ms 50 --no-graph-timing"
_C4_ARGS = "--only c4 --steps 4 --warmup 2 --no-cpu --warm-ms 0 --no-graph-timing"
_TRAFFIC_ARGS = "--only gemm,quant,f32,copy --steps 3 --warmup 1 --no-cpu --warm-ms 0 --no-graph-timing"
PROFILE_RUNS = {
    "trace": ("--kernel-trace --stats", "--no-cpu --warm-ms 50 --no-graph-timing"),
    "fetch": ("--pmc FETCH_SIZE", _TRAFFIC_ARGS),
    "write": ("--pmc WRITE_SIZE", _TRAFFIC_ARGS),
    "gemm_p1": ("--pmc SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY "
                "SQ_INSTS_MFMA SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS", _GEMM_ARGS),
    "gemm_p2": ("--pmc TCP_TCC_READ_REQ_sum TCP_TCC_READ_REQ_LATENCY_sum TCP_PENDING_STALL_CYCLES_sum TCC_HIT_sum "
                "TCC_MISS_sum TA_BUFFER_READ_LDS_WAVEFRONTS_sum TD_TC_STALL_sum TD_TD_BUSY_sum", _GEMM_ARGS),
    "gemm_p3": ("--pmc GRBM_COUNT GRBM_GUI_ACTIVE SQ_CYCLES", _GEMM_ARGS),
    "c4_trace": ("--kernel-trace --stats", "--no-cpu --only c4 --steps 10 --warmup 20 --no-graph-timing"),
    "c4row_trace": ("--kernel-trace --stats", "--no-cpu --only c4row --steps 40 --warmup 20 --no-graph-timing"),
    "c4_p1": ("--pmc SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_LDS_BANK_CONFLICT "
              "SQ_INSTS_VALU SQ_WAIT_ANY SQ_ACTIVE_INST_LDS", _C4_ARGS),
    "c4_p2": ("--pmc SQ_INSTS_MFMA SQ_INSTS_LDS SQ_WAVES SQ_INSTS_VMEM_WR SQ_INSTS_VMEM_RD GRBM_GUI_ACTIVE GRBM_COUNT",
              _C4_ARGS),
    "c4_p3": ("--pmc FETCH_SIZE", _C4_ARGS),
    "c4_p4": ("--pmc WRITE_SIZE", _C4_ARGS),
}
for _M, _K, _N in C5_ROWS:
    _row = f"--only skinny --c5-rows {_M}:{_K}:{_N} --steps 20 --warmup 3 --no-cpu --warm-ms 0 --no-graph-timing"
    PROFILE_RUNS[f"c5_{_M}_{_K}_{_N}_fetch"] = ("--pmc FETCH_SIZE", _row)
    PROFILE_RUNS[f"c5_{_M}_{_K}_{_N}_write"] = ("--pmc WRITE_SIZE", _row)
    PROFILE_RUNS[f"c5_{_M}_{_K}_{_N}_l2"] = ("--pmc TCP_TCC_READ_REQ_sum TCC_HIT_sum TCC_MISS_sum "
                                             "TCP_PENDING_STALL_CYCLES_sum", _row)
    PROFILE_RUNS[f"c5_{_M}_{_K}_{_N}_sq"] = ("--pmc SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA "
                                             "GRBM_COUNT", _row)


def profile_command(name, out="OUT"):
    prof, args = PROFILE_RUNS[name]
    return f"rocprofv3 {prof} -d {out}/{name} -o run --output-format csv -- python3 bench.py {args}"


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


def _short(name):
    """A kernel's name without namespaces, return type and arguments."""
    k = name.replace("void ", "").replace("(anonymous namespace)::", "").replace("kh::", "")
    return k[:k.find("(")] if "(" in k else k


def _grid(r):
    g = r.get("Grid_Size") or r.get("Grid_Size_X") or "0"
    return int(g)


def _per_dispatch(root, names):
    """Counter values per dispatch from the runs `names` under root:
    {dispatch key: {"kernel", "grid", "wg", "ns", counter: value}}, keyed by
    (run, Dispatch_Id); counters summed over their instances."""
    out = {}
    for name in names:
        cc = _find(os.path.join(root, name), "counter_collection.csv")
        if not cc:
            continue
        for r in _read_csv(cc):
            key = (name, r["Dispatch_Id"])
            d = out.setdefault(key, {"kernel": _short(r["Kernel_Name"]), "grid": _grid(r),
                                     "wg": int(r.get("Workgroup_Size") or 0),
                                     "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def _by_kernel(disp):
    """Per (kernel, grid): the median duration and the mean of each counter."""
    groups = {}
    for d in disp.values():
        groups.setdefault((d["kernel"], d["grid"], d["wg"]), []).append(d)
    res = {}
    for key, ds in groups.items():
        ctrs = {}
        for d in ds:
            for c, v in d.items():
                if c not in ("kernel", "grid", "wg", "ns"):
                    ctrs.setdefault(c, []).append(v)
        res[key] = {"n": len(ds), "us": float(np.median([d["ns"] for d in ds])) / 1e3,
                    **{c: sum(v) / len(v) for c, v in ctrs.items()}}
    return res


def _calibration(root):
    """FETCH_SIZE / WRITE_SIZE readings of the 1 GiB copy -> bytes factors."""
    disp = _per_dispatch(root, ["fetch", "write"])
    f = [d["FETCH_SIZE"] for d in disp.values() if "copy16_kernel" in d["kernel"] and "FETCH_SIZE" in d]
    w = [d["WRITE_SIZE"] for d in disp.values() if "copy16_kernel" in d["kernel"] and "WRITE_SIZE" in d]
    if not f or not w:
        return None
    cf, cw = sum(f) / len(f), sum(w) / len(w)
    return {"copy_bytes": COPY_BYTES, "FETCH_SIZE_KiB": cf, "WRITE_SIZE_KiB": cw,
            "fetch_factor": COPY_BYTES / (cf * 1024), "write_factor": COPY_BYTES / (cw * 1024)}


_GRAPH_NOTE = ("Every run passes `--no-graph-timing`: no HIP graph is launched under the profiler, so the "
               "graph-replayed figures of the bench line (C1, C5, C4) have no trace of their own and these runs "
               "time the same calls issued one by one. rocprofv3's kernel trace has died with a host SIGSEGV "
               "inside `hipGraphLaunch` on such graphs (intermittently, the same command also running clean); "
               "a review of the library's graph handling (handles live until `kh_graph_destroy`, which "
               "synchronizes first; every buffer a graph names stays pinned or retired while it lives) found "
               "nothing that could fault on the host there, so the tool's graph instrumentation is held "
               "responsible.")


def _write_profile(fname, title, commands, body):
    path = os.path.join(ROOT, "profiles", fname)
    cmd = "\n".join("    " + c for c in commands)
    text = (f"# {title}\n\nGenerated by `python3 bench.py --summarize OUT` from the runs below (run from the "
            f"repository root, OUT a scratch directory):\n\n{cmd}\n\n{_GRAPH_NOTE}\n\n{body.rstrip()}\n")
    with open(path, "w") as f:
        f.write(text)
    print(f"wrote {path}")


def _md_table(header, rows):
    lines = ["| " + " | ".join(header) + " |", "|" + "---|" * len(header)]
    lines += ["| " + " | ".join(str(c) for c in r) + " |" for r in rows]
    return "\n".join(lines)


def _summarize_trace(root):
    stats = _find(os.path.join(root, "trace"), "kernel_stats.csv")
    if not stats:
        return
    # Median per kernel from the dispatch trace: the average also counts each
    # leg's warm-up launches, made while the shader clock is still ramping.
    trace = _find(os.path.join(root, "trace"), "kernel_trace.csv")
    durs = {}
    for r in (_read_csv(trace) if trace else []):
        durs.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]),
                                                      int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    # The trace run times each leg over the bench's default 50 steps after
    # its warm-up: for a kernel that only its leg launches (the C3a GEMM),
    # its last 50 dispatches are the timed ones.
    steps = 50

    def timed(name):
        d = [t for _, t in sorted(durs[name])][-steps:]
        return f"{float(np.mean(d)) / 1e3:.2f}"

    rows = [(f"`{_short(r['Name'])[:90]}`", r["Calls"], f"{float(r['AverageNs']) / 1e3:.2f}",
             f"{float(np.median([t for _, t in durs[r['Name']]])) / 1e3:.2f}" if r["Name"] in durs else "",
             timed(r["Name"]) if r["Name"] in durs else "",
             f"{float(r['MinNs']) / 1e3:.2f}", f"{float(r['MaxNs']) / 1e3:.2f}", f"{float(r['Percentage']):.1f}")
            for r in _read_csv(stats)]
    _write_profile("bench_kernels_mi355x.md", "Kernel trace of `bench.py` on one MI355X (gfx950)",
                   [profile_command("trace")],
                   "Every bench leg (`run_kernel_stats.csv`, medians from `run_kernel_trace.csv`); durations include "
                   "the profiler's per-dispatch timestamps. The average counts each leg's warm-up launches (this "
                   "run warms each leg for at least 50 ms, the first of them while the shader clock is still "
                   f"ramping); the median, and the average of a kernel's last {steps} dispatches (the leg's timed "
                   "steps, for a kernel only one leg launches, such as the C3a GEMM), are the figures to set "
                   "beside the bench line.\n\n"
                   + _md_table(["kernel", "calls", "avg us", "median us", f"avg of last {steps} us", "min us",
                                "max us", "% time"], rows))


def _summarize_traffic(root, traffic):
    cal = _calibration(root)
    if not cal:
        return
    traffic["_calibration"] = cal
    ff, wf = cal["fetch_factor"], cal["write_factor"]
    disp = _per_dispatch(root, ["fetch", "write"])
    rows = []
    for key, frag in KERNELS.items():
        f = [d["FETCH_SIZE"] for d in disp.values() if frag in d["kernel"] and "FETCH_SIZE" in d]
        w = [d["WRITE_SIZE"] for d in disp.values() if frag in d["kernel"] and "WRITE_SIZE" in d]
        if not f or not w or key == "copy_1GiB":
            continue
        fk, wk = sum(f) / len(f), sum(w) / len(w)
        b = fk * 1024 * ff + wk * 1024 * wf
        traffic[key] = {"FETCH_SIZE_KiB": fk, "WRITE_SIZE_KiB": wk, "bytes_per_launch": b,
                        "algorithmic_bytes": ALGO_BYTES[key], "ratio": b / ALGO_BYTES[key]}
        rows.append((key, f"{fk:.0f}", f"{wk:.0f}", f"{b / 1e9:.3f}", f"{ALGO_BYTES[key] / 1e9:.3f}",
                     f"{b / ALGO_BYTES[key]:.3f}"))
    # C5 rows: each call's kernels (one or two launches) summed.
    c5 = []
    for M, K, N in C5_ROWS:
        d5 = _per_dispatch(root, [f"c5_{M}_{K}_{N}_fetch", f"c5_{M}_{K}_{N}_write"])
        per = _by_kernel({k: v for k, v in d5.items()
                          if not v["kernel"].startswith(_SETUP_KERNELS + ("stream_read",))})
        f = sum(v.get("FETCH_SIZE", 0.0) for v in per.values())
        w = sum(v.get("WRITE_SIZE", 0.0) for v in per.values())
        if not per or not f:
            continue
        b = f * 1024 * ff + w * 1024 * wf
        algo = N * K + 8 * N + 4 * M * K + 2 * M * K + 4 * M * N
        key = f"c5_M{M}_K{K}_N{N}"
        traffic[key] = {"FETCH_SIZE_KiB": f, "WRITE_SIZE_KiB": w, "bytes_per_launch": b, "algorithmic_bytes": algo,
                        "ratio": b / algo, "kernels": sorted(f"{k[0]} x{k[1] // max(k[2], 1)}" for k in per)}
        c5.append((key, ", ".join(f"`{k[0]}` ({k[1] // max(k[2], 1)} WGs)" for k in sorted(per)), f"{f:.0f}",
                   f"{w:.0f}", f"{b / 1e6:.2f}", f"{algo / 1e6:.2f}", f"{b / algo:.3f}"))
    body = (f"Calibration: the library's `copy16_kernel` copying 1 GiB reads FETCH_SIZE = {cal['FETCH_SIZE_KiB']:.0f} "
            f"KiB and WRITE_SIZE = {cal['WRITE_SIZE_KiB']:.0f} KiB per dispatch for 1,048,576 KiB moved each way, so "
            f"FETCH_SIZE is scaled by {ff:.4f} and WRITE_SIZE by {wf:.4f} to give bytes.\n\n"
            + _md_table(["kernel", "FETCH_SIZE KiB", "WRITE_SIZE KiB", "HBM GB/launch", "algorithmic GB", "ratio"], rows))
    cmds = [profile_command("fetch"), profile_command("write")]
    if c5:
        body += ("\n\nC5 rows (`kh_linear_i8`, per call: the per-row quantize and the skinny GEMM for M > 2, the "
                 "fused decode kernel for M <= 3; algorithmic bytes N*K + 8N + 6MK + 4MN):\n\n"
                 + _md_table(["row", "kernels", "FETCH_SIZE KiB", "WRITE_SIZE KiB", "HBM MB/call", "algorithmic MB",
                              "ratio"], c5))
        cmds += [profile_command(f"c5_{M}_{K}_{N}_{w}") for M, K, N in C5_ROWS for w in ("fetch", "write")]
    _write_profile("hbm_traffic_mi355x.md", "HBM traffic per launch (rocprofv3 --pmc), one MI355X", cmds, body)


def _counter_table(per, cal):
    """Markdown table of derived quantities per (kernel, grid); a column is
    shown only when some kernel has the counters it needs."""
    ff = cal["fetch_factor"] if cal else 2.0
    wf = cal["write_factor"] if cal else 1.0
    cols = [("kernel", None), ("WGs", None), ("dispatches", None), ("us (median)", "{:.1f}"), ("clock MHz", "{:.0f}"),
            ("MFMA busy", "{:.2f}"), ("MFMA busy at that clock", "{:.2f}"), ("VALU issue", "{:.2f}"), ("fetched MB", "{:.1f}"), ("written MB", "{:.1f}"),
            ("L1->L2 reads", "{:.0f}"), ("L1->L2 latency (cycles)", "{:.0f}"), ("L2 hit", "{:.2f}"),
            ("L1 pending-stall share", "{:.2f}"), ("TD busy share", "{:.2f}"), ("LDS-DMA wave loads", "{:.3g}"),
            ("LDS bank-conflict cycles", "{:.3g}")]
    rows = []
    for (k, g, wg), v in sorted(per.items(), key=lambda kv: -kv[1]["us"] * kv[1]["n"]):
        us = v["us"]
        cyc = us * 1e-6 * 2.4e9
        r = {"kernel": f"`{k}`", "WGs": g // max(wg, 1), "dispatches": v["n"], "us (median)": us}
        # the clock only for launches long enough that the counting window is the kernel
        if us >= 100 and "SQ_CYCLES" in v:
            r["clock MHz"] = v["SQ_CYCLES"] / 32 / (us * 1e-6) / 1e6
        elif us >= 100 and "GRBM_COUNT" in v:
            r["clock MHz"] = v["GRBM_COUNT"] / 8 / (us * 1e-6) / 1e6
        if "SQ_VALU_MFMA_BUSY_CYCLES" in v:
            r["MFMA busy"] = v["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024 / cyc
            if "clock MHz" in r:
                r["MFMA busy at that clock"] = v["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024 / (us * r["clock MHz"])
        if "SQ_INSTS_VALU" in v:
            r["VALU issue"] = (v["SQ_INSTS_VALU"] - v.get("SQ_INSTS_MFMA", 0.0)) * 4 / 1024 / cyc
        if "FETCH_SIZE" in v:
            r["fetched MB"] = v["FETCH_SIZE"] * 1024 * ff / 1e6
        if "WRITE_SIZE" in v:
            r["written MB"] = v["WRITE_SIZE"] * 1024 * wf / 1e6
        if "TCP_TCC_READ_REQ_sum" in v:
            r["L1->L2 reads"] = v["TCP_TCC_READ_REQ_sum"]
            if "TCP_TCC_READ_REQ_LATENCY_sum" in v and v["TCP_TCC_READ_REQ_sum"] > 0:
                r["L1->L2 latency (cycles)"] = v["TCP_TCC_READ_REQ_LATENCY_sum"] / v["TCP_TCC_READ_REQ_sum"]
        if "TCC_HIT_sum" in v and v["TCC_HIT_sum"] + v.get("TCC_MISS_sum", 0.0) > 0:
            r["L2 hit"] = v["TCC_HIT_sum"] / (v["TCC_HIT_sum"] + v.get("TCC_MISS_sum", 0.0))
        if "TCP_PENDING_STALL_CYCLES_sum" in v:
            r["L1 pending-stall share"] = v["TCP_PENDING_STALL_CYCLES_sum"] / 256 / cyc
        if "TD_TD_BUSY_sum" in v:
            r["TD busy share"] = v["TD_TD_BUSY_sum"] / 256 / cyc
        if "TA_BUFFER_READ_LDS_WAVEFRONTS_sum" in v:
            r["LDS-DMA wave loads"] = v["TA_BUFFER_READ_LDS_WAVEFRONTS_sum"]
        if "SQ_LDS_BANK_CONFLICT" in v:
            r["LDS bank-conflict cycles"] = v["SQ_LDS_BANK_CONFLICT"]
        rows.append(r)
    shown = [(c, f) for c, f in cols if any(c in r for r in rows)]
    body = [[(r[c] if f is None else f.format(r[c])) if c in r else "" for c, f in shown] for r in rows]
    return _md_table([c for c, _ in shown], body)


_COUNTER_NOTE = ("Per dispatch, averaged over the runs.  us: median duration under the counter runs.  clock (launches "
                 "of 100 us or more): SQ_CYCLES / 32 shader engines, or GRBM_COUNT / 8 XCDs, over the duration.  MFMA "
                 "busy: SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / (duration x 2.4 GHz), and the same over the "
                 "measured clock's cycles where there is one; VALU issue: (SQ_INSTS_VALU - SQ_INSTS_MFMA) x 4 cycles "
                 "/ 1024 / (duration x 2.4 GHz); the L1 pending-stall and TD busy shares are per CU over the same "
                 "cycles -- all but the second against the peak clock, so lower bounds.  Bytes: FETCH_SIZE "
                 "and WRITE_SIZE scaled by the 1 GiB copy calibration (`hbm_traffic_mi355x.md`).  L1->L2 reads: "
                 "TCP_TCC_READ_REQ_sum (requests of up to 128 B).\n\n")

# Kernels that only build the model (weight quantization at construction) or
# calibrate: left out of the per-leg counter tables.
_SETUP_KERNELS = ("col_absmax", "pack_quant", "fill_u32", "fill_f64", "copy16", "__amd")


def _summarize_counters(root, runs, fname, title, cal, select=None):
    disp = _per_dispatch(root, runs)
    disp = {k: v for k, v in disp.items()
            if not v["kernel"].startswith(_SETUP_KERNELS) and (select is None or select(v))}
    if not disp:
        return
    _write_profile(fname, title, [profile_command(r) for r in runs if os.path.isdir(os.path.join(root, r))],
                   _COUNTER_NOTE + _counter_table(_by_kernel(disp), cal))


def _summarize_c4_forward(root, run="c4_trace", fname="c4_forward_mi355x.md",
                          title="C4 int8 char-LM forward: kernel time per forward on one MI355X (gfx950)",
                          which="the default `CharLM` forward"):
    """The C4 forward's kernel time per forward: the trace split at each
    embedding launch, the segments with the modal number of launches (one
    forward each; the others include the bench's per-GEMM re-runs), and per
    kernel and grid the median of its launches' time per forward."""
    tr = _find(os.path.join(root, run), "kernel_trace.csv")
    if not tr:
        return
    rows = sorted(_read_csv(tr), key=lambda r: int(r["Start_Timestamp"]))
    segs, cur = [], None
    for r in rows:
        k = _short(r["Kernel_Name"])
        if k.startswith("embedding"):
            if cur:
                segs.append(cur)
            cur = []
        if cur is not None:
            cur.append((k, _grid(r) // max(int(r.get("Workgroup_Size") or r.get("Workgroup_Size_X") or 1), 1),
                        (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    if cur:
        segs.append(cur)
    if not segs:
        return
    counts = {}
    for s_ in segs:
        counts[len(s_)] = counts.get(len(s_), 0) + 1
    mode = max(counts, key=counts.get)
    good = [s_ for s_ in segs if len(s_) == mode]
    order = {}
    for i, (k, g, _) in enumerate(good[0]):
        order.setdefault((k, g), []).append(i)
    table, total = [], 0.0
    for (k, g), idx in order.items():
        per = float(np.median([sum(s_[i][2] for i in idx) for s_ in good]))
        each = float(np.median([s_[i][2] for s_ in good for i in idx]))
        table.append((per, (f"`{k}`", g, len(idx), f"{each:.1f}", f"{per:.1f}")))
        total += per
    table.sort(key=lambda t: -t[0])
    body = (f"Workload: config C4 (vocab 65, d_model 384, 6 heads, 6 layers, FFN 1536, batch 64 x seq 256), the "
            f"{which} run eagerly (the kernels a HIP-graph replay launches; rocprofv3's kernel "
            f"trace has crashed inside hipGraphLaunch).  The trace is split into forwards at each embedding "
            f"launch; the {len(good)} segments holding exactly one forward's {mode} launches give the medians "
            f"below (durations include the profiler's per-dispatch timestamps).\n\n"
            + _md_table(["kernel", "WGs", "launches per forward", "us each", "us per forward"], [t[1] for t in table])
            + f"\n\nSum: {total:.1f} us of kernel time per forward.")
    _write_profile(fname, title, [profile_command(run)], body)


def summarize(root):
    """Regenerates profiles/*.md and profiles/traffic.json from the rocprofv3
    CSV output of the PROFILE_RUNS under root (each file only when its runs
    are present)."""
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    try:
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f)
    except (OSError, ValueError):
        traffic = {}
    _summarize_trace(root)
    _summarize_traffic(root, traffic)
    cal = traffic.get("_calibration")
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(traffic, f, indent=1, sort_keys=True)
    _summarize_counters(root, ["gemm_p1", "gemm_p2", "gemm_p3"], "gemm_i8_counters_mi355x.md",
                        "`gemm_i8_pingpong_kernel` (C3a, int8 8192^3, fused dequantize): hardware counters, one MI355X",
                        cal, select=lambda d: "gemm_i8_pingpong" in d["kernel"])
    _summarize_counters(root, ["c4_p1", "c4_p2", "c4_p3", "c4_p4"], "c4_counters_mi355x.md",
                        "C4 forward: hardware counters per kernel on one MI355X (gfx950)", cal)
    c5runs = [f"c5_{M}_{K}_{N}_{w}" for M, K, N in C5_ROWS for w in ("fetch", "write", "l2", "sq")]
    _summarize_counters(root, c5runs, "c5_counters_mi355x.md",
                        "C5 decode rows (`kh_linear_i8`): hardware counters per kernel, one MI355X", cal,
                        select=lambda d: not d["kernel"].startswith("copy16"))
    _summarize_c4_forward(root)
    _summarize_c4_forward(root, "c4row_trace", "c4_forward_per_token_mi355x.md",
                          "C4 int8 char-LM forward with per-token activation scales: kernel time per forward on one "
                          "MI355X (gfx950)", '`CharLM(act_granularity="row")` forward')
    return traffic


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


def _timed_slabs(fn, budget_s, max_calls):
    """Calls fn() until budget_s of wall time or max_calls; returns (calls, s)."""
    n = 0
    t0 = time.perf_counter()
    while n < max_calls and (n == 0 or time.perf_counter() - t0 < budget_s):
        fn()
        n += 1
    return n, time.perf_counter() - t0


def _c2_slab(rows, cols=16384, seed=2024):
    gen = np.random.Generator(np.random.PCG64(seed))
    x = gen.standard_normal((rows, cols), dtype=np.float32)
    n_out = rows * cols // 1000
    idx = gen.choice(rows * cols, size=n_out, replace=False)
    x.reshape(-1)[idx] = np.where(gen.random(n_out) < 0.5, -50.0, 50.0).astype(np.float32)
    return x


def cpu_c2(budget_s=3.0):
    """C2 on one host core: the per-row quantize and the dequantize of
    python/kansai/quantize.py:66-70 and :76 (binary64 scale and division,
    ties to even, clamp; binary64 product narrowed to binary32), as the
    oracle's C restatement, over slabs of 64 rows of the C2 distribution."""
    from oracle import oracle as O
    x = _c2_slab(64)
    q, s = O.ko_quantize_rows(x)
    nq, tq = _timed_slabs(lambda: O.ko_quantize_rows(x), budget_s, 1 << 20)
    nd, td = _timed_slabs(lambda: O.ko_dequantize_rows(q, s), budget_s, 1 << 20)
    el = x.size
    return {"quantize_GB/s": round(5.0 * el * nq / tq / 1e9, 3), "dequantize_GB/s": round(5.0 * el * nd / td / 1e9, 3),
            "cores": 1, "kind": "port",
            "sample": f"{nq} and {nd} passes over a [64, 16384] slab of C2's distribution (0.1 % +-50 outliers) through "
                      f"the C restatement of quantize.py:66-76 (the reference's own path is CPython list comprehensions, "
                      f"slower still); 5 B per element"}


def cpu_c3b(budget_s=4.0):
    """C3b on one host core: the reference's compiled fp32 i-k-j matmul
    (backend/cpu/src/Ops.cpp:322-339, oracle/_ref) on 4-row slabs of the
    4096^3 problem."""
    from oracle import oracle as O
    n = 4096
    gen = np.random.Generator(np.random.PCG64(4))
    b = gen.standard_normal((n, n), dtype=np.float32)
    a = gen.standard_normal((4, n), dtype=np.float32)
    use_ref = O.ref_available()
    mm = O.ref_matmul if use_ref else O.ko_matmul_f32
    calls, dt = _timed_slabs(lambda: mm(a, b), budget_s, 256)
    rows = 4 * calls
    return {"TFLOP/s": round(2.0 * rows * n * n / dt / 1e12, 6), "cores": 1, "kind": "reference" if use_ref else "port",
            "sample": f"{rows} rows x 4096 x 4096 of C3b through Ops.cpp's i-k-j loop (-O3, 1 thread), {dt:.1f} s, "
                      f"scaled linearly in rows"}


def cpu_c4(budget_s=4.0):
    """C4 on one host core as the reference computes it: one pre-LN block
    (python/kansai/nn.py:466-478) for one sequence of 256 tokens, the
    Linears as its QLinear does (x @ dequantize(W) + b, quantize.py:115-122)
    and the attention products (nn.py:381-427) through its compiled i-k-j
    matmul (oracle/_ref); LayerNorm, softmax and GELU elementwise in numpy
    float32.  The forward's time is that block's time x 6 layers x 64
    sequences plus the final LayerNorm and head."""
    from oracle import charlm_ref as R
    from oracle import oracle as O
    from kansaiml_amd.charlm import CharLMWeights
    w = CharLMWeights(seed=0)
    use_ref = O.ref_available()
    mm = O.ref_matmul if use_ref else O.ko_matmul_f32
    add = O.ref_add_bias if use_ref else O.ko_add_bias
    T, D, H = 256, w.d_model, w.heads
    dk = D // H

    def deq(wm):
        q, s = O.ko_quantize_cols_packed(wm)
        return np.ascontiguousarray((q.T.astype(np.float64) * s[None, :]).astype(np.float32))

    p = w.blocks[0]
    wq = deq(np.concatenate([p["w_q"], p["w_k"], p["w_v"]], axis=1))
    wo, w1, w2, wh = deq(p["w_o"]), deq(p["fc1_w"]), deq(p["fc2_w"]), deq(w.head_w)
    ids = np.random.Generator(np.random.PCG64(9)).integers(0, 65, T)
    x0 = (w.tok[ids] + w.pos[:T]).astype(np.float32)
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], np.float32(0), np.float32(-1e9))

    def block(x):
        h = R.layer_norm(x, p["ln1_w"], p["ln1_b"])
        qkv = mm(h, wq)
        heads = []
        for hh in range(H):
            q = np.ascontiguousarray(qkv[:, hh * dk:(hh + 1) * dk])
            k = np.ascontiguousarray(qkv[:, D + hh * dk:D + (hh + 1) * dk].T)
            v = np.ascontiguousarray(qkv[:, 2 * D + hh * dk:2 * D + (hh + 1) * dk])
            sc = mm(q, k) * np.float32(1.0 / np.sqrt(dk)) + mask
            sc = sc - sc.max(axis=-1, keepdims=True)
            e = np.exp(sc)
            heads.append(mm((e / e.sum(axis=-1, keepdims=True)).astype(np.float32), v))
        x = (x + mm(np.concatenate(heads, axis=1), wo)).astype(np.float32)
        h = R.layer_norm(x, p["ln2_w"], p["ln2_b"])
        f = R.gelu(add(mm(h, w1), p["fc1_b"]))
        return (x + add(mm(f, w2), p["fc2_b"])).astype(np.float32)

    nb, tb = _timed_slabs(lambda: block(x0), budget_s, 64)
    nh, th = _timed_slabs(lambda: add(mm(R.layer_norm(x0, w.lnf_w, w.lnf_b), wh), w.head_b), 0.5, 64)
    ms = (tb / nb * w.layers + th / nh) * 64 * 1e3
    return {"ms_per_forward": round(ms, 1), "tokens_per_s": round(64 * 256 / (ms * 1e-3), 1), "cores": 1,
            "kind": "reference" if use_ref else "port",
            "sample": f"{nb} passes of one pre-LN block over one 256-token sequence ({tb / nb * 1e3:.1f} ms each) and "
                      f"{nh} of the head, scaled x6 layers x64 sequences; Linears and attention products through "
                      f"Ops.cpp's i-k-j matmul on dequantized weights (the reference's QLinear), elementwise in numpy"}


def cpu_c5(rows, budget_s=0.6):
    """C5 on one host core, the reference's path for a quantized decode
    Linear: x @ dequantize(W) + b (quantize.py:115-122) through its compiled
    i-k-j matmul (oracle/_ref) on the dequantized per-channel weight."""
    from oracle import oracle as O
    use_ref = O.ref_available()
    mm = O.ref_matmul if use_ref else O.ko_matmul_f32
    add = O.ref_add_bias if use_ref else O.ko_add_bias
    out = {}
    gen = np.random.Generator(np.random.PCG64(6))
    for K, N in sorted({(k, n) for _, k, n in rows}):
        q, s = O.ko_quantize_cols_packed(c5_host_weight(K, N))
        wd = np.ascontiguousarray((q.T.astype(np.float64) * s[None, :]).astype(np.float32))
        del q
        b = np.zeros(N, np.float32)
        for M, k2, n2 in rows:
            if (k2, n2) != (K, N):
                continue
            x = gen.standard_normal((M, K), dtype=np.float32)
            calls, dt = _timed_slabs(lambda: add(mm(x, wd), b), budget_s, 1000)
            us = dt / calls * 1e6
            out[(M, K, N)] = {"us": round(us, 1), "cores": 1, "kind": "reference" if use_ref else "port",
                              "sample": f"{calls} calls of x @ dequantize(W) + b (Ops.cpp i-k-j, 1 thread)"}
    return out


def main():
    global WARM_MS, GRAPH_TIMING
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
    ap.add_argument("--warm-ms", type=float, default=WARM_MS,
                    help="minimum untimed warm-up per leg in ms (0 under counter runs, which serialise dispatches)")
    ap.add_argument("--profile-commands", metavar="DIR",
                    help="print the rocprofv3 commands whose output --summarize reads, and exit")
    ap.add_argument("--no-graph-timing", action="store_true",
                    help="time C1 and C5 from Python-issued calls only (for profiler runs)")
    ap.add_argument("--c5-rows", default=None,
                    help="C5 rows to run as M:K:N,... (default: all six); for per-row counter runs")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    if args.profile_commands:
        for name in PROFILE_RUNS:
            print(profile_command(name, args.profile_commands))
        return
    WARM_MS = args.warm_ms
    GRAPH_TIMING = not args.no_graph_timing
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

    # The latency-bound legs first: right after the power-heavy GEMM legs their
    # microsecond launches measured up to 2x slower.
    c1 = None
    if "c1" in only:
        log("C1 int8 quantized Linear ...")
        c1 = bench_c1(max(50, args.steps), args.warmup)
        log(f"C1: {c1['us_kernels_back_to_back']:.2f} us per call (one launch, back to back as a graph; "
            f"{c1['us_kernels_stream']:.2f} us issued from Python; two launches {c1['us_two_launch']:.2f} us), "
            f"{c1['us_eager_call']:.2f} us eager")
    skinny = None
    if "skinny" in only:
        log("skinny decode GEMMs C5 ...")
        c5_rows = ([tuple(int(v) for v in r.split(":")) for r in args.c5_rows.split(",")] if args.c5_rows
                   else C5_ROWS)
        skinny = bench_skinny(max(20, args.steps), args.warmup, c5_rows)
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
    c4 = None
    if "c4" in only:
        log("C4 int8 char-LM forward ...")
        c4 = bench_c4(max(5, args.steps // 4), max(2, args.warmup // 10))
        log(f"C4 forward: {c4['ms_per_forward']:.3f} ms ({c4['timing']}; {c4['tokens_per_s']:.0f} tokens/s), "
            f"{c4['ms_per_forward_eager']:.3f} ms eager")
        Nn.call("kh_pool_trim")
    c4row = None
    if "c4row" in only:
        log("C4 forward with per-token activation scales ...")
        c4row = bench_c4_per_token(max(5, args.steps // 4), max(2, args.warmup // 10))
        log(f"C4 per-token forward: {c4row['ms_per_forward']:.3f} ms ({c4row['timing']})")
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

    cpu = cpu_c2v = cpu_c3bv = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline()
        log(f"CPU baseline {cpu['value']:.6f} TOPS")
        if c1 is not None:
            c1["cpu"] = cpu_c1()
            log(f"C1 on the CPU: {c1['cpu']['us_per_call']:.1f} us per call")
        if "quant" in only:
            cpu_c2v = cpu_c2()
            log(f"C2 on the CPU: quantize {cpu_c2v['quantize_GB/s']} GB/s, dequantize {cpu_c2v['dequantize_GB/s']} GB/s")
        if "f32" in only:
            cpu_c3bv = cpu_c3b()
            log(f"C3b on the CPU: {cpu_c3bv['TFLOP/s']} TFLOP/s")
        if c4 is not None:
            c4["cpu"] = cpu_c4()
            log(f"C4 on the CPU: {c4['cpu']['ms_per_forward']} ms per forward")
        if skinny:
            c5cpu = cpu_c5([(r["M"], r["K"], r["N"]) for r in skinny])
            for r in skinny:
                r["cpu"] = c5cpu[(r["M"], r["K"], r["N"])]
            log("C5 on the CPU: " + ", ".join(f"M={r['M']} N={r['N']} {r['cpu']['us']} us" for r in skinny))
    attainable_frac = (round(g_tops / probe["TOPS"], 4) if probe and probe.get("TOPS") and g_tops == g_tops
                       else None)

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
                     "attainable": probe, "frac_of_attainable": attainable_frac},
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
            "cpu": cpu_c2v,
        },
        "fp32_matmul": {"workload": "C3b fp32 matmul 4096^3", "ms": round(f_ms, 5), "TFLOP/s": round(f_tflops, 2),
                        "roofline": {"bound": "mfma", "achieved": round(f_tflops, 2), "peak": PEAK_FP32_TFLOPS,
                                     "unit": "TFLOP/s", "frac": round(f_tflops / PEAK_FP32_TFLOPS, 4),
                                     "traffic": measured_traffic("fp32_matmul_4096")},
                        "cpu": cpu_c3bv},
        "skinny_decode": {"workload": "C5 kh_linear_i8: per-token quantize + int8 GEMM, per-channel weights",
                          "bytes": "N*K + 8N + 4MK + 2MK + 4MN", "rows": skinny},
        "c1_linear": c1,
        "c4_forward": c4,
        "c4_forward_per_token": c4row,
        "host_buffers": host_buffers,
        "cpu_baseline": cpu,
        "warmup_per_leg": {"min_ms": WARM_MS, **WARMUP_LOG},
        "device": info,
    }
    print(json.dumps(result).replace("NaN", "null"))


if __name__ == "__main__":
    main()
