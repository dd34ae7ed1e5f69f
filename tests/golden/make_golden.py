"""Writes the golden fixtures in tests/golden/*.npz.

Expected outputs are computed by a pure-Python evaluation of the
reference's own formulas (python/kansai/quantize.py:66-70 and :76 of the
reference, executed here with CPython's binary64 floats and its round(),
which is ties-to-even) -- NOT by the C oracle, so the fixtures pin the
oracle and the GPU kernels independently.  Nothing from /root/reference
is imported; the formulas are restated in oracle/oracle.py (py_*).

Inputs reproduce the reference tests' own data where it is Python-seeded
(tests/test_quantize.py:41-43: random.Random(0), 1000 x uniform(-3, 3),
narrowed to fp32 by from_flat) and use numpy PCG64 seeds otherwise.  The
inputs are stored inside each fixture, so the tests need no RNG.

Run:  python tests/golden/make_golden.py
"""

import os
import random
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))

from oracle.oracle import f32, py_quantize_symmetric, py_dequantize  # noqa: E402


def quant_fixture(vals):
    """vals: list of fp32-representable floats -> (q int8 array, scale, deq fp32 array)."""
    q, scale = py_quantize_symmetric(vals)
    deq = py_dequantize(q, scale)
    return np.array(q, np.int8), scale, np.array(deq, np.float32)


def save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, {k: v.shape for k, v in arrays.items()})


def _near_tie_values(gen, m, n):
    """n fp32 values (plus m itself first) whose quotient by m/127 lies
    within a few fp32 ulps of a half-integer."""
    s = m / 127.0
    vals = [f32(m)]
    while len(vals) < n + 1:
        k = int(gen.integers(-127, 127))
        t = (k + 0.5) * s
        v0 = np.float32(t)
        for v in (np.nextafter(v0, np.float32(-np.inf)), v0, np.nextafter(v0, np.float32(np.inf))):
            if abs(float(v)) <= m:
                vals.append(float(v))
    return vals[: n + 1]


def _near_tie_tensor(gen, m, n):
    vals = _near_tie_values(gen, f32(m), n)
    q, s, d = quant_fixture(vals)
    return dict(x=np.array(vals, np.float32), q=q, scale=np.array([s]), deq=d)


def per_tensor_cases():
    # 1. The reference test's own input: tests/test_quantize.py:41-43.
    rng = random.Random(0)
    vals = [f32(rng.uniform(-3.0, 3.0)) for _ in range(1000)]
    q, s, d = quant_fixture(vals)
    save("ref_test_quantize_1000", x=np.array(vals, np.float32), q=q, scale=np.array([s]), deq=d)

    # 2. tests/test_quantize.py:58-59: exact zero -> q = 0.
    vals = [0.0, 1.0, -1.0]
    q, s, d = quant_fixture(vals)
    save("zero_maps_to_zero", x=np.array(vals, np.float32), q=q, scale=np.array([s]), deq=d)

    # 3. Ties: with max |v| = 127 the scale is exactly 1.0, so v = k + 0.5
    #    divides to an exact half and round() must go to the even k.  With
    #    max |v| = 63.5 the scale is exactly 0.5.  Round-half-away-from-zero
    #    fails every one of these.
    ties = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, -126.5, 100.5, -0.0, 0.0]
    q, s, d = quant_fixture([f32(v) for v in ties])
    save("ties_scale_one", x=np.array(ties, np.float32), q=q, scale=np.array([s]), deq=d)
    ties2 = [63.5, 0.25, 0.75, 1.25, -1.25, 62.25, -62.75, 31.25]
    q, s, d = quant_fixture([f32(v) for v in ties2])
    save("ties_scale_half", x=np.array(ties2, np.float32), q=q, scale=np.array([s]), deq=d)

    # 3b. Near-ties: the fp32 neighbours of (k + 0.5) * scale.  Their exact
    #     quotients straddle the half-integer by a few fp32 ulps, so binary32
    #     division or a reciprocal multiply rounds some of them the wrong
    #     way while the reference's binary64 division does not.
    save("near_ties", **_near_tie_tensor(np.random.Generator(np.random.PCG64(21)), 3.7, 4000))

    # 4. All-zero tensor: scale 1.0 (quantize.py:68), every code 0.
    q, s, d = quant_fixture([0.0] * 17)
    save("all_zero", x=np.zeros(17, np.float32), q=q, scale=np.array([s]), deq=d)

    # 5. Reduction sizes straddling a block width, from the reference's
    #    tests/test_metal_backend.py:263-273 (1, 4, 255, 256, 257, 1000,
    #    100000), N(0,1) with a few planted outliers.
    gen = np.random.Generator(np.random.PCG64(5))
    for n in (1, 4, 255, 256, 257, 1000, 100000):
        x = gen.standard_normal(n).astype(np.float32)
        if n > 10:
            idx = gen.choice(n, size=max(1, n // 1000), replace=False)
            x[idx] = np.where(gen.random(idx.size) < 0.5, -50.0, 50.0).astype(np.float32)
        q, s, d = quant_fixture([float(v) for v in x])
        save(f"per_tensor_n{n}", x=x, q=q, scale=np.array([s]), deq=d)


def per_row_and_col_cases():
    gen = np.random.Generator(np.random.PCG64(7))
    # Per-row (per-token) quantize, including an all-zero row, a row whose
    # max is negative, a single-element row and planted +-50 outliers.
    for rows, cols in ((5, 33), (16, 1024), (3, 1), (64, 4099)):
        x = gen.standard_normal((rows, cols)).astype(np.float32)
        if rows > 1:
            x[1, :] = 0.0
        if cols > 8:
            x[0, 3] = -50.0
            x[rows - 1, cols // 2] = 50.0
        qs, ss, ds = [], [], []
        for r in range(rows):
            q, s, d = quant_fixture([float(v) for v in x[r]])
            qs.append(q)
            ss.append(s)
            ds.append(d)
        save(f"per_row_{rows}x{cols}", x=x, q=np.stack(qs), scale=np.array(ss), deq=np.stack(ds))

    # Per-row near-ties: every row has its own max (so its own scale) and
    # values a few ulps either side of (k + 0.5) * scale.
    rows, cols = 24, 1024
    xs, qs, ss, ds = [], [], [], []
    for r in range(rows):
        m = f32(float(gen.uniform(0.01, 80.0)))
        vals = _near_tie_values(gen, m, cols - 1)
        perm = gen.permutation(cols)
        vals = [vals[i] for i in perm]
        q, s, d = quant_fixture(vals)
        xs.append(np.array(vals, np.float32))
        qs.append(q)
        ss.append(s)
        ds.append(d)
    save("per_row_near_ties_24x1024", x=np.stack(xs), q=np.stack(qs), scale=np.array(ss), deq=np.stack(ds))

    # Per-output-channel quantize of an [in, out] weight (nn.py:77 layout),
    # codes packed K-contiguous ([out, in]).
    for k, n in ((19, 15), (64, 48)):
        w = (gen.standard_normal((k, n)) * 0.02).astype(np.float32)
        w[:, 2] *= 20.0  # an outlier column
        qs, ss = [], []
        for j in range(n):
            q, s, _ = quant_fixture([float(v) for v in w[:, j]])
            qs.append(q)
            ss.append(s)
        save(f"per_col_{k}x{n}", w=w, q_packed=np.stack(qs), scale=np.array(ss))


def gemm_cases():
    """int8 GEMM accumulators (exact Python ints) and the dequantize
    epilogue out = f32(acc * (sa*sb)) + bias (bias added in binary32), at
    the reference's own non-tile-aligned sizes (DEVLOG.md:362-366:
    17x15x19, 100x50x77, 1x1x1) plus C1's per-tensor int8 Linear shape at
    a reduced batch."""
    gen = np.random.Generator(np.random.PCG64(11))
    for (M, N, K, per_row, per_col) in ((17, 15, 19, False, False), (100, 50, 77, True, True),
                                        (1, 1, 1, False, False), (8, 512, 512, False, False),
                                        (33, 40, 130, True, False)):
        a = gen.integers(-127, 128, size=(M, K), dtype=np.int8)
        bt = gen.integers(-127, 128, size=(N, K), dtype=np.int8)
        sa = gen.uniform(0.001, 0.05, size=M if per_row else 1)
        sb = gen.uniform(0.001, 0.05, size=N if per_col else 1)
        bias = gen.standard_normal(N).astype(np.float32)
        al = a.tolist()
        bl = bt.tolist()
        acc = [[sum(x * y for x, y in zip(al[i], bl[j])) for j in range(N)] for i in range(M)]
        out = np.empty((M, N), np.float32)
        for i in range(M):
            si = float(sa[i if per_row else 0])
            for j in range(N):
                s = si * float(sb[j if per_col else 0])
                y = np.float32(f32(acc[i][j] * s)) + bias[j]  # binary32 add
                out[i, j] = y
        save(f"gemm_i8_{M}x{N}x{K}", a=a, bt=bt, sa=sa, sb=sb, bias=bias,
             acc=np.array(acc, np.int32), out=out)


def epilogue_order_case():
    """A GEMM whose diagonal outputs land on binary32 rounding midpoints, so
    the epilogue's association order is observable: acc * (sa_i * sb_j)
    (the definition) and (acc * sa_i) * sb_j round to different binary32
    values there.  K = 4 with a single nonzero per row/column, so
    acc[i, i] = a_i (small odd integers) and off-diagonals are 0 + bias."""
    gen = np.random.Generator(np.random.PCG64(31))
    n = 16
    a = np.zeros((n, 4), np.int8)
    bt = np.zeros((n, 4), np.int8)
    sa = np.empty(n)
    sb = np.empty(n)
    i = 0
    while i < n:
        av = int(gen.choice([3, 5, 7, 9, 11, 13, -3, -7]))
        s_a = float(gen.uniform(0.001, 0.05))
        f = np.float32(av * s_a * 0.02)
        y = float(f) + float(np.spacing(f)) / 2.0  # an exact binary32 midpoint
        s_b = y / (av * s_a)
        good = f32(av * (s_a * s_b))
        other = f32((av * s_a) * s_b)
        if good != other:
            a[i, 0] = av
            bt[i, 0] = 1
            sa[i] = s_a
            sb[i] = s_b
            i += 1
    bias = np.zeros(n, np.float32)
    acc = (a.astype(np.int64) @ bt.astype(np.int64).T).astype(np.int32)
    out = np.empty((n, n), np.float32)
    for r in range(n):
        for c in range(n):
            out[r, c] = np.float32(f32(int(acc[r, c]) * (float(sa[r]) * float(sb[c])))) + bias[c]
    save("gemm_i8_epilogue_order_16x16x4", a=a, bt=bt, sa=sa, sb=sb, bias=bias, acc=acc, out=out)


if __name__ == "__main__":
    per_tensor_cases()
    per_row_and_col_cases()
    gemm_cases()
    epilogue_order_case()
