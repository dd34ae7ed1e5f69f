/*
 * kansai_oracle.c -- CPU restatement of the reference's int8 quantize ->
 * int8 matmul -> dequantize path and of its fp32 matmul + bias.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (kansaiml_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, as the checker.
 *
 * Every function states the reference file:line it restates.  The
 * reference quantizer is Python (python/kansai/quantize.py); its arithmetic
 * is IEEE binary64 with round-half-to-even, which C99 gives directly:
 *   - Python `v / scale` on floats      == C `(double)v / scale`
 *   - Python `round(x)` (float -> int)  == C `nearbyint(x)` in the default
 *     FE_TONEAREST mode (ties to even); NOT C `round()` (ties away).
 *   - `core.from_flat` converts each binary64 to binary32 with
 *     round-to-nearest-even, which is C's `(float)d`.
 * Build with -O3 -fno-fast-math -ffp-contract=off so no FMA contraction
 * or reassociation changes a result.
 *
 * Parity pins (tests/test_oracle.py): the reference test's own known-answer
 * checks (tests/test_quantize.py:41-59 and :66-72 of the reference), the
 * golden fixtures in tests/golden/ (made by a pure-Python evaluation of the
 * reference formula with CPython's own round()), hand-built ties, and
 * independent library routines (numpy int64 matmul for the int8 GEMM,
 * numpy float64 for the epilogue, the reference's own compiled Ops.cpp
 * from oracle/_ref for the fp32 loop).
 */
#include "kansai_oracle.h"

#include <math.h>
#include <string.h>

/* quantize.py:67-69 for one slice of n values with element stride
 * `stride`: m = max |v| (default 0.0); scale = m/127.0 if m > 0 else 1.0;
 * q = clamp(round(v/scale), -127, 127).  Returns KO_NONFINITE if any value
 * is NaN or +-inf (the reference raises ValueError/OverflowError from
 * round() there); codes are then left as 0 and the scale as NaN. */
static int quantize_slice(const float* v, int64_t n, int64_t stride,
                          int8_t* q, int64_t qstride, double* scale_out) {
    double m = 0.0;
    int bad = 0;
    for (int64_t i = 0; i < n; ++i) {
        double a = fabs((double)v[i * stride]);
        if (!isfinite(a)) bad = 1;
        else if (a > m) m = a;
    }
    if (bad) {
        for (int64_t i = 0; i < n; ++i) q[i * qstride] = 0;
        *scale_out = NAN;
        return KO_NONFINITE;
    }
    const double scale = (m > 0.0) ? m / 127.0 : 1.0;  /* quantize.py:68 */
    for (int64_t i = 0; i < n; ++i) {                  /* quantize.py:69 */
        double r = nearbyint((double)v[i * stride] / scale);
        if (r > 127.0) r = 127.0;
        if (r < -127.0) r = -127.0;
        q[i * qstride] = (int8_t)r;
    }
    *scale_out = scale;
    return KO_OK;
}

/* quantize.py:50-70, per tensor (one scale for all n values). */
int ko_quantize_tensor(const float* x, int64_t n, int8_t* q, double* scale) {
    return quantize_slice(x, n, 1, q, 1, scale);
}

/* quantize.py:50-70 applied to each row of a row-major [rows, cols]
 * matrix (per-token activations; config C2's per-row scales). */
int ko_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, double* scales) {
    int rc = KO_OK;
    for (int64_t r = 0; r < rows; ++r) {
        int e = quantize_slice(x + r * cols, cols, 1, q + r * cols, 1, &scales[r]);
        if (e != KO_OK) rc = e;
    }
    return rc;
}

/* quantize.py:50-70 applied to each column j of a row-major [k, n] matrix
 * (an nn.Linear weight, laid out [in, out] by python/kansai/nn.py:77, so
 * one column is one output channel).  Codes are written packed
 * K-contiguous: q_packed[j * k + i] = code of w[i, j]. */
int ko_quantize_cols_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scales) {
    int rc = KO_OK;
    for (int64_t j = 0; j < n; ++j) {
        int e = quantize_slice(w + j, k, n, q_packed + j * k, 1, &scales[j]);
        if (e != KO_OK) rc = e;
    }
    return rc;
}

/* Per-tensor scale (quantize.py:50-70 on the whole [k, n] weight) with the
 * same K-contiguous packing as ko_quantize_cols_packed. */
int ko_quantize_tensor_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scale) {
    double m = 0.0;
    int bad = 0;
    for (int64_t i = 0; i < k * n; ++i) {
        double a = fabs((double)w[i]);
        if (!isfinite(a)) bad = 1;
        else if (a > m) m = a;
    }
    if (bad) {
        memset(q_packed, 0, (size_t)(k * n));
        *scale = NAN;
        return KO_NONFINITE;
    }
    const double s = (m > 0.0) ? m / 127.0 : 1.0;
    for (int64_t i = 0; i < k; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double r = nearbyint((double)w[i * n + j] / s);
            if (r > 127.0) r = 127.0;
            if (r < -127.0) r = -127.0;
            q_packed[j * k + i] = (int8_t)r;
        }
    *scale = s;
    return KO_OK;
}

/* quantize.py:73-77: flat = [q*scale] in binary64, then core.from_flat
 * narrows each to binary32 (round to nearest even). */
void ko_dequantize_tensor(const int8_t* q, int64_t n, double scale, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = (float)((double)q[i] * scale);
}

void ko_dequantize_rows(const int8_t* q, int64_t rows, int64_t cols, const double* scales, float* out) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c)
            out[r * cols + c] = (float)((double)q[r * cols + c] * scales[r]);
}

/* int8 x int8 -> int32 GEMM.  The reference has none (quantize.py:115-122
 * dequantizes instead); this is the closed form acc[i,j] = sum_k a[i,k] *
 * bt[j,k], exact in int32 for k <= 133144 since |a*b| <= 127*127.
 * a: [M, K] row-major, bt: [N, K] row-major (the packed weight). */
void ko_gemm_i8(const int8_t* a, const int8_t* bt, int64_t M, int64_t N, int64_t K, int32_t* acc) {
    for (int64_t i = 0; i < M; ++i) {
        const int8_t* ar = a + i * K;
        for (int64_t j = 0; j < N; ++j) {
            const int8_t* br = bt + j * K;
            int32_t s = 0;
            for (int64_t kk = 0; kk < K; ++kk) s += (int32_t)ar[kk] * (int32_t)br[kk];
            acc[i * N + j] = s;
        }
    }
}

/* The dequantize epilogue of the int8 GEMM, defined as the reference's
 * dequantize (quantize.py:76: binary64 product, narrowed to binary32)
 * applied to the accumulator with the combined scale, followed by the
 * reference's fp32 bias add (Ops.cpp:34-38):
 *   out[i,j] = (float)((double)acc[i,j] * (sa_i * sb_j)) + bias[j]
 * sa has M entries (per row / per token) or 1 (per tensor); likewise sb
 * has N entries (per output channel) or 1.  bias may be NULL. */
void ko_epilogue(const int32_t* acc, int64_t M, int64_t N,
                 const double* sa, int64_t sa_n, const double* sb, int64_t sb_n,
                 const float* bias, float* out) {
    for (int64_t i = 0; i < M; ++i) {
        const double si = sa[sa_n == 1 ? 0 : i];
        for (int64_t j = 0; j < N; ++j) {
            const double s = si * sb[sb_n == 1 ? 0 : j];
            float y = (float)((double)acc[i * N + j] * s);
            if (bias) y = y + bias[j];
            out[i * N + j] = y;
        }
    }
}

/* backend/cpu/src/Ops.cpp:322-339, the Linux (non-Accelerate) branch:
 * fill 0, then i-k-j accumulation in binary32. */
void ko_matmul_f32(const float* a, const float* b, float* out, int64_t M, int64_t K, int64_t N) {
    for (int64_t i = 0; i < M * N; ++i) out[i] = 0.0f;
    for (int64_t i = 0; i < M; ++i)
        for (int64_t kk = 0; kk < K; ++kk) {
            const float av = a[i * K + kk];
            const float* brow = b + kk * N;
            float* orow = out + i * N;
            for (int64_t j = 0; j < N; ++j) orow[j] += av * brow[j];
        }
}

/* backend/cpu/src/Ops.cpp:34-38 (Tensor::add's bias branch,
 * core/src/Tensor.cpp:158-166). */
void ko_add_bias(const float* x, const float* bias, float* out, int64_t batch, int64_t features) {
    for (int64_t i = 0; i < batch; ++i)
        for (int64_t j = 0; j < features; ++j)
            out[i * features + j] = x[i * features + j] + bias[j];
}
