/*
 * oracle_selftest.c -- drives every function of kansai_oracle.c on small
 * and edge-case inputs, for a build under AddressSanitizer and
 * UndefinedBehaviorSanitizer (`make -C oracle sanitize`).
 *
 * TEST INFRASTRUCTURE ONLY (a checker of the checker).  Each check is a
 * closed form or an independent recomputation, not the oracle's formula
 * retyped: ties to even (python/kansai/quantize.py:69 uses Python's round),
 * the zero tensor's scale 1.0 (quantize.py:68), per-row / per-column results
 * equal to the per-tensor quantize of that slice, the packed per-tensor
 * weight equal to the transposed per-tensor quantize, the int8 GEMM against
 * an int64 loop in another order, the epilogue against a binary64
 * recomputation, and the fp32 matmul against binary64 within the i-k-j
 * loop's rounding bound.  Prints "oracle selftest: ok" and exits 0 on
 * success; any failure (or sanitizer report) exits nonzero.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kansai_oracle.h"

static int failures = 0;

#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                 \
            fputc('\n', stderr);                          \
            ++failures;                                   \
        }                                                 \
    } while (0)

/* A small deterministic generator (xorshift64*), so the test needs no libc
 * random state. */
static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {
    rng_state ^= rng_state >> 12;
    rng_state ^= rng_state << 25;
    rng_state ^= rng_state >> 27;
    return rng_state * 2685821657736338717ull;
}
static float uniform(float lo, float hi) {
    return lo + (hi - lo) * (float)((next_u64() >> 40) * (1.0 / 16777216.0));
}
static int8_t code(void) { return (int8_t)((int)(next_u64() % 255) - 127); }

/* Exact heap allocations (no slack), so an off-by-one read or write is an
 * ASan report. */
static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static void test_quantize_tensor(void) {
    /* scale 1.0 (max 127): v / s is v itself, so the ties are exact */
    const float v[] = {127.0f, 0.5f, 1.5f, 2.5f, -0.5f, -1.5f, -126.5f, 3.0f};
    const int8_t want[] = {127, 0, 2, 2, 0, -2, -126, 3};
    int8_t q[8];
    double s = 0;
    CHECK(ko_quantize_tensor(v, 8, q, &s) == KO_OK, "rc");
    CHECK(s == 1.0, "scale %g", s);
    for (int i = 0; i < 8; ++i) CHECK(q[i] == want[i], "tie %d: %d != %d", i, q[i], want[i]);

    /* zero tensor and empty tensor: scale 1.0, codes 0 */
    float z[5] = {0.0f, -0.0f, 0.0f, 0.0f, 0.0f};
    int8_t qz[5];
    CHECK(ko_quantize_tensor(z, 5, qz, &s) == KO_OK && s == 1.0, "zero scale %g", s);
    for (int i = 0; i < 5; ++i) CHECK(qz[i] == 0, "zero code");
    CHECK(ko_quantize_tensor(z, 0, qz, &s) == KO_OK && s == 1.0, "empty scale %g", s);

    /* +-max maps to +-127; |v - q s| <= s / 2 */
    const int n = 1001;
    float* x = xmalloc(sizeof(float) * n);
    int8_t* qx = xmalloc((size_t)n);
    for (int i = 0; i < n; ++i) x[i] = uniform(-3.0f, 3.0f);
    x[17] = -4.0f;
    CHECK(ko_quantize_tensor(x, n, qx, &s) == KO_OK, "rc");
    CHECK(s == 4.0 / 127.0, "scale %.17g", s);
    CHECK(qx[17] == -127, "max code %d", qx[17]);
    for (int i = 0; i < n; ++i) CHECK(fabs((double)x[i] - qx[i] * s) <= s / 2, "error bound at %d", i);

    /* non-finite input is refused */
    x[3] = NAN;
    CHECK(ko_quantize_tensor(x, n, qx, &s) == KO_NONFINITE, "NaN accepted");
    x[3] = INFINITY;
    CHECK(ko_quantize_tensor(x, n, qx, &s) == KO_NONFINITE, "inf accepted");
    free(x);
    free(qx);
}

static void test_slices(void) {
    const int64_t k = 37, n = 29;
    float* w = xmalloc(sizeof(float) * k * n);
    float* col = xmalloc(sizeof(float) * k);
    int8_t* qp = xmalloc((size_t)(k * n));
    int8_t* qr = xmalloc((size_t)(k * n));
    int8_t* qt = xmalloc((size_t)(k * n));
    int8_t* qc = xmalloc((size_t)k);
    double* sc = xmalloc(sizeof(double) * n);
    double* sr = xmalloc(sizeof(double) * k);
    double s1 = 0, st = 0;
    for (int64_t i = 0; i < k * n; ++i) w[i] = uniform(-1.0f, 1.0f) * (1.0f + (float)(i % 7));
    for (int64_t i = 0; i < k; ++i) w[i * n + 5] = 0.0f; /* an all-zero column */

    /* per column, packed: equal to the per-tensor quantize of that column */
    CHECK(ko_quantize_cols_packed(w, k, n, qp, sc) == KO_OK, "rc");
    for (int64_t j = 0; j < n; ++j) {
        for (int64_t i = 0; i < k; ++i) col[i] = w[i * n + j];
        CHECK(ko_quantize_tensor(col, k, qc, &s1) == KO_OK, "rc");
        CHECK(sc[j] == s1, "col scale %lld", (long long)j);
        for (int64_t i = 0; i < k; ++i) CHECK(qp[j * k + i] == qc[i], "col code");
    }
    CHECK(sc[5] == 1.0, "zero column scale %g", sc[5]);

    /* per row: equal to the per-tensor quantize of that row */
    CHECK(ko_quantize_rows(w, k, n, qr, sr) == KO_OK, "rc");
    for (int64_t i = 0; i < k; ++i) {
        CHECK(ko_quantize_tensor(w + i * n, n, qc, &s1) == KO_OK, "rc");
        CHECK(sr[i] == s1, "row scale");
        for (int64_t j = 0; j < n; ++j) CHECK(qr[i * n + j] == qc[j], "row code");
    }

    /* per tensor, packed: the per-tensor quantize, transposed */
    CHECK(ko_quantize_tensor_packed(w, k, n, qp, &st) == KO_OK, "rc");
    CHECK(ko_quantize_tensor(w, k * n, qt, &s1) == KO_OK, "rc");
    CHECK(st == s1, "packed scale");
    for (int64_t i = 0; i < k; ++i)
        for (int64_t j = 0; j < n; ++j) CHECK(qp[j * k + i] == qt[i * n + j], "packed code");
    w[3] = -INFINITY;
    CHECK(ko_quantize_tensor_packed(w, k, n, qp, &st) == KO_NONFINITE, "inf accepted");
    CHECK(ko_quantize_cols_packed(w, k, n, qp, sc) == KO_NONFINITE, "inf accepted");
    CHECK(ko_quantize_rows(w, k, n, qr, sr) == KO_NONFINITE, "inf accepted");

    /* dequantize: q * s in binary64, narrowed once */
    float* out = xmalloc(sizeof(float) * k * n);
    for (int64_t i = 0; i < k * n; ++i) qt[i] = code();
    ko_dequantize_tensor(qt, k * n, 0.0123, out);
    for (int64_t i = 0; i < k * n; ++i) CHECK(out[i] == (float)(qt[i] * 0.0123), "dequantize");
    ko_dequantize_rows(qt, k, n, sr, out);
    free(w);
    free(col);
    free(qp);
    free(qr);
    free(qt);
    free(qc);
    free(sc);
    free(sr);
    free(out);
}

static void test_gemm(void) {
    const int64_t M = 33, N = 40, K = 130;
    int8_t* a = xmalloc((size_t)(M * K));
    int8_t* bt = xmalloc((size_t)(N * K));
    int32_t* acc = xmalloc(sizeof(int32_t) * M * N);
    float* out = xmalloc(sizeof(float) * M * N);
    float* bias = xmalloc(sizeof(float) * N);
    double* sa = xmalloc(sizeof(double) * M);
    double* sb = xmalloc(sizeof(double) * N);
    for (int64_t i = 0; i < M * K; ++i) a[i] = code();
    for (int64_t i = 0; i < N * K; ++i) bt[i] = code();
    for (int64_t i = 0; i < M; ++i) sa[i] = uniform(1e-3f, 1e-2f);
    for (int64_t j = 0; j < N; ++j) {
        sb[j] = uniform(1e-3f, 1e-2f);
        bias[j] = uniform(-1.0f, 1.0f);
    }
    a[0] = -127; /* the extreme product */
    bt[0] = -127;
    ko_gemm_i8(a, bt, M, N, K, acc);
    /* k-outer int64 accumulation: a different order, no overflow possible */
    int64_t* ref = calloc((size_t)(M * N), sizeof(int64_t));
    for (int64_t kk = 0; kk < K; ++kk)
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j) ref[i * N + j] += (int64_t)a[i * K + kk] * bt[j * K + kk];
    for (int64_t i = 0; i < M * N; ++i) CHECK(acc[i] == ref[i], "acc %lld", (long long)i);

    ko_epilogue(acc, M, N, sa, M, sb, N, bias, out);
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            const float y = (float)((double)ref[i * N + j] * (sa[i] * sb[j])) + bias[j];
            CHECK(out[i * N + j] == y, "epilogue %lld,%lld", (long long)i, (long long)j);
        }
    ko_epilogue(acc, M, N, sa, 1, sb, 1, NULL, out); /* per-tensor scales, no bias */
    for (int64_t i = 0; i < M * N; ++i) CHECK(out[i] == (float)((double)ref[i] * (sa[0] * sb[0])), "epilogue pt");
    free(ref);
    free(a);
    free(bt);
    free(acc);
    free(out);
    free(bias);
    free(sa);
    free(sb);
}

static void test_matmul(void) {
    const int64_t M = 19, K = 67, N = 23;
    float* a = xmalloc(sizeof(float) * M * K);
    float* b = xmalloc(sizeof(float) * K * N);
    float* out = xmalloc(sizeof(float) * M * N);
    float* bias = xmalloc(sizeof(float) * N);
    float* ob = xmalloc(sizeof(float) * M * N);
    for (int64_t i = 0; i < M * K; ++i) a[i] = uniform(-2.0f, 2.0f);
    for (int64_t i = 0; i < K * N; ++i) b[i] = uniform(-2.0f, 2.0f);
    for (int64_t j = 0; j < N; ++j) bias[j] = uniform(-1.0f, 1.0f);
    ko_matmul_f32(a, b, out, M, K, N);
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double e = 0, mag = 0;
            for (int64_t kk = 0; kk < K; ++kk) {
                e += (double)a[i * K + kk] * b[kk * N + j];
                mag += fabs((double)a[i * K + kk] * b[kk * N + j]);
            }
            CHECK(fabs(out[i * N + j] - e) <= K * 1.2e-7 * mag, "matmul %lld,%lld", (long long)i, (long long)j);
        }
    ko_add_bias(out, bias, ob, M, N);
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) CHECK(ob[i * N + j] == out[i * N + j] + bias[j], "bias");
    free(a);
    free(b);
    free(out);
    free(bias);
    free(ob);
}

int main(void) {
    test_quantize_tensor();
    test_slices();
    test_gemm();
    test_matmul();
    if (failures) {
        fprintf(stderr, "oracle selftest: %d failures\n", failures);
        return 1;
    }
    printf("oracle selftest: ok\n");
    return 0;
}
