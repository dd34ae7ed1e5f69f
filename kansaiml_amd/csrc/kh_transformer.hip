// kh_transformer.hip -- the fp32 pieces of a decoder block around the int8
// Linear layers (config C4): token + position embedding, LayerNorm, GELU, and
// multi-head attention (causal or unmasked).
//
// Semantics follow the reference's modules (python/kansai/nn.py):
//   Embedding      out[r] = tok[id[r]] + pos[r % T]        (nn.py:624-646, the
//                  sum of train_shakespeare_large.py:72-75)
//   LayerNorm      mean and biased variance over the last axis, eps 1e-5,
//                  (x - mean) / sqrt(var + eps) * w + b     (nn.py:308-331)
//   GELU           x * 0.5 * (1 + erf(x / sqrt(2)))         (Ops.cpp:250-256)
//   attention      softmax(Q K^T / sqrt(d_k) + mask) V per head, mask 0 on and
//                  below the diagonal and -1e9 above (nn.py:381-427;
//                  train_shakespeare_large.py:69-70); the softmax subtracts the
//                  row max (Tensor.cpp:906-913).  exp(-1e9 - max) is exactly 0
//                  in binary32, so masked keys are skipped; every row keeps
//                  its diagonal key.  BigGPT adds the mask only when the
//                  sequence fills its position table (:86); shorter
//                  sequences attend over all T keys (causal = 0).
// All fp32 (float accumulation order differs from the reference's CPU loops,
// and LayerNorm multiplies by 1 / sqrt(var + eps) rather than dividing, so
// results agree to rounding, not bit for bit).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "kh_common.h"
#include "kh_act.h"
#include "kh_pipeline.h"
#include "kh_quant_math.h"
// kh_quant_math.h turns FP contraction off for the exact quantize arithmetic
// it defines; the fp32 kernels of this file keep the compiler's default.
#pragma clang fp contract(fast)

namespace {

// ---------------------------------------------------------------------------
// Embedding: one thread per output element (embedding_kernel), or per four
// (embedding4_kernel: D % 4 == 0, 16-byte aligned tables and output).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embedding_kernel(const int32_t* __restrict__ ids,
                                                        const float* __restrict__ tok, const float* __restrict__ pos,
                                                        int64_t rows, int T, int D, int V, float* __restrict__ out,
                                                        unsigned* __restrict__ fault) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= rows * D) return;
    const int64_t r = e / D;
    const int c = (int)(e % D);
    const int id = ids[r];
    if (id < 0 || id >= V) {
        atomicOr(fault, kh::kFaultBadIndex);
        out[e] = 0.0f;
        return;
    }
    out[e] = tok[(int64_t)id * D + c] + pos[(int64_t)(r % T) * D + c];
}

__global__ __launch_bounds__(256) void embedding4_kernel(const int32_t* __restrict__ ids,
                                                         const float* __restrict__ tok, const float* __restrict__ pos,
                                                         int rows, int T, int D4, int V, float* __restrict__ out,
                                                         unsigned* __restrict__ fault) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)rows * D4) return;
    const int r = (int)(e / D4), c = (int)(e - (int64_t)r * D4);
    const int id = ids[r];
    f4* o = reinterpret_cast<f4*>(out) + e;
    if (id < 0 || id >= V) {
        atomicOr(fault, kh::kFaultBadIndex);
        *o = f4{0.f, 0.f, 0.f, 0.f};
        return;
    }
    *o = reinterpret_cast<const f4*>(tok)[(int64_t)id * D4 + c] + reinterpret_cast<const f4*>(pos)[(int64_t)(r % T) * D4 + c];
}

// Rows of D = 128 * KH floats (D = 128 .. 512, 16-byte aligned tables and
// output): half a wave per row, KH float4 per lane, each wave four rows (two
// pairs) with every id and table load issued before the first store, so a
// launch of rows / 16 workgroups is resident at once and each wave waits
// for two round trips (ids, then tables) instead of the one-float4-per-
// thread kernel's many short-lived waves each waiting for both.
template <int KH>
__global__ __launch_bounds__(256) void embedding_rows_kernel(const int32_t* __restrict__ ids,
                                                             const float* __restrict__ tok,
                                                             const float* __restrict__ pos, int rows, int T, int V,
                                                             float* __restrict__ out, unsigned* __restrict__ fault) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int P = 2, D4 = 32 * KH;
    const int lane = threadIdx.x & 63, half = lane >> 5, hl = lane & 31;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (2 * P);
    int id[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = row0 + 2 * p + half;
        id[p] = r < rows ? ids[r] : 0;
    }
    f4 tv[P][KH], pv[P][KH];
    bool bad[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = row0 + 2 * p + half;
        bad[p] = id[p] < 0 || id[p] >= V;
        const int idc = bad[p] ? 0 : id[p];
#pragma unroll
        for (int i = 0; i < KH; ++i) {
            tv[p][i] = reinterpret_cast<const f4*>(tok)[(int64_t)idc * D4 + hl + 32 * i];
            pv[p][i] = reinterpret_cast<const f4*>(pos)[(int64_t)((r < rows ? r : 0) % T) * D4 + hl + 32 * i];
        }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = row0 + 2 * p + half;
        if (r >= rows) continue;
        if (bad[p] && hl == 0) atomicOr(fault, kh::kFaultBadIndex);
#pragma unroll
        for (int i = 0; i < KH; ++i)
            reinterpret_cast<f4*>(out)[(int64_t)r * D4 + hl + 32 * i] =
                bad[p] ? f4{0.f, 0.f, 0.f, 0.f} : tv[p][i] + pv[p][i];
    }
}

// ---------------------------------------------------------------------------
// LayerNorm: one wave per row; the row lives in registers (D <= 64 * 16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) { return kh::lanes::wave_sum(v); }

constexpr int kLnMaxPerLane = 16;

// Max over a 256-thread workgroup (4 waves); every thread gets the result.
__device__ __forceinline__ unsigned block4_max(unsigned v, unsigned* wmax) {
    v = kh::lanes::wave_max(v);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = v;
    __syncthreads();
    return max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
}

// One row of LayerNorm by one wave (any D <= 1024; the scalar path for rows
// that are not float4-aligned); returns this lane's largest |out| bits.  MODE
// (kh::quant::kOut*): store the fp32 row to `out`, only reduce its absmax, or
// store its int8 codes under scale `sc` to `q`.  The centred values are
// multiplied by the row's 1 / sqrt(var + eps), as in layernorm_rows_vec.
template <int MODE>
__device__ __forceinline__ unsigned layernorm_row(const float* __restrict__ x, int64_t row, int D,
                                                  const float* __restrict__ w, const float* __restrict__ b, float eps,
                                                  float* __restrict__ out, int8_t* __restrict__ q,
                                                  const kh::quant::Scale& sc, int lane) {
    using namespace kh::quant;
    const float* xr = x + row * D;
    float* orow = out + row * D;
    int8_t* qrow = q + row * D;
    unsigned mx = 0;
    float v[kLnMaxPerLane];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kLnMaxPerLane; ++i) {
        const int c = lane + i * 64;
        v[i] = c < D ? xr[c] : 0.0f;
        s += v[i];
    }
    const float mean = wave_sum(s) / (float)D;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kLnMaxPerLane; ++i) {
        const int c = lane + i * 64;
        const float cv = c < D ? v[i] - mean : 0.0f;
        v[i] = cv;
        ss += cv * cv;
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < kLnMaxPerLane; ++i) {
        const int c = lane + i * 64;
        if (c < D) {
            const float y = v[i] * inv * w[c] + b[c];
            if (MODE == kOutStore) orow[c] = y;
            if (MODE == kOutQuant) qrow[c] = (int8_t)quant_one(y, sc);
            mx = max(mx, kh::abs_bits32(y));
        }
    }
    return mx;
}

// The vectorized LayerNorm of kLnRowsPerWave consecutive rows by one wave
// (D % 4 == 0, D <= 256 * KV, 16-byte aligned rows): every row's loads are
// issued before any arithmetic and the weight and bias once, so the wave
// waits one memory round trip for all of its rows.  Mean and variance as in
// layernorm_row; the centred values are multiplied by the row's correctly
// rounded 1 / sqrt(var + eps) instead of divided by sqrt(var + eps) (within
// 1 ulp of the quotient; the division's ~10-instruction sequence per element
// made the kernel compute-bound).  Rows >= `rows` are computed on zeros and
// not stored.
constexpr int kLnRowsPerWave = 4;
// LayerNorm output quantized per row (per token): each row's own absmax,
// binary64 scale (quantize.py:67-69 applied to the row) and codes, in one
// pass -- a wave owns whole rows, so no other workgroup is involved.
constexpr int kLnRowQuant = 3;

template <int KV, int MODE>
__device__ __forceinline__ unsigned layernorm_rows_vec(const float* __restrict__ x, int64_t row0, int64_t rows,
                                                       int D, const float* __restrict__ w,
                                                       const float* __restrict__ b, float eps,
                                                       float* __restrict__ out, int8_t* __restrict__ q,
                                                       const kh::quant::Scale& sc, double* __restrict__ rscales,
                                                       unsigned* __restrict__ fault, int lane) {
    using namespace kh::quant;
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int R = kLnRowsPerWave;
    const int D4 = D / 4;
    f4 v[R][KV];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < KV; ++i) {
            const int c4 = lane + i * 64;
            v[r][i] = (row0 + r < rows && c4 < D4) ? reinterpret_cast<const f4*>(x + (row0 + r) * D)[c4]
                                                   : f4{0.f, 0.f, 0.f, 0.f};
        }
    f4 wv[KV], bv[KV];
#pragma unroll
    for (int i = 0; i < KV; ++i) {
        const int c4 = lane + i * 64;
        wv[i] = c4 < D4 ? reinterpret_cast<const f4*>(w)[c4] : f4{0.f, 0.f, 0.f, 0.f};
        bv[i] = c4 < D4 ? reinterpret_cast<const f4*>(b)[c4] : f4{0.f, 0.f, 0.f, 0.f};
    }
    float mean[R], sumsq[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < KV; ++i) s += (v[r][i].x + v[r][i].y) + (v[r][i].z + v[r][i].w);
        mean[r] = s;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) mean[r] = wave_sum(mean[r]) / (float)D;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < KV; ++i) {
            if (lane + i * 64 < D4) {
                v[r][i] -= mean[r];
                ss += (v[r][i].x * v[r][i].x + v[r][i].y * v[r][i].y) + (v[r][i].z * v[r][i].z + v[r][i].w * v[r][i].w);
            }
        }
        sumsq[r] = ss;
    }
    float inv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) inv[r] = 1.0f / sqrtf(wave_sum(sumsq[r]) / (float)D + eps);
    unsigned mx = 0;
    if constexpr (MODE == kLnRowQuant) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            unsigned rm = 0;
#pragma unroll
            for (int i = 0; i < KV; ++i) {
                if (lane + i * 64 < D4) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[r][i][e] = v[r][i][e] * inv[r] * wv[i][e] + bv[i][e];
                        rm = max(rm, kh::abs_bits32(v[r][i][e]));
                    }
                }
            }
            const Scale rs = make_scale(wave_max(rm));
            if (row0 + r >= rows) continue;
            if (lane == 0) {
                rscales[row0 + r] = rs.s;
                if (rs.bad) flag_nonfinite(fault);
            }
#pragma unroll
            for (int i = 0; i < KV; ++i) {
                const int c4 = lane + i * 64;
                if (c4 < D4) reinterpret_cast<unsigned*>(q + (row0 + r) * D)[c4] = pack4(v[r][i], rs);
            }
        }
        return 0;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (row0 + r >= rows) continue;
#pragma unroll
        for (int i = 0; i < KV; ++i) {
            const int c4 = lane + i * 64;
            if (c4 < D4) {
                f4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = v[r][i][e] * inv[r] * wv[i][e] + bv[i][e];
                    mx = max(mx, kh::abs_bits32(y[e]));
                }
                if (MODE == kOutStore) reinterpret_cast<f4*>(out + (row0 + r) * D)[c4] = y;
                if (MODE == kOutQuant) reinterpret_cast<unsigned*>(q + (row0 + r) * D)[c4] = pack4(y, sc);
            }
        }
    }
    return mx;
}

// The LayerNorm of kLnRowsPerWave consecutive rows by one wave, two rows at a
// time (D == 128 * KH, 16-byte aligned rows): lanes 0-31 hold row 2p and
// lanes 32-63 row 2p + 1 of pair p, KH float4 each, so every lane carries
// data in every instruction and a row's mean, variance and 1 / sqrt(var +
// eps) are computed once per pair; the reductions stay in the VALU
// (kh::lanes::half_sum).  Otherwise as layernorm_rows_vec: all loads before any
// arithmetic, the centred values multiplied by the correctly rounded
// 1 / sqrt(var + eps).  Rows >= `rows` are computed on a copy of the last row
// and their results discarded (each row's sums stay within its half-wave).
// Leaves the normalized values in v and each pair's largest |value| bits in rm.
constexpr int kLnPairs = kLnRowsPerWave / 2;

template <int KH>
__device__ __forceinline__ void layernorm_half_loads(const float* __restrict__ x, int64_t row0, int64_t rows, int D,
                                                     const float* __restrict__ w, const float* __restrict__ b,
                                                     kh::quant::f32x4 (&v)[kLnPairs][KH], kh::quant::f32x4 (&wv)[KH],
                                                     kh::quant::f32x4 (&bv)[KH], int lane) {
    using kh::quant::f32x4;
    constexpr int P = kLnPairs;
    const int half = lane >> 5, hl = lane & 31;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        // A row past the end loads the last row (rows >= 1): every load is
        // unconditional, so no branch splits them and they all go out before
        // the first wait.
        const int64_t row = min(row0 + 2 * p + half, rows - 1);
#pragma unroll
        for (int i = 0; i < KH; ++i) v[p][i] = reinterpret_cast<const f32x4*>(x + row * D)[hl + 32 * i];
    }
#pragma unroll
    for (int i = 0; i < KH; ++i) {
        wv[i] = reinterpret_cast<const f32x4*>(w)[hl + 32 * i];
        bv[i] = reinterpret_cast<const f32x4*>(b)[hl + 32 * i];
    }
}

template <int KH>
__device__ __forceinline__ void layernorm_half_math(int D, float eps, kh::quant::f32x4 (&v)[kLnPairs][KH],
                                                    const kh::quant::f32x4 (&wv)[KH],
                                                    const kh::quant::f32x4 (&bv)[KH], unsigned (&rm)[kLnPairs]) {
    constexpr int P = kLnPairs;
    float mean[P], inv[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < KH; ++i) s += (v[p][i].x + v[p][i].y) + (v[p][i].z + v[p][i].w);
        mean[p] = kh::lanes::half_sum(s) / (float)D;
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < KH; ++i) {
            v[p][i] -= mean[p];
            ss += (v[p][i].x * v[p][i].x + v[p][i].y * v[p][i].y) + (v[p][i].z * v[p][i].z + v[p][i].w * v[p][i].w);
        }
        inv[p] = 1.0f / sqrtf(kh::lanes::half_sum(ss) / (float)D + eps);
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        rm[p] = 0;
#pragma unroll
        for (int i = 0; i < KH; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[p][i][e] = v[p][i][e] * inv[p] * wv[i][e] + bv[i][e];
                rm[p] = max(rm[p], kh::abs_bits32(v[p][i][e]));
            }
    }
}

// layernorm_half_loads and layernorm_half_math, then MODE's output; returns
// this lane's largest |out| bits over its rows < `rows`.  MODE kOutQuant
// reduces the pass-1 partials qparts[0..nqparts) to the tensor's scale here
// (workgroup 0 stores it to *scales; `red`: 4 words of LDS), with their
// loads issued behind the rows': the LayerNorm arithmetic waits only for the
// rows, and one memory round trip covers both.  kLnRowQuant stores each
// row's scale to scales[row].  Every thread of the workgroup calls it.
template <int KH, int MODE>
__device__ __forceinline__ unsigned layernorm_rows_half(const float* __restrict__ x, int64_t row0, int64_t rows,
                                                        int D, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps,
                                                        float* __restrict__ out, int8_t* __restrict__ q,
                                                        const unsigned* __restrict__ qparts, int nqparts,
                                                        unsigned* red, double* __restrict__ scales,
                                                        unsigned* __restrict__ fault, int lane) {
    using namespace kh::quant;
    constexpr int P = kLnPairs;
    const int half = lane >> 5, hl = lane & 31;
    f32x4 v[P][KH], wv[KH], bv[KH];
    unsigned rm[P];
    layernorm_half_loads<KH>(x, row0, rows, D, w, b, v, wv, bv, lane);
    unsigned m8[8];
    if constexpr (MODE == kOutQuant) partials_first_loads(qparts, nqparts, m8);
    layernorm_half_math<KH>(D, eps, v, wv, bv, rm);
    Scale sc{};
    if constexpr (MODE == kOutQuant) {
        sc = make_scale(partials_finish(qparts, nqparts, m8, red));
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *scales = sc.s;
            if (sc.bad) flag_nonfinite(fault);
        }
    }
    unsigned mx = 0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int64_t row = row0 + 2 * p + half;
        if constexpr (MODE == kLnRowQuant) {
            // The row's own scale (quantize.py:67-69 applied to the row).
            const Scale rs = make_scale(kh::lanes::half_max(rm[p]));
            if (row >= rows) continue;
            if (hl == 0) {
                scales[row] = rs.s;
                if (rs.bad) flag_nonfinite(fault);
            }
#pragma unroll
            for (int i = 0; i < KH; ++i) reinterpret_cast<unsigned*>(q + row * D)[hl + 32 * i] = pack4(v[p][i], rs);
        } else {
            if (row >= rows) continue;
            mx = max(mx, rm[p]);
#pragma unroll
            for (int i = 0; i < KH; ++i) {
                if (MODE == kOutStore) reinterpret_cast<f32x4*>(out + row * D)[hl + 32 * i] = v[p][i];
                if (MODE == kOutQuant) reinterpret_cast<unsigned*>(q + row * D)[hl + 32 * i] = pack4(v[p][i], sc);
            }
        }
    }
    return mx;
}

// A 256-thread workgroup normalizes kLnRowsPerBlock rows, each wave one row
// at a time, and (when parts is given) writes the max |out| of its rows.
// MODE kOutQuant reduces the pass-1 partials qparts[0..nqparts) to the
// tensor's scale (workgroup 0 stores it to *qscale): first, or on the
// two-rows-per-wave path once its row loads are issued.
constexpr int kLnRowsPerBlock = 16;

// KV: 0 for the scalar path, else float4 columns per lane of the vectorized
// path (2 for D <= 512, 4 for D <= 1024); HALF: the two-rows-per-wave path
// with KV float4 per lane (D == 128 * KV).
template <int KV, int MODE, bool HALF = false>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, int64_t rows, int D,
                                                        const float* __restrict__ w, const float* __restrict__ b,
                                                        float eps, float* __restrict__ out,
                                                        unsigned* __restrict__ parts, int8_t* __restrict__ q,
                                                        const unsigned* __restrict__ qparts, int nqparts,
                                                        double* __restrict__ qscale, unsigned* __restrict__ fault) {
    using namespace kh::quant;
    __shared__ unsigned wmax[4];
    const int lane = threadIdx.x & 63;
    Scale sc{};
    if (MODE == kOutQuant && !(KV > 0 && HALF)) {
        sc = make_scale(block_reduce_partials(qparts, nqparts, wmax));
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *qscale = sc.s;
            if (sc.bad) flag_nonfinite(fault);
        }
    }
    unsigned mx = 0;
    if constexpr (KV > 0) {
        static_assert(kLnRowsPerBlock == 4 * kLnRowsPerWave, "four waves");
        const int64_t row0 = (int64_t)blockIdx.x * kLnRowsPerBlock + (threadIdx.x >> 6) * kLnRowsPerWave;
        if constexpr (HALF)
            mx = layernorm_rows_half<KV, MODE>(x, row0, rows, D, w, b, eps, out, q, qparts, nqparts, wmax, qscale,
                                               fault, lane);
        else
            mx = layernorm_rows_vec<KV, MODE>(x, row0, rows, D, w, b, eps, out, q, sc, qscale, fault, lane);
    } else {
        static_assert(MODE != kLnRowQuant, "per-row codes: vectorized path only");
#pragma unroll 1
        for (int k = threadIdx.x >> 6; k < kLnRowsPerBlock; k += 4) {
            const int64_t row = (int64_t)blockIdx.x * kLnRowsPerBlock + k;
            if (row < rows) mx = max(mx, layernorm_row<MODE>(x, row, D, w, b, eps, out, q, sc, lane));
        }
    }
    if (MODE != kOutQuant && parts) {
        // Per-workgroup max |out| bits, for a following per-tensor quantize.
        mx = block4_max(mx, wmax);
        if (threadIdx.x == 0) parts[blockIdx.x] = mx;
    }
}

// ---------------------------------------------------------------------------
// GELU (kh::gelu: the erf form of the reference, evaluated through erfc).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gelu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = kh::gelu(x[i]);
}

// ---------------------------------------------------------------------------
// Attention, fp32, flash-style (online softmax) on fp32 MFMA; CAUSAL masks
// keys after the query, otherwise only keys past T are left out.
//
// qkv: [B*T, 3*D] row-major, the fused Q|K|V projection output (head h of Q
// at columns h*dk .. h*dk+dk-1, K at D + h*dk, V at 2D + h*dk).  out: [B*T, D],
// head h written to its own columns (heads are merged in place).  dk = 64.
//
// A workgroup owns 64 queries of one (batch, head); wave w owns queries
// 16w .. 16w+15 of them, lane l query 16w + l % 16.  Keys go through LDS 64
// at a time, K and V each as [key][d]: 256-byte rows whose 16-byte chunk c
// sits at position c ^ att_swz(key % 16), brought in by LDS-DMA from a buffer
// resource spanning the batch's rows (keys past T read as 0).  LDS bank
// conflicts of ds_read_b128 on gfx950, measured with a probe kernel: none when
// each 16-lane group reads one 256-byte row at 16 distinct positions and the
// two groups of a half-wave read rows of different parity, two-way when a
// half-wave's lanes read 16 different rows as the K reads below must (one key
// per lane).  The key order att_key gives the V reads the first form; the K
// reads keep the two-way conflict (about 0.8 M conflict cycles per launch at
// C4's shape, hidden behind the MFMAs: the launch time did not change when
// the V reads' conflicts were removed).  Each has one buffer and its own point in the
// iteration: V of tile i is loaded while S of tile i is computed and
// softmaxed, K of tile i+1 while P V of tile i is computed, so no wave waits
// on HBM once the pipeline runs.  Both products run on
// v_mfma_f32_16x16x4_f32 (D[i][j] += sum over k of A[i][k] B[k][j]; lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16]; result register r of lane
// l is D[4 * (l / 16) + r][l % 16]).  The reduction index of each product is
// order-free, so it is mapped to keep operands in registers:
//   S^T = K Q^T (k = head dim; step s of lane group g = l / 16 takes
//   d = 16g + s; A's row i is key att_key(i) of the subtile): lane l ends up
//   holding, for its own query, the scores of keys 16t + att_key(4g + r)
//   (t, r = 0..3) of the tile;
//   O^T = V^T P^T (k = key; step (t, r) of lane group g takes key
//   16t + att_key(4g + r); product j's row i is d = 4i + j): P^T's operand is exactly
//   the probabilities lane l holds, so P never leaves registers, V^T's
//   operands for the four products are one 16-byte read of V's row, and lane
//   l ends up holding d = 16g .. 16g+15 of its query's output.
// The softmax of a query reduces over its lane's 16 scores and the 4 lanes
// l % 16 + 16g (lane swaps, kh_lanes.h).  Scores are kept in base-2 units:
// Q is scaled by log2(e) / sqrt(dk) = log2(e) / 8 (one rounding), so the
// softmax's exponentials are bare v_exp_f32 (2^x).
//
// Workgroups are ordered so that the query blocks of one (batch, head) run on
// one XCD (its L2 holds their shared K and V; workgroup i runs on XCD i % 8)
// and, within an XCD, the blocks with the most key tiles go first.
// ---------------------------------------------------------------------------
constexpr int kDk = 64;
constexpr int kAttQ = 64;  // queries per workgroup (16 per wave)
constexpr int kAttK = 64;  // keys per LDS tile
constexpr float kLog2eOver8 = 0.18033688011112042f;  // log2(e) / sqrt(64)
constexpr float kLog2e = 1.4426950408889634f;

// A caller's additive mask (nn.py:421-422: scores + mask, broadcast to
// [batch, heads, query, key]): element strides of the batch, head and query
// axes (0 where the axis broadcasts; keys contiguous), read through a buffer
// resource of `bytes` (reads past it, for keys or queries past T, give 0).
struct AttMask {
    const float* m;
    uint32_t bytes;
    int sb, sh, sq;
};

typedef float f32x4v __attribute__((ext_vector_type(4)));

// LDS position of a row's 16-byte chunks: chunk c of key k (k % 16) at
// c ^ att_swz(k), a different permutation of the 16 positions per key.
__device__ __forceinline__ int att_swz(int k) { return (k & 10) | ((k >> 2) & 1); }
// Key of row i of a 16-key subtile in the products: rows 4g + r take key
// 4g + (r ^ (g & 1)), so the two lane groups of a half-wave read V rows of
// different parity (different 256-byte halves of the bank window).
__device__ __forceinline__ int att_key(int i) { return i ^ ((i >> 2) & 1); }

// max / sum over the 4 lanes l % 16 + 16g holding one query's scores (the
// same lane of each 16-lane row: one row swap, one half swap; every one of
// the 4 lanes gets the same bits).
__device__ __forceinline__ float query4_max(float v) {
    return kh::lanes::swap32(kh::lanes::swap16(v, kh::lanes::MaxF{}), kh::lanes::MaxF{});
}
__device__ __forceinline__ float query4_sum(float v) {
    return kh::lanes::swap32(kh::lanes::swap16(v, kh::lanes::AddF{}), kh::lanes::AddF{});
}

// One 64-key tile of K or V (rows of the batch's qkv at byte offset `col`)
// into `tile` by LDS-DMA: wave w's instruction i fills rows 16i + 4w .. +3,
// lane l row 16i + 4w + l / 16 at position l % 16, loading the chunk that
// belongs there.
__device__ __forceinline__ void attention_tile_dma(__amdgpu_buffer_rsrc_t r, float* tile, int k0, int row_bytes,
                                                   int col, int wave, int lane) {
    const int row = 4 * wave + (lane >> 4);  // 16i + row, i = 0..3
    const int voff = (k0 + row) * row_bytes + col + 16 * ((lane & 15) ^ att_swz(row));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        kh::pipe::lds_dma16(r, reinterpret_cast<char*>(tile) + (16 * i + 4 * wave) * kDk * 4,
                            voff + 16 * i * row_bytes, 0);
}

// S^T = K Q^T for key subtiles t < NT of the tile in `ks` (st[t][r] = score of
// key 16t + att_key(4g + r)); subtiles t >= NT are left as they are.
template <int NT>
__device__ __forceinline__ void attention_scores(const float* ks, const float (&qf)[16], int li, int g,
                                                 f32x4v (&st)[4]) {
    const int kr = att_key(li), ksw = att_swz(kr);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        f32x4v kv[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
            kv[t] = *reinterpret_cast<const f32x4v*>(&ks[(16 * t + kr) * kDk + 4 * ((4 * g + c) ^ ksw)]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < NT; ++t)
                st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][e], qf[4 * c + e], st[t], 0, 0, 0);
    }
}

// O^T += V^T P^T over key subtiles t < NT of the tile in `vs`: product j,
// A = V^T (d 4 li + j, key 16t + att_key(4g + r)), B = P^T (in registers).
template <int NT>
__device__ __forceinline__ void attention_pv(const float* vs, const f32x4v (&st)[4], int li, int g, f32x4v (&o)[4]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        f32x4v va[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            va[r] = *reinterpret_cast<const f32x4v*>(
                &vs[(16 * t + att_key(4 * g + r)) * kDk + 4 * (li ^ att_swz(att_key(4 * g + r)))]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[r][j], st[t][r], o[j], 0, 0, 0);
    }
}

template <bool CAUSAL, bool MASK = false>
__global__ __launch_bounds__(256, 3) void attention_mfma_kernel(const float* __restrict__ qkv, int B, int T, int H,
                                                             float* __restrict__ out, unsigned* __restrict__ parts,
                                                             unsigned* __restrict__ rparts, AttMask am) {
    __shared__ __attribute__((aligned(1024))) float ks[kAttK * kDk];
    __shared__ __attribute__((aligned(1024))) float vs[kAttK * kDk];
    using kh::pipe::wait_imm;
    const int D = H * kDk;
    const int nq = (T + kAttQ - 1) / kAttQ, pairs = B * H;
    int qb, pair;
    if (pairs % kh::pipe::kXcds == 0) {
        const int per = pairs / kh::pipe::kXcds, s = blockIdx.x / kh::pipe::kXcds;
        qb = nq - 1 - s / per;
        pair = (blockIdx.x % kh::pipe::kXcds) * per + s % per;
    } else {
        qb = nq - 1 - blockIdx.x / pairs;
        pair = blockIdx.x % pairs;
    }
    const int b = pair / H, h = pair - b * H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, g = lane >> 4;
    const float* bq = qkv + (int64_t)b * T * 3 * D;
    const int q0 = qb * kAttQ + wave * 16;  // this wave's first query
    const int q = q0 + li;                  // this lane's query
    const int row_bytes = 3 * D * 4;
    const __amdgpu_buffer_rsrc_t rsrc = kh::pipe::make_rsrc(bq, (uint32_t)(T * row_bytes));
    const int kcol = (D + h * kDk) * 4, vcol = kcol + D * 4;
    // MASK: this lane's query row of the mask (in elements).
    const __amdgpu_buffer_rsrc_t rmask = kh::pipe::make_rsrc(am.m, am.bytes);
    const int mrow = b * am.sb + h * am.sh + q * am.sq;

    // Q operand: query q, d = 16g .. 16g+15, scaled by log2(e) / 8.
    float qf[16];
    {
        const f32x4v* qr = reinterpret_cast<const f32x4v*>(bq + (int64_t)min(q, T - 1) * 3 * D + h * kDk + 16 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4v v = qr[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[4 * c + e] = q < T ? v[e] * kLog2eOver8 : 0.0f;
        }
    }
    attention_tile_dma(rsrc, ks, 0, row_bytes, kcol, wave, lane);
    f32x4v o[4];  // O^T: register r of o[j] is O[q][16g + 4r + j]
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    float m = -3.0e38f, l = 0.0f;

    // Causal: key tiles through the workgroup's last query; otherwise all of them.
    const int tiles = ((CAUSAL ? min(T, (qb + 1) * kAttQ) : T) - 1) / kAttK + 1;
    // The last key any of this wave's queries attends to.  Key subtiles
    // beyond it (the diagonal tile's upper subtiles, keys past T) hold only
    // masked scores, whose probabilities are exactly 0: their products are
    // skipped (the same results: the mask below still covers their scores).
    const int last_key = __builtin_amdgcn_readfirstlane(CAUSAL ? min(q0 + 15, T - 1) : T - 1);
    for (int it = 0; it < tiles; ++it) {
        const int k0 = it * kAttK;
        // Key subtiles with a key <= last_key: 1..4 (k0 <= last_key for
        // every tile the loop visits).
        const int nt = min(4, (last_key - k0) / 16 + 1);
        // K(it) has landed for every wave, and every wave is done with V(it-1).
        __builtin_amdgcn_s_waitcnt(wait_imm(0, 15));
        __syncthreads();
        attention_tile_dma(rsrc, vs, k0, row_bytes, vcol, wave, lane);

        // S^T = K Q^T, 4 subtiles of 16 keys: st[t][r] = score of key 16t + att_key(4g + r).
        f32x4v st[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) st[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
        if (nt == 4) attention_scores<4>(ks, qf, li, g, st);
        else if (nt == 3) attention_scores<3>(ks, qf, li, g, st);
        else if (nt == 2) attention_scores<2>(ks, qf, li, g, st);
        else attention_scores<1>(ks, qf, li, g, st);
        if constexpr (MASK) {
            // The caller's mask, in the scores' base-2 units: keys
            // 16t + 4g + e of the tile (register e ^ (g & 1), att_key's order).
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float mv = __uint_as_float(
                        __builtin_amdgcn_raw_buffer_load_b32(rmask, (mrow + k0 + 16 * t + 4 * g + e) * 4, 0, 0));
                    st[t][e ^ (g & 1)] += mv * kLog2e;
                }
        }
        // Causal mask (key > query) and keys past T -- only where the tile
        // reaches this wave's diagonal or the sequence end.  Under a caller's
        // mask these scores are -inf: a row whose every visible key the
        // caller masked with -inf then has no real score, m stays at its
        // -3e38 start, and -inf keeps their probabilities 0 (l = 0, a NaN
        // row, as the reference's softmax of an all -inf row gives).
        constexpr float kOff = MASK ? -__builtin_inff() : -3.0e38f;
        if (!((!CAUSAL || k0 + kAttK - 1 <= q0) && k0 + kAttK <= T)) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * t + att_key(4 * g + r);
                    st[t][r] = ((CAUSAL && key > q) || key >= T) ? kOff : st[t][r];
                }
        }
        float mx = -3.0e38f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[t][r]);
        mx = query4_max(mx);
        const float m_new = fmaxf(m, mx);
        const float corr = __builtin_amdgcn_exp2f(m - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // A masked score (-3e38) gives exactly 0: m_new is a real
                // score (the first tile holds key 0, which every query sees),
                // so the exponent is about -3e38 and 2^x underflows to 0.
                const float p = __builtin_amdgcn_exp2f(st[t][r] - m_new);
                st[t][r] = p;
                sum += p;
            }
        l = l * corr + query4_sum(sum);
        m = m_new;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= corr;

        // V(it) has landed for every wave, and every wave is done with K(it).
        __builtin_amdgcn_s_waitcnt(wait_imm(0, 15));
        __syncthreads();
        if (it + 1 < tiles) attention_tile_dma(rsrc, ks, k0 + kAttK, row_bytes, kcol, wave, lane);

        // O^T += V^T P^T.
        if (nt == 4) attention_pv<4>(vs, st, li, g, o);
        else if (nt == 3) attention_pv<3>(vs, st, li, g, o);
        else if (nt == 2) attention_pv<2>(vs, st, li, g, o);
        else attention_pv<1>(vs, st, li, g, o);
    }
    unsigned mxo = 0;
    if (q < T) {
        const float inv = 1.0f / l;
        float* orow = out + ((int64_t)b * T + q) * D + h * kDk + 16 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f32x4v y = f32x4v{o[0][r], o[1][r], o[2][r], o[3][r]} * inv;
            *reinterpret_cast<f32x4v*>(orow + 4 * r) = y;
#pragma unroll
            for (int e = 0; e < 4; ++e) mxo = max(mxo, kh::abs_bits32(y[e]));
        }
    }
    if (rparts) {
        // Per-(row, head) max |out| bits, for a following per-row quantize:
        // the lanes li, li + 16, li + 32, li + 48 hold query q's 64 outputs.
        unsigned mr = mxo;
        mr = max(mr, (unsigned)__shfl_xor((int)mr, 16));
        mr = max(mr, (unsigned)__shfl_xor((int)mr, 32));
        if (g == 0 && q < T) rparts[((int64_t)b * T + q) * H + h] = mr;
    }
    if (parts) {
        // Per-workgroup max |out| bits, for a following per-tensor quantize.
        __shared__ unsigned wmax[4];
        mxo = block4_max(mxo, wmax);
        if (tid == 0) parts[blockIdx.x] = mxo;
    }
}

// Launches the LayerNorm kernel in the layout the row length takes: two rows
// per wave for D = 128, 256, 384 or 512 (16-byte aligned), one row per wave
// otherwise (float4 columns where aligned, scalar for the rest).  Every mode
// of one D takes the same layout, so a fused pass computes exactly the values
// the plain LayerNorm stores.
template <int MODE>
void launch_layernorm(kh::Device* d, bool vec, int64_t blocks, const float* x, int64_t rows, int D, const float* w,
                      const float* b, float eps, float* out, unsigned* parts, int8_t* q, const unsigned* qparts,
                      int nqparts, double* qscale) {
    auto go = [&](auto kv, auto half) {
        layernorm_kernel<decltype(kv)::value, MODE, decltype(half)::value><<<(unsigned)blocks, 256, 0, d->stream>>>(
            x, rows, D, w, b, eps, out, parts, q, qparts, nqparts, qscale, d->fault);
    };
    using yes = std::true_type;
    using no = std::false_type;
    if (vec && D % 128 == 0 && D <= 512) {
        if (D == 128) go(std::integral_constant<int, 1>{}, yes{});
        else if (D == 256) go(std::integral_constant<int, 2>{}, yes{});
        else if (D == 384) go(std::integral_constant<int, 3>{}, yes{});
        else go(std::integral_constant<int, 4>{}, yes{});
    } else if (vec && D <= 512) {
        go(std::integral_constant<int, 2>{}, no{});
    } else if (vec) {
        go(std::integral_constant<int, 4>{}, no{});
    } else if constexpr (MODE != kLnRowQuant) {
        go(std::integral_constant<int, 0>{}, no{});
    }
}

}  // namespace

extern "C" {

int kh_embedding(const int32_t* ids, int64_t rows, int T, const float* tok, int V, const float* pos, int D,
                 float* out) {
    KH_REQUIRE(rows >= 0 && T > 0 && V > 0 && D > 0, "kh_embedding: bad shape");
    if (rows == 0) return KH_OK;
    KH_REQUIRE(ids && tok && pos && out, "kh_embedding: null pointer");
    KH_DEVICE_OR_RETURN(d);
    const int64_t n = rows * D;
    const bool vec = D % 4 == 0 && rows <= 0x7FFFFFFF && kh::aligned(tok, 16) && kh::aligned(pos, 16) &&
                     kh::aligned(out, 16);
    if (vec && D % 128 == 0 && D <= 512 && rows <= 0x7FFFFFFF - 16) {
        const unsigned blocks = (unsigned)((rows + 15) / 16);
        auto go = [&](auto kh_) {
            embedding_rows_kernel<decltype(kh_)::value><<<blocks, 256, 0, d->stream>>>(ids, tok, pos, (int)rows, T, V,
                                                                                     out, d->fault);
        };
        if (D == 128) go(std::integral_constant<int, 1>{});
        else if (D == 256) go(std::integral_constant<int, 2>{});
        else if (D == 384) go(std::integral_constant<int, 3>{});
        else go(std::integral_constant<int, 4>{});
        return kh::launch_status("embedding");
    }
    if (vec && n / 4 <= 0xFFFFFFFFLL * 256) {
        embedding4_kernel<<<(unsigned)((n / 4 + 255) / 256), 256, 0, d->stream>>>(ids, tok, pos, (int)rows, T, D / 4,
                                                                                  V, out, d->fault);
        return kh::launch_status("embedding");
    }
    embedding_kernel<<<(unsigned)((n + 255) / 256), 256, 0, d->stream>>>(ids, tok, pos, rows, T, D, V, out, d->fault);
    return kh::launch_status("embedding");
}

int kh_layernorm_ex(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps, float* out,
                    unsigned* absmax_parts, int max_parts, int* nparts) {
    KH_REQUIRE(rows >= 0 && D > 0, "kh_layernorm: bad shape");
    KH_REQUIRE(D <= 64 * kLnMaxPerLane, "kh_layernorm: rows longer than 1024 are not supported");
    KH_REQUIRE(!absmax_parts || (max_parts > 0 && nparts), "kh_layernorm_ex: partials need max_parts and nparts");
    if (nparts) *nparts = 0;
    if (rows == 0) return KH_OK;
    KH_REQUIRE(x && weight && bias && out, "kh_layernorm: null pointer");
    KH_DEVICE_OR_RETURN(d);
    const int64_t blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    KH_REQUIRE(blocks <= 0x7FFFFFFFLL, "kh_layernorm: too many rows");
    const bool fused = absmax_parts && blocks <= max_parts;
    const bool vec = D % 4 == 0 && kh::aligned(x, 16) && kh::aligned(out, 16) && kh::aligned(weight, 16) &&
                     kh::aligned(bias, 16);
    using kh::quant::kOutStore;
    unsigned* parts = fused ? absmax_parts : nullptr;
    launch_layernorm<kOutStore>(d, vec, blocks, x, rows, D, weight, bias, eps, out, parts, nullptr, nullptr, 0,
                                nullptr);
    int rc = kh::launch_status("layernorm");
    if (rc || !absmax_parts) return rc;
    if (fused) {
        *nparts = (int)blocks;
        return KH_OK;
    }
    return kh_absmax_parts(out, rows * D, absmax_parts, max_parts, nparts);
}

int kh_layernorm(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps, float* out) {
    return kh_layernorm_ex(x, rows, D, weight, bias, eps, out, nullptr, 0, nullptr);
}

int kh_layernorm_quant(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps,
                       int8_t* q, double* scale) {
    KH_REQUIRE(rows >= 0 && D > 0, "kh_layernorm_quant: bad shape");
    KH_REQUIRE(D <= 64 * kLnMaxPerLane, "kh_layernorm_quant: rows longer than 1024 are not supported");
    KH_REQUIRE(scale, "kh_layernorm_quant: null scale");
    KH_DEVICE_OR_RETURN(d);
    if (rows == 0) {
        // The reference's quantize of an empty tensor: max 0, scale 1.0.
        const double one = 1.0;
        return kh_memcpy_h2d(scale, &one, sizeof(one));
    }
    KH_REQUIRE(x && weight && bias && q, "kh_layernorm_quant: null pointer");
    const int64_t blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    KH_REQUIRE(blocks <= 0x7FFFFFFFLL, "kh_layernorm_quant: too many rows");
    auto* parts = static_cast<unsigned*>(kh::scratch_area(d, (size_t)blocks * sizeof(unsigned)));
    if (!parts) return KH_ERR_OOM;
    const bool vec = D % 4 == 0 && kh::aligned(x, 16) && kh::aligned(q, 4) && kh::aligned(weight, 16) &&
                     kh::aligned(bias, 16);
    using kh::quant::kOutMaxOnly;
    using kh::quant::kOutQuant;
    // Pass 1 reduces the normalized values' absmax into one partial per
    // workgroup without storing them; pass 2 recomputes them (the same
    // arithmetic, so the same values) and stores their codes.
    launch_layernorm<kOutMaxOnly>(d, vec, blocks, x, rows, D, weight, bias, eps, nullptr, parts, nullptr, nullptr, 0,
                                  nullptr);
    launch_layernorm<kOutQuant>(d, vec, blocks, x, rows, D, weight, bias, eps, nullptr, nullptr, q, parts,
                                (int)blocks, scale);
    return kh::launch_status("layernorm_quant");
}

int kh_layernorm_quant_rows(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps,
                            int8_t* q, double* scales) {
    KH_REQUIRE(rows >= 0 && D > 0, "kh_layernorm_quant_rows: bad shape");
    KH_REQUIRE(D <= 64 * kLnMaxPerLane, "kh_layernorm_quant_rows: rows longer than 1024 are not supported");
    if (rows == 0) return KH_OK;
    KH_REQUIRE(x && weight && bias && q && scales, "kh_layernorm_quant_rows: null pointer");
    KH_DEVICE_OR_RETURN(d);
    const int64_t blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    KH_REQUIRE(blocks <= 0x7FFFFFFFLL, "kh_layernorm_quant_rows: too many rows");
    const bool vec = D % 4 == 0 && kh::aligned(x, 16) && kh::aligned(q, 4) && kh::aligned(weight, 16) &&
                     kh::aligned(bias, 16);
    if (!vec) {
        // Other shapes: the fp32 LayerNorm into a pool buffer, then the
        // per-row quantize of it (the same values, so the same codes).
        void* tmp = nullptr;
        int rc = kh_alloc((size_t)rows * D * sizeof(float), &tmp);
        if (rc) return rc;
        rc = kh_layernorm(x, rows, D, weight, bias, eps, static_cast<float*>(tmp));
        if (!rc) rc = kh_quantize_rows(static_cast<float*>(tmp), rows, D, q, scales);
        const int frc = kh_free(tmp);
        return rc ? rc : frc;
    }
    launch_layernorm<kLnRowQuant>(d, vec, blocks, x, rows, D, weight, bias, eps, nullptr, nullptr, q, nullptr, 0,
                                  scales);
    return kh::launch_status("layernorm_quant_rows");
}

int kh_gelu(const float* x, float* out, int64_t n) {
    KH_REQUIRE(n >= 0, "kh_gelu: negative size");
    if (n == 0) return KH_OK;
    KH_REQUIRE(x && out, "kh_gelu: null pointer");
    KH_DEVICE_OR_RETURN(d);
    int64_t g = (n + 1023) / 1024;
    if (g > 65536) g = 65536;
    gelu_kernel<<<(unsigned)g, 256, 0, d->stream>>>(x, out, n);
    return kh::launch_status("gelu");
}

static int attention_impl(const float* qkv, int B, int T, int H, int dk, int causal, float* out,
                          unsigned* absmax_parts, int max_parts, int* nparts, unsigned* row_parts,
                          const AttMask* mask = nullptr) {
    KH_REQUIRE(B > 0 && T > 0 && H > 0, "kh_attention: bad shape");
    KH_REQUIRE(dk == kDk, "kh_attention: only head dimension 64 is supported");
    KH_REQUIRE(causal == 0 || causal == 1, "kh_attention: causal must be 0 or 1");
    KH_REQUIRE(qkv && out, "kh_attention: null pointer");
    KH_REQUIRE(!absmax_parts || (max_parts > 0 && nparts), "kh_attention_ex: partials need max_parts and nparts");
    if (nparts) *nparts = 0;
    KH_DEVICE_OR_RETURN(d);
    KH_REQUIRE(kh::aligned(qkv, 16) && kh::aligned(out, 16), "kh_attention: 16-byte aligned buffers required");
    // Key offsets within a batch's rows, up to the last tile's padding, are
    // 32-bit buffer offsets.
    const int64_t nq = (T + kAttQ - 1) / kAttQ;
    KH_REQUIRE((nq * kAttQ) * 3 * (int64_t)H * kDk * 4 <= 0x7FFFFFFFLL,
               "kh_attention: one batch's qkv rows must stay under 2 GiB");
    const int64_t blocks = nq * H * B;
    KH_REQUIRE(blocks <= 0x7FFFFFFFLL, "kh_attention: too many query blocks");
    const bool fused = absmax_parts && blocks <= max_parts;
    // 1/sqrt(d_k) = 1/8 for dk = 64 (the reference's binary64 Python float,
    // nn.py:413, is exactly representable in binary32); the kernel applies it
    // to Q together with log2(e), keeping the scores in base-2 units.
    unsigned* pp = fused ? absmax_parts : nullptr;
    const AttMask am = mask ? *mask : AttMask{nullptr, 0, 0, 0, 0};
    if (mask && causal)
        attention_mfma_kernel<true, true><<<(unsigned)blocks, 256, 0, d->stream>>>(qkv, B, T, H, out, pp, row_parts, am);
    else if (mask)
        attention_mfma_kernel<false, true><<<(unsigned)blocks, 256, 0, d->stream>>>(qkv, B, T, H, out, pp, row_parts, am);
    else if (causal)
        attention_mfma_kernel<true><<<(unsigned)blocks, 256, 0, d->stream>>>(qkv, B, T, H, out, pp, row_parts, am);
    else
        attention_mfma_kernel<false><<<(unsigned)blocks, 256, 0, d->stream>>>(qkv, B, T, H, out, pp, row_parts, am);
    int rc = kh::launch_status("attention");
    if (rc || !absmax_parts) return rc;
    if (fused) {
        *nparts = (int)blocks;
        return KH_OK;
    }
    return kh_absmax_parts(out, (int64_t)B * T * H * kDk, absmax_parts, max_parts, nparts);
}

int kh_attention_ex(const float* qkv, int B, int T, int H, int dk, int causal, float* out, unsigned* absmax_parts,
                    int max_parts, int* nparts) {
    return attention_impl(qkv, B, T, H, dk, causal, out, absmax_parts, max_parts, nparts, nullptr);
}

int kh_attention_rows(const float* qkv, int B, int T, int H, int dk, int causal, float* out, unsigned* row_parts) {
    KH_REQUIRE(row_parts, "kh_attention_rows: null row_parts");
    return attention_impl(qkv, B, T, H, dk, causal, out, nullptr, 0, nullptr, row_parts);
}

int kh_attention_masked(const float* qkv, int B, int T, int H, int dk, int causal, const float* mask,
                        int64_t mask_elems, int64_t stride_b, int64_t stride_h, int64_t stride_q, float* out,
                        unsigned* row_parts) {
    KH_REQUIRE(mask && mask_elems > 0, "kh_attention_masked: null or empty mask");
    KH_REQUIRE(kh::aligned(mask, 4), "kh_attention_masked: the mask must be 4-byte aligned");
    KH_REQUIRE(stride_b >= 0 && stride_h >= 0 && stride_q >= 0, "kh_attention_masked: negative stride");
    KH_REQUIRE(mask_elems <= 0x7FFFFFFFLL / 4 && stride_b <= 0x7FFFFFFFLL && stride_h <= 0x7FFFFFFFLL &&
                   stride_q <= 0x7FFFFFFFLL,
               "kh_attention_masked: the mask must stay under 2 GiB of offsets");
    KH_REQUIRE(B > 0 && T > 0 && H > 0, "kh_attention: bad shape");
    // The last element any (batch, head, query, key) reads must be inside
    // the mask; every offset (up to a padded query's last key) a 32-bit
    // byte offset.
    // (Bounded in binary64 first: the int64 sums below cannot overflow once
    // it is under the mask's size.)
    const int64_t nq = (T + kAttQ - 1) / kAttQ;
    KH_REQUIRE((double)(B - 1) * stride_b + (double)(H - 1) * stride_h + (double)(nq * kAttQ) * stride_q +
                       (double)(nq * kAttQ + kAttK) <= (double)(0x7FFFFFFFLL / 4),
               "kh_attention_masked: the mask must stay under 2 GiB of offsets");
    const int64_t last = (B - 1) * stride_b + (H - 1) * stride_h + (T - 1) * stride_q + (T - 1);
    KH_REQUIRE(last < mask_elems, "kh_attention_masked: the mask's strides reach past its elements");
    const int64_t reach = (B - 1) * stride_b + (H - 1) * stride_h + (nq * kAttQ) * stride_q + nq * kAttQ + kAttK;
    KH_REQUIRE(mask_elems * 4 <= 0x7FFFFFFFLL && reach * 4 <= 0x7FFFFFFFLL,
               "kh_attention_masked: the mask must stay under 2 GiB of offsets");
    const AttMask am{mask, (uint32_t)(mask_elems * 4), (int)stride_b, (int)stride_h, (int)stride_q};
    return attention_impl(qkv, B, T, H, dk, causal, out, nullptr, 0, nullptr, row_parts, &am);
}

int kh_causal_attention_ex(const float* qkv, int B, int T, int H, int dk, float* out, unsigned* absmax_parts,
                           int max_parts, int* nparts) {
    return kh_attention_ex(qkv, B, T, H, dk, 1, out, absmax_parts, max_parts, nparts);
}

int kh_causal_attention(const float* qkv, int B, int T, int H, int dk, float* out) {
    return kh_attention_ex(qkv, B, T, H, dk, 1, out, nullptr, 0, nullptr);
}

}  // extern "C"
