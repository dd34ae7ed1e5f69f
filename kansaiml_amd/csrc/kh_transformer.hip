// kh_transformer.hip -- the fp32 pieces of a decoder block around the int8
// Linear layers (config C4): token + position embedding, LayerNorm, exact-erf
// GELU, and causal multi-head attention.
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
//                  its diagonal key.
// All fp32 (float accumulation order differs from the reference's CPU loops,
// so results agree to rounding, not bit for bit).
#include <hip/hip_runtime.h>

#include "kh_common.h"

namespace {

// ---------------------------------------------------------------------------
// Embedding: one thread per output element.
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

// ---------------------------------------------------------------------------
// LayerNorm: one wave per row; the row lives in registers (D <= 64 * 16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

constexpr int kLnMaxPerLane = 16;

__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, int64_t rows, int D,
                                                        const float* __restrict__ w, const float* __restrict__ b,
                                                        float eps, float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + row * D;
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
    const float var = wave_sum(ss) / (float)D;
    const float denom = sqrtf(var + eps);
    float* orow = out + row * D;
#pragma unroll
    for (int i = 0; i < kLnMaxPerLane; ++i) {
        const int c = lane + i * 64;
        if (c < D) orow[c] = v[i] / denom * w[c] + b[c];
    }
}

// ---------------------------------------------------------------------------
// GELU (exact erf).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gelu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const float kInvSqrt2 = 0.70710678118654752440f;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const float xi = x[i];
        const float cdf = 0.5f * (1.0f + erff(xi * kInvSqrt2));
        out[i] = xi * cdf;
    }
}

// ---------------------------------------------------------------------------
// Causal attention, fp32, flash-style (online softmax).
//
// qkv: [B*T, 3*D] row-major, the fused Q|K|V projection output (head h of Q
// at columns h*dk .. h*dk+dk-1, K at D + h*dk, V at 2D + h*dk).  out: [B*T, D],
// head h written to its own columns (heads are merged in place).
// One thread per query: the query row and its output accumulator live in
// registers; K and V rows are staged in LDS 64 keys at a time and every lane
// of a wave reads the same K/V row (an LDS broadcast), so each 16-byte LDS
// read feeds four FMAs per lane.  The softmax is rescaled once per chunk of
// 16 keys.  A workgroup owns kQ queries of one (batch, head).  dk = 64.
// ---------------------------------------------------------------------------
constexpr int kDk = 64;
constexpr int kQ = 128;  // queries (threads) per workgroup
constexpr int kKT = 64;  // keys per LDS tile
constexpr int kChunk = 16;

typedef float f32x4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kQ) void attention_kernel(const float* __restrict__ qkv, int B, int T, int H,
                                                       float scale, float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) float ks[kKT][kDk];
    __shared__ __attribute__((aligned(16))) float vs[kKT][kDk];
    const int D = H * kDk;
    const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int q = qb * kQ + tid;
    const bool qvalid = q < T;
    const int64_t row0 = (int64_t)b * T;

    float qv[kDk], o[kDk];
    {
        const f32x4v* qr = reinterpret_cast<const f32x4v*>(qkv + (row0 + (qvalid ? q : 0)) * 3 * D + h * kDk);
#pragma unroll
        for (int d4 = 0; d4 < kDk / 4; ++d4) {
            const f32x4v v = qr[d4];
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[4 * d4 + e] = qvalid ? v[e] * scale : 0.0f;
        }
    }
#pragma unroll
    for (int d = 0; d < kDk; ++d) o[d] = 0.0f;
    float m = -3.0e38f, l = 0.0f;

    const int q_last = min(T, (qb + 1) * kQ) - 1;
    for (int k0 = 0; k0 <= q_last; k0 += kKT) {
        __syncthreads();
        for (int e = tid; e < kKT * kDk / 4; e += kQ) {
            const int kk = e / (kDk / 4), d4 = e % (kDk / 4);
            const int key = k0 + kk;
            const bool ok = key < T;
            const float* kr = qkv + (row0 + (ok ? key : 0)) * 3 * D;
            const f32x4v zero = {0.f, 0.f, 0.f, 0.f};
            reinterpret_cast<f32x4v*>(ks[kk])[d4] = ok ? reinterpret_cast<const f32x4v*>(kr + D + h * kDk)[d4] : zero;
            reinterpret_cast<f32x4v*>(vs[kk])[d4] = ok ? reinterpret_cast<const f32x4v*>(kr + 2 * D + h * kDk)[d4] : zero;
        }
        __syncthreads();
        if (!qvalid || q < k0) continue;
        const int n_keys = min(kKT, q - k0 + 1);  // keys <= q in this tile
        for (int c0 = 0; c0 < n_keys; c0 += kChunk) {
            float s[kChunk];
            float cmax = -3.0e38f;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                const f32x4v* kr = reinterpret_cast<const f32x4v*>(ks[c0 + j]);
                float acc = 0.0f;
#pragma unroll
                for (int d4 = 0; d4 < kDk / 4; ++d4) {
                    const f32x4v kv = kr[d4];
                    acc += qv[4 * d4] * kv[0];
                    acc += qv[4 * d4 + 1] * kv[1];
                    acc += qv[4 * d4 + 2] * kv[2];
                    acc += qv[4 * d4 + 3] * kv[3];
                }
                s[j] = (c0 + j < n_keys) ? acc : -3.0e38f;
                cmax = fmaxf(cmax, s[j]);
            }
            const float m_new = fmaxf(m, cmax);
            const float corr = __expf(m - m_new);
            l *= corr;
#pragma unroll
            for (int d = 0; d < kDk; ++d) o[d] *= corr;
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                const float p = (c0 + j < n_keys) ? __expf(s[j] - m_new) : 0.0f;
                l += p;
                const f32x4v* vr = reinterpret_cast<const f32x4v*>(vs[c0 + j]);
#pragma unroll
                for (int d4 = 0; d4 < kDk / 4; ++d4) {
                    const f32x4v vv = vr[d4];
                    o[4 * d4] += p * vv[0];
                    o[4 * d4 + 1] += p * vv[1];
                    o[4 * d4 + 2] += p * vv[2];
                    o[4 * d4 + 3] += p * vv[3];
                }
            }
            m = m_new;
        }
    }
    if (!qvalid) return;
    const float inv = 1.0f / l;
    f32x4v* orow = reinterpret_cast<f32x4v*>(out + (row0 + q) * D + h * kDk);
#pragma unroll
    for (int d4 = 0; d4 < kDk / 4; ++d4)
        orow[d4] = f32x4v{o[4 * d4] * inv, o[4 * d4 + 1] * inv, o[4 * d4 + 2] * inv, o[4 * d4 + 3] * inv};
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
    embedding_kernel<<<(unsigned)((n + 255) / 256), 256, 0, d->stream>>>(ids, tok, pos, rows, T, D, V, out, d->fault);
    return kh::launch_status("embedding");
}

int kh_layernorm(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps, float* out) {
    KH_REQUIRE(rows >= 0 && D > 0, "kh_layernorm: bad shape");
    KH_REQUIRE(D <= 64 * kLnMaxPerLane, "kh_layernorm: rows longer than 1024 are not supported");
    if (rows == 0) return KH_OK;
    KH_REQUIRE(x && weight && bias && out, "kh_layernorm: null pointer");
    KH_DEVICE_OR_RETURN(d);
    layernorm_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, d->stream>>>(x, rows, D, weight, bias, eps, out);
    return kh::launch_status("layernorm");
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

int kh_causal_attention(const float* qkv, int B, int T, int H, int dk, float* out) {
    KH_REQUIRE(B > 0 && T > 0 && H > 0, "kh_causal_attention: bad shape");
    KH_REQUIRE(dk == kDk, "kh_causal_attention: only head dimension 64 is supported");
    KH_REQUIRE(B <= 65535 && H <= 65535, "kh_causal_attention: too many batches or heads");
    KH_REQUIRE(qkv && out, "kh_causal_attention: null pointer");
    KH_DEVICE_OR_RETURN(d);
    KH_REQUIRE(kh::aligned(qkv, 16) && kh::aligned(out, 16), "kh_causal_attention: 16-byte aligned buffers required");
    dim3 grid((unsigned)((T + kQ - 1) / kQ), (unsigned)H, (unsigned)B);
    // 1/sqrt(d_k) as the reference forms it: a binary64 Python float narrowed
    // to binary32 by from_flat (nn.py:413).
    const float scale = (float)(1.0 / 8.0);
    attention_kernel<<<grid, kQ, 0, d->stream>>>(qkv, B, T, H, scale, out);
    return kh::launch_status("attention");
}

}  // extern "C"
