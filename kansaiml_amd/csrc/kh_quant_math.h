// kh_quant_math.h -- the element arithmetic of symmetric int8 quantization,
// shared by the quantize kernels (kh_quant.hip) and the decode GEMM that
// quantizes its activations in-kernel (kh_gemm_i8.hip).  Internal header.
//
// Semantics are the reference's, bit for bit (python/kansai/quantize.py:66-70):
//   m = max|v|;  s = m / 127.0 in binary64 (1.0 when m == 0);
//   q = clamp(round_half_even(fl64(v / s)), -127, 127).
// The fast path and its exactness argument are described in kh_quant.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "kh_common.h"
#include "kh_lanes.h"

#pragma clang fp contract(off)

namespace kh {
namespace quant {

// Native clang vectors (the nontemporal builtins reject HIP's struct vectors).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr float kTieEps = 1.0f / 32768.0f;
// |v * rf - k| <= kFastHalf  <=>  v * rf is at least kTieEps from a half-integer.
constexpr float kFastHalf = 0.5f - kTieEps;
constexpr unsigned kFastMinBits = 0x1F800000u;  // 2^-64
// 1.5 * 2^23: for |x| < 2^22, fl32(x + kMagic) = kMagic + rint(x) (binary32
// spacing is 1 there; kMagic is even so ties go to the even integer), and the
// low byte of its bit pattern is rint(x) as a two's-complement int8.
constexpr float kMagic = 12582912.0f;

__device__ __forceinline__ unsigned abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// Running absmax over raw bit patterns without masking each value: the
// unsigned max is dominated by negative values (sign bit set) and the signed
// max by positive ones.  Both keep NaN/inf patterns, which compare above
// every finite magnitude.
struct AbsMax {
    unsigned umax = 0;
    int smax = 0;
    __device__ __forceinline__ void add4(f32x4 v) {
        const unsigned b0 = __float_as_uint(v.x), b1 = __float_as_uint(v.y);
        const unsigned b2 = __float_as_uint(v.z), b3 = __float_as_uint(v.w);
        umax = max(umax, max(max(b0, b1), max(b2, b3)));
        smax = max(smax, max(max((int)b0, (int)b1), max((int)b2, (int)b3)));
    }
    __device__ __forceinline__ void add1(float v) {
        const unsigned b = __float_as_uint(v);
        umax = max(umax, b);
        smax = max(smax, (int)b);
    }
    // |max| as bits (>= 0x7F800000 if any value was NaN or inf).
    __device__ __forceinline__ unsigned bits() const { return max(umax & 0x7FFFFFFFu, (unsigned)max(smax, 0)); }
};

// Max over the wave, in every lane (whole wave active).
__device__ __forceinline__ unsigned wave_max(unsigned v) { return kh::lanes::wave_max(v); }

struct Scale {
    double s;    // the reference's binary64 scale
    float rf;    // binary32 reciprocal for the fast path
    bool fast;   // fast path allowed for this slice
    bool bad;    // slice holds NaN or +-inf
};

// quantize.py:67-68 from the absmax bit pattern.
__device__ __forceinline__ Scale make_scale(unsigned mbits) {
    Scale r;
    r.bad = mbits >= KH_NONFINITE_BITS;
    const float m = __uint_as_float(mbits);
    r.s = r.bad ? __longlong_as_double(0x7FF8000000000000LL) : (m > 0.0f ? (double)m / 127.0 : 1.0);
    r.rf = r.bad ? 0.0f : (float)(1.0 / r.s);
    r.fast = !r.bad && mbits >= kFastMinBits;
    return r;
}

__device__ __forceinline__ void flag_nonfinite(unsigned* fault) { atomicOr(fault, kh::kFaultNonFinite); }

// quantize.py:69 exactly: binary64 divide, rint (ties to even), clamp.
__device__ __forceinline__ int quant_exact(float v, double s) {
    const int q = (int)rint((double)v / s);
    return min(127, max(-127, q));
}

// Fast path for one value: a's low byte is the code; `ok` is cleared when
// the exact path is needed.
__device__ __forceinline__ unsigned quant_fast(float v, float rf, bool& ok) {
    const float a = __builtin_fmaf(v, rf, kMagic);
    const float d = __builtin_fmaf(v, rf, -(a - kMagic));
    ok = ok && (fabsf(d) <= kFastHalf);
    return __float_as_uint(a);
}

__device__ __forceinline__ int quant_one(float v, const Scale& sc) {
    if (sc.bad) return 0;
    if (sc.fast) {
        bool ok = true;
        const unsigned a = quant_fast(v, sc.rf, ok);
        if (ok) return (int)(int8_t)(a & 0xFFu);
    }
    return quant_exact(v, sc.s);
}

// Four values -> four packed codes (byte e = code of v[e]) by the fast path.
__device__ __forceinline__ unsigned pack4_fast(f32x4 v, float rf, bool& ok) {
    const unsigned a0 = quant_fast(v.x, rf, ok);
    const unsigned a1 = quant_fast(v.y, rf, ok);
    const unsigned a2 = quant_fast(v.z, rf, ok);
    const unsigned a3 = quant_fast(v.w, rf, ok);
    // v_perm_b32: byte 0 of each source into bytes 0..3.
    return __builtin_amdgcn_perm(a1, a0, 0x0c0c0400u) | __builtin_amdgcn_perm(a3, a2, 0x04000c0cu);
}

// Four values -> four packed codes, each by the fast path where it is
// decisive and by the exact path otherwise.
__device__ __forceinline__ unsigned pack4_checked(f32x4 v, const Scale& sc) {
    if (sc.bad) return 0u;
    const unsigned b0 = (unsigned)(quant_one(v.x, sc) & 0xFF);
    const unsigned b1 = (unsigned)(quant_one(v.y, sc) & 0xFF);
    const unsigned b2 = (unsigned)(quant_one(v.z, sc) & 0xFF);
    const unsigned b3 = (unsigned)(quant_one(v.w, sc) & 0xFF);
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

__device__ __forceinline__ unsigned pack4(f32x4 v, const Scale& sc) {
    if (sc.fast) {
        bool ok = true;
        const unsigned w = pack4_fast(v, sc.rf, ok);
        if (ok) return w;
    }
    return pack4_checked(v, sc);
}

// block_reduce_partials in two halves, so a kernel can issue other loads
// around the partials' and wait for all of them together.  The first issues
// this thread's first eight loads (an index past the end reads the last
// partial again, which leaves the maximum unchanged; count >= 1).
__device__ __forceinline__ void partials_first_loads(const unsigned* __restrict__ partials, int count,
                                                     unsigned (&m8)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) m8[u] = partials[min((int)threadIdx.x + u * (int)blockDim.x, count - 1)];
}

// The second: the rest of the partials, eight loads at a time, then the
// workgroup's maximum (every thread of the workgroup calls it).
__device__ __forceinline__ unsigned partials_finish(const unsigned* __restrict__ partials, int count,
                                                    unsigned (&m8)[8], unsigned* red) {
    const int step = blockDim.x;
    for (int i = threadIdx.x + 8 * step; i < count; i += 8 * step) {
#pragma unroll
        for (int u = 0; u < 8; ++u) m8[u] = max(m8[u], partials[min(i + u * step, count - 1)]);
    }
    unsigned mb = max(max(max(m8[0], m8[1]), max(m8[2], m8[3])), max(max(m8[4], m8[5]), max(m8[6], m8[7])));
    mb = wave_max(mb);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = mb;
    __syncthreads();
    mb = red[0];
    for (int i = 1; i < (int)(blockDim.x / 64); ++i) mb = max(mb, red[i]);
    return mb;
}

// Reduces per-workgroup absmax partials[0..count) across the block (any
// multiple of 64 threads up to 1024; `red` holds blockDim.x / 64 words of
// LDS); every thread gets the max bits.
__device__ __forceinline__ unsigned block_reduce_partials(const unsigned* __restrict__ partials, int count,
                                                          unsigned* red) {
    // Eight loads per thread issued before any is used: the partials are L2
    // resident, and loads that each wait for the one before cost one L2
    // round trip apiece.
    unsigned m8[8];
    partials_first_loads(partials, count, m8);
    return partials_finish(partials, count, m8, red);
}

// What a kernel producing the input of a per-tensor quantize does with each
// value it computes: store it (fp32), only reduce its absmax into the
// workgroup's partial (pass 1 of a fused producer + quantize), or quantize
// it with the scale reduced from those partials and store the int8 code
// (pass 2: the fp32 tensor is never written).
constexpr int kOutStore = 0;
constexpr int kOutMaxOnly = 1;
constexpr int kOutQuant = 2;

}  // namespace quant
}  // namespace kh
