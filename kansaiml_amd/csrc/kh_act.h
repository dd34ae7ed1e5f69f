// kh_act.h -- fp32 activation arithmetic shared by the stand-alone kernels
// and the fused GEMM epilogues, so a fused and an unfused graph produce the
// same bits.  Internal header.
#pragma once

#include <hip/hip_runtime.h>

namespace kh {

// GELU with the exact erf, as the reference's cpu::gelu
// (backend/cpu/src/Ops.cpp:250-256): x * 0.5 * (1 + erf(x / sqrt(2))),
// evaluated in binary32.
__device__ __forceinline__ float gelu_exact(float x) {
    const float kInvSqrt2 = 0.70710678118654752440f;
    const float cdf = 0.5f * (1.0f + erff(x * kInvSqrt2));
    return x * cdf;
}

// |x| as an unsigned bit pattern: for finite values the unsigned order of
// these bits is the numeric order of |x|; NaN/inf patterns compare above
// every finite magnitude (the absmax partials the per-tensor quantizer reads).
__device__ __forceinline__ unsigned abs_bits32(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

}  // namespace kh
