// kh_act.h -- fp32 activation arithmetic shared by the stand-alone kernels
// and the fused GEMM epilogues, so a fused and an unfused graph produce the
// same bits.  Internal header.
#pragma once

#include <hip/hip_runtime.h>

namespace kh {

// GELU, x * Phi(x) with Phi the standard normal CDF -- the reference's
// cpu::gelu (backend/cpu/src/Ops.cpp:250-256), x * 0.5 * (1 + erf(x / sqrt(2))),
// evaluated without erf and without branches.  With a = |x| and
// u = Phi(-a) = erfc(a / sqrt(2)) / 2: GELU(x) = x * (1 - u) for x >= 0 and
// x * u for x < 0 (no cancellation in 1 + erf for x < 0).  erfc(z) in the
// form t * exp(-z^2 + P(t)), t = 1 / (1 + z / 2) (Numerical Recipes, 2nd ed.,
// section 6.2), with P fitted by Chebyshev interpolation of degree 8 on
// z in [0, 4.4] (gen_gelu_coeffs.py: relative error of erfc 1.5e-8 there;
// beyond it u < 1e-9), written in h = 1 / (2 + z) about 0.328125 with
// log2(e) folded in:  u = h * 2^(Q(h - 0.328125) - a^2 * log2(e) / 2).
// One reciprocal, one exp2 and 16 other VALU operations, where the library
// erff took two branches of 7 and ~20 (a wave of mixed magnitudes runs both).
// Absolute error against binary64 GELU about 1e-7 * max(1, |x|) (the
// reference's binary32 formula, even with a correctly rounded erf: 1.1e-7).
// +-0, +-inf and NaN as that formula: GELU(-inf) = -inf * 0 = NaN.
// The operations are spelled out (explicit fmaf, contraction off in the
// body), so every translation unit computes the same bits whatever its own
// contraction setting.
__device__ __forceinline__ float gelu(float x) {
#pragma clang fp contract(off)
    const float a = fabsf(x);
    const float h = __builtin_amdgcn_rcpf(fmaf(a, 0.70710678f, 2.0f));  // 1 / (2 + a / sqrt(2))
    const float s = h - 0.328125f;
    float e = 59.52790069580078f;
    e = fmaf(e, s, -24.029563903808594f);
    e = fmaf(e, s, -13.704853057861328f);
    e = fmaf(e, s, 11.420587539672852f);
    e = fmaf(e, s, 1.5131943225860596f);
    e = fmaf(e, s, -4.644575595855713f);
    e = fmaf(e, s, 0.00912492722272873f);
    e = fmaf(e, s, 3.9687139987945557f);
    e = fmaf(e, s, -0.6614291667938232f);
    e = fmaf(-a, a * 0.7213475204444817f, e);  // - a^2 log2(e) / 2
    const float p = __builtin_amdgcn_exp2f(e);
    return x * (x >= 0.0f ? fmaf(-h, p, 1.0f) : h * p);  // x * (1 - u) or x * u, u = h * p
}

// |x| as an unsigned bit pattern: for finite values the unsigned order of
// these bits is the numeric order of |x|; NaN/inf patterns compare above
// every finite magnitude (the absmax partials the per-tensor quantizer reads).
__device__ __forceinline__ unsigned abs_bits32(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

}  // namespace kh
