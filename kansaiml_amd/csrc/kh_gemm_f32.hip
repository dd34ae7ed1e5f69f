// kh_gemm_f32.hip -- fp32 matmul (+ fused bias) on gfx950 fp32 MFMA.
//
// out (M, N) = a (M, K) @ b (K, N) [+ bias (N)], row-major fp32: the op
// kan::cpu::matmul computes (backend/cpu/src/Ops.cpp:322-339) and the
// reference's Metal backend dispatches to MPS (MetalOps.mm:427-472), with the
// bias add of Ops.cpp:34-38 folded into the store.  Accumulation is fp32 in a
// different order than the reference's i-k-j loop, so results agree to a
// K-scaled rounding bound, not bit for bit.
//
// Structure: a workgroup owns a BM x BN tile (256x256 for large shapes,
// 128x128 otherwise), walks K in BK steps through
// double-buffered LDS.  A is stored transposed in LDS (k-major) so the MFMA
// operand read -- lane l takes A[row l%32][k l/32] -- is a contiguous
// 32-float read; B keeps its natural k-major layout for the same reason.
// Each wave owns (BM/WM) x (BN/WN) outputs as 32x32 blocks of
// v_mfma_f32_32x32x2_f32 (2 k per instruction).
#include <hip/hip_runtime.h>

#include "kh_common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int BM, int BN, int BK, int WM, int WN, bool VEC>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f32_kernel(const float* __restrict__ A,
                                                                const float* __restrict__ B, float* __restrict__ C,
                                                                const float* __restrict__ bias, int64_t M, int64_t N,
                                                                int64_t K) {
    constexpr int kThreads = WM * WN * 64;
    constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    constexpr int kTM = kWaveM / 32, kTN = kWaveN / 32;
    constexpr int kApad = BM + 4;  // floats per LDS row of A^T
    constexpr int kBpad = BN + 4;
    constexpr int kAVec = BM * BK / 4 / kThreads;  // float4 per thread
    constexpr int kBVec = BK * BN / 4 / kThreads;
    static_assert(kAVec >= 1 && kBVec >= 1, "tile too small for the block");
    __shared__ __attribute__((aligned(16))) float As[2][BK][kApad];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][kBpad];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;

    f32x16 acc[kTM][kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) acc[a][b] = f32x16{0};

    f32x4 ra[kAVec], rb[kBVec];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int c = 0; c < kAVec; ++c) {
            const int idx = tid + c * kThreads;
            const int r = idx / (BK / 4), kc = (idx % (BK / 4)) * 4;
            const int64_t gi = m0 + r, gk = k0 + kc;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                if (gi < M && gk < K) v = *reinterpret_cast<const f32x4*>(A + gi * K + gk);
            } else if (gi < M) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gk + e < K) v[e] = A[gi * K + gk + e];
            }
            ra[c] = v;
        }
#pragma unroll
        for (int c = 0; c < kBVec; ++c) {
            const int idx = tid + c * kThreads;
            const int r = idx / (BN / 4), nc = (idx % (BN / 4)) * 4;
            const int64_t gk = k0 + r, gj = n0 + nc;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                if (gk < K && gj < N) v = *reinterpret_cast<const f32x4*>(B + gk * N + gj);
            } else if (gk < K) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gj + e < N) v[e] = B[gk * N + gj + e];
            }
            rb[c] = v;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int c = 0; c < kAVec; ++c) {
            const int idx = tid + c * kThreads;
            const int r = idx / (BK / 4), kc = (idx % (BK / 4)) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) As[buf][kc + e][r] = ra[c][e];
        }
#pragma unroll
        for (int c = 0; c < kBVec; ++c) {
            const int idx = tid + c * kThreads;
            const int r = idx / (BN / 4), nc = (idx % (BN / 4)) * 4;
            *reinterpret_cast<f32x4*>(&Bs[buf][r][nc]) = rb[c];
        }
    };

    const int64_t nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    const int fr = lane & 31;
    const int fk = lane >> 5;
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int buf = (int)(kt & 1);
        if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float fa[kTM], fb[kTN];
#pragma unroll
            for (int a = 0; a < kTM; ++a) fa[a] = As[buf][kk + fk][wm * kWaveM + a * 32 + fr];
#pragma unroll
            for (int b = 0; b < kTN; ++b) fb[b] = Bs[buf][kk + fk][wn * kWaveN + b * 32 + fr];
#pragma unroll
            for (int a = 0; a < kTM; ++a)
#pragma unroll
                for (int b = 0; b < kTN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    const int64_t row_base = m0 + wm * kWaveM + 4 * (lane >> 5);
    const int64_t col_base = n0 + wn * kWaveN + (lane & 31);
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) {
            const int64_t j = col_base + b * 32;
            if (j >= N) continue;
            const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t i = row_base + a * 32 + 8 * (r >> 2) + (r & 3);
                if (i < M) C[i * N + j] = bias ? acc[a][b][r] + bj : acc[a][b][r];
            }
        }
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_f32(kh::Device* d, const float* A, const float* B, float* C, const float* bias, int64_t M, int64_t N,
               int64_t K, bool vec) {
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    if (vec)
        gemm_f32_kernel<BM, BN, BK, WM, WN, true><<<grid, WM * WN * 64, 0, d->stream>>>(A, B, C, bias, M, N, K);
    else
        gemm_f32_kernel<BM, BN, BK, WM, WN, false><<<grid, WM * WN * 64, 0, d->stream>>>(A, B, C, bias, M, N, K);
    return kh::launch_status("gemm_f32");
}

__global__ void bias_fill_kernel(float* __restrict__ C, const float* __restrict__ bias, int64_t M, int64_t N) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < M * N) C[i] = bias ? bias[i % N] : 0.0f;
}

}  // namespace

extern "C" int kh_matmul_f32(const float* a, const float* b, float* out, int64_t M, int64_t K, int64_t N,
                             const float* bias) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_matmul_f32: negative shape");
    if (M == 0 || N == 0) return KH_OK;
    KH_REQUIRE(out, "kh_matmul_f32: null out");
    KH_REQUIRE(K == 0 || (a && b), "kh_matmul_f32: null operand");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_matmul_f32: shape too large");
    KH_DEVICE_OR_RETURN(d);
    if (K == 0) {
        // Ops.cpp:330: fill 0 (then the bias add).
        bias_fill_kernel<<<(unsigned)((M * N + 255) / 256), 256, 0, d->stream>>>(out, bias, M, N);
        return kh::launch_status("bias_fill");
    }
    const bool vec = (K % 4 == 0) && (N % 4 == 0) && kh::aligned(a, 16) && kh::aligned(b, 16);
    // 256x256 tiles (8 waves of 128x64) where the grid still covers every CU
    // once: C3b's 4096^3 runs at 130.9 TFLOP/s there against 121 with
    // 128x128 (measured; 256x128, 128x256, BK 8 and 32 and 16 waves all
    // within 127-131).  The k order of each output is the same in every
    // tiling, so results do not depend on the choice.
    const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles >= d->cus) return launch_f32<256, 256, 16, 2, 4>(d, a, b, out, bias, M, N, K, vec);
    return launch_f32<128, 128, 16, 2, 2>(d, a, b, out, bias, M, N, K, vec);
}
