// kh_gemm_i8.hip -- int8 x int8 -> int32 GEMM on gfx950 MFMA with a fused
// dequantize + bias epilogue.
//
// The reference has no int8 GEMM: its qlinear dequantizes the weight and runs
// the fp32 matmul (python/kansai/quantize.py:115-122).  This kernel computes
//   acc[i, j] = sum_k a[i, k] * b[j, k]                       (exact int32)
//   out[i, j] = (float)((double)acc[i, j] * (sa_i * sb_j)) + bias[j]
// i.e. the reference's dequantize (quantize.py:76: binary64 product narrowed
// to binary32) applied to the accumulator with the combined scale, then the
// reference's fp32 bias add (backend/cpu/src/Ops.cpp:34-38).
//
// Layout: a [M, K] row-major (activations, K-contiguous); b [N, K] row-major
// (the packed weight, K-contiguous); out/acc [M, N] row-major.
//
// Structure: a workgroup owns a BM x BN output tile and walks K in BK steps.
// Each step's A and B tiles are staged in LDS (double-buffered; the next
// tile's global loads are in flight while the current one is multiplied).
// Waves are arranged WM x WN; each wave owns (BM/WM) x (BN/WN) outputs as
// 32x32 blocks of v_mfma_i32_32x32x32_i8 (one MFMA consumes 32 k: lane l
// supplies 16 consecutive k of A row l%32 and of B column l%32).  LDS rows
// are padded by 16 bytes so the 16-byte ds_read of 8 consecutive rows hits
// distinct banks.
#include <hip/hip_runtime.h>

#include "kh_common.h"

#pragma clang fp contract(off)

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

struct Epilogue {
    const double* sa;
    const double* sb;
    const float* bias;
    float* out;
    int32_t* acc;
    int sa_per_row;
    int sb_per_col;
};

// One output element of the epilogue (see the file comment).
__device__ __forceinline__ void epilogue_store(const Epilogue& ep, int64_t i, int64_t j, int64_t N, int32_t acc) {
    if (ep.acc) ep.acc[i * N + j] = acc;
    if (ep.out) {
        const double s = ep.sa[ep.sa_per_row ? i : 0] * ep.sb[ep.sb_per_col ? j : 0];
        float y = (float)((double)acc * s);
        if (ep.bias) y = y + ep.bias[j];
        ep.out[i * N + j] = y;
    }
}

template <int BM, int BN, int BK, int WM, int WN>
struct GemmCfg {
    static constexpr int kThreads = WM * WN * 64;
    static constexpr int kPad = 16;
    static constexpr int kLdsRow = BK + kPad;  // bytes per LDS row
    static constexpr int kWaveM = BM / WM;
    static constexpr int kWaveN = BN / WN;
    static constexpr int kTM = kWaveM / 32;
    static constexpr int kTN = kWaveN / 32;
    static constexpr int kChunksPerRow = BK / 16;
    static constexpr int kAChunks = BM * kChunksPerRow / kThreads;  // 16-byte chunks per thread
    static constexpr int kBChunks = BN * kChunksPerRow / kThreads;
    static constexpr int kLdsA = BM * kLdsRow;
    static constexpr int kLdsB = BN * kLdsRow;
    static_assert(BM % (WM * 32) == 0 && BN % (WN * 32) == 0, "wave tile must be a multiple of 32");
    static_assert(BK % 32 == 0, "BK must be a multiple of 32");
    static_assert((BM * kChunksPerRow) % kThreads == 0 && (BN * kChunksPerRow) % kThreads == 0, "chunking");
};

// Loads one 16-byte chunk of a K-contiguous operand (zero outside the matrix).
// VEC16: K % 16 == 0 and the base is 16-byte aligned, so a chunk is either
// fully inside or fully outside; otherwise bytes are gathered one by one.
template <bool VEC16>
__device__ __forceinline__ i32x4 load_chunk(const int8_t* __restrict__ base, int64_t row, int64_t rows, int64_t k,
                                            int64_t K) {
    if (VEC16) {
        if (row < rows && k < K) return *reinterpret_cast<const i32x4*>(base + row * K + k);
        return i32x4{0, 0, 0, 0};
    } else {
        unsigned w[4] = {0, 0, 0, 0};
        if (row < rows) {
            const int8_t* p = base + row * K;
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (k + e < K) w[e >> 2] |= ((unsigned)(uint8_t)p[k + e]) << (8 * (e & 3));
        }
        return i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool VEC16>
__global__ __launch_bounds__(WM * WN * 64) void gemm_i8_kernel(const int8_t* __restrict__ A,
                                                               const int8_t* __restrict__ B, int64_t M, int64_t N,
                                                               int64_t K, Epilogue ep) {
    using C = GemmCfg<BM, BN, BK, WM, WN>;
    __shared__ __attribute__((aligned(16))) int8_t lds[2][C::kLdsA + C::kLdsB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;

    i32x16 acc[C::kTM][C::kTN];
#pragma unroll
    for (int a = 0; a < C::kTM; ++a)
#pragma unroll
        for (int b = 0; b < C::kTN; ++b) acc[a][b] = i32x16{0};

    i32x4 ra[C::kAChunks], rb[C::kBChunks];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int c = 0; c < C::kAChunks; ++c) {
            const int idx = tid + c * C::kThreads;
            const int r = idx / C::kChunksPerRow, kc = idx % C::kChunksPerRow;
            ra[c] = load_chunk<VEC16>(A, m0 + r, M, k0 + kc * 16, K);
        }
#pragma unroll
        for (int c = 0; c < C::kBChunks; ++c) {
            const int idx = tid + c * C::kThreads;
            const int r = idx / C::kChunksPerRow, kc = idx % C::kChunksPerRow;
            rb[c] = load_chunk<VEC16>(B, n0 + r, N, k0 + kc * 16, K);
        }
    };
    auto lstore = [&](int buf) {
        int8_t* la = lds[buf];
        int8_t* lb = lds[buf] + C::kLdsA;
#pragma unroll
        for (int c = 0; c < C::kAChunks; ++c) {
            const int idx = tid + c * C::kThreads;
            const int r = idx / C::kChunksPerRow, kc = idx % C::kChunksPerRow;
            *reinterpret_cast<i32x4*>(la + r * C::kLdsRow + kc * 16) = ra[c];
        }
#pragma unroll
        for (int c = 0; c < C::kBChunks; ++c) {
            const int idx = tid + c * C::kThreads;
            const int r = idx / C::kChunksPerRow, kc = idx % C::kChunksPerRow;
            *reinterpret_cast<i32x4*>(lb + r * C::kLdsRow + kc * 16) = rb[c];
        }
    };

    const int64_t nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 16;
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int buf = (int)(kt & 1);
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const int8_t* la = lds[buf] + (wm * C::kWaveM + frag_row) * C::kLdsRow + frag_k;
        const int8_t* lb = lds[buf] + C::kLdsA + (wn * C::kWaveN + frag_row) * C::kLdsRow + frag_k;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            i32x4 fa[C::kTM], fb[C::kTN];
#pragma unroll
            for (int a = 0; a < C::kTM; ++a) fa[a] = *reinterpret_cast<const i32x4*>(la + a * 32 * C::kLdsRow + kk);
#pragma unroll
            for (int b = 0; b < C::kTN; ++b) fb[b] = *reinterpret_cast<const i32x4*>(lb + b * 32 * C::kLdsRow + kk);
#pragma unroll
            for (int a = 0; a < C::kTM; ++a)
#pragma unroll
                for (int b = 0; b < C::kTN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // 32x32 MFMA result layout: register r of lane l holds row
    // 8*(r/4) + 4*(l/32) + r%4 and column l%32 of the block.
    const int64_t row_base = m0 + wm * C::kWaveM + 4 * (lane >> 5);
    const int64_t col_base = n0 + wn * C::kWaveN + (lane & 31);
#pragma unroll
    for (int a = 0; a < C::kTM; ++a)
#pragma unroll
        for (int b = 0; b < C::kTN; ++b) {
            const int64_t j = col_base + b * 32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t i = row_base + a * 32 + 8 * (r >> 2) + (r & 3);
                if (i < M && j < N) epilogue_store(ep, i, j, N, acc[a][b][r]);
            }
        }
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_gemm(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K, const Epilogue& ep,
                bool vec16) {
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    if (vec16)
        gemm_i8_kernel<BM, BN, BK, WM, WN, true><<<grid, WM * WN * 64, 0, d->stream>>>(A, B, M, N, K, ep);
    else
        gemm_i8_kernel<BM, BN, BK, WM, WN, false><<<grid, WM * WN * 64, 0, d->stream>>>(A, B, M, N, K, ep);
    return kh::launch_status("gemm_i8");
}

}  // namespace

extern "C" {

int kh_gemm_i8(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
               int sa_per_row, const double* sb, int sb_per_col, const float* bias, float* out, int32_t* acc_out) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8: negative shape");
    KH_REQUIRE(out || acc_out, "kh_gemm_i8: neither out nor acc_out given");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8: shape too large");
    if (M == 0 || N == 0) return KH_OK;
    KH_REQUIRE(K == 0 || (a && b_packed), "kh_gemm_i8: null operand");
    KH_REQUIRE(!out || (sa && sb), "kh_gemm_i8: scales required when out is given");
    KH_DEVICE_OR_RETURN(d);
    Epilogue ep{sa, sb, bias, out, acc_out, sa_per_row, sb_per_col};
    const bool vec16 = (K % 16 == 0) && kh::aligned(a, 16) && kh::aligned(b_packed, 16);
    if (M >= 2048 && N >= 2048)
        return launch_gemm<256, 256, 64, 2, 4>(d, a, b_packed, M, N, K, ep, vec16);
    return launch_gemm<128, 128, 64, 2, 2>(d, a, b_packed, M, N, K, ep, vec16);
}

int kh_linear_i8(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N, const double* sb,
                 int sb_per_col, const float* bias, int8_t* q_scratch, double* sx_scratch, float* out) {
    KH_REQUIRE(out, "kh_linear_i8: null out");
    int rc = kh_quantize_rows(x, M, K, q_scratch, sx_scratch);
    if (rc) return rc;
    return kh_gemm_i8(q_scratch, b_packed, M, N, K, sx_scratch, 1, sb, sb_per_col, bias, out, nullptr);
}

}  // extern "C"
