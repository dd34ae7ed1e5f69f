// kh_gemm_f32.hip -- fp32 matmul (+ fused bias) on gfx950 fp32 MFMA.
//
// out (M, N) = a (M, K) @ b (K, N) [+ bias (N)], row-major fp32: the op
// kan::cpu::matmul computes (backend/cpu/src/Ops.cpp:322-339) and the
// reference's Metal backend dispatches to MPS (MetalOps.mm:427-472), with the
// bias add of Ops.cpp:34-38 folded into the store.  Accumulation is fp32 in a
// different order than the reference's i-k-j loop, so results agree to a
// K-scaled rounding bound, not bit for bit.
//
// Structure (gemm_f32_kernel; large shapes with K % 16 == 0 take the
// ping-pong kernel below): a workgroup owns a BM x BN tile (256x256 for large
// shapes, 128x128 otherwise), walks K in BK steps through
// double-buffered LDS.  A is stored transposed in LDS (k-major) so the MFMA
// operand read -- lane l takes A[row l%32][k l/32] -- is a contiguous
// 32-float read; B keeps its natural k-major layout for the same reason.
// Each wave owns (BM/WM) x (BN/WN) outputs as 32x32 blocks of
// v_mfma_f32_32x32x2_f32 (2 k per instruction).
#include <hip/hip_runtime.h>

#include "kh_common.h"
#include "kh_pipeline.h"

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

// ---------------------------------------------------------------------------
// Ping-pong fp32 GEMM for large shapes (K % 16 == 0, N % 4 == 0): the int8
// kernel's pipeline (kh_gemm_i8.hip) with fp32 operands.
//
// * 256x256 workgroup tile, 8 waves as 2 (M) x 4 (N), each 128x64 outputs as
//   4x2 blocks of v_mfma_f32_32x32x2_f32; K staged 16 floats (64 bytes of
//   each A row, 16 B rows) at a time in a ring of NS LDS stages of 32 KB,
//   filled by LDS-DMA with no VGPR staging.
// * Operands stay in their natural layouts.  The MFMA takes A[i][k] from
//   lane i % 32 + 32 g and B[k][j] from lane j % 32 + 32 g for its two k
//   (g = 0, 1).  Lane group g reads 8 consecutive floats of its A row (two
//   16-byte reads, k = 8g .. 8g + 7), and MFMA s (0..7) of a stage uses
//   element s: k = 8g + s, with B[8g + s][j] read as one dword.  The sum over
//   k is the same, in a different order (fp32: within the rounding bound).
// * A rows: 16-byte chunks XOR-swizzled by (row >> 2) & 3 on the global side
//   (LDS-DMA lane l lands at M0 + 16 l), as in the int8 kernel.  B rows are
//   1 KB (256 floats); rows 8..15 are rotated by 8 chunks so the two lane
//   groups of a dword read (rows s and 8 + s) fall in different banks.
// * Two wave groups (waves 0-3 and 4-7, one of each per SIMD) alternate
//   memory phase (fragment reads for stage k, LDS-DMA for stage k + NS - 1)
//   and compute phase (64 MFMAs), one barrier apart.
// * Rows past M read zeros (buffer resource bound); columns past N get an
//   offset past the resource and read zeros too.
// ---------------------------------------------------------------------------
template <int NS>
__global__ __launch_bounds__(512, 2) void gemm_f32_pingpong_kernel(const float* __restrict__ A,
                                                                   const float* __restrict__ B,
                                                                   float* __restrict__ C,
                                                                   const float* __restrict__ bias, int M, int N,
                                                                   int K) {
    using namespace kh::pipe;
    constexpr int BM = 256, BN = 256, BK = 16, WM = 2, WN = 4, kWaves = WM * WN;
    constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    constexpr int kTM = kWaveM / 32, kTN = kWaveN / 32;
    constexpr int kLdsA = BM * BK * 4;            // bytes: 256 rows x 64 B
    constexpr int kStage = kLdsA + BK * BN * 4;   // + 16 rows x 1 KB
    constexpr int kAInst = BM / 16 / kWaves;      // 16 A rows per DMA instruction
    constexpr int kBInst = BK / kWaves;           // one B row per DMA instruction
    constexpr int kLoads = kAInst + kBInst;
    constexpr int D = NS - 1;
    static_assert(NS >= 3 && NS <= 4, "wait_loads_beyond covers up to 3 stages ahead");
    __shared__ __attribute__((aligned(1024))) char lds[NS * kStage];

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int group = wm;

    const int rows_a = min(BM, M - tm * BM);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A + (int64_t)tm * BM * K, (uint32_t)rows_a * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)K * (uint32_t)N * 4u);
    auto swz = [](int r) { return (r >> 2) & 3; };

    // A: instruction i of this wave fills rows (wave * kAInst + i) * 16 + l / 4,
    // slot chunk l % 4 (holding global chunk (l % 4) ^ swz(row)).
    int a_voff[kAInst];
#pragma unroll
    for (int i = 0; i < kAInst; ++i) {
        const int r = (wave * kAInst + i) * 16 + (lane >> 2);
        a_voff[i] = r * K * 4 + (((lane & 3) ^ swz(r)) << 4);
    }
    // B: instruction i fills k-row kr = wave * kBInst + i; slot chunk l holds
    // global chunk (l + 8 [kr >= 8]) % 64 of the tile's 256 columns.
    int b_voff[kBInst];
    bool b_live[kBInst];
#pragma unroll
    for (int i = 0; i < kBInst; ++i) {
        const int kr = wave * kBInst + i;
        const int col = tn * BN + (((lane + (kr >= 8 ? 8 : 0)) & 63) << 2);
        b_live[i] = col < N;
        b_voff[i] = (kr * N + col) * 4;
    }
    auto issue_stage = [&](int kt) {
        char* base = lds + (kt % NS) * kStage;
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < kAInst; ++i) lds_dma16(ra, base + (wave * kAInst + i) * 1024, a_voff[i], k0 * 4);
#pragma unroll
        for (int i = 0; i < kBInst; ++i) {
            // offsets past the resource read zeros; 0x7FFFFFF0 >= K * N * 4
            const int off = b_live[i] ? b_voff[i] + k0 * N * 4 : 0x7FFFFFF0;
            lds_dma16(rb, base + kLdsA + (wave * kBInst + i) * 1024, off, 0);
        }
    };

    // Fragments: A block a, lane (g = l / 32, row l % 32) reads chunks 2g and
    // 2g + 1 of its row; B block b, step s reads row 8g + s, column j.
    const int fr = lane & 31, g = lane >> 5;
    int a_off[kTM], b_off[kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a) {
        const int r = wm * kWaveM + a * 32 + fr;
        a_off[a] = r * 64 + (((2 * g) ^ swz(r)) << 4);
    }
#pragma unroll
    for (int b = 0; b < kTN; ++b) {
        const int c = wn * kWaveN + b * 32 + fr;
        b_off[b] = kLdsA + (8 * g) * 1024 + ((((c >> 2) - 8 * g) & 63) << 4) + (c & 3) * 4;
    }
    f32x4 fa[kTM][2];
    float fb[kTN][8];
    auto read_stage = [&](int kt) {
        const char* base = lds + (kt % NS) * kStage;
#pragma unroll
        for (int a = 0; a < kTM; ++a) {
            fa[a][0] = *reinterpret_cast<const f32x4*>(base + a_off[a]);
            fa[a][1] = *reinterpret_cast<const f32x4*>(base + (a_off[a] ^ 16));
        }
#pragma unroll
        for (int b = 0; b < kTN; ++b)
#pragma unroll
            for (int s = 0; s < 8; ++s) fb[b][s] = *reinterpret_cast<const float*>(base + b_off[b] + s * 1024);
    };

    f32x16 acc[kTM][kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) acc[a][b] = f32x16{0};

    const int nk = K / BK;
#pragma unroll
    for (int st = 0; st < D; ++st)
        if (st < nk) issue_stage(st);
    wait_loads_beyond<kLoads>(min(D - 1, nk - 1));  // stage 0 landed
    __builtin_amdgcn_s_barrier();
    if (group == 1) __builtin_amdgcn_s_barrier();  // stagger: group 1 runs one phase behind
    __builtin_amdgcn_sched_barrier(0);
    for (int k = 0; k < nk; ++k) {
        // memory phase
        read_stage(k);
        if (k + D < nk) issue_stage(k + D);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));          // fragments in registers
        wait_loads_beyond<kLoads>(min(D - 1, nk - 2 - k));  // stage k + 1 landed
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // compute phase
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int a = 0; a < kTM; ++a)
#pragma unroll
                for (int b = 0; b < kTN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][s >> 2][s & 3], fb[b][s], acc[a][b], 0,
                                                                     0, 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (group == 0) __builtin_amdgcn_s_barrier();  // both groups end on 2 * nk + 2 barriers

    // 32x32 result layout: register r of lane l holds row 8 (r / 4) + 4 (l / 32)
    // + r % 4, column l % 32.
    const int64_t row_base = (int64_t)tm * BM + wm * kWaveM + 4 * g;
    const int64_t col_base = (int64_t)tn * BN + wn * kWaveN + fr;
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
    // once: the ping-pong kernel where its layout conditions hold (C3b's
    // 4096^3: 136 TFLOP/s), else the register-staged kernel at the same tile
    // (131; 121 with 128x128 tiles; 256x128, 128x256, BK 8 and 32 and 16
    // waves all measured within 127-131).
    const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256);
    const bool pp = K % 16 == 0 && N % 4 == 0 && kh::aligned(a, 16) && kh::aligned(b, 16) &&
                    K * N * 4 < 0x7FFFFFF0LL && 256 * K * 4 < 0x7FFFFFFFLL && M <= 0x7FFFFFFF;
    if (big_tiles >= d->cus && pp) {
        gemm_f32_pingpong_kernel<4><<<(unsigned)big_tiles, 512, 0, d->stream>>>(a, b, out, bias, (int)M, (int)N,
                                                                                 (int)K);
        return kh::launch_status("gemm_f32_pingpong");
    }
    if (big_tiles >= d->cus) return launch_f32<256, 256, 16, 2, 4>(d, a, b, out, bias, M, N, K, vec);
    return launch_f32<128, 128, 16, 2, 2>(d, a, b, out, bias, M, N, K, vec);
}
