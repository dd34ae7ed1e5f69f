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

// Stores one 32x32 MFMA result block (register r of lane l holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32, relative to (i0, j)).  The column's
// scale and bias are read once per block.
__device__ __forceinline__ void store_block32(const Epilogue& ep, int64_t i0, int64_t j, int64_t N, const i32x16& v) {
    const double sbj = ep.sb ? ep.sb[ep.sb_per_col ? j : 0] : 0.0;
    const float bj = ep.bias ? ep.bias[j] : 0.0f;
    const double sa0 = (ep.sa && !ep.sa_per_row) ? ep.sa[0] * sbj : 0.0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t i = i0 + 8 * (r >> 2) + (r & 3);
        if (ep.acc) ep.acc[i * N + j] = v[r];
        if (ep.out) {
            const double s = ep.sa_per_row ? ep.sa[i] * sbj : sa0;
            float y = (float)((double)v[r] * s);
            if (ep.bias) y = y + bj;
            ep.out[i * N + j] = y;
        }
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

// ---------------------------------------------------------------------------
// Full-tile kernel (M % BM == 0, N % BN == 0, K % BK == 0, 16-byte aligned
// operands): no bounds tests in the main loop.
//
// * Global loads are raw buffer loads: one VGPR offset per chunk, the k
//   advance in an SGPR.
// * LDS rows are BK = 128 bytes (8 chunks of 16 B) with no padding; chunk c
//   of row r is stored at chunk slot c ^ swz(r), an XOR swizzle under which
//   the MFMA fragment reads (32 consecutive rows, one chunk) and the
//   row-contiguous fragment writes are both free of bank conflicts.
// * MFMA fragments are double-buffered in registers across the four 32-k
//   substeps of a BK step, so LDS latency hides behind the previous
//   substep's MFMAs.
// * Workgroups are launched on a 1-D grid; hardware deals consecutive
//   workgroup ids round-robin to the 8 XCDs, so the id is remapped to give
//   each XCD a contiguous band of tiles, walked in groups of kGroupM tile rows
//   so that concurrently resident tiles share A and B panels in that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kXcds = 8;
constexpr int kBufferFlags = 0x00020000;  // dword 3 of a raw gfx9 buffer resource

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

__device__ __forceinline__ int lds_swz(int r) { return ((r >> 1) ^ (r << 2)) & 7; }

// Workgroup id -> (tile row, tile col).
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    int t = bid;
    if (total % kXcds == 0) t = (bid % kXcds) * (total / kXcds) + bid / kXcds;
    const int per_group = group_m * tiles_n;
    const int g = t / per_group;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_g = t - g * per_group;
    tm = first_m + in_g % gm;
    tn = in_g / gm;
}

// Swizzle for BK-byte LDS rows (BK / 16 chunks): conflict-free for 8- and
// 16-lane groups reading one chunk of consecutive rows.
template <int BK>
__device__ __forceinline__ int tile_swz(int r) {
    if (BK == 128) return ((r >> 1) ^ (r << 2)) & 7;
    return ((r >> 1) ^ (r >> 3)) & 3;
}

// Scheduling hint: interleave `n` (1 MFMA, 1 LDS read) pairs.
#define KH_SCHED_MFMA_DS(n)                                   \
    do {                                                      \
        _Pragma("unroll") for (int _i = 0; _i < (n); ++_i) {  \
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); \
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
        }                                                     \
    } while (0)

// HINT: interleave LDS reads between MFMAs with scheduling barriers.
// PRIO: raise the wave's issue priority while it issues an MFMA cluster, so
// the SIMD's other wave does its memory work in the gaps.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int HINT, int PRIO>
__global__ __launch_bounds__(WM * WN * 64) void gemm_i8_tiled_kernel(const int8_t* __restrict__ A,
                                                                     const int8_t* __restrict__ B, int M, int N,
                                                                     int K, int group_m, Epilogue ep) {
    constexpr int kCh = BK / 16;  // 16-byte chunks per LDS row
    constexpr int kSub = BK / 32;  // MFMA k-substeps per stage
    constexpr int kThreads = WM * WN * 64;
    constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    constexpr int kTM = kWaveM / 32, kTN = kWaveN / 32;
    constexpr int kAChunks = BM * kCh / kThreads;
    constexpr int kBChunks = BN * kCh / kThreads;
    constexpr int kLdsA = BM * BK, kLdsB = BN * BK, kStage = kLdsA + kLdsB;
    static_assert(kAChunks >= 1 && kBChunks >= 1, "tile too small for the block");
    static_assert(STAGES >= 2, "at least two LDS stages");
    __shared__ __attribute__((aligned(16))) int8_t lds[STAGES * kStage];

    int tm, tn;
    tile_of(blockIdx.x, M / BM, N / BN, group_m, tm, tn);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A + (int64_t)tm * BM * K, (uint32_t)BM * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + (int64_t)tn * BN * K, (uint32_t)BN * (uint32_t)K);

    int a_goff[kAChunks], a_loff[kAChunks], b_goff[kBChunks], b_loff[kBChunks];
#pragma unroll
    for (int c = 0; c < kAChunks; ++c) {
        const int idx = tid + c * kThreads, r = idx / kCh, kc = idx % kCh;
        a_goff[c] = r * K + kc * 16;
        a_loff[c] = r * BK + ((kc ^ tile_swz<BK>(r)) << 4);
    }
#pragma unroll
    for (int c = 0; c < kBChunks; ++c) {
        const int idx = tid + c * kThreads, r = idx / kCh, kc = idx % kCh;
        b_goff[c] = r * K + kc * 16;
        b_loff[c] = kLdsA + r * BK + ((kc ^ tile_swz<BK>(r)) << 4);
    }
    i32x4 sa_[kAChunks], sb_[kBChunks];
    auto gload = [&](int k0) {
#pragma unroll
        for (int c = 0; c < kAChunks; ++c) sa_[c] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_goff[c], k0, 0);
#pragma unroll
        for (int c = 0; c < kBChunks; ++c) sb_[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_goff[c], k0, 0);
    };
    auto lstore = [&](int stage) {
        int8_t* base = lds + stage * kStage;
#pragma unroll
        for (int c = 0; c < kAChunks; ++c) *reinterpret_cast<i32x4*>(base + a_loff[c]) = sa_[c];
#pragma unroll
        for (int c = 0; c < kBChunks; ++c) *reinterpret_cast<i32x4*>(base + b_loff[c]) = sb_[c];
    };

    const int fr = lane & 31, fh = lane >> 5;
    // LDS byte offsets (within a stage) of this lane's fragment rows.
    int a_row[kTM], b_row[kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a) a_row[a] = wm * kWaveM + a * 32 + fr;
#pragma unroll
    for (int b = 0; b < kTN; ++b) b_row[b] = wn * kWaveN + b * 32 + fr;
    auto read_frags = [&](int stage, int sub, i32x4* fa, i32x4* fb) {
        const int8_t* base = lds + stage * kStage;
#pragma unroll
        for (int a = 0; a < kTM; ++a) {
            const int r = a_row[a];
            fa[a] = *reinterpret_cast<const i32x4*>(base + r * BK + (((2 * sub + fh) ^ tile_swz<BK>(r)) << 4));
        }
#pragma unroll
        for (int b = 0; b < kTN; ++b) {
            const int r = b_row[b];
            fb[b] = *reinterpret_cast<const i32x4*>(base + kLdsA + r * BK + (((2 * sub + fh) ^ tile_swz<BK>(r)) << 4));
        }
    };

    i32x16 acc[kTM][kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) acc[a][b] = i32x16{0};

    const int nk = K / BK;
    // Prologue: stages 0 .. STAGES-2 into LDS, k-step STAGES-1 into registers.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
        if (s < nk) {
            gload(s * BK);
            lstore(s);
        }
    }
    if (STAGES - 1 < nk) gload((STAGES - 1) * BK);
    __syncthreads();

    i32x4 fa[2][kTM], fb[2][kTN];
    read_frags(0, 0, fa[0], fb[0]);
    for (int kt = 0; kt < nk; ++kt) {
        const int stage = kt % STAGES;
        const int next_stage = (kt + 1) % STAGES;
#pragma unroll
        for (int sub = 0; sub < kSub; ++sub) {
            const int cur = sub & 1;
            // Prefetch the next substep's fragments -- from the next stage
            // after the last substep (visible since the previous barrier).
            if (sub + 1 < kSub)
                read_frags(stage, sub + 1, fa[cur ^ 1], fb[cur ^ 1]);
            else if (kt + 1 < nk && STAGES > 2)
                read_frags(next_stage, 0, fa[cur ^ 1], fb[cur ^ 1]);
            if (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int a = 0; a < kTM; ++a)
#pragma unroll
                for (int b = 0; b < kTN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[cur][a], fb[cur][b], acc[a][b], 0, 0, 0);
            if (HINT) KH_SCHED_MFMA_DS(kTM + kTN);
            if (PRIO) __builtin_amdgcn_s_setprio(0);
        }
        // Registers hold k-step kt + STAGES - 1: store it into the stage that
        // was read during k-step kt - 1 (every wave passed the last barrier).
        if (kt + STAGES - 1 < nk) {
            lstore((kt + STAGES - 1) % STAGES);
            if (kt + STAGES < nk) gload((kt + STAGES) * BK);
        }
        __syncthreads();
        if (STAGES == 2 && kt + 1 < nk) read_frags(next_stage, 0, fa[kSub & 1], fb[kSub & 1]);
    }

    // With 128x128 wave tiles the accumulators fill all 256 AGPRs; keep them
    // there until each block is stored (otherwise every block is copied to
    // VGPRs at once on loop exit).
    if (kTM * kTN * 16 > 128) {
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) asm volatile("" : "+a"(acc[a][b]));
    }
    const int64_t row_base = (int64_t)tm * BM + wm * kWaveM + 4 * fh;
    const int64_t col_base = (int64_t)tn * BN + wn * kWaveN + fr;
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) {
            store_block32(ep, row_base + a * 32, col_base + b * 32, N, acc[a][b]);
            __builtin_amdgcn_sched_barrier(0);
        }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for decode-style shapes (M <= 32): weight streaming.
//
// A workgroup owns 16 output columns for all M rows; its SKW waves split K,
// each streaming its slice of those 16 packed weight rows (16 B per lane per
// 64-k step) through v_mfma_i32_16x16x64_i8 with up to two 16-row tiles of
// activations.  Rows >= M read zeros: their buffer offsets fall past the
// activation resource, whose loads return 0.  The waves' partial int32
// accumulators are summed through LDS (integer sums are exact in any order)
// and the first wave applies the epilogue.  Bound: HBM bytes of the weight,
// N*K, plus the activations (L2 resident) and the output.
// ---------------------------------------------------------------------------
typedef int i32x4v __attribute__((ext_vector_type(4)));
constexpr int kSkinnyWaves = 8;

template <int MT>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_i8_skinny_kernel(const int8_t* __restrict__ A,
                                                                           const int8_t* __restrict__ B, int M,
                                                                           int N, int K, Epilogue ep) {
    __shared__ i32x4v red[kSkinnyWaves][MT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int col = n0 + (lane & 15);
    const int kg = (lane >> 4) * 16;
    const int kper = K / kSkinnyWaves;
    const int k_begin = wave * kper;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    const int b_off = min(col, N - 1) * K + kg;
    int a_off[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) a_off[t] = (t * 16 + (lane & 15)) * K + kg;

    i32x4v acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = i32x4v{0, 0, 0, 0};
#pragma unroll 8
    for (int k = k_begin; k < k_begin + kper; k += 64) {
        const i32x4v b = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off, k, 0);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const i32x4v a = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t], k, 0);
            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[t], 0, 0, 0);
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave != 0) return;
    // 16x16 MFMA result layout: register r of lane l holds row 4*(l/16) + r,
    // column l%16.
    const int64_t j = col;
    if (j >= N) return;
    const double sbj = ep.sb ? ep.sb[ep.sb_per_col ? j : 0] : 0.0;
    const float bj = ep.bias ? ep.bias[j] : 0.0f;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        i32x4v sum = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < kSkinnyWaves; ++w) sum += red[w][t][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t i = t * 16 + 4 * (lane >> 4) + r;
            if (i >= M) continue;
            if (ep.acc) ep.acc[i * N + j] = sum[r];
            if (ep.out) {
                const double s = ep.sa[ep.sa_per_row ? i : 0] * sbj;
                float y = (float)((double)sum[r] * s);
                if (ep.bias) y = y + bj;
                ep.out[i * N + j] = y;
            }
        }
    }
}

bool skinny_fits(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K) {
    return M >= 1 && M <= 32 && K > 0 && K % (64 * kSkinnyWaves) == 0 && kh::aligned(A, 16) &&
           kh::aligned(B, 16) && M * K <= 0xFFFFFFFFLL && N * K <= 0xFFFFFFFFLL && N <= 0x7FFFFFFF;
}

int launch_skinny(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                  const Epilogue& ep) {
    const unsigned blocks = (unsigned)((N + 15) / 16);
    if (M <= 16)
        gemm_i8_skinny_kernel<1><<<blocks, kSkinnyWaves * 64, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
    else
        gemm_i8_skinny_kernel<2><<<blocks, kSkinnyWaves * 64, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
    return kh::launch_status("gemm_i8_skinny");
}

template <int BM, int BN, int BK, int WM, int WN, int STAGES, int HINT, int PRIO>
int launch_tiled(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                 const Epilogue& ep, int group_m) {
    const unsigned tiles = (unsigned)((M / BM) * (N / BN));
    gemm_i8_tiled_kernel<BM, BN, BK, WM, WN, STAGES, HINT, PRIO>
        <<<tiles, WM * WN * 64, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep);
    return kh::launch_status("gemm_i8_tiled");
}

// True when the full-tile kernel applies to this shape.
template <int BM, int BN, int BK>
bool tiled_fits(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K) {
    return M % BM == 0 && N % BN == 0 && K % BK == 0 && K > 0 && kh::aligned(A, 16) && kh::aligned(B, 16) &&
           (int64_t)BM * K <= 0xFFFFFFFFLL && (int64_t)BN * K <= 0xFFFFFFFFLL && M <= 0x7FFFFFFF && N <= 0x7FFFFFFF &&
           (M / BM) * (N / BN) <= 0x7FFFFFFF;
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
    if (skinny_fits(a, b_packed, M, N, K)) return launch_skinny(d, a, b_packed, M, N, K, ep);
    if (tiled_fits<256, 256, 128>(a, b_packed, M, N, K))
        return launch_tiled<256, 256, 128, 2, 4, 2, 1, 0>(d, a, b_packed, M, N, K, ep, 8);
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
