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

#include <type_traits>

#include "kh_common.h"
#include "kh_quant_math.h"
#include "kh_act.h"
#include "kh_pipeline.h"

#pragma clang fp contract(off)

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct Epilogue {
    const double* sa;
    const double* sb;
    const float* bias;
    float* out;
    int32_t* acc;
    int sa_per_row;
    int sb_per_col;
    int act;                // kActNone or kActGelu, applied after the bias
    const float* residual;  // [M, N]: out = residual + y (the graph's x.add(linear(..)))
    // Output mode kOutQuant (the fp32 result quantized per tensor, never
    // stored): codes [M, N], the pass-1 absmax partials, the scale's slot.
    int8_t* q;
    const unsigned* qparts;
    int nqparts;
    double* qscale;
    unsigned* fault;
    // 1: the full-tile fp32 stores are non-temporal (an output too large
    // to stay in the last-level cache); 0: ordinary stores.
    int stream_out;
};

constexpr int kActNone = 0;
constexpr int kActGelu = 1;

// The fp32 output of one accumulator (see the file comment), then the fused
// activation and residual add in the order the unfused graph applies them;
// `resid` is residual[i, j] (read by the caller, ignored without a residual).
// FUSED = false compiles the plain epilogue only (no activation or residual
// code: the kernels that never fuse keep their register budget).
template <bool FUSED = true>
__device__ __forceinline__ float epilogue_finish(const Epilogue& ep, int32_t acc, double s, float bj, float resid) {
    float y = (float)((double)acc * s);
    if (ep.bias) y = y + bj;
    if (FUSED) {
        if (ep.act == kActGelu) y = kh::gelu(y);
        if (ep.residual) y = resid + y;
    }
    return y;
}

template <bool FUSED = true>
__device__ __forceinline__ float epilogue_value(const Epilogue& ep, int64_t i, int64_t j, int64_t N, int32_t acc,
                                                double s, float bj) {
    const float resid = (FUSED && ep.residual) ? ep.residual[i * N + j] : 0.0f;
    return epilogue_finish<FUSED>(ep, acc, s, bj, resid);
}

// One output element of the epilogue (see the file comment).
__device__ __forceinline__ void epilogue_store(const Epilogue& ep, int64_t i, int64_t j, int64_t N, int32_t acc) {
    if (ep.acc) ep.acc[i * N + j] = acc;
    if (ep.out) {
        const double s = ep.sa[ep.sa_per_row ? i : 0] * ep.sb[ep.sb_per_col ? j : 0];
        ep.out[i * N + j] = epilogue_value(ep, i, j, N, acc, s, ep.bias ? ep.bias[j] : 0.0f);
    }
}

// Stores one 32x32 MFMA result block (register r of lane l holds row
// 8*(r/4) + 4*(l/32) + r%4, column l%32, relative to (i0, j)); MASKED skips
// rows >= M and columns >= N.  The column's scale and bias are read once per
// block.  The residual is read RG rows at a time, each group before any of
// its stores: the output may alias nothing the compiler can prove, so a load
// left after a store would wait for it (one memory round trip per element
// instead of one per group).  Returns the largest |out| bits stored (for the
// absmax partials of a following per-tensor quantize).
template <bool FUSED, int RG, bool MASKED, int MODE>
__device__ __forceinline__ unsigned store_block32_impl(const Epilogue& ep, int64_t i0, int64_t j, int64_t M,
                                                       int64_t N, const i32x16& v, const kh::quant::Scale& sc) {
    static_assert(16 % RG == 0, "residual group");
    if (MASKED && j >= N) return 0;
    const double sbj = ep.sb ? ep.sb[ep.sb_per_col ? j : 0] : 0.0;
    const float bj = ep.bias ? ep.bias[j] : 0.0f;
    const double sa0 = (ep.sa && !ep.sa_per_row) ? ep.sa[0] * sbj : 0.0;
    unsigned mx = 0;
#pragma unroll
    for (int g0 = 0; g0 < 16; g0 += RG) {
        float res[RG];
#pragma unroll
        for (int rr = 0; rr < RG; ++rr) {
            const int r = g0 + rr;
            const int64_t i = i0 + 8 * (r >> 2) + (r & 3);
            res[rr] = (FUSED && ep.residual && (!MASKED || i < M)) ? ep.residual[i * N + j] : 0.0f;
        }
#pragma unroll
        for (int rr = 0; rr < RG; ++rr) {
            const int r = g0 + rr;
            const int64_t i = i0 + 8 * (r >> 2) + (r & 3);
            if (MASKED && i >= M) continue;
            if (MODE != kh::quant::kOutStore) {
                // The value the fp32 epilogue would store: its absmax
                // (pass 1) or its per-tensor code (pass 2).
                const double s = ep.sa_per_row ? ep.sa[i] * sbj : sa0;
                const float y = epilogue_finish<FUSED>(ep, v[r], s, bj, res[rr]);
                mx = max(mx, kh::abs_bits32(y));
                if (MODE == kh::quant::kOutQuant) ep.q[i * N + j] = (int8_t)kh::quant::quant_one(y, sc);
                continue;
            }
            if (ep.acc) ep.acc[i * N + j] = v[r];
            if (ep.out) {
                const double s = ep.sa_per_row ? ep.sa[i] * sbj : sa0;
                const float y = epilogue_finish<FUSED>(ep, v[r], s, bj, res[rr]);
                ep.out[i * N + j] = y;
                mx = max(mx, kh::abs_bits32(y));
            }
        }
    }
    return mx;
}

template <bool FUSED = true, int RG = 16, int MODE = kh::quant::kOutStore>
__device__ __forceinline__ unsigned store_block32(const Epilogue& ep, int64_t i0, int64_t j, int64_t N,
                                                  const i32x16& v, const kh::quant::Scale& sc) {
    return store_block32_impl<FUSED, RG, false, MODE>(ep, i0, j, 0, N, v, sc);
}

// store_block32 for a block that may extend past row M or column N.
template <bool FUSED = true, int RG = 16, int MODE = kh::quant::kOutStore>
__device__ __forceinline__ unsigned store_block32_masked(const Epilogue& ep, int64_t i0, int64_t j, int64_t M,
                                                         int64_t N, const i32x16& v, const kh::quant::Scale& sc) {
    return store_block32_impl<FUSED, RG, true, MODE>(ep, i0, j, M, N, v, sc);
}

// max |GELU(y)| over 16 values as bits, with GELU evaluated once instead of
// 16 times: kh::gelu, as the hardware computes it, is non-decreasing on
// [0, +inf), and |GELU(x)| for every negative x is below GELU(0.3) (both
// checked over every binary32 value by tests/test_gpu_charlm.py), so when the
// largest value is >= 0.3 its GELU is the largest in magnitude.  Otherwise
// every value's GELU is evaluated.  A NaN or +-inf among the values gives a
// non-finite result, as GELU would (GELU of NaN, +inf, -inf: NaN, +inf, NaN).
constexpr int kGeluMonoBits = 0x3E99999A;  // 0.3f

__device__ __forceinline__ unsigned gelu_absmax_bits(const float (&y)[16]) {
    kh::quant::AbsMax am;
#pragma unroll
    for (int r = 0; r < 16; ++r) am.add1(y[r]);
    const unsigned m = am.bits();
    if (m >= KH_NONFINITE_BITS) return m;
    if (am.smax >= kGeluMonoBits) return kh::abs_bits32(kh::gelu(__int_as_float(am.smax)));
    unsigned g = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) g = max(g, kh::abs_bits32(kh::gelu(y[r])));
    return g;
}

// store_block32 for a block inside the matrix in the common configuration --
// fp32 output only (or one of the quantize passes), per-tensor activation
// scale, or per-row scales (ROWSA: sa[i] * sb[j] per row, as in
// store_block32_impl) -- with the uniform choices (bias, activation, residual) taken once
// per block instead of per element, and raw buffer accesses whose row offsets
// are scalar (8*(r/4) + r%4 rows of N floats), so no element needs address
// arithmetic.  Same arithmetic, in the same order, as store_block32_impl.
// (rowblk, colblk): the block's first row and column; N <= 2^24.
// The column scale sb[j] and bias[j] of lane l's column colblk + l % 32 (0
// without them), loaded by the kernels before their main loop.
struct ColEpi {
    double sb;
    float bias;
};
__device__ __forceinline__ ColEpi col_epi(const Epilogue& ep, int64_t j) {
    return ColEpi{ep.sb ? ep.sb[ep.sb_per_col ? j : 0] : 0.0, ep.bias ? ep.bias[j] : 0.0f};
}

// The int8 codes of a 32x32 block (lane l's 16 values: column l % 32, rows
// 4 (l / 32) + 8 (r / 4) + r % 4, the low byte of c[r] each) through `rq`,
// a resource over the block's 32 rows of N codes (from column -col0).  Codes of rows 8g + t
// (t = 0..3) of this lane's column, packed (byte t = row t), then transposed
// across each quad of lanes so that lane 4p + t holds row 8g + t of columns
// 4p .. 4p + 3: one dword store per group instead of four byte stores (N and
// the codes' base 4-byte aligned).
__device__ __forceinline__ void store_codes_block32(__amdgpu_buffer_rsrc_t rq, int N, int lane,
                                                    const unsigned (&c)[16], int col0 = 0) {
    const int fr = lane & 31, fh = lane >> 5;
    const unsigned sel_a = (fr & 1) ? 0x03070105u : 0x06020400u;  // with lane ^ 1: bytes (0,2) or (1,3)
    const unsigned sel_b = (fr & 2) ? 0x03020706u : 0x05040100u;  // with lane ^ 2: halves 0 or 1
    const int qoff = (4 * fh + (fr & 3)) * N + (fr & ~3) + col0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const unsigned p = __builtin_amdgcn_perm(c[4 * g + 1], c[4 * g], 0x0c0c0400u) |
                           __builtin_amdgcn_perm(c[4 * g + 3], c[4 * g + 2], 0x04000c0cu);
        const unsigned a = __builtin_amdgcn_perm(kh::lanes::quad_perm<0xB1>(p), p, sel_a);
        const unsigned t = __builtin_amdgcn_perm(kh::lanes::quad_perm<0x4E>(a), a, sel_b);
        __builtin_amdgcn_raw_buffer_store_b32(t, rq, qoff, 8 * g * N, 0);
    }
}

template <bool FUSED, int MODE, bool ROWSA = false>
__device__ __forceinline__ unsigned store_block32_full(const Epilogue& ep, int64_t rowblk, int64_t colblk, int N,
                                                       int lane, double sa, const i32x16& v,
                                                       const kh::quant::Scale& sc, ColEpi ce,
                                                       const double* sa_rows = nullptr, int sa_row0 = 0) {
    const int fr = lane & 31, fh = lane >> 5;
    const double sbj = ce.sb;
    const double s = sa * sbj;
    const int64_t base = rowblk * N + colblk;
    const uint32_t span = (uint32_t)N * 32u * 4u;  // the block's 32 rows, in bytes
    const int voff = (4 * fh * N + fr) * 4;
    auto row_off = [&](int r) { return (8 * (r >> 2) + (r & 3)) * N * 4; };
    float res[16];
    if (FUSED && ep.residual) {
        const __amdgpu_buffer_rsrc_t rr = kh::pipe::make_rsrc(ep.residual + base, span);
#pragma unroll
        for (int r = 0; r < 16; ++r) res[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rr, voff, row_off(r), 0));
    }
    float y[16];
    if constexpr (ROWSA) {
        // Value r of this lane is row rowblk + 4*fh + 8*(r/4) + r%4: four
        // row scales at a time (sa[i] * sb[j], then the product), so only
        // four binary64 scales are live at once.
        // (sa_rows: the block's row scales elsewhere, first row at sa_row0.)
        const double* sar = (sa_rows ? sa_rows + sa_row0 : ep.sa + rowblk) + 4 * fh;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            double s4[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) s4[rr] = sar[8 * g + rr] * sbj;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) y[4 * g + rr] = (float)((double)v[4 * g + rr] * s4[rr]);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) y[r] = (float)((double)v[r] * s);
    }
    if (ep.bias) {
#pragma unroll
        for (int r = 0; r < 16; ++r) y[r] = y[r] + ce.bias;
    }
    if constexpr (FUSED && MODE == kh::quant::kOutMaxOnly) {
        if (ep.act == kActGelu && !ep.residual) return gelu_absmax_bits(y);
    }
    if (FUSED && ep.act == kActGelu) {
#pragma unroll
        for (int r = 0; r < 16; ++r) y[r] = kh::gelu(y[r]);
    }
    if (FUSED && ep.residual) {
#pragma unroll
        for (int r = 0; r < 16; ++r) y[r] = res[r] + y[r];
    }
    unsigned mx = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = max(mx, kh::abs_bits32(y[r]));
    if (MODE == kh::quant::kOutStore) {
        // Non-temporal stores (cache policy nt) for a large output: it
        // streams out without taking L2 lines from the operand tiles other
        // workgroups are still reading (8192^3: 2370 -> 2390 TOPS).
        // Ordinary stores for the rest: C4's forward, whose GEMM outputs
        // are at most 100.7 MB, runs 0.5-1.3 % faster with them.
        const __amdgpu_buffer_rsrc_t ro = kh::pipe::make_rsrc(ep.out + base, span);
        if (ep.stream_out) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y[r]), ro, voff, row_off(r), 2);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y[r]), ro, voff, row_off(r), 0);
        }
    } else if (MODE == kh::quant::kOutQuant) {
        // The codes of quant_one: the fast path for all 16 values, and the
        // exact path for all 16 in a lane holding an undecided value (or
        // everywhere when the scale rules the fast path out).
        unsigned c[16];
        bool ok = sc.fast;
#pragma unroll
        for (int r = 0; r < 16; ++r) c[r] = kh::quant::quant_fast(y[r], sc.rf, ok);  // low byte: the code
        if (!ok) {
#pragma unroll
            for (int r = 0; r < 16; ++r) c[r] = sc.bad ? 0u : (unsigned)kh::quant::quant_exact(y[r], sc.s);
        }
        store_codes_block32(kh::pipe::make_rsrc(ep.q + base, span / 4u), N, lane, c);
    }
    return mx;
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
// Full-tile kernel (M % 256 == 0, N % 256 == 0, K % 64 == 0, 16-byte aligned
// operands), scheduled for the MI355X power envelope: with random int8
// operands the shader clock settles near 1.3-1.6 GHz under MFMA load, so the
// kernel's job is to keep the MFMA pipe issuing at that clock.
//
// * 256x256 workgroup tile, 8 waves as 2 (M) x 4 (N); each wave owns 128x64
//   outputs as 4x2 blocks of v_mfma_i32_32x32x32_i8 (128 int32 accumulators).
// * K is staged 64 bytes at a time in a ring of NS LDS stages (32 KB each).
//   Operands move global -> LDS by LDS-DMA (buffer_load_dwordx4 ... lds):
//   no VGPR staging and no ds_write.  Lane l of one instruction lands at
//   M0 + 16*l, so the XOR swizzle is applied on the global side: LDS slot
//   (row r, chunk c') holds global chunk c' ^ swz(r), swz(r) = (r >> 2) & 3,
//   under which the MFMA fragment reads (16 consecutive rows, one chunk per
//   lane) hit 64 distinct banks.
// * Ping-pong: waves 0-3 (group 0, one per SIMD) and waves 4-7 (group 1) run
//   the same sequence -- memory phase (fragment reads for K-step k, LDS-DMA
//   for step k + NS - 1), barrier, compute phase (16 MFMAs), barrier -- with
//   group 1 one barrier behind, so on every SIMD one wave's MFMAs cover the
//   other wave's memory phase.  Every wave executes 2 * nk + 2 barriers.
// * Before the barrier that ends its memory phase for step k a wave waits
//   for its own LDS-DMA of stage k + 1 (vmcnt counts the later stages still
//   allowed in flight) and for its fragment reads (lgkmcnt 0), so the
//   barrier publishes stage k + 1 and retires every read of stage k - 1,
//   whose slot the next memory phase refills.
// * Workgroups are launched on a 1-D grid; hardware deals consecutive ids
//   round-robin to the 8 XCDs, so the id is remapped to give each XCD a
//   contiguous band of tiles, walked in groups of `group_m` tile rows so that
//   concurrently resident tiles share A and B panels in that XCD's L2.
// ---------------------------------------------------------------------------
using namespace kh::pipe;

// FUSED: the epilogue may apply an activation and a residual add.  EPI:
// kEpiGeneral, every epilogue path; kEpiFull / kEpiFullRows, the launch
// guarantees full tiles, no int32 output and N <= 2^24 with a per-tensor /
// per-row activation scale, so only that store_block32_full is compiled in.  Waves per
// SIMD: 2 for 256-wide N tiles (128 accumulators per wave); 4 for the
// 256x128 tile; 6 (three resident workgroups per CU, 80 registers) for the
// 128x128 tile unless the general fused epilogue is compiled in, which needs 4
// (128 registers: its per-element residual and masking paths spill heavily
// at 80).  At K = 384 the third workgroup's main loop covers the other two's
// epilogues.
constexpr int kEpiGeneral = 0, kEpiFull = 1, kEpiFullRows = 2;

template <int BM, int BN, int NS, bool FUSED, int MODE = kh::quant::kOutStore, int EPI = kEpiGeneral>
__global__ __launch_bounds__(512, BN == 256 ? 2 : ((BM == 256 || NS >= 4 || (FUSED && EPI == kEpiGeneral)) ? 4 : 6)) void gemm_i8_pingpong_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K, int group_m, Epilogue ep,
    unsigned* parts) {
    constexpr int BK = 64, WM = 2, WN = 4, kWaves = WM * WN;
    static_assert((BM == 128 || BM == 256) && (BN == 128 || BN == 256), "tile");
    constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    constexpr int kTM = kWaveM / 32, kTN = kWaveN / 32;
    constexpr int kLdsA = BM * BK, kStage = (BM + BN) * BK;
    constexpr int kAInst = BM / 16 / kWaves, kBInst = BN / 16 / kWaves;  // 1 KB = 16 rows per instruction
    constexpr int kLoads = kAInst + kBInst;  // LDS-DMA instructions per wave per stage
    constexpr int D = NS - 1;                // prefetch distance in stages
    // Residual rows read ahead of their stores in the fused epilogue: all 16
    // of a block where the register budget allows, 4 in the 256x128 tile
    // (4 waves per SIMD leave it no room for 16).
    constexpr int kResidRows = (BM == 256 && BN == 128) ? 4 : 16;
    static_assert(NS >= 3 && NS <= 5, "wait_loads_beyond covers up to 3 stages ahead");
    __shared__ __attribute__((aligned(1024))) int8_t lds[NS * kStage];

    // kOutQuant: the tensor's scale from the pass-1 partials, before the
    // pipeline starts (workgroup 0 stores it for the caller).
    kh::quant::Scale sc{};
    if constexpr (MODE == kh::quant::kOutQuant) {
        __shared__ unsigned qred[kWaves];
        sc = kh::quant::make_scale(kh::quant::block_reduce_partials(ep.qparts, ep.nqparts, qred));
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            *ep.qscale = sc.s;
            if (sc.bad) kh::quant::flag_nonfinite(ep.fault);
        }
    }

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, group_m, tm, tn);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int group = wm;  // waves 0-3 and 4-7: one of each per SIMD

    // Rows past M (N) lie outside the resource: their loads return zeros.
    const int rows_a = min(BM, M - tm * BM), rows_b = min(BN, N - tn * BN);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A + (int64_t)tm * BM * K, (uint32_t)rows_a * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + (int64_t)tn * BN * K, (uint32_t)rows_b * (uint32_t)K);
    auto swz = [](int r) { return (r >> 2) & 3; };

    // LDS-DMA sources: instruction i of this wave fills rows
    // (wave * kXInst + i) * 16 + l / 4, slot chunk l % 4.
    const int lr = lane >> 2, lc = lane & 3;
    int a_voff[kAInst], b_voff[kBInst];
#pragma unroll
    for (int i = 0; i < kAInst; ++i) {
        const int r = (wave * kAInst + i) * 16 + lr;
        a_voff[i] = r * K + ((lc ^ swz(r)) << 4);
    }
#pragma unroll
    for (int i = 0; i < kBInst; ++i) {
        const int r = (wave * kBInst + i) * 16 + lr;
        b_voff[i] = r * K + ((lc ^ swz(r)) << 4);
    }
    auto issue_stage = [&](int kt) {
        int8_t* base = lds + (kt % NS) * kStage;
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < kAInst; ++i) lds_dma16(ra, base + (wave * kAInst + i) * 1024, a_voff[i], k0);
#pragma unroll
        for (int i = 0; i < kBInst; ++i) lds_dma16(rb, base + kLdsA + (wave * kBInst + i) * 1024, b_voff[i], k0);
    };

    // Fragment of 32x32 block row/col r for 32-k substep s: lane l reads
    // 16 bytes of row r + l % 32 at chunk 2s + l / 32, i.e. LDS byte
    // r * 64 + (((l / 32) ^ swz) << 4), with bit 5 flipped for s = 1.
    const int fr = lane & 31, fh = lane >> 5;
    // The full-tile epilogue's column scales, biases and activation scale,
    // requested before the main loop (the epilogue then waits for nothing).
    ColEpi ce[kTN];
    double sa_t = 0.0;
    if constexpr (EPI != kEpiGeneral) {
#pragma unroll
        for (int b = 0; b < kTN; ++b) ce[b] = col_epi(ep, (int64_t)tn * BN + wn * kWaveN + b * 32 + fr);
        if constexpr (EPI == kEpiFull) sa_t = ep.sa[0];
    }
    int a_off[kTM], b_off[kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a) {
        const int r = wm * kWaveM + a * 32 + fr;
        a_off[a] = r * BK + ((fh ^ swz(r)) << 4);
    }
#pragma unroll
    for (int b = 0; b < kTN; ++b) {
        const int r = wn * kWaveN + b * 32 + fr;
        b_off[b] = kLdsA + r * BK + ((fh ^ swz(r)) << 4);
    }
    i32x4 fa[2][kTM], fb[2][kTN];
    auto read_stage = [&](int kt) {
        const int8_t* base = lds + (kt % NS) * kStage;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int a = 0; a < kTM; ++a) fa[s][a] = *reinterpret_cast<const i32x4*>(base + (a_off[a] ^ (s << 5)));
#pragma unroll
            for (int b = 0; b < kTN; ++b) fb[s][b] = *reinterpret_cast<const i32x4*>(base + (b_off[b] ^ (s << 5)));
        }
    };

    i32x16 acc[kTM][kTN];
#pragma unroll
    for (int a = 0; a < kTM; ++a)
#pragma unroll
        for (int b = 0; b < kTN; ++b) acc[a][b] = i32x16{0};

    const int nk = K / BK;
#pragma unroll
    for (int s = 0; s < D; ++s)
        if (s < nk) issue_stage(s);
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
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int a = 0; a < kTM; ++a)
#pragma unroll
                for (int b = 0; b < kTN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s][a], fb[s][b], acc[a][b], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (group == 0) __builtin_amdgcn_s_barrier();  // both groups end on 2 * nk + 2 barriers

    const int64_t row_base = (int64_t)tm * BM + wm * kWaveM + 4 * fh;
    const int64_t col_base = (int64_t)tn * BN + wn * kWaveN + fr;
    unsigned mx = 0;
    const bool full = rows_a == BM && rows_b == BN;
    if constexpr (EPI != kEpiGeneral) {
        constexpr bool kRows = EPI == kEpiFullRows;
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) {
                mx = max(mx, store_block32_full<FUSED, MODE, kRows>(ep, (int64_t)tm * BM + wm * kWaveM + a * 32,
                                                                    (int64_t)tn * BN + wn * kWaveN + b * 32, N,
                                                                    lane, sa_t, acc[a][b], sc, ce[b]));
                __builtin_amdgcn_sched_barrier(0);
            }
    } else if (full && !ep.acc && !ep.sa_per_row && (MODE != kh::quant::kOutStore || ep.out) && N <= (1 << 24) &&
               (MODE != kh::quant::kOutQuant || ((N & 3) == 0 && ((uintptr_t)ep.q & 3) == 0))) {
        // (The quantize pass of store_block32_full writes a dword of four
        // codes per lane: it needs every row of q 4-byte aligned.)
        const double sa = ep.sa[0];
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) {
                const int64_t cb = (int64_t)tn * BN + wn * kWaveN + b * 32;
                mx = max(mx, store_block32_full<FUSED, MODE>(ep, (int64_t)tm * BM + wm * kWaveM + a * 32, cb, N,
                                                             lane, sa, acc[a][b], sc, col_epi(ep, cb + fr)));
                __builtin_amdgcn_sched_barrier(0);
            }
    } else if (full && !ep.acc && ep.sa_per_row && MODE == kh::quant::kOutStore && ep.out && N <= (1 << 24)) {
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) {
                const int64_t cb = (int64_t)tn * BN + wn * kWaveN + b * 32;
                mx = max(mx, store_block32_full<FUSED, MODE, true>(ep, (int64_t)tm * BM + wm * kWaveM + a * 32, cb, N,
                                                                   lane, 0.0, acc[a][b], sc, col_epi(ep, cb + fr)));
                __builtin_amdgcn_sched_barrier(0);
            }
    } else if (full) {
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) {
                mx = max(mx, store_block32<FUSED, kResidRows, MODE>(ep, row_base + a * 32, col_base + b * 32, N,
                                                                    acc[a][b], sc));
                __builtin_amdgcn_sched_barrier(0);
            }
    } else {
#pragma unroll
        for (int a = 0; a < kTM; ++a)
#pragma unroll
            for (int b = 0; b < kTN; ++b) {
                mx = max(mx, store_block32_masked<FUSED, kResidRows, MODE>(ep, row_base + a * 32, col_base + b * 32,
                                                                           M, N, acc[a][b], sc));
                __builtin_amdgcn_sched_barrier(0);
            }
    }
    if (MODE != kh::quant::kOutQuant && parts) {
        // Per-workgroup max |out| bits, for a following per-tensor quantize.
        unsigned* wmax = reinterpret_cast<unsigned*>(lds);  // every stage's last reader passed the final barrier
        mx = kh::quant::wave_max(mx);
        if (lane == 0) wmax[wave] = mx;
        __syncthreads();
        if (tid == 0) {
            unsigned m = wmax[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) m = max(m, wmax[w]);
            parts[blockIdx.x] = m;
        }
    }
}

// ---------------------------------------------------------------------------
// Quantize-on-load GEMM: out = epilogue(quantize_tensor(X) . B^T) for fp32 X
// [M, K] whose per-tensor scale comes from the absmax partials its producer
// wrote.  The codes of X are made in the main loop and never stored: where the
// two-step path reads X (4 bytes per value), writes its codes (1) and reads
// them back once per N-tile (1 each), this reads X once.
//
// * Workgroup tile kQlBM = 64 rows x BN = 128 NB columns (C4's N = 384 in one
//   tile, so X is read once); 8 waves as 2 (M) x 4 (N), each 32 x 32 NB
//   outputs (NB blocks of v_mfma_i32_32x32x32_i8).
// * K in steps of 64 through a ring of NS LDS stages, each A codes 64 x 64
//   and B codes BN x 64 in the ping-pong kernel's layout (64-byte rows, chunk
//   c of row r at slot c ^ ((r >> 2) & 3)).  B arrives by LDS-DMA.  For A,
//   thread t loads 8 floats of row t / 8 (two 16-byte loads, D = NS - 1 steps
//   ahead, into a register ring), quantizes them with the shared element
//   arithmetic (pack4: the fast path, the exact binary64 path where it is not
//   decisive) and writes the 8 codes to the stage (ds_write_b64).
// * Per step: wait for this wave's loads of the step, quantize and write A,
//   barrier (publishes A and B of the step; every read of the stage that the
//   next loads refill is done), issue the loads of step k + D, read the
//   fragments and multiply.
// * Epilogue: store_block32_full with the tensor's scale as the per-tensor
//   activation scale -- the same values as kh_quantize_tensor_parts followed
//   by kh_gemm_i8_ex.
// ---------------------------------------------------------------------------
constexpr int kQlBM = 64;

template <int NB, int NS, bool FUSED, bool ROWS = false, int NK = 0>
__global__ __launch_bounds__(512, 2) void gemm_i8_qload_kernel(const float* __restrict__ X, int M, int N, int K,
                                                               const unsigned* __restrict__ xparts, int nxparts,
                                                               const int8_t* __restrict__ B, Epilogue ep,
                                                               unsigned* parts) {
    using kh::quant::f32x4;
    constexpr int BK = 64, BN = 128 * NB, WN = 4, kWaves = 8, D = NS - 1;
    constexpr int kLdsA = kQlBM * BK;
    constexpr int kStage = kLdsA + BN * BK;
    constexpr int kBInst = BN / 16 / kWaves;  // 1 KB = 16 rows per LDS-DMA instruction
    constexpr int kLoads = kBInst + 2;        // loads per wave per stage
    static_assert(NS >= 2 && NS <= 5, "wait_loads_beyond covers up to 3 stages ahead");
    __shared__ __attribute__((aligned(1024))) int8_t lds[NS * kStage];
    __shared__ unsigned red[kWaves];
    // ROWS: the workgroup's 64 row scales (quantize.py:67-68 per row).
    __shared__ double row_s[ROWS ? kQlBM : 1];
    __shared__ float row_rf[ROWS ? kQlBM : 1];
    __shared__ unsigned row_flags[ROWS ? kQlBM : 1];

    const int tiles_n = N / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    auto swz = [](int r) { return (r >> 2) & 3; };
    // A: 8 floats of row t / 8 at k = 8 (t % 8) of each step; their codes go
    // to bytes 8 (t % 2) of chunk (t % 8) / 2.
    const int arow = tid >> 3, aq = tid & 7;

    kh::quant::Scale sc;
    if constexpr (!ROWS) {
        // The tensor's scale (quantize.py:67-68), the same in every workgroup.
        sc = kh::quant::make_scale(kh::quant::block_reduce_partials(xparts, nxparts, red));
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            if (ep.qscale) *ep.qscale = sc.s;
            if (sc.bad) kh::quant::flag_nonfinite(ep.fault);
        }
    } else {
        // Row r's scale from the producer's nxparts (<= 16) words of row r,
        // all issued at once through one resource for the workgroup's rows
        // (a resource per lane would be a loop over the lanes); indices past
        // the row read its last word again, which leaves the maximum
        // unchanged.  The tn == 0 workgroups report the scales.
        if (tid < kQlBM) {
            const int64_t gr = (int64_t)tm * kQlBM + tid;
            const __amdgpu_buffer_rsrc_t rp =
                make_rsrc(xparts + (int64_t)tm * kQlBM * nxparts, (uint32_t)(kQlBM * nxparts) * 4u);
            unsigned w[16];
#pragma unroll
            for (int p = 0; p < 16; ++p)
                w[p] = __builtin_amdgcn_raw_buffer_load_b32(rp, (tid * nxparts + min(p, nxparts - 1)) * 4, 0, 0);
            unsigned mb = 0;
#pragma unroll
            for (int p = 0; p < 16; ++p) mb = max(mb, w[p]);
            const kh::quant::Scale s = kh::quant::make_scale(mb);
            row_s[tid] = s.s;
            row_rf[tid] = s.rf;
            row_flags[tid] = (s.fast ? 1u : 0u) | (s.bad ? 2u : 0u);
            if (tn == 0) {
                if (ep.qscale) ep.qscale[gr] = s.s;
                if (s.bad) kh::quant::flag_nonfinite(ep.fault);
            }
        }
        __syncthreads();
        sc.s = row_s[arow];
        sc.rf = row_rf[arow];
        sc.fast = (row_flags[arow] & 1u) != 0;
        sc.bad = (row_flags[arow] & 2u) != 0;
    }

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(X + (int64_t)tm * kQlBM * K, (uint32_t)kQlBM * (uint32_t)K * 4u);
    const int a_voff = (arow * K + aq * 8) * 4;
    const int a_lds = arow * BK + (((aq >> 1) ^ swz(arow)) << 4) + 8 * (aq & 1);
    // B: instruction i of this wave fills rows (wave kBInst + i) 16 + l / 4,
    // slot chunk l % 4 (the ping-pong kernel's LDS-DMA).
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + (int64_t)tn * BN * K, (uint32_t)BN * (uint32_t)K);
    const int lr = lane >> 2, lc = lane & 3;
    int b_voff[kBInst];
#pragma unroll
    for (int i = 0; i < kBInst; ++i) {
        const int r = (wave * kBInst + i) * 16 + lr;
        b_voff[i] = r * K + ((lc ^ swz(r)) << 4);
    }
    auto issue = [&](int kt, f32x4 (&xa)[2]) {
        int8_t* base = lds + (kt % NS) * kStage + kLdsA;
#pragma unroll
        for (int i = 0; i < kBInst; ++i) lds_dma16(rb, base + (wave * kBInst + i) * 1024, b_voff[i], kt * BK);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            xa[h] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff + 16 * h, kt * BK * 4, 0));
    };

    // Fragments (as the ping-pong kernel): lane l reads 16 bytes of row
    // r + l % 32 at chunk 2s + l / 32.
    const int fr = lane & 31, fh = lane >> 5;
    const int ar = wm * 32 + fr;
    const int a_off = ar * BK + ((fh ^ swz(ar)) << 4);
    int b_off[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int r = wn * 32 * NB + b * 32 + fr;
        b_off[b] = kLdsA + r * BK + ((fh ^ swz(r)) << 4);
    }
    i32x16 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = i32x16{0};
    ColEpi ce[NB];  // requested before the main loop
#pragma unroll
    for (int b = 0; b < NB; ++b) ce[b] = col_epi(ep, (int64_t)tn * BN + wn * 32 * NB + b * 32 + fr);

    const int nk = NK ? NK : K / BK;
    f32x4 xa[D][2];
#pragma unroll
    for (int s = 0; s < D; ++s)
        if (s < nk) issue(s, xa[s]);
    // Unrolled whole where the step count is fixed (NK), not otherwise.
    constexpr int kOuter = NK ? (NK + D - 1) / D : 1;
#pragma unroll kOuter
    for (int k0 = 0; k0 < nk; k0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int k = k0 + j;
            if (k >= nk) break;
            int8_t* stage = lds + (k % NS) * kStage;
            wait_loads_beyond<kLoads>(min(D - 1, nk - 1 - k));  // this wave's A and B of step k landed
            const unsigned c0 = kh::quant::pack4(xa[j][0], sc), c1 = kh::quant::pack4(xa[j][1], sc);
            const unsigned st_addr = (unsigned)(uintptr_t)(__attribute__((address_space(3))) int8_t*)stage;
            // Inline LDS accesses: as plain ones the compiler would wait for
            // every LDS-DMA in flight (the later steps' B) before each.
            asm volatile("ds_write_b64 %0, %1" : : "v"(st_addr + a_lds), "v"(u32x2{c0, c1}) : "memory");
            __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            i32x4 fa[2], fb[2][NB];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                asm volatile("ds_read_b128 %0, %1" : "=v"(fa[s]) : "v"(st_addr + (a_off ^ (s << 5))) : "memory");
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    asm volatile("ds_read_b128 %0, %1" : "=v"(fb[s][b]) : "v"(st_addr + (b_off[b] ^ (s << 5))) : "memory");
            }
            __builtin_amdgcn_sched_barrier(0);
            if (k + D < nk) issue(k + D, xa[j]);
            __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));  // the fragments in registers
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s], fb[s][b], acc[b], 0, 0, 0);
            }
        }
    }

    unsigned mx = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if constexpr (ROWS)
            mx = max(mx, store_block32_full<FUSED, kh::quant::kOutStore, true>(
                             ep, (int64_t)tm * kQlBM + wm * 32, (int64_t)tn * BN + wn * 32 * NB + b * 32, N, lane,
                             0.0, acc[b], sc, ce[b], row_s, wm * 32));
        else
            mx = max(mx, store_block32_full<FUSED, kh::quant::kOutStore>(ep, (int64_t)tm * kQlBM + wm * 32,
                                                                          (int64_t)tn * BN + wn * 32 * NB + b * 32, N,
                                                                          lane, sc.s, acc[b], sc, ce[b]));
        __builtin_amdgcn_sched_barrier(0);
    }
    if (parts) {
        // Per-workgroup max |out| bits, for a following per-tensor quantize.
        mx = kh::quant::wave_max(mx);
        __syncthreads();  // red's scale reduction is read by every wave before this point
        if (lane == 0) red[wave] = mx;
        __syncthreads();
        if (tid == 0) {
            unsigned m = red[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) m = max(m, red[w]);
            parts[blockIdx.x] = m;
        }
    }
}

// ---------------------------------------------------------------------------
// Per-row (per-token) producer quantize: an int8 Linear's epilogue (bias,
// GELU) quantized per row inside the GEMM, the fp32 result never written
// (kh_gemm_i8_quant_rows: quantize.py:50-70 applied to each row of qlinear's
// output, quantize.py:115-144).  A row's scale needs all N of its values, so
// a workgroup owns 32 whole rows and keeps their results in registers: the
// weight streams through LDS in units of 256 columns x 128 bytes of K
// (LDS-DMA, 128 contiguous bytes per row, a ring of four units), each of the
// 8 waves multiplies its 32 columns of the unit (v_mfma_i32_32x32x32_i8,
// activation fragments held in registers), and after a chunk's last unit
// turns its 32 x 32 accumulators into the epilogue's values (the fp32
// epilogue of store_block32_full with per-row scales, then GELU), kept in
// registers.  The rows' absmax is then reduced across the lanes and waves
// (LDS) and the same registers are quantized with each row's scale.
// ---------------------------------------------------------------------------
constexpr int kRqRows = 32, kRqWaves = 8, kRqCols = 256, kRqSlab = 128, kRqRing = 4;

template <bool GELU, int NC, int KS>
__global__ __launch_bounds__(kRqWaves * 64, 2) void gemm_i8_quant_rows_kernel(const int8_t* __restrict__ A,
                                                                              const int8_t* __restrict__ B, int M,
                                                                              int N, int K, Epilogue ep) {
    constexpr int kSlabs = KS / 4;  // 128-byte k-slabs per chunk of 256 columns
    constexpr int kUnits = NC * kSlabs;
    constexpr int kAhead = kRqRing - 1;
    static_assert(KS % 4 == 0, "K must be a multiple of 128");
    __shared__ __attribute__((aligned(1024))) int8_t b_lds[kRqRing][kRqCols * kRqSlab];
    __shared__ unsigned red[kRqWaves][kRqRows];
    __shared__ double row_sa[kRqWaves][kRqRows];  // each wave's own copy
    __shared__ double row_s[kRqRows];
    __shared__ float row_rf[kRqRows];
    __shared__ unsigned row_fl[kRqRows];  // bit 0: fast path allowed, bit 1: non-finite
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int fr = lane & 31, fh = lane >> 5;
    const int m0 = blockIdx.x * kRqRows;
    const int rows_valid = min(kRqRows, M - m0);
    // Rows past M read zeros (buffer bound); their codes are dropped below.
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A + (int64_t)m0 * K, (uint32_t)rows_valid * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    // Row r of a unit holds its 8 granules of 16 bytes with granule g in slot
    // g ^ swz(r): a fragment read (16 consecutive rows, one granule) then
    // hits 16 distinct 16-byte slots of 256 bytes.
    auto swz = [](int r) { return (r >> 1) & 7; };

    // Unit u = (chunk u / kSlabs, slab u % kSlabs): this wave's 32 rows of
    // it, 8 rows (of 128 bytes) per LDS-DMA instruction.
    const int dr = lane >> 3, dg = lane & 7;
    auto issue = [&](int u) {
        const int c = u / kSlabs, sl = u % kSlabs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 32 * wave + 8 * i + dr;
            lds_dma16(rb, b_lds[u % kRqRing] + (32 * wave + 8 * i) * kRqSlab,
                      (kRqCols * c + r) * K + ((dg ^ swz(r)) << 4), kRqSlab * sl);
        }
    };
    // The loads in the order they are needed: row fr's activation scale
    // (written to LDS once unit 0 has landed), the first units, the
    // activation fragments (substep t: lane l supplies k = 32 t + 16 (l / 32)
    // .. + 15 of activation row l % 32, as of weight column l % 32 of its
    // block) and the epilogue's column operands (chunk c: column 256 c + 32
    // wave + fr).
    const double my_sa = ep.sa[ep.sa_per_row ? min(m0 + fr, M - 1) : 0];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kAhead && u < kUnits; ++u) issue(u);
    __builtin_amdgcn_sched_barrier(0);
    i32x4 af[KS];
#pragma unroll
    for (int t = 0; t < KS; ++t)
        af[t] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, fr * K + 16 * fh, 32 * t, 0));
    double sbj[NC];
    float bj[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int j = kRqCols * c + 32 * wave + fr;
        sbj[c] = ep.sb[ep.sb_per_col ? j : 0];
        bj[c] = ep.bias ? ep.bias[j] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    // The LDS this wave touches while its LDS-DMAs are in flight -- its units'
    // rows and its copy of the row scales -- is accessed by inline ds_read /
    // ds_write with explicit waits: as plain LDS accesses the compiler would
    // wait for every LDS-DMA in flight (the next units') before each.
    const unsigned sa_lds = (unsigned)(uintptr_t)(__attribute__((address_space(3))) double*)row_sa[wave];

    const int br = 32 * wave + fr;
    const int b_off = br * kRqSlab;
    float g[NC][16];
    unsigned mx[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) mx[r] = 0;
    // Chunk c's values (value r of the block is row 4 fh + 8 (r / 4) + r % 4)
    // in four groups of four rows, each with its four rows' scales.
    i32x16 acc[2];  // chunk c accumulates in acc[c % 2]
    auto finish = [&](int c, int g4) {
        double s4[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            asm volatile("ds_read_b64 %0, %1" : "=v"(s4[rr]) : "v"(sa_lds + 8 * (4 * fh + 8 * g4 + rr)) : "memory");
        __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) s4[rr] = s4[rr] * sbj[c];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int r = 4 * g4 + rr;
            float y = (float)((double)acc[c & 1][r] * s4[rr]);
            if (ep.bias) y = y + bj[c];
            if (GELU) y = kh::gelu(y);
            g[c][r] = y;
            mx[r] = max(mx[r], kh::abs_bits32(y));
        }
    };
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
        // This wave's loads of unit u have landed (those of the units after
        // it, 4 instructions each, may be in flight).  A wave reads only the
        // rows of a unit it loaded itself, so the waves need no barrier
        // here and drift apart (one's MFMAs overlap another's epilogue).
        if (u + 2 < kUnits) __builtin_amdgcn_s_waitcnt(wait_imm(8, 15));
        else if (u + 1 < kUnits) __builtin_amdgcn_s_waitcnt(wait_imm(4, 15));
        else __builtin_amdgcn_s_waitcnt(wait_imm(0, 15));
        asm volatile("" ::: "memory");  // the unit's LDS reads stay after the wait
        if (u == 0 && fh == 0) asm volatile("ds_write_b64 %0, %1" : : "v"(sa_lds + 8 * fr), "v"(my_sa) : "memory");
        // The unit's fragments, then (the reads issued) slot (u + 3) % 4 --
        // read by this wave in step u - 1 -- takes unit u + 3.
        const int8_t* base = b_lds[u % kRqRing] + b_off;
        const int c = u / kSlabs, sl = u % kSlabs;
        // (Inline ds_read_b128: read as plain LDS loads, the compiler would
        // wait for every LDS-DMA in flight -- the next units' -- before them;
        // the explicit wait below covers these four.)
        i32x4 bfr[4];
        const unsigned lds_row = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)base;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            asm volatile("ds_read_b128 %0, %1"
                         : "=v"(bfr[q])
                         : "v"(lds_row + (((2 * q + fh) ^ swz(br)) << 4))
                         : "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (u + kAhead < kUnits) issue(u + kAhead);
        __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));  // the four fragments in registers
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            acc[c & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[4 * sl + q], bfr[q],
                                                               sl == 0 && q == 0 ? i32x16{0} : acc[c & 1], 0, 0, 0);
        // The previous chunk's values, spread over this chunk's units (group
        // g4 in unit g4 kSlabs / 4) so that the epilogue's arithmetic runs
        // while the next units' weights are in flight.
        if (c > 0) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
                if (g4 * kSlabs / 4 == sl) finish(c - 1, g4);
        }
    }
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) finish(NC - 1, g4);

    // Each row's largest |value| bits (NaN and +-inf above every finite
    // value): over the lane's chunks, the 32 lanes of its half, the waves.
#pragma unroll
    for (int r = 0; r < 16; ++r) mx[r] = kh::lanes::half_max(mx[r]);
    if (fr == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave][4 * fh + 8 * (r >> 2) + (r & 3)] = mx[r];
    }
    __syncthreads();
    if (tid < kRqRows) {
        unsigned m = red[0][tid];
#pragma unroll
        for (int w = 1; w < kRqWaves; ++w) m = max(m, red[w][tid]);
        const kh::quant::Scale sc = kh::quant::make_scale(m);
        row_s[tid] = sc.s;
        row_rf[tid] = sc.rf;
        row_fl[tid] = (sc.fast ? 1u : 0u) | (sc.bad ? 2u : 0u);
        if (tid < rows_valid) {
            ep.qscale[m0 + tid] = sc.s;
            if (sc.bad) kh::quant::flag_nonfinite(ep.fault);
        }
    }
    __syncthreads();
    double rs[16];
    float rrf[16];
    bool all_fast = true;
    unsigned rbad = 0;  // bit r: row of value r non-finite
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 4 * fh + 8 * (r >> 2) + (r & 3);
        rs[r] = row_s[row];
        rrf[r] = row_rf[row];
        const unsigned f = row_fl[row];
        all_fast = all_fast && (f & 1u);
        rbad |= ((f >> 1) & 1u) << r;
    }
    // quant_one with each row's scale: the fast path where every row of the
    // lane allows it and each value is decisive, the exact one otherwise.
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(ep.q + (int64_t)m0 * N, (uint32_t)rows_valid * (uint32_t)N);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        unsigned cq[16];
        bool ok = all_fast;
#pragma unroll
        for (int r = 0; r < 16; ++r) cq[r] = kh::quant::quant_fast(g[c][r], rrf[r], ok);
        if (!ok) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                cq[r] = ((rbad >> r) & 1u) ? 0u : (unsigned)kh::quant::quant_exact(g[c][r], rs[r]);
        }
        store_codes_block32(rq, N, lane, cq, kRqCols * c + 32 * wave);
    }
}

// N = 256 NC (NC = 2, 4, 6) and K = 32 KS (KS = 8, 12): the C4 model's
// per-token fc1 (K = 384, N = 1536) and the shapes around it.
bool quant_rows_fits(const int8_t* A, const int8_t* B, const int8_t* q, int64_t M, int64_t N, int64_t K) {
    return M >= 1 && (N == 512 || N == 1024 || N == 1536) && (K == 256 || K == 384) && kh::aligned(A, 16) &&
           kh::aligned(B, 16) && kh::aligned(q, 4) && (M + kRqRows) * K <= 0x7FFFFFFFLL &&
           (M + kRqRows) * N <= 0x7FFFFFFFLL;
}

template <bool GELU, int NC>
void launch_quant_rows_nc(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                          const Epilogue& ep) {
    const unsigned grid = (unsigned)((M + kRqRows - 1) / kRqRows);
    if (K == 256)
        gemm_i8_quant_rows_kernel<GELU, NC, 8><<<grid, kRqWaves * 64, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
    else
        gemm_i8_quant_rows_kernel<GELU, NC, 12><<<grid, kRqWaves * 64, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
}

template <bool GELU>
void launch_quant_rows_act(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                           const Epilogue& ep) {
    if (N == 512)
        launch_quant_rows_nc<GELU, 2>(d, A, B, M, N, K, ep);
    else if (N == 1024)
        launch_quant_rows_nc<GELU, 4>(d, A, B, M, N, K, ep);
    else
        launch_quant_rows_nc<GELU, 6>(d, A, B, M, N, K, ep);
}

int launch_quant_rows(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                      const Epilogue& ep) {
    if (ep.act == kActGelu)
        launch_quant_rows_act<true>(d, A, B, M, N, K, ep);
    else
        launch_quant_rows_act<false>(d, A, B, M, N, K, ep);
    return kh::launch_status("gemm_i8_quant_rows");
}

// ---------------------------------------------------------------------------
// Skinny GEMM for decode-style and small shapes (M <= 64): weight streaming.
//
// A workgroup owns 16 output columns for all M rows; its SKW waves split K,
// each streaming its slice of those 16 packed weight rows (16 B per lane per
// 64-k step) through v_mfma_i32_16x16x64_i8 with up to two 16-row tiles of
// activations.  Where the slice is one chunk of 4 or 8 steps (K = 2048 or
// 4096) and a workgroup has one column tile, the weights are read whole rows
// at a time (2 rows x 512 B per wave instruction at K = 4096, the pattern of
// a plain streaming read) and rearranged into B fragments through the wave's
// own LDS region; otherwise each load is one B fragment (16 rows x 64 B).  Each wave takes its slice in chunks of C steps (8 where the
// slice allows) and issues a chunk's loads, the activations (its first batch
// of them) and the epilogue's operands first and then the weights, before its
// first MFMA (scheduling barriers keep the compiler from interleaving them
// with the MFMAs' waits), so the HBM stream and the L2-resident activations
// are in flight together; loads return in issue order, so activations issued
// behind the weights would arrive only after the last weight byte (M = 32,
// N = 4096: 12.28 -> 11.67 us per kh_linear_i8 call).  Rows >= M read zeros: their buffer offsets fall past the activation
// resource, whose loads return 0.  The waves' partial int32 accumulators are
// summed through LDS (integer sums are exact in any order) and the first MT
// waves apply the epilogue, one 16-row tile each.  Bound: HBM bytes of the
// weight, N*K, plus the activations (L2 resident) and the output.
// ---------------------------------------------------------------------------
typedef int i32x4v __attribute__((ext_vector_type(4)));
constexpr int kSkinnyWaves = 8;

template <int MT, int NT, int C, bool ONE, bool LEAN = false>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_i8_skinny_kernel(const int8_t* __restrict__ A,
                                                                           const int8_t* __restrict__ B, int M,
                                                                           int N, int K, int kslice, Epilogue ep) {
    static_assert(MT * NT <= kSkinnyWaves, "one epilogue wave per 16x16 tile");
    __shared__ i32x4v red[kSkinnyWaves][MT * NT][64];
    // TP: the wave's weight slice is read whole rows at a time (16 / C rows
    // x 64 C bytes per instruction) and turned into B fragments through the
    // wave's own LDS region (C KiB: one pass of full-wave writes, then the
    // fragment reads).
    constexpr bool TP = ONE && NT == 1 && MT <= 2 && (C == 4 || C == 8);
    __shared__ i32x4v wt[TP ? kSkinnyWaves : 1][TP ? C : 1][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16 * NT;
    const int kg = (lane >> 4) * 16;
    // The launch guarantees kslice % (512 * C) == 0 and kslice > 0; saying so
    // lets the compiler load every kernel argument before the first weight
    // load instead of after a loop-skip branch.
    __builtin_assume(kslice >= 64 * kSkinnyWaves * C);
    // Activation loads in batches of up to 4 steps, each batch issued whole
    // before its MFMAs (all C at once measured slower at N = 11008).
    constexpr int AC = C < 4 ? C : 4;
    // Split K: workgroup (x, y) sums k in [y kslice, (y + 1) kslice) (kslice
    // = K without a split) and writes its int32 sums as partial y.
    const int kper = kslice / kSkinnyWaves;  // a multiple of 64 * C; exactly 64 * C when ONE
    const int k_begin = blockIdx.y * kslice + wave * kper;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    int b_off[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) b_off[u] = min(n0 + u * 16 + (lane & 15), N - 1) * K + kg;
    int a_off[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        a_off[t] = (t * 16 + (lane & 15)) * K + kg;
        // Kept in a register from here: recomputed later, the offset was
        // built from a register the compiler shared with a loaded epilogue
        // operand, and waited for every load in flight.
        asm volatile("" : "+v"(a_off[t]));
    }

    i32x4v acc[MT][NT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int u = 0; u < NT; ++u) acc[t][u] = i32x4v{0, 0, 0, 0};
    // The epilogue's operands (scales, bias, residual), loaded by the waves
    // that finish the tiles while the weights stream in, rather than a
    // dependent round trip after the reduction.
    const int et = wave / NT;
    const int64_t ej = n0 + (wave % NT) * 16 + (lane & 15);
    const int64_t ejc = min(ej, (int64_t)N - 1);
    double sbj = 0.0, sai[4] = {0.0, 0.0, 0.0, 0.0};
    float bj = 0.0f, res[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto prefetch_epilogue = [&]() {
        if (wave >= MT * NT) return;
        sbj = ep.sb ? ep.sb[ep.sb_per_col ? ejc : 0] : 0.0;
        bj = ep.bias ? ep.bias[ejc] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t i = min((int64_t)(et * 16 + 4 * (lane >> 4) + r), (int64_t)M - 1);
            sai[r] = ep.out ? ep.sa[ep.sa_per_row ? i : 0] : 0.0;
            res[r] = ep.residual ? ep.residual[i * N + ejc] : 0.0f;
        }
    };
    auto chunk_tp = [&](int k0) {
        constexpr int R = 16 / C;  // rows per load instruction
        // The activation steps, all ahead of the MFMAs, or with LEAN (two
        // row tiles on a grid of more than one workgroup per CU) four at a
        // time: 144 -> 114 VGPRs for two row tiles, two workgroups per CU.
        // Issued before the weights, with the epilogue's operands: loads
        // return in issue order, so behind the weights these L2 hits would
        // arrive only after the last weight byte.
        constexpr int AB = LEAN && C > 4 ? 4 : C;
        i32x4v a[MT][C];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int c = 0; c < AB; ++c) a[t][c] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t], k0 + 64 * c, 0);
        prefetch_epilogue();
        __builtin_amdgcn_sched_barrier(0);
        i32x4v b[C];
        const int ch = lane % (4 * C);  // the 16-byte chunk of its rows this lane reads
#pragma unroll
        for (int i = 0; i < C; ++i)
            b[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, min(n0 + i * R + lane / (4 * C), N - 1) * K + ch * 16,
                                                         k0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // Slot of fragment lane l in step st's 1 KiB block: l with bits 0-1
        // XORed by l / 16 and bits 2-3 by st, so a write quarter (one row, 4
        // steps x 4 chunks) and a read quarter (16 rows, one chunk) each
        // cover the 16 distinct 16-byte bank groups.
        auto slot = [](int l, int st) { return l ^ ((l >> 4) & 3) ^ ((st & 3) << 2); };
        const int st = ch >> 2, q = ch & 3;
        i32x4v bf[C];
#pragma unroll
        for (int i = 0; i < C; ++i) wt[wave][st][slot(i * R + lane / (4 * C) + 16 * q, st)] = b[i];
        asm volatile("" ::: "memory");
#pragma unroll
        for (int c = 0; c < C; ++c) bf[c] = wt[wave][c][slot(lane, c)];
        asm volatile("" ::: "memory");
#pragma unroll
        for (int c = 0; c < AB; ++c)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[t][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t][c], bf[c], acc[t][0], 0, 0, 0);
        if constexpr (AB < C) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = AB; c < C; ++c)
                    a[t][c] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t], k0 + 64 * c, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = AB; c < C; ++c)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t][c], bf[c], acc[t][0], 0, 0, 0);
        }
    };
    auto chunk = [&](int k0) {
        // The first batch of activation steps (and, for a single chunk, the
        // epilogue's operands) ahead of the weights: loads return in issue
        // order, so these L2 hits would otherwise wait for the weight stream.
        i32x4v a[MT][AC];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int c = 0; c < AC; ++c) a[t][c] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t], k0 + 64 * c, 0);
        if constexpr (ONE) prefetch_epilogue();
        __builtin_amdgcn_sched_barrier(0);
        i32x4v b[NT][C];
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
            for (int c = 0; c < C; ++c) b[u][c] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[u], k0 + 64 * c, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c0 = 0; c0 < C; c0 += AC) {
            if (c0 > 0) {
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int c = 0; c < AC; ++c)
                        a[t][c] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t], k0 + 64 * (c0 + c), 0);
            }
            // All of the batch's loads ahead of its MFMAs (left to itself the
            // scheduler issues each load just before its MFMA: one L2 round
            // trip per step).
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < AC; ++c)
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int u = 0; u < NT; ++u)
                        acc[t][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t][c], b[u][c0 + c], acc[t][u], 0, 0, 0);
        }
    };
    // A wave's whole slice as one chunk where it fits (measured ~1 us faster
    // than the same loads under a loop, even one that runs once).
    if constexpr (TP) {
        chunk_tp(k_begin);
    } else if constexpr (ONE) {
        chunk(k_begin);
    } else {
        prefetch_epilogue();
        for (int k0 = k_begin; k0 < k_begin + kper; k0 += 64 * C) chunk(k0);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int u = 0; u < NT; ++u) red[wave][t * NT + u][lane] = acc[t][u];
    __syncthreads();
    if (wave >= MT * NT) return;
    // Wave w finishes row tile w / NT of column tile w % NT (operands loaded
    // by prefetch_epilogue).  16x16 MFMA result layout: register r of lane l
    // holds row 4*(l/16) + r, column l%16.
    const int t = et;
    const int64_t j = ej;
    if (j >= N) return;
    i32x4v sum = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < kSkinnyWaves; ++w) sum += red[w][wave][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t i = t * 16 + 4 * (lane >> 4) + r;
        if (i >= M) continue;
        if (ep.acc) ep.acc[((int64_t)blockIdx.y * M + i) * N + j] = sum[r];
        if (ep.out) ep.out[i * N + j] = epilogue_finish(ep, sum[r], sai[r] * sbj, bj, res[r]);
    }
}

// The split-K partials [S, M, N] (int32) summed -- exact in any order -- and
// the epilogue applied, as the unsplit kernel does (epilogue_store: the same
// sa_i * sb_j product, bias, activation and residual).
__global__ __launch_bounds__(256) void skinny_splitk_epilogue_kernel(const int32_t* __restrict__ P, int S, int M,
                                                                     int N, Epilogue ep) {
    const int64_t mn = (int64_t)M * N;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= mn) return;
    int32_t sum = 0;
    for (int s = 0; s < S; ++s) sum += P[s * mn + idx];
    epilogue_store(ep, idx / N, idx % N, N, sum);
}

bool skinny_fits(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K) {
    return M >= 1 && M <= 64 && K > 0 && K % (64 * kSkinnyWaves) == 0 && kh::aligned(A, 16) &&
           kh::aligned(B, 16) && M * K <= 0xFFFFFFFFLL && N * K <= 0xFFFFFFFFLL && N <= 0x7FFFFFFF;
}

// Split-K factor for a skinny launch: with one 16-column tile per workgroup a
// narrow N leaves CUs idle (N = 1024: 64 workgroups on 256 CUs, each
// streaming 16 K bytes of weight), so K is split over up to 8 workgroups per
// tile until the grid covers the CUs, keeping each wave at least one 64-k
// step, for K >= kSplitMinK (below it the weight is small enough that the
// second launch costs more than the idle CUs).  1 where the caller cannot
// allocate (the partials live in pooled device memory).
constexpr int64_t kSplitMinK = 8192;
int skinny_split(const kh::Device* d, int64_t N, int64_t K, bool may_alloc) {
    const int64_t tiles = (N + 15) / 16, steps = K / (64 * kSkinnyWaves);
    int S = 1;
    if (!may_alloc || K < kSplitMinK) return 1;
    while (S < 8 && tiles * S * 2 <= d->cus && steps % (2 * S) == 0) S *= 2;
    return S;
}

int launch_skinny(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                  const Epilogue& ep, bool may_alloc = true) {
    const int S = skinny_split(d, N, K, may_alloc);
    const int64_t kslice = K / S;
    const int64_t steps = kslice / (64 * kSkinnyWaves);  // 64-k steps per wave
    Epilogue eps = ep;
    void* parts = nullptr;
    if (S > 1) {
        int rc = kh_alloc((size_t)S * (size_t)(M * N) * sizeof(int32_t), &parts);
        if (rc) return rc;
        eps.out = nullptr;
        eps.acc = static_cast<int32_t*>(parts);
    }
    // One 16-column tile per workgroup.  (32 columns, each activation
    // fragment feeding two weight tiles, measured faster for two row tiles
    // at N = 11008 before the whole-row weight reads; with them the
    // 16-column tiles with LEAN loads are faster: 22.96 -> 21.37 us.)
    const bool lean = M > 16 && (N + 15) / 16 > d->cus;
    auto go = [&](auto mt, auto nt, auto c, auto one, auto leanv) {
        constexpr int NT = decltype(nt)::value;
        const dim3 blocks((unsigned)((N + 16 * NT - 1) / (16 * NT)), (unsigned)S);
        gemm_i8_skinny_kernel<decltype(mt)::value, NT, decltype(c)::value, decltype(one)::value,
                              decltype(leanv)::value><<<blocks, kSkinnyWaves * 64, 0, d->stream>>>(
            A, B, (int)M, (int)N, (int)K, (int)kslice, eps);
    };
    auto pick = [&](auto mt) {
        using T = std::true_type;
        using F = std::false_type;
        using N1 = std::integral_constant<int, 1>;
        switch (steps) {
            case 1: return go(mt, N1(), std::integral_constant<int, 1>(), T(), F());
            case 2: return go(mt, N1(), std::integral_constant<int, 2>(), T(), F());
            case 4: return go(mt, N1(), std::integral_constant<int, 4>(), T(), F());
            case 8:
                if (lean) return go(mt, N1(), std::integral_constant<int, 8>(), T(), T());
                return go(mt, N1(), std::integral_constant<int, 8>(), T(), F());
            case 16: return go(mt, N1(), std::integral_constant<int, 16>(), T(), F());
            default: break;
        }
        if (steps % 8 == 0) go(mt, N1(), std::integral_constant<int, 8>(), F(), F());
        else if (steps % 4 == 0) go(mt, N1(), std::integral_constant<int, 4>(), F(), F());
        else if (steps % 2 == 0) go(mt, N1(), std::integral_constant<int, 2>(), F(), F());
        else go(mt, N1(), std::integral_constant<int, 1>(), F(), F());
    };
    if (M <= 16) pick(std::integral_constant<int, 1>());
    else if (M <= 32) pick(std::integral_constant<int, 2>());
    else pick(std::integral_constant<int, 4>());
    int rc = kh::launch_status("gemm_i8_skinny");
    if (S > 1) {
        if (!rc) {
            skinny_splitk_epilogue_kernel<<<(unsigned)((M * N + 255) / 256), 256, 0, d->stream>>>(
                static_cast<const int32_t*>(parts), S, (int)M, (int)N, ep);
            rc = kh::launch_status("skinny_splitk_epilogue");
        }
        kh_free(parts);  // stream-ordered: reused only by work queued after the epilogue
    }
    return rc;
}

// ---------------------------------------------------------------------------
// Narrow-N GEMM: many rows, at most 128 output columns (C4's vocabulary head,
// M = 16384, N = 65, K = 384).  A 128 x 128 ping-pong tile there computes 128
// columns for 65 and gives the chip one tile per 128 rows (128 workgroups on
// 256 CUs).  Here a workgroup owns 64 rows and every column: the whole packed
// weight (N rows of K bytes, zero rows up to 16 NT) goes into LDS once; each
// 16-row group of A has two waves, each multiplying the group's
// v_mfma_i32_16x16x64_i8 A fragments (loaded straight from memory, all of
// them before the weight is staged) with half of the NT 16-column B
// fragments read from LDS, then applying the epilogue of the other kernels
// (epilogue_finish: the same binary64 dequantize, bias, activation and
// residual).  Bound: the A and output bytes, M K + 4 M N (C4's head: 8.47 ->
// 7.36 us against the 128 x 128 ping-pong tiles, graph-replayed; 6.44 us with
// every load unconditional and the weight's requested first).  LDS rows
// are K + 16 bytes apart, so the 16 rows of a fragment read fall on distinct
// banks.  Non-temporal output stores measured slower (7.93 us).
// ---------------------------------------------------------------------------
constexpr int kNarrowRows = 64;
constexpr int kNarrowMaxK = 512;
// Two waves per 16-row group, each with half of the column tiles: 8 waves
// per workgroup (7.36 us for the C4 head against 7.93 with one wave per
// group and all of its tiles).
constexpr int kNarrowWN = 2;

template <int NT, bool FUSED>
__global__ __launch_bounds__(256 * kNarrowWN) void gemm_i8_narrow_kernel(const int8_t* __restrict__ A,
                                                             const int8_t* __restrict__ B, int M, int N, int K,
                                                             Epilogue ep) {
    extern __shared__ __attribute__((aligned(16))) int8_t bs[];  // [16 NT][K + 16]
    // Chunks of 16 bytes of the weight per thread: 16 NT rows x K / 16 <= 32
    // chunks each, over the workgroup's threads.
    constexpr int kMaxChunks = (16 * NT * (kNarrowMaxK / 16) + 256 * kNarrowWN - 1) / (256 * kNarrowWN);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = K >> 6;  // 64-k steps, 1..8
    const int kc16 = K >> 4;
    const int ldb = K + 16;
    constexpr int NTW = (NT + kNarrowWN - 1) / kNarrowWN;  // column tiles per wave
    const int m0 = blockIdx.x * kNarrowRows + (wave % 4) * 16;
    const int t0 = (wave / 4) * NTW;
    // Every load before any is used, in the order they are needed (loads
    // return in issue order): the thread's chunks of the weight (rows >= N
    // read zero: buffer bound; L2-resident and staged into LDS first), the
    // epilogue's column and row operands, then the A fragments of all
    // k-steps (rows >= M read zero).  Every load is unconditional -- a chunk
    // or k-step past the end re-reads the last one (a cache hit, never used,
    // or stored again to the same LDS slot with the same bytes): loads under
    // a condition made the compiler wait for each one where the branches
    // join, one memory round trip per k-step.
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    const int chunks = 16 * NT * kc16;
    i32x4v bv[kMaxChunks];
    int bdst[kMaxChunks];
#pragma unroll
    for (int u = 0; u < kMaxChunks; ++u) {
        const int c = min(tid + 256 * kNarrowWN * u, chunks - 1);
        const int n = c / kc16, kc = c - n * kc16;
        bv[u] = __builtin_amdgcn_raw_buffer_load_b128(rb, n * K + kc * 16, 0, 0);
        bdst[u] = n * ldb + kc * 16;
    }
    double sbj[NT];
    float bj[NT];
#pragma unroll
    for (int tt = 0; tt < NTW; ++tt) {
        const int t = t0 + tt;
        const int jc = min(16 * t + (lane & 15), N - 1);
        sbj[tt] = ep.sb ? ep.sb[ep.sb_per_col ? jc : 0] : 0.0;
        bj[tt] = ep.bias ? ep.bias[jc] : 0.0f;
    }
    double sai[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        sai[r] = ep.out ? ep.sa[ep.sa_per_row ? min(m0 + 4 * (lane >> 4) + r, M - 1) : 0] : 0.0;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
    const int a_off = (m0 + (lane & 15)) * K + (lane >> 4) * 16;
    i32x4v a[kNarrowMaxK / 64];
#pragma unroll
    for (int s = 0; s < kNarrowMaxK / 64; ++s)
        a[s] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off, 64 * min(s, ks - 1), 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kMaxChunks; ++u) *reinterpret_cast<i32x4v*>(bs + bdst[u]) = bv[u];
    __syncthreads();
    i32x4v acc[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[t] = i32x4v{0, 0, 0, 0};
    const int8_t* bl = bs + (lane & 15) * ldb + (lane >> 4) * 16;
#pragma unroll
    for (int s = 0; s < kNarrowMaxK / 64; ++s) {
        if (s < ks) {
#pragma unroll
            for (int tt = 0; tt < NTW; ++tt)
                if (t0 + tt < NT)
                    acc[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        a[s], *reinterpret_cast<const i32x4v*>(bl + 16 * (t0 + tt) * ldb + 64 * s), acc[tt], 0, 0, 0);
        }
    }
    // 16x16 result layout: register r of lane l is row 4 (l / 16) + r,
    // column l % 16 of the tile.
#pragma unroll
    for (int tt = 0; tt < NTW; ++tt) {
        const int t = t0 + tt;
        const int64_t j = 16 * t + (lane & 15);
        if (t >= NT || j >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t i = m0 + 4 * (lane >> 4) + r;
            if (i >= M) continue;
            if (ep.acc) ep.acc[i * N + j] = acc[tt][r];
            if (ep.out) {
                const float resid = (FUSED && ep.residual) ? ep.residual[i * N + j] : 0.0f;
                ep.out[i * N + j] = epilogue_finish<FUSED>(ep, acc[tt][r], sai[r] * sbj[tt], bj[tt], resid);
            }
        }
    }
}

// The weight's LDS copy (16 NT rows of K + 16 bytes) within 64 KiB, 32-bit
// offsets into A, and enough rows for the chip (2048 rows: 32 workgroups).
bool narrow_fits(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K) {
    const int64_t lds = ((N + 15) / 16) * 16 * (K + 16);
    return N >= 1 && N <= 128 && M >= 2048 && K >= 64 && K <= kNarrowMaxK && K % 64 == 0 && lds <= 65536 &&
           kh::aligned(A, 16) && kh::aligned(B, 16) && (M + kNarrowRows) * K <= 0x7FFFFFFFLL;
}

int launch_narrow(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                  const Epilogue& ep) {
    const unsigned blocks = (unsigned)((M + kNarrowRows - 1) / kNarrowRows);
    const bool fused = ep.act != kActNone || ep.residual;
    auto go = [&](auto nt) {
        constexpr int NT = decltype(nt)::value;
        const size_t lds = (size_t)16 * NT * (K + 16);
        if (fused)
            gemm_i8_narrow_kernel<NT, true><<<blocks, 256 * kNarrowWN, lds, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
        else
            gemm_i8_narrow_kernel<NT, false><<<blocks, 256 * kNarrowWN, lds, d->stream>>>(A, B, (int)M, (int)N, (int)K, ep);
    };
    if (N <= 16) go(std::integral_constant<int, 1>());
    else if (N <= 32) go(std::integral_constant<int, 2>());
    else if (N <= 48) go(std::integral_constant<int, 3>());
    else if (N <= 64) go(std::integral_constant<int, 4>());
    else if (N <= 80) go(std::integral_constant<int, 5>());
    else if (N <= 96) go(std::integral_constant<int, 6>());
    else if (N <= 112) go(std::integral_constant<int, 7>());
    else go(std::integral_constant<int, 8>());
    return kh::launch_status("gemm_i8_narrow");
}

// fp32 outputs above this many bytes (half the MI355X's 256 MB last-level
// cache) are stored non-temporally: C3a's 256 MiB output streams, C4's
// outputs (at most fc1's 100.7 MB) take ordinary stores.
constexpr int64_t kStreamOutBytes = 128ll << 20;

template <int BM, int BN, int NS>
int launch_pingpong_cfg(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                        const Epilogue& ep, unsigned* parts, int* nparts, int mode) {
    using namespace kh::quant;
    const unsigned tiles = (unsigned)(((M + BM - 1) / BM) * ((N + BN - 1) / BN));
    // Tile rows per group of the XCD-banded walk: 2 for the 256x256 tile
    // (8192^3: 2320 TOPS against 2230-2260 with 4-8 rows and 2030 with 1 or
    // 32), 8 elsewhere (no measurable difference at C4's shapes).
    constexpr int group_m = (BM == 256 && BN == 256) ? 2 : 8;
    // Every tile full and the common epilogues: the full-tile kernels.
    const bool full = M % BM == 0 && N % BN == 0 && N <= (1 << 24) && !ep.acc;
    const bool fast = full && !ep.sa_per_row && (mode != kOutStore || ep.out) &&
                      (mode != kOutQuant || kh::aligned(ep.q, 4));
    const bool fast_rows = full && ep.sa_per_row && mode == kOutStore && ep.out;
    if (fast) {
        if constexpr (BM == 128 && BN == 128) {
            if (mode == kOutMaxOnly)
                gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutMaxOnly, kEpiFull>
                    <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
            else if (mode == kOutQuant)
                gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutQuant, kEpiFull>
                    <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, nullptr);
        }
        if (mode != kOutStore) {
            // launched above (launch_pingpong routes the quantize passes to the 128x128 tile)
        } else if (ep.act != kActNone || ep.residual)
            gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutStore, kEpiFull>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
        else
            gemm_i8_pingpong_kernel<BM, BN, NS, false, kOutStore, kEpiFull>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
        if (nparts) *nparts = (int)tiles;
        return kh::launch_status("gemm_i8_pingpong");
    }
    if (fast_rows) {
        if (ep.act != kActNone || ep.residual)
            gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutStore, kEpiFullRows>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
        else
            gemm_i8_pingpong_kernel<BM, BN, NS, false, kOutStore, kEpiFullRows>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
        if (nparts) *nparts = (int)tiles;
        return kh::launch_status("gemm_i8_pingpong");
    }
    if constexpr (BM == 128 && BN == 128) {
        if (mode == kOutMaxOnly)
            gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutMaxOnly>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
        else if (mode == kOutQuant)
            gemm_i8_pingpong_kernel<BM, BN, NS, true, kOutQuant>
                <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, nullptr);
    }
    if (mode != kOutStore) {
        // The quantize passes exist for the 128x128 tile only (launch_pingpong
        // routes them there; in the 256-row tiles the pass-1 epilogue spills).
    } else if (ep.act != kActNone || ep.residual)
        gemm_i8_pingpong_kernel<BM, BN, NS, true>
            <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
    else
        gemm_i8_pingpong_kernel<BM, BN, NS, false>
            <<<tiles, 512, 0, d->stream>>>(A, B, (int)M, (int)N, (int)K, group_m, ep, parts);
    if (nparts) *nparts = (int)tiles;
    return kh::launch_status("gemm_i8_pingpong");
}

// The largest tile that still gives the chip at least 1.5 tiles per CU;
// the smallest tile otherwise.  Short K (<= 512: a handful of K-steps, where
// writing the fp32 tile dominates) takes 128x128 tiles, several resident per
// CU, so one workgroup's epilogue overlaps another's main loop.  Short K gets
// a 3-stage ring.  The two passes of a fused quantize (mode kOutMaxOnly,
// then kOutQuant) both take 128x128 tiles.
int launch_pingpong(kh::Device* d, const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                    const Epilogue& ep_in, unsigned* parts = nullptr, int* nparts = nullptr,
                    int mode = kh::quant::kOutStore) {
    Epilogue ep = ep_in;
    ep.stream_out = M * N * (int64_t)sizeof(float) > kStreamOutBytes;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    const int64_t want = (int64_t)d->cus * 3 / 2;
    // At most two 128x128 tiles per CU: LDS holds two workgroups of a
    // 4-stage ring, one stage more in flight per K-step.
    const bool deep = tiles(128, 128) <= 2 * (int64_t)d->cus && K >= 192;
    if (K <= 512 || mode != kh::quant::kOutStore) {
        if (deep) return launch_pingpong_cfg<128, 128, 4>(d, A, B, M, N, K, ep, parts, nparts, mode);
        return launch_pingpong_cfg<128, 128, 3>(d, A, B, M, N, K, ep, parts, nparts, mode);
    }
    if (tiles(256, 256) >= want) {
        if (K >= 1024) return launch_pingpong_cfg<256, 256, 4>(d, A, B, M, N, K, ep, parts, nparts, mode);
        return launch_pingpong_cfg<256, 256, 3>(d, A, B, M, N, K, ep, parts, nparts, mode);
    }
    if (tiles(256, 128) >= want) return launch_pingpong_cfg<256, 128, 3>(d, A, B, M, N, K, ep, parts, nparts, mode);
    if (deep) return launch_pingpong_cfg<128, 128, 4>(d, A, B, M, N, K, ep, parts, nparts, mode);
    return launch_pingpong_cfg<128, 128, 3>(d, A, B, M, N, K, ep, parts, nparts, mode);
}

// True when the ping-pong kernel applies to this shape (any M and N; K a
// multiple of 64; 16-byte aligned operands; 32-bit offsets).
bool pingpong_fits(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K) {
    return M > 0 && N > 0 && K % 64 == 0 && K > 0 && kh::aligned(A, 16) && kh::aligned(B, 16) &&
           256 * K <= 0x7FFFFFFFLL && M <= 0x7FFFFFFF && N <= 0x7FFFFFFF &&
           ((M + 127) / 128) * ((N + 127) / 128) <= 0x7FFFFFFF;
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

// ---------------------------------------------------------------------------
// Decode Linear for one to three tokens (kh_linear_i8 with M <= 3): the
// per-token quantize of the fp32 activations is fused into the weight-
// streaming GEMV, so a decode step is one launch instead of two dependent
// ones.
//
// A workgroup (8 waves) owns 16 consecutive weight rows (output columns), 16K
// contiguous bytes, and reads them 8 KiB per load instruction -- the fastest
// streaming pattern measured (an MFMA operand layout, 16 rows x 64 B per
// wave instruction, read the same bytes ~20 % slower).  So lane t of
// instruction i holds 16 bytes of row i * (8192 / K) + t / (K / 16) at the
// k offset 16 * (t % (K / 16)), the same offset in every instruction; the
// products are VALU v_dot4_i32_i8 against the lane's 16 activation codes
// (read once from LDS), exact in int32 in any order.  Each row's lanes are
// whole waves: a wave sums its lanes in the VALU (for up to two tokens one
// wave_sum per partial, for MAXM = 4 token rows the transposed butterfly over
// half of the rows' partials at a time), the row's waves through LDS.  Each workgroup loads the fp32 activations first (L2-resident after
// the first workgroup), then issues all of its weight loads, so the
// in-order vmcnt wait for the activations does not wait for the weights;
// while the weights stream in it reduces each row's absmax (wave shuffles
// and an LDS table) and quantizes the row with the reference's arithmetic
// into LDS codes (workgroup 0 also writes the codes and scales to q_out /
// sx_out, the outputs kh_linear_i8 documents).  Groups with an undecided
// element take the exact path out of line, from memory.
// ---------------------------------------------------------------------------
template <int S, int MAXM>
__global__ __launch_bounds__(512) void linear_i8_decode_kernel(const float* __restrict__ x, int M,
                                                               const int8_t* __restrict__ B, int N,
                                                               const double* __restrict__ sb, int sb_per_col,
                                                               const float* __restrict__ bias,
                                                               float* __restrict__ out, int8_t* __restrict__ q_out,
                                                               double* __restrict__ sx_out,
                                                               unsigned* __restrict__ fault) {
    using namespace kh::quant;
    constexpr int W = 8, T = W * 64;
    constexpr int K = 512 * S;
    constexpr int XH = K / 4 / T;         // float4 of each activation row per thread
    constexpr int kLanesPerRow = K / 16;  // 16 weight bytes per lane
    constexpr int kRowsPerInst = T / kLanesPerRow;
    constexpr int kWavesPerRow = kLanesPerRow / 64;
    static_assert(XH >= 1 && MAXM * XH <= 32 && kRowsPerInst * S == 16 && kWavesPerRow >= 1, "shape");
    // More than two tokens: the partial products of half the wave's rows at
    // a time (MAXM * S / 2 per lane) summed by the transposed butterfly.
    constexpr bool kTransposed = MAXM > 2;
    constexpr int kHalfP = MAXM * S / 2;
    __shared__ __attribute__((aligned(16))) int8_t codes[MAXM * K];
    __shared__ unsigned rmax[W][MAXM];
    __shared__ int red[kTransposed ? 1 : W][MAXM][S];
    __shared__ int redt[kTransposed ? W : 1][2][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)M * (uint32_t)K * 4u);
    f32x4 xv[MAXM][XH];
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
#pragma unroll
        for (int h = 0; h < XH; ++h)
            xv[m][h] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (m * K + (tid + h * T) * 4) * 4, 0, 0));

    // The epilogue's column scale and bias (thread j < 16 * MAXM finishes
    // row j % 16 of token j / 16), in flight with the weights.  Every thread
    // loads them (16 addresses per workgroup), unconditionally and before the
    // weights: the in-order vmcnt wait for the activations then counts
    // exactly and does not wait for any weight load.
    const int erow = tid & 15;
    const int ecol = min((int)blockIdx.x * 16 + erow, N - 1);
    const double sbj = sb[sb_per_col ? ecol : 0];
    const float bj = bias ? bias[ecol] : 0.0f;
    // Rows past N read zeros (buffer-resource bound; the launch keeps
    // (N + 16) * K within 32 bits).
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    const uint32_t wbase = (uint32_t)blockIdx.x * 16u * (uint32_t)K + (uint32_t)tid * 16u;
    i32x4 b[S];
#pragma unroll
    for (int i = 0; i < S; ++i) b[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, wbase, i * 8192, 0);

#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        AbsMax am;
#pragma unroll
        for (int h = 0; h < XH; ++h) am.add4(xv[m][h]);
        const unsigned mb = wave_max(am.bits());
        if (lane == 0) rmax[wave][m] = mb;
    }
    __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
    __builtin_amdgcn_s_barrier();

    unsigned redo = 0;
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        if (m >= M) break;
        unsigned mb = rmax[0][m];
#pragma unroll
        for (int w = 1; w < W; ++w) mb = max(mb, rmax[w][m]);
        const Scale sc = make_scale(mb);
        if (blockIdx.x == 0 && tid == 0) {
            sx_out[m] = sc.s;
            if (sc.bad) flag_nonfinite(fault);
        }
#pragma unroll
        for (int h = 0; h < XH; ++h) {
            const int e4 = tid + h * T;
            bool ok = sc.fast;
            const unsigned w4 = pack4_fast(xv[m][h], sc.rf, ok);
            if (!ok) redo |= 1u << (m * XH + h);
            *reinterpret_cast<unsigned*>(codes + m * K + e4 * 4) = w4;
            if (blockIdx.x == 0) *reinterpret_cast<unsigned*>(q_out + (int64_t)m * K + e4 * 4) = w4;
        }
    }
    while (redo) {
        const int bit = __builtin_ctz(redo);
        redo &= redo - 1;
        const int m = bit / XH, h = bit % XH;
        unsigned mb = rmax[0][m];
        for (int w = 1; w < W; ++w) mb = max(mb, rmax[w][m]);
        const Scale sc = make_scale(mb);
        const int e4 = tid + h * T;
        const f32x4 vv =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (m * K + e4 * 4) * 4, 0, 0));
        const unsigned w4 = pack4(vv, sc);
        *reinterpret_cast<unsigned*>(codes + m * K + e4 * 4) = w4;
        if (blockIdx.x == 0) *reinterpret_cast<unsigned*>(q_out + (int64_t)m * K + e4 * 4) = w4;
    }
    __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
    __builtin_amdgcn_s_barrier();

    // Partial dot products: the lane's 16 codes of each token against its
    // 16 bytes of every row it loaded.
    const int kk = (tid % kLanesPerRow) * 16;
    i32x4 a[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
        a[m] = (m < M) ? *reinterpret_cast<const i32x4*>(codes + m * K + kk) : i32x4{0, 0, 0, 0};
    if constexpr (kTransposed) {
        // Value m * S / 2 + j of half h: token m against instruction
        // h * S / 2 + j (int32 sums are exact in any order).
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int p[kHalfP];
#pragma unroll
            for (int m = 0; m < MAXM; ++m)
#pragma unroll
                for (int j = 0; j < S / 2; ++j) {
                    int acc = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_sdot4(a[m][e], b[h * (S / 2) + j][e], acc, false);
                    p[m * (S / 2) + j] = acc;
                }
            kh::lanes::wave_sum_transposed(p, lane);
            redt[wave][h][lane] = p[0];
        }
    } else {
        int p[MAXM][S];
#pragma unroll
        for (int i = 0; i < S; ++i)
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
                p[m][i] = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) p[m][i] = __builtin_amdgcn_sdot4(a[m][e], b[i][e], p[m][i], false);
            }
        // Wave sums of all S * MAXM partials, in the VALU (independent chains
        // the compiler interleaves; int32 sums are exact in any order).
#pragma unroll
        for (int m = 0; m < MAXM; ++m)
#pragma unroll
            for (int i = 0; i < S; ++i) p[m][i] = kh::lanes::wave_sum(p[m][i]);
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MAXM; ++m)
#pragma unroll
                for (int i = 0; i < S; ++i) red[wave][m][i] = p[m][i];
        }
    }
    __syncthreads();
    if (tid >= 16 * MAXM) return;
    // Row erow of the workgroup came from instruction erow / kRowsPerInst,
    // waves [sub * kWavesPerRow, (sub + 1) * kWavesPerRow).
    const int m = tid >> 4;
    const int n = (int)blockIdx.x * 16 + erow;
    if (m >= M || n >= N) return;
    const int i = erow / kRowsPerInst, sub = erow % kRowsPerInst;
    int sum = 0;
    if constexpr (kTransposed) {
        const int h = i / (S / 2);
        const int l = kh::lanes::transposed_lane<kHalfP>(m * (S / 2) + i % (S / 2));
#pragma unroll
        for (int w = 0; w < kWavesPerRow; ++w) sum += redt[sub * kWavesPerRow + w][h][l];
    } else {
#pragma unroll
        for (int w = 0; w < kWavesPerRow; ++w) sum += red[sub * kWavesPerRow + w][m][i];
    }
    unsigned mb = rmax[0][m];
#pragma unroll
    for (int w = 1; w < W; ++w) mb = max(mb, rmax[w][m]);
    float y = (float)((double)sum * (make_scale(mb).s * sbj));
    if (bias) y = y + bj;
    out[(int64_t)m * N + n] = y;
}

template <int S>
int launch_decode(kh::Device* d, const float* x, int64_t M, const int8_t* B, int64_t N, const double* sb,
                  int sb_per_col, const float* bias, float* out, int8_t* q, double* sx) {
    const unsigned blocks = (unsigned)((N + 15) / 16);
    if (M == 1)
        linear_i8_decode_kernel<S, 1><<<blocks, 512, 0, d->stream>>>(x, (int)M, B, (int)N, sb, sb_per_col, bias, out, q,
                                                                      sx, d->fault);
    else if (M == 2)
        linear_i8_decode_kernel<S, 2><<<blocks, 512, 0, d->stream>>>(x, (int)M, B, (int)N, sb, sb_per_col, bias, out, q,
                                                                      sx, d->fault);
    else if constexpr (S <= 8) {
        if (M > 3) return kh::fail(KH_ERR_INVALID_ARG, "linear_i8_decode: more than three tokens");
        linear_i8_decode_kernel<S, 4><<<blocks, 512, 0, d->stream>>>(x, (int)M, B, (int)N, sb, sb_per_col, bias, out, q,
                                                                      sx, d->fault);
    } else {
        // The four-row kernel's activations do not fit its registers at this K.
        return kh::fail(KH_ERR_INVALID_ARG, "linear_i8_decode: three tokens need K <= 4096");
    }
    return kh::launch_status("linear_i8_decode");
}

// True when the fused decode kernel covers this call: one or two tokens
// with K = 2048, 4096 or 8192, three with K = 2048 or 4096.  Back to back
// against the two-launch path (N = 4096 / 11008, K = 4096): M = 3 8.1 / 12.6
// against 9.3 / 14.3 us; M = 4 8.4 / 15.9 against 9.4 / 15.0; M = 8 (the
// same design with 8 token rows) 11.9 / 23.4 against 9.8 / 15.7.
bool decode_fits(const float* x, int64_t M, int64_t K, const int8_t* B, int64_t N, const int8_t* q) {
    const bool k_ok = M <= 2 ? (K == 2048 || K == 4096 || K == 8192) : (K == 2048 || K == 4096);
    return M >= 1 && M <= 3 && k_ok && N >= 1 && (N + 16) * K <= 0xFFFFFFFFLL && kh::aligned(x, 16) &&
           kh::aligned(B, 16) && kh::aligned(q, 4);
}

// ---------------------------------------------------------------------------
// Small int8 Linear with a per-tensor activation scale in one launch
// (kh_linear_i8_tensor; config C1's x [64, 512]): quantize.py:50-70 on the
// whole of x, then the GEMM with the dequantize and bias fused.  x is at most
// kTensorSmallElems values, so every workgroup reads all of it (an L2 hit
// after the first few), reduces the absmax over the workgroup and writes the
// codes into LDS itself: no workgroup waits for another and there is no
// second launch.  The GEMM is the skinny kernel's: 16 output columns per
// workgroup, the 8 waves splitting K into C 64-k steps each, MT 16-row tiles
// of v_mfma_i32_16x16x64_i8 with the A fragments read from LDS (chunk j of
// row m at chunk j ^ (m & 15), so a fragment's 16 rows fall on distinct
// banks), partial sums reduced through LDS.  Each wave issues its share of
// x first and its weight fragments after it, so the in-order vmcnt wait for
// x does not wait for the weights.  Workgroup 0 writes the codes and the
// scale (the outputs kh_linear_i8_tensor documents); an undecided element
// takes the exact path inside pack4.
// ---------------------------------------------------------------------------
constexpr int kTensorSmallElems = 32768;

template <int MT, int C>
__global__ __launch_bounds__(512) void linear_i8_tensor_small_kernel(const float* __restrict__ x, int M,
                                                                     const int8_t* __restrict__ B, int N,
                                                                     const double* __restrict__ sb, int sb_per_col,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ out, int8_t* __restrict__ q_out,
                                                                     double* __restrict__ sx_out,
                                                                     unsigned* __restrict__ fault) {
    using namespace kh::quant;
    constexpr int W = kSkinnyWaves, T = W * 64;
    constexpr int K = 64 * W * C;
    constexpr int XH = kTensorSmallElems / 4 / T;  // float4 of x per thread at most
    __shared__ __attribute__((aligned(16))) int8_t codes[kTensorSmallElems];
    __shared__ i32x4v red[W][MT][64];
    __shared__ unsigned wmax[W];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * 16;
    const int nx4 = M * K / 4;  // float4 of x

    // x: float4 tid + T h (past the end: zeros from the resource bound).
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)nx4 * 16u);
    f32x4 xv[XH];
#pragma unroll
    for (int h = 0; h < XH; ++h)
        xv[h] = (h * T < nx4) ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (tid + h * T) * 16,
                                                                                                 0, 0))
                              : f32x4{0.f, 0.f, 0.f, 0.f};
    // The epilogue's column operands, then the weight fragments of this
    // wave's K slice (16 rows x 64 B per instruction; rows past N read row N-1).
    const int ej = min(n0 + (lane & 15), N - 1);
    const double sbj = sb[sb_per_col ? ej : 0];
    const float bj = bias ? bias[ej] : 0.0f;
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
    const int kg = (lane >> 4) * 16;
    const int k_begin = wave * 64 * C;
    i32x4v b[C];
#pragma unroll
    for (int c = 0; c < C; ++c) b[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, ej * K + kg, k_begin + 64 * c, 0);
    __builtin_amdgcn_sched_barrier(0);

    AbsMax am;
#pragma unroll
    for (int h = 0; h < XH; ++h) am.add4(xv[h]);
    const unsigned wb = wave_max(am.bits());
    if (lane == 0) wmax[wave] = wb;
    __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
    __builtin_amdgcn_s_barrier();
    unsigned mb = wmax[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mb = max(mb, wmax[w]);
    const Scale sc = make_scale(mb);
    if (blockIdx.x == 0 && tid == 0) {
        *sx_out = sc.s;
        if (sc.bad) flag_nonfinite(fault);
    }
    // Element 4 e4 is row e4 / (K / 4), column 4 (e4 % (K / 4)).
    auto code_at = [](int e4) {
        const int m = e4 / (K / 4), k4 = e4 % (K / 4);
        return m * K + ((((k4 >> 2) ^ (m & 15))) << 4) + ((k4 & 3) << 2);
    };
#pragma unroll
    for (int h = 0; h < XH; ++h) {
        const int e4 = tid + h * T;
        if (h * T < nx4 && e4 < nx4) {
            const unsigned w4 = pack4(xv[h], sc);
            *reinterpret_cast<unsigned*>(codes + code_at(e4)) = w4;
            if (blockIdx.x == 0) *reinterpret_cast<unsigned*>(q_out + (int64_t)e4 * 4) = w4;
        }
    }
    __builtin_amdgcn_s_waitcnt(wait_imm(63, 0));
    __builtin_amdgcn_s_barrier();

    // A fragments: lane l holds 16 codes of row 16 t + l % 16 (zero past M)
    // at k = k_begin + 64 c + 16 (l / 16).
    i32x4v acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = i32x4v{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int row = t * 16 + (lane & 15);
            i32x4v a = i32x4v{0, 0, 0, 0};
            if (row < M) a = *reinterpret_cast<const i32x4v*>(codes + code_at(row * (K / 4) + ((k_begin + 64 * c + kg) >> 2)));
            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[c], acc[t], 0, 0, 0);
        }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    if (wave >= MT) return;
    const int j = n0 + (lane & 15);
    if (j >= N) return;
    i32x4v sum = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < W; ++w) sum += red[w][wave][lane];
    // 16x16 MFMA result layout: register r of lane l holds row 4*(l/16) + r.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = wave * 16 + 4 * (lane >> 4) + r;
        if (i >= M) continue;
        float y = (float)((double)sum[r] * (sc.s * sbj));
        if (bias) y = y + bj;
        out[(int64_t)i * N + j] = y;
    }
}

// True when the one-launch per-tensor Linear covers this call.
bool tensor_small_fits(const float* x, int64_t M, int64_t K, const int8_t* B, int64_t N, const int8_t* q) {
    return M >= 1 && M <= 64 && (K == 512 || K == 1024 || K == 2048 || K == 4096) && M * K <= kTensorSmallElems &&
           N >= 1 &&
           N * K <= 0xFFFFFFFFLL && N <= 0x7FFFFFFF && kh::aligned(x, 16) && kh::aligned(B, 16) && kh::aligned(q, 4);
}

int launch_tensor_small(kh::Device* d, const float* x, int64_t M, int64_t K, const int8_t* B, int64_t N,
                        const double* sb, int sb_per_col, const float* bias, float* out, int8_t* q, double* sx) {
    const unsigned blocks = (unsigned)((N + 15) / 16);
    auto go = [&](auto mt, auto c) {
        linear_i8_tensor_small_kernel<decltype(mt)::value, decltype(c)::value><<<blocks, 512, 0, d->stream>>>(
            x, (int)M, B, (int)N, sb, sb_per_col, bias, out, q, sx, d->fault);
    };
    auto pick_c = [&](auto mt) {
        switch (K / 512) {
            case 1: return go(mt, std::integral_constant<int, 1>());
            case 2: return go(mt, std::integral_constant<int, 2>());
            case 4: return go(mt, std::integral_constant<int, 4>());
            case 8: return go(mt, std::integral_constant<int, 8>());
            default: break;
        }
    };
    const int64_t c = K / 512;
    if (c != 1 && c != 2 && c != 4 && c != 8) return kh::fail(KH_ERR_INVALID_ARG, "linear_i8_tensor: internal K case");
    if (M <= 16) pick_c(std::integral_constant<int, 1>());
    else if (M <= 32) pick_c(std::integral_constant<int, 2>());
    else pick_c(std::integral_constant<int, 4>());
    return kh::launch_status("linear_i8_tensor_small");
}

// NB (128-column blocks per tile) of the quantize-on-load kernel for this
// shape, 0 when it does not take it: M a multiple of 64, N = 128, 256 or a
// multiple of 384, K of 64, 16-byte aligned X and B, 32-bit offsets.
int qload_nb(const float* x, const int8_t* b, int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || M % kQlBM || N <= 0 || K <= 0 || K % 64 || !kh::aligned(x, 16) || !kh::aligned(b, 16)) return 0;
    if ((int64_t)kQlBM * K * 4 > 0xFFFFFFFFLL || 384 * K > 0x7FFFFFFFLL || M > 0x7FFFFFFFLL) return 0;
    if ((M / kQlBM) * (N / 128) > 0x7FFFFFFFLL) return 0;
    if (N == 128 || N == 256) return (int)(N / 128);
    return N % 384 == 0 ? 3 : 0;
}

template <int NB, bool ROWS = false>
int launch_qload(kh::Device* d, const float* x, int64_t M, int64_t N, int64_t K, const unsigned* xparts,
                 int nxparts, const int8_t* b, const Epilogue& ep_in, unsigned* parts) {
    Epilogue ep = ep_in;
    ep.stream_out = M * N * (int64_t)sizeof(float) > kStreamOutBytes;
    const unsigned grid = (unsigned)((M / kQlBM) * (N / (128 * NB)));
    const bool fused = ep.act != kActNone || ep.residual;
    if (K == 384) {
        if (fused)
            gemm_i8_qload_kernel<NB, 5, true, ROWS, 6><<<grid, 512, 0, d->stream>>>(x, (int)M, (int)N, (int)K, xparts,
                                                                                    nxparts, b, ep, parts);
        else
            gemm_i8_qload_kernel<NB, 5, false, ROWS, 6><<<grid, 512, 0, d->stream>>>(x, (int)M, (int)N, (int)K,
                                                                                     xparts, nxparts, b, ep, parts);
    } else if (fused)
        gemm_i8_qload_kernel<NB, 5, true, ROWS><<<grid, 512, 0, d->stream>>>(x, (int)M, (int)N, (int)K, xparts,
                                                                             nxparts, b, ep, parts);
    else
        gemm_i8_qload_kernel<NB, 5, false, ROWS><<<grid, 512, 0, d->stream>>>(x, (int)M, (int)N, (int)K, xparts,
                                                                              nxparts, b, ep, parts);
    return kh::launch_status("gemm_i8_qload");
}

}  // namespace

extern "C" {

// may_alloc = false: no pool allocation (the skinny kernel then never splits K).
static int gemm_i8_impl(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
                        int sa_per_row, const double* sb, int sb_per_col, const float* bias, float* out,
                        int32_t* acc_out, int act, const float* residual, unsigned* parts, int max_parts,
                        int* nparts, bool may_alloc = true) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8: negative shape");
    KH_REQUIRE(out || acc_out, "kh_gemm_i8: neither out nor acc_out given");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8: shape too large");
    KH_REQUIRE(act == kActNone || act == kActGelu, "kh_gemm_i8_ex: unknown activation");
    KH_REQUIRE(!(act || residual || parts) || out, "kh_gemm_i8_ex: activation, residual and partials need out");
    KH_REQUIRE(!parts || (nparts && max_parts > 0), "kh_gemm_i8_ex: partials need max_parts > 0 and nparts");
    if (nparts) *nparts = 0;
    if (M == 0 || N == 0) return KH_OK;
    KH_REQUIRE(K == 0 || (a && b_packed), "kh_gemm_i8: null operand");
    KH_REQUIRE(!out || (sa && sb), "kh_gemm_i8: scales required when out is given");
    KH_DEVICE_OR_RETURN(d);
    Epilogue ep{sa, sb, bias, out, acc_out, sa_per_row, sb_per_col, act, residual};
    int rc;
    bool parts_done = false;
    if (skinny_fits(a, b_packed, M, N, K)) {
        rc = launch_skinny(d, a, b_packed, M, N, K, ep, may_alloc);
    } else if (!parts && narrow_fits(a, b_packed, M, N, K)) {
        rc = launch_narrow(d, a, b_packed, M, N, K, ep);
    } else if (pingpong_fits(a, b_packed, M, N, K)) {
        // The ping-pong kernel writes one partial per workgroup when they fit.
        const int64_t worst = ((M + 127) / 128) * ((N + 127) / 128);
        const bool fused = parts && worst <= max_parts;
        rc = launch_pingpong(d, a, b_packed, M, N, K, ep, fused ? parts : nullptr, fused ? nparts : nullptr);
        parts_done = fused;
    } else {
        const bool vec16 = (K % 16 == 0) && kh::aligned(a, 16) && kh::aligned(b_packed, 16);
        if (M >= 2048 && N >= 2048)
            rc = launch_gemm<256, 256, 64, 2, 4>(d, a, b_packed, M, N, K, ep, vec16);
        else
            rc = launch_gemm<128, 128, 64, 2, 2>(d, a, b_packed, M, N, K, ep, vec16);
    }
    if (rc || !parts || parts_done) return rc;
    return kh_absmax_parts(out, M * N, parts, max_parts, nparts);
}

int kh_gemm_i8(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
               int sa_per_row, const double* sb, int sb_per_col, const float* bias, float* out, int32_t* acc_out) {
    return gemm_i8_impl(a, b_packed, M, N, K, sa, sa_per_row, sb, sb_per_col, bias, out, acc_out, kActNone,
                        nullptr, nullptr, 0, nullptr);
}

int kh_gemm_i8_ex(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
                  int sa_per_row, const double* sb, int sb_per_col, const float* bias, int act, const float* residual,
                  float* out, unsigned* absmax_parts, int max_parts, int* nparts) {
    return gemm_i8_impl(a, b_packed, M, N, K, sa, sa_per_row, sb, sb_per_col, bias, out, nullptr, act, residual,
                        absmax_parts, max_parts, nparts);
}

int kh_gemm_i8_quant(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
                     int sa_per_row, const double* sb, int sb_per_col, const float* bias, int act,
                     const float* residual, int8_t* q, double* scale) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8_quant: negative shape");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8_quant: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8_quant: shape too large");
    KH_REQUIRE(act == kActNone || act == kActGelu, "kh_gemm_i8_quant: unknown activation");
    KH_REQUIRE(scale, "kh_gemm_i8_quant: null scale");
    KH_DEVICE_OR_RETURN(d);
    if (M == 0 || N == 0) {
        const double one = 1.0;  // the reference's quantize of an empty tensor
        return kh_memcpy_h2d(scale, &one, sizeof(one));
    }
    KH_REQUIRE(q && sa && sb && (K == 0 || (a && b_packed)), "kh_gemm_i8_quant: null pointer");
    if (pingpong_fits(a, b_packed, M, N, K) && !skinny_fits(a, b_packed, M, N, K)) {
        // Pass 1: the epilogue's values reduced to one absmax partial per
        // workgroup, nothing stored.  Pass 2: the same GEMM and epilogue
        // (so the same values), quantized with the scale of those partials;
        // the fp32 result never reaches memory.
        const int64_t worst = ((M + 127) / 128) * ((N + 127) / 128);
        auto* parts = static_cast<unsigned*>(kh::scratch_area(d, (size_t)worst * sizeof(unsigned)));
        if (!parts) return KH_ERR_OOM;
        Epilogue ep{sa, sb, bias, nullptr, nullptr, sa_per_row, sb_per_col, act, residual,
                    q, parts, 0, scale, d->fault};
        int nparts = 0;
        int rc = launch_pingpong(d, a, b_packed, M, N, K, ep, parts, &nparts, kh::quant::kOutMaxOnly);
        if (rc) return rc;
        ep.nqparts = nparts;
        return launch_pingpong(d, a, b_packed, M, N, K, ep, nullptr, nullptr, kh::quant::kOutQuant);
    }
    // Other shapes: the fp32 result through a pooled temporary, then the
    // per-tensor quantize.
    void* tmp = nullptr;
    int rc = kh_alloc((size_t)(M * N) * sizeof(float), &tmp);
    if (rc) return rc;
    float* out = static_cast<float*>(tmp);
    rc = gemm_i8_impl(a, b_packed, M, N, K, sa, sa_per_row, sb, sb_per_col, bias, out, nullptr, act, residual,
                      nullptr, 0, nullptr);
    if (!rc) rc = kh_quantize_tensor(out, M * N, q, scale);
    kh_free(tmp);  // stream-ordered reuse: later work is queued behind the quantize
    return rc;
}

int kh_gemm_i8_quant_rows(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K, const double* sa,
                          int sa_per_row, const double* sb, int sb_per_col, const float* bias, int act, int8_t* q,
                          double* scales) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8_quant_rows: negative shape");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8_quant_rows: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8_quant_rows: shape too large");
    KH_REQUIRE(act == kActNone || act == kActGelu, "kh_gemm_i8_quant_rows: unknown activation");
    if (M == 0) return KH_OK;
    KH_REQUIRE(scales, "kh_gemm_i8_quant_rows: null scales");
    if (N == 0) return kh_quantize_rows(nullptr, M, 0, q, scales);  // every row's scale 1.0
    KH_REQUIRE(q && sa && sb && (K == 0 || (a && b_packed)), "kh_gemm_i8_quant_rows: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (quant_rows_fits(a, b_packed, q, M, N, K)) {
        Epilogue ep{sa, sb, bias, nullptr, nullptr, sa_per_row, sb_per_col, act, nullptr,
                    q, nullptr, 0, scales, d->fault};
        return launch_quant_rows(d, a, b_packed, M, N, K, ep);
    }
    // Other shapes: the fp32 result through a pooled temporary, then the
    // per-row quantize.
    void* tmp = nullptr;
    int rc = kh_alloc((size_t)(M * N) * sizeof(float), &tmp);
    if (rc) return rc;
    float* out = static_cast<float*>(tmp);
    rc = gemm_i8_impl(a, b_packed, M, N, K, sa, sa_per_row, sb, sb_per_col, bias, out, nullptr, act, nullptr,
                      nullptr, 0, nullptr);
    if (!rc) rc = kh_quantize_rows(out, M, N, q, scales);
    kh_free(tmp);  // stream-ordered reuse: later work is queued behind the quantize
    return rc;
}

int kh_gemm_i8_qload(const float* x, int64_t M, int64_t N, int64_t K, const unsigned* x_parts, int x_nparts,
                     const int8_t* b_packed, const double* sb, int sb_per_col, const float* bias, int act,
                     const float* residual, float* out, double* x_scale, unsigned* absmax_parts, int max_parts,
                     int* nparts) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8_qload: negative shape");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8_qload: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8_qload: shape too large");
    KH_REQUIRE(act == kActNone || act == kActGelu, "kh_gemm_i8_qload: unknown activation");
    KH_REQUIRE(M * K == 0 || (x && x_parts && x_nparts > 0),
               "kh_gemm_i8_qload: x and the producer's absmax partials are required");
    KH_REQUIRE(!absmax_parts || (nparts && max_parts > 0), "kh_gemm_i8_qload: partials need max_parts and nparts");
    if (nparts) *nparts = 0;
    KH_DEVICE_OR_RETURN(d);
    if (M * K == 0) {
        // An empty X quantizes with scale 1.0 (quantize.py:68); the product is zero.
        void* tmp = nullptr;
        int rc = x_scale ? KH_OK : kh_alloc(sizeof(double), &tmp);
        if (rc) return rc;
        double* sc = x_scale ? x_scale : static_cast<double*>(tmp);
        const double one = 1.0;
        rc = kh_memcpy_h2d(sc, &one, sizeof(one));
        if (!rc && M && N)
            rc = kh_gemm_i8_ex(nullptr, b_packed, M, N, 0, sc, 0, sb, sb_per_col, bias, act, residual, out,
                               absmax_parts, max_parts, nparts);
        const int frc = tmp ? kh_free(tmp) : KH_OK;
        return rc ? rc : frc;
    }
    if (N == 0) {
        // Nothing to multiply; the scale is still the tensor's.
        if (!x_scale) return KH_OK;
        void* tmp = nullptr;
        int rc = kh_alloc((size_t)(M * K), &tmp);
        if (rc) return rc;
        rc = kh_quantize_tensor_parts(x, M * K, x_parts, x_nparts, static_cast<int8_t*>(tmp), x_scale);
        const int frc = kh_free(tmp);
        return rc ? rc : frc;
    }
    KH_REQUIRE(b_packed && sb && out, "kh_gemm_i8_qload: null pointer");
    const int nb = qload_nb(x, b_packed, M, N, K);
    const int64_t grid = nb ? (M / kQlBM) * (N / (128 * nb)) : 0;
    if (nb && (!absmax_parts || grid <= max_parts)) {
        Epilogue ep{nullptr, sb, bias, out, nullptr, 0, sb_per_col, act, residual, nullptr, nullptr, 0, x_scale,
                    d->fault};
        int rc = nb == 1   ? launch_qload<1>(d, x, M, N, K, x_parts, x_nparts, b_packed, ep, absmax_parts)
                 : nb == 2 ? launch_qload<2>(d, x, M, N, K, x_parts, x_nparts, b_packed, ep, absmax_parts)
                           : launch_qload<3>(d, x, M, N, K, x_parts, x_nparts, b_packed, ep, absmax_parts);
        if (!rc && absmax_parts) *nparts = (int)grid;
        return rc;
    }
    // Other shapes: the codes (and the scale, when the caller wants none)
    // through a pooled temporary, then the GEMM.
    void* tmp = nullptr;
    int rc = kh_alloc((size_t)(M * K) + 8, &tmp);
    if (rc) return rc;
    double* sc = x_scale ? x_scale : static_cast<double*>(tmp);
    int8_t* q = static_cast<int8_t*>(tmp) + 8;
    rc = kh_quantize_tensor_parts(x, M * K, x_parts, x_nparts, q, sc);
    if (!rc)
        rc = kh_gemm_i8_ex(q, b_packed, M, N, K, sc, 0, sb, sb_per_col, bias, act, residual, out, absmax_parts,
                           max_parts, nparts);
    const int frc = kh_free(tmp);  // stream-ordered reuse: later work is queued behind the GEMM
    return rc ? rc : frc;
}

int kh_gemm_i8_qload_rows(const float* x, int64_t M, int64_t N, int64_t K, const unsigned* row_parts,
                          int parts_per_row, const int8_t* b_packed, const double* sb, int sb_per_col,
                          const float* bias, int act, const float* residual, float* out, double* x_scales) {
    KH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "kh_gemm_i8_qload_rows: negative shape");
    KH_REQUIRE(K <= 133144, "kh_gemm_i8_qload_rows: K > 133144 could overflow the int32 accumulator");
    KH_REQUIRE(M <= 0xFFFFLL * 128 && N <= 0x7FFFFFFFLL, "kh_gemm_i8_qload_rows: shape too large");
    KH_REQUIRE(act == kActNone || act == kActGelu, "kh_gemm_i8_qload_rows: unknown activation");
    KH_REQUIRE(parts_per_row >= 1, "kh_gemm_i8_qload_rows: parts_per_row must be >= 1");
    if (M == 0) return KH_OK;
    KH_REQUIRE(x && row_parts && b_packed && sb && (out || N == 0), "kh_gemm_i8_qload_rows: null pointer");
    KH_DEVICE_OR_RETURN(d);
    const int nb = parts_per_row <= 16 && K > 0 ? qload_nb(x, b_packed, M, N, K) : 0;
    if (nb) {
        Epilogue ep{nullptr, sb, bias, out, nullptr, 1, sb_per_col, act, residual, nullptr, nullptr, 0, x_scales,
                    d->fault};
        return nb == 1   ? launch_qload<1, true>(d, x, M, N, K, row_parts, parts_per_row, b_packed, ep, nullptr)
               : nb == 2 ? launch_qload<2, true>(d, x, M, N, K, row_parts, parts_per_row, b_packed, ep, nullptr)
                         : launch_qload<3, true>(d, x, M, N, K, row_parts, parts_per_row, b_packed, ep, nullptr);
    }
    // Other shapes: the per-row quantize (the same row scales: each is the
    // row's absmax, which the partials only hold in pieces) and the GEMM.
    void* tmp = nullptr;
    int rc = kh_alloc((size_t)(M * K) + (size_t)M * 8, &tmp);
    if (rc) return rc;
    double* sc = x_scales ? x_scales : static_cast<double*>(tmp);
    int8_t* q = static_cast<int8_t*>(tmp) + (size_t)M * 8;
    rc = kh_quantize_rows(x, M, K, q, sc);
    if (!rc && N)
        rc = kh_gemm_i8_ex(q, b_packed, M, N, K, sc, 1, sb, sb_per_col, bias, act, residual, out, nullptr, 0, nullptr);
    const int frc = kh_free(tmp);  // stream-ordered reuse: later work is queued behind the GEMM
    return rc ? rc : frc;
}

// kh_linear_i8's work with the codes and scales in q_scratch / sx_scratch.
// With may_alloc = false it allocates nothing: the decode kernel,
// kh_quantize_rows and the GEMM without absmax partials and without a K
// split use no library scratch and no pooled memory.
static int linear_i8_impl(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N, const double* sb,
                          int sb_per_col, const float* bias, int8_t* q_scratch, double* sx_scratch, float* out,
                          bool may_alloc = true) {
    if (M >= 1 && N >= 1 && x && b_packed && sb && q_scratch && sx_scratch &&
        decode_fits(x, M, K, b_packed, N, q_scratch)) {
        KH_DEVICE_OR_RETURN(d);
        switch (K) {
            case 2048: return launch_decode<4>(d, x, M, b_packed, N, sb, sb_per_col, bias, out, q_scratch, sx_scratch);
            case 4096: return launch_decode<8>(d, x, M, b_packed, N, sb, sb_per_col, bias, out, q_scratch, sx_scratch);
            default: return launch_decode<16>(d, x, M, b_packed, N, sb, sb_per_col, bias, out, q_scratch, sx_scratch);
        }
    }
    int rc = kh_quantize_rows(x, M, K, q_scratch, sx_scratch);
    if (rc) return rc;
    return gemm_i8_impl(q_scratch, b_packed, M, N, K, sx_scratch, 1, sb, sb_per_col, bias, out, nullptr, kActNone,
                        nullptr, nullptr, 0, nullptr, may_alloc);
}

int kh_linear_i8_tensor(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N, const double* sb,
                        int sb_per_col, const float* bias, int8_t* q_scratch, double* sx_scratch, float* out) {
    KH_REQUIRE(out, "kh_linear_i8_tensor: null out");
    KH_REQUIRE(M >= 0 && K >= 0 && N >= 0, "kh_linear_i8_tensor: negative shape");
    if (M >= 1 && N >= 1 && x && b_packed && sb && q_scratch && sx_scratch &&
        tensor_small_fits(x, M, K, b_packed, N, q_scratch)) {
        KH_DEVICE_OR_RETURN(d);
        return launch_tensor_small(d, x, M, K, b_packed, N, sb, sb_per_col, bias, out, q_scratch, sx_scratch);
    }
    KH_REQUIRE(M * K == 0 || (M <= INT64_MAX / K), "kh_linear_i8_tensor: M * K overflows");
    int rc = kh_quantize_tensor(x, M * K, q_scratch, sx_scratch);
    if (rc) return rc;
    return kh_gemm_i8(q_scratch, b_packed, M, N, K, sx_scratch, 0, sb, sb_per_col, bias, out, nullptr);
}

int kh_linear_i8(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N, const double* sb,
                 int sb_per_col, const float* bias, int8_t* q_scratch, double* sx_scratch, float* out) {
    KH_REQUIRE(out, "kh_linear_i8: null out");
    return linear_i8_impl(x, M, K, b_packed, N, sb, sb_per_col, bias, q_scratch, sx_scratch, out);
}

int kh_linear_i8_noalloc(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N, const double* sb,
                         int sb_per_col, const float* bias, float* out) {
    KH_REQUIRE(out, "kh_linear_i8_noalloc: null out");
    KH_REQUIRE(M >= 0 && K >= 0, "kh_linear_i8_noalloc: negative shape");
    KH_REQUIRE(M <= kh::kNoAllocRows,
               "kh_linear_i8_noalloc: M = " + std::to_string(M) + " exceeds the fixed scratch's " +
                   std::to_string(kh::kNoAllocRows) + " rows");
    KH_REQUIRE(K <= (int64_t)kh::kNoAllocCodeBytes && M * K <= (int64_t)kh::kNoAllocCodeBytes,
               "kh_linear_i8_noalloc: M * K = " + std::to_string(M * K) + " codes exceed the fixed scratch's " +
                   std::to_string(kh::kNoAllocCodeBytes) + " bytes");
    // Never initialises the device (that allocates): kh_init first.
    kh::Device* d = kh::current_initialized();
    if (!d) return KH_ERR_NO_DEVICE;
    int8_t* q = reinterpret_cast<int8_t*>(d->noalloc);
    double* sx = reinterpret_cast<double*>(d->noalloc + kh::kNoAllocCodeBytes);
    return linear_i8_impl(x, M, K, b_packed, N, sb, sb_per_col, bias, q, sx, out, /*may_alloc=*/false);
}

}  // extern "C"
