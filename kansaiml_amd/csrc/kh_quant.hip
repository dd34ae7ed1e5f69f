// kh_quant.hip -- symmetric int8 quantize / dequantize kernels for gfx950.
//
// Semantics are the reference's, bit for bit (python/kansai/quantize.py:66-70
// and :76):
//   m = max|v|;  s = m / 127.0 in binary64 (1.0 when m == 0);
//   q = clamp(round_half_even(fl64(v / s)), -127, 127);
//   dequantized = (float)((double)q * s).
//
// Exact division without paying a binary64 divide per element: with
// rf = (float)(1.0 / s), the binary32 FMA a = fl32(v * rf + 1.5*2^23) rounds
// the EXACT product v * rf to the nearest integer k (ties to even) and
// d = fl32(v * rf - k) is its distance to k.  |v * rf - v / s| <= 7.6e-6 for
// |v| <= m (rf carries one binary64 and one binary32 rounding, relative
// 6e-8, on a quotient of magnitude <= 127.0000001), and fl64(v / s) is within
// 1.5e-14 of v / s, so when |d| <= 0.5 - kTieEps (kTieEps = 2^-15, four
// times that bound) k is the reference's round(fl64(v / s)).  Elements that
// fail the test take the exact path: a correctly rounded binary64 divide and
// rint (ties to even).  Rows whose max is below 2^-64 (where 127/m could
// overflow binary32) take the exact path throughout.  The fast path cannot
// leave [-127, 127] (|v * rf| <= 127 * (1 + 2^-23)), so only the exact path
// clamps.
//
// Memory layout: x, q row-major contiguous; per-row kernels keep the whole
// row in registers between the absmax and the quantize step, so each fp32
// value crosses HBM once (5 bytes moved per element: 4 read + 1 written).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kh_common.h"

#pragma clang fp contract(off)

#include "kh_quant_math.h"

using namespace kh::quant;

namespace {

// ---------------------------------------------------------------------------
// Per-row quantize, row held in registers.  ROW_THREADS = 64 * WAVES_PER_ROW
// threads own one row; a 256-thread block owns 256 / ROW_THREADS rows.
// Requires cols % 4 == 0, x 16-byte and q 4-byte aligned, cols <= ROW_THREADS * 4 * VPT.
// ---------------------------------------------------------------------------
// Buffer resources (V#) over one row: loads beyond num_records return 0 and
// stores beyond it are dropped, so the row edge needs no per-access test,
// and each access needs one VGPR offset (the per-step offset is an SGPR).
constexpr int kBufferFlags = 0x00020000;  // dword 3 of a raw gfx9 buffer resource (32-bit data)
constexpr int kCacheNontemporal = 2;      // buffer instruction cache-policy operand: nt

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

template <int WAVES_PER_ROW, int VPT>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                                             double* __restrict__ scales, int64_t rows,
                                                             int64_t cols, unsigned* __restrict__ fault) {
    constexpr int ROW_THREADS = 64 * WAVES_PER_ROW;
    constexpr int ROWS_PER_BLOCK = 256 / ROW_THREADS;
    __shared__ unsigned red[4];
    const int lt = threadIdx.x % ROW_THREADS;
    // A wave lies within one row's threads: the row, and so each row's
    // buffer resource, is wave-uniform.  Said explicitly, the resources live
    // in scalar registers; derived from threadIdx.x they were vector values,
    // and every store became a loop over the lanes' distinct resources.
    const int sub = __builtin_amdgcn_readfirstlane((int)threadIdx.x / ROW_THREADS);
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + sub;
    const bool active = row < rows;
    // An inactive slot (past the last row) gets an empty resource: loads read 0.
    const __amdgpu_buffer_rsrc_t xr = row_rsrc(x + (active ? row : 0) * cols, active ? cols * 4 : 0);

    // Each value is read once: nontemporal loads (the row is not read again
    // unless a group takes the exact path); the codes are stored normally.
    f32x4 v[VPT];
    AbsMax am;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        v[i] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, lt * 16, i * ROW_THREADS * 16, kCacheNontemporal));
        am.add4(v[i]);
    }
    unsigned mb = wave_max(am.bits());
    if (WAVES_PER_ROW > 1) {
        const int w = threadIdx.x / 64;
        if ((threadIdx.x & 63) == 0) red[w] = mb;
        __syncthreads();
        const int w0 = sub * WAVES_PER_ROW;
        mb = red[w0];
#pragma unroll
        for (int i = 1; i < WAVES_PER_ROW; ++i) mb = max(mb, red[w0 + i]);
    }
    if (!active) return;
    const Scale sc = make_scale(mb);
    if (lt == 0) {
        scales[row] = sc.s;
        if (sc.bad) flag_nonfinite(fault);
    }
    // Fast path for every element, stored as it is produced; the registers
    // holding the row die group by group.  A group of four holding an
    // undecided element (|d| within kTieEps of a half; about one per 30k
    // elements) is then redone from memory by the exact path and stored again.
    const __amdgpu_buffer_rsrc_t qr = row_rsrc(q + row * cols, cols);
    unsigned redo = sc.fast ? 0u : (VPT >= 32 ? ~0u : ((1u << VPT) - 1u));
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        bool ok = true;
        const unsigned w = pack4_fast(v[i], sc.rf, ok);
        if (!ok) redo |= 1u << i;
        __builtin_amdgcn_raw_buffer_store_b32(w, qr, lt * 4, i * ROW_THREADS * 4, 0);
    }
    while (redo) {
        const int i = __builtin_ctz(redo);
        redo &= redo - 1;
        const f32x4 vv =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, lt * 16, i * ROW_THREADS * 16, 0));
        __builtin_amdgcn_raw_buffer_store_b32(pack4(vv, sc), qr, lt * 4, i * ROW_THREADS * 4, 0);
    }
}

// Per-row quantize for any shape/alignment: one block per row, two passes
// (the second pass re-reads the row, normally from L2).
__global__ __launch_bounds__(256) void quant_rows_generic_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                                                 double* __restrict__ scales, int64_t cols,
                                                                 unsigned* __restrict__ fault) {
    __shared__ unsigned red[4];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * cols;
    AbsMax am;
    for (int64_t c = threadIdx.x; c < cols; c += 256) am.add1(xr[c]);
    unsigned mb = wave_max(am.bits());
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = mb;
    __syncthreads();
    mb = max(max(red[0], red[1]), max(red[2], red[3]));
    const Scale sc = make_scale(mb);
    if (threadIdx.x == 0) {
        scales[row] = sc.s;
        if (sc.bad) flag_nonfinite(fault);
    }
    int8_t* qr = q + row * cols;
    for (int64_t c = threadIdx.x; c < cols; c += 256) qr[c] = (int8_t)quant_one(xr[c], sc);
}

// ---------------------------------------------------------------------------
// Per-tensor quantize: pass 1 writes one absmax (as bits) per block into
// `partials`; pass 2 reduces the partials in every block, then quantizes.
// VEC: x 16-byte aligned and q 4-byte aligned (float4 body, scalar tail).
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void absmax_partials_kernel(const float* __restrict__ x, int64_t n,
                                                              unsigned* __restrict__ partials) {
    __shared__ unsigned red[4];
    AbsMax am;
    const int64_t stride = (int64_t)gridDim.x * 256;
    if (VEC) {
        const int64_t n4 = n >> 2;
        const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) am.add4(x4[i]);
        if (blockIdx.x == 0)
            for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += 256) am.add1(x[i]);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) am.add1(x[i]);
    }
    unsigned mb = wave_max(am.bits());
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = mb;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = max(max(red[0], red[1]), max(red[2], red[3]));
}

constexpr int kTensorUnroll = 4;

template <bool VEC>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const float* __restrict__ x, int64_t n,
                                                           int8_t* __restrict__ q, double* __restrict__ scale,
                                                           const unsigned* __restrict__ partials, int nparts,
                                                           unsigned* __restrict__ fault) {
    __shared__ unsigned red[4];
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t n4 = n >> 2;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    // kTensorUnroll float4 per thread in flight before the first code is
    // stored (one load at a time per wave left HBM idle between them).  The
    // first batch is requested before the partials, so the workgroup waits
    // for one memory round trip before its first store, not two.
    constexpr int U = kTensorUnroll;
    const int64_t first = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
    f32x4 v[U];
    auto load = [&](int64_t i0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * 256;
            v[u] = i < n4 ? x4[i] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    if (VEC) load(first);
    const unsigned mb = block_reduce_partials(partials, nparts, red);
    const Scale sc = make_scale(mb);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scale[0] = sc.s;
        if (sc.bad) flag_nonfinite(fault);
    }
    if (VEC) {
        unsigned* q4 = reinterpret_cast<unsigned*>(q);
        for (int64_t i0 = first; i0 < n4; i0 += stride * U) {
            if (i0 != first) load(i0);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = i0 + (int64_t)u * 256;
                if (i < n4) q4[i] = pack4(v[u], sc);
            }
        }
        if (blockIdx.x == 0)
            for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += 256) q[i] = (int8_t)quant_one(x[i], sc);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) q[i] = (int8_t)quant_one(x[i], sc);
    }
}

// Per-tensor quantize of a small tensor (n <= kSmallPer * 4 * 1024, x 16-byte
// and q 4-byte aligned) in one launch: one 1024-thread workgroup holds the
// values in registers, reduces the absmax, and stores the codes -- the same
// arithmetic as the two-pass path, without the second launch (latency-bound
// sizes such as a Linear's activations).
constexpr int kSmallThreads = 1024;
constexpr int kSmallPer = 16;  // float4 per thread
constexpr int64_t kSmallTensor = (int64_t)kSmallPer * 4 * kSmallThreads;

__global__ __launch_bounds__(kSmallThreads) void quant_tensor_small_kernel(const float* __restrict__ x, int64_t n,
                                                                           int8_t* __restrict__ q,
                                                                           double* __restrict__ scale,
                                                                           unsigned* __restrict__ fault) {
    __shared__ unsigned red[kSmallThreads / 64];
    const int tid = threadIdx.x;
    const int n4 = (int)(n >> 2), tail = (int)(n - 4 * (int64_t)n4);
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
    f32x4 v[kSmallPer];
    AbsMax am;
#pragma unroll
    for (int i = 0; i < kSmallPer; ++i) {
        const int idx = tid + i * kSmallThreads;
        v[i] = idx < n4 ? x4[idx] : f32x4{0.f, 0.f, 0.f, 0.f};
        if (idx < n4) am.add4(v[i]);
    }
    const float xt = tid < tail ? x[4 * (int64_t)n4 + tid] : 0.0f;
    if (tid < tail) am.add1(xt);
    unsigned mb = wave_max(am.bits());
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    mb = red[0];
#pragma unroll
    for (int w = 1; w < kSmallThreads / 64; ++w) mb = max(mb, red[w]);
    const Scale sc = make_scale(mb);
    if (tid == 0) {
        scale[0] = sc.s;
        if (sc.bad) flag_nonfinite(fault);
    }
    unsigned* q4 = reinterpret_cast<unsigned*>(q);
#pragma unroll
    for (int i = 0; i < kSmallPer; ++i) {
        const int idx = tid + i * kSmallThreads;
        if (idx < n4) q4[idx] = pack4(v[i], sc);
    }
    if (tid < tail) q[4 * (int64_t)n4 + tid] = (int8_t)quant_one(xt, sc);
}

// ---------------------------------------------------------------------------
// Per-column (per output channel) absmax of a [k, n] weight, and the
// transpose-quantize that packs codes K-contiguous ([n, k]).
// ---------------------------------------------------------------------------
__global__ void fill_u32_kernel(unsigned* __restrict__ p, int64_t count, unsigned value) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

constexpr int kColRowsPerBlock = 128;

__global__ __launch_bounds__(256) void col_absmax_kernel(const float* __restrict__ w, int64_t k, int64_t n,
                                                         unsigned* __restrict__ colmax) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const int64_t i0 = (int64_t)blockIdx.y * kColRowsPerBlock;
    const int64_t i1 = min(k, i0 + kColRowsPerBlock);
    AbsMax am;
    for (int64_t i = i0; i < i1; ++i) am.add1(w[i * n + j]);
    atomicMax(colmax + j, am.bits());
}

constexpr int kTile = 64;

// PER_COL: maxbits = colmax[n]; otherwise maxbits = partials[nparts] reduced
// to one per-tensor absmax.  Writes q_packed[j * k + i] and the scales.
template <bool PER_COL>
__global__ __launch_bounds__(256) void pack_quant_kernel(const float* __restrict__ w, int64_t k, int64_t n,
                                                         const unsigned* __restrict__ maxbits, int nparts,
                                                         int8_t* __restrict__ qp, double* __restrict__ scales,
                                                         unsigned* __restrict__ fault) {
    __shared__ __attribute__((aligned(16))) int8_t tile[kTile][kTile + 4];
    __shared__ double s_col[kTile];
    __shared__ float rf_col[kTile];
    __shared__ unsigned char flags_col[kTile];  // bit0 fast, bit1 bad
    __shared__ unsigned red[4];
    const int64_t i0 = (int64_t)blockIdx.y * kTile;
    const int64_t j0 = (int64_t)blockIdx.x * kTile;
    const int t = threadIdx.x;

    if (PER_COL) {
        if (t < kTile) {
            const int64_t j = j0 + t;
            const Scale sc = make_scale(j < n ? maxbits[j] : 0u);
            s_col[t] = sc.s;
            rf_col[t] = sc.rf;
            flags_col[t] = (sc.fast ? 1 : 0) | (sc.bad ? 2 : 0);
            if (blockIdx.y == 0 && j < n) {
                scales[j] = sc.s;
                if (sc.bad) flag_nonfinite(fault);
            }
        }
    } else {
        const unsigned mb = block_reduce_partials(maxbits, nparts, red);
        const Scale sc = make_scale(mb);
        if (t < kTile) {
            s_col[t] = sc.s;
            rf_col[t] = sc.rf;
            flags_col[t] = (sc.fast ? 1 : 0) | (sc.bad ? 2 : 0);
        }
        if (blockIdx.x == 0 && blockIdx.y == 0 && t == 0) {
            scales[0] = sc.s;
            if (sc.bad) flag_nonfinite(fault);
        }
    }
    __syncthreads();

    // Read: thread (r = t / 64, c = t % 64) covers rows r, r+4, ..., column c.
    const int c = t & 63;
    const int r0 = t >> 6;
    Scale sc;
    sc.s = s_col[c];
    sc.rf = rf_col[c];
    sc.fast = flags_col[c] & 1;
    sc.bad = flags_col[c] & 2;
    const int64_t j = j0 + c;
#pragma unroll 4
    for (int r = r0; r < kTile; r += 4) {
        const int64_t i = i0 + r;
        int code = 0;
        if (i < k && j < n) code = quant_one(w[i * n + j], sc);
        tile[c][r] = (int8_t)code;
    }
    __syncthreads();

    // Write: thread (jj = t / 4, part = t % 4) writes 16 consecutive k of column j0 + jj.
    const int jj = t >> 2;
    const int ii = (t & 3) * 16;
    const int64_t jo = j0 + jj;
    if (jo >= n) return;
    const int64_t io = i0 + ii;
    int8_t* dst = qp + jo * k + io;
    if (io + 16 <= k && kh::aligned(dst, 16)) {
        uint4 v;
        v.x = *reinterpret_cast<const unsigned*>(&tile[jj][ii + 0]);
        v.y = *reinterpret_cast<const unsigned*>(&tile[jj][ii + 4]);
        v.z = *reinterpret_cast<const unsigned*>(&tile[jj][ii + 8]);
        v.w = *reinterpret_cast<const unsigned*>(&tile[jj][ii + 12]);
        *reinterpret_cast<uint4*>(dst) = v;
    } else {
        for (int e = 0; e < 16 && io + e < k; ++e) dst[e] = tile[jj][ii + e];
    }
}

// ---------------------------------------------------------------------------
// Dequantize (quantize.py:76): out = (float)((double)q * s).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float deq_one(int8_t q, double s) { return (float)((double)q * s); }

__device__ __forceinline__ f32x4 deq4(unsigned w, double s) {
    return f32x4{deq_one((int8_t)(w & 0xFF), s), deq_one((int8_t)((w >> 8) & 0xFF), s),
                 deq_one((int8_t)((w >> 16) & 0xFF), s), deq_one((int8_t)(w >> 24), s)};
}

// Vector dequantize.  Block (bx, row) covers kDeqPerBlock consecutive codes of
// one row (per-row scale uniform over the block; per-tensor: rows == 1).
// Each lane reads 4 codes (one u32) and writes one 16-byte float4 per step,
// so every load and store instruction covers a contiguous span of the wave.
// Codes load through the cache normally; the fp32 output is written with
// nontemporal stores (measured fastest of the four load/store policy pairs).
// Requires cols % 4 == 0, q 4-byte and out 16-byte aligned.
// STEPS of 1024 codes per block: 4 for rows of more than 3072 codes, fewer
// for shorter rows, so that a block issues no steps past its row's end.
constexpr int kDeqSteps = 4;
typedef int i32x4raw __attribute__((ext_vector_type(4)));  // a 16-byte buffer store's data
constexpr int kDeqPerBlock = 256 * 4 * kDeqSteps;

template <int STEPS>
__global__ __launch_bounds__(256) void dequant_vec_kernel(const int8_t* __restrict__ q, int64_t cols,
                                                          const double* __restrict__ scales, int per_row,
                                                          float* __restrict__ out) {
    const int64_t row = blockIdx.y;
    const double s = scales[per_row ? row : 0];
    // The block's span of the row, as buffer resources: every step's load is
    // issued before the first conversion (loads past the row's end read 0,
    // stores past it are dropped).  With a bounds test around each step the
    // compiler waited for each load before issuing the next.
    constexpr int kPerBlock = 1024 * STEPS;
    const int64_t c0 = (int64_t)blockIdx.x * kPerBlock;
    const int span = (int)min((int64_t)kPerBlock, cols - c0);
    const __amdgpu_buffer_rsrc_t rq = row_rsrc(q + row * cols + c0, span);
    const __amdgpu_buffer_rsrc_t ro = row_rsrc(out + row * cols + c0, (int64_t)span * 4);
    unsigned w[STEPS];
#pragma unroll
    for (int step = 0; step < STEPS; ++step)
        w[step] = __builtin_amdgcn_raw_buffer_load_b32(rq, threadIdx.x * 4, step * 1024, 0);
#pragma unroll
    for (int step = 0; step < STEPS; ++step)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4raw, deq4(w[step], s)), ro, threadIdx.x * 16,
                                               step * 4096, kCacheNontemporal);
}

// Any shape / alignment.
__global__ __launch_bounds__(256) void dequant_generic_kernel(const int8_t* __restrict__ q, int64_t n, int64_t cols,
                                                              const double* __restrict__ scales, int per_row,
                                                              float* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        out[i] = deq_one(q[i], scales[per_row ? i / cols : 0]);
}

// out[i, j] = (float)((double)qp[j * k + i] * s_j), back to the [k, n] layout.
__global__ __launch_bounds__(256) void dequant_packed_kernel(const int8_t* __restrict__ qp, int64_t k, int64_t n,
                                                             const double* __restrict__ scales, int64_t scales_n,
                                                             float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) int8_t tile[kTile][kTile + 4];
    const int64_t i0 = (int64_t)blockIdx.y * kTile;
    const int64_t j0 = (int64_t)blockIdx.x * kTile;
    const int t = threadIdx.x;
    // Read codes: thread (jj = t / 4) reads 16 k of column j0 + jj.
    {
        const int jj = t >> 2;
        const int ii = (t & 3) * 16;
        for (int e = 0; e < 16; ++e) {
            const int64_t i = i0 + ii + e, j = j0 + jj;
            tile[jj][ii + e] = (i < k && j < n) ? qp[j * k + i] : (int8_t)0;
        }
    }
    __syncthreads();
    const int c = t & 63;
    const int64_t j = j0 + c;
    if (j >= n) return;
    const double s = scales[scales_n == 1 ? 0 : j];
    for (int r = t >> 6; r < kTile; r += 4) {
        const int64_t i = i0 + r;
        if (i < k) out[i * n + j] = deq_one(tile[c][r], s);
    }
}

int grid_for(int64_t work_items, int per_thread, int cap) {
    int64_t g = (work_items + 256LL * per_thread - 1) / (256LL * per_thread);
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

constexpr int kMaxPartials = 1024;

}  // namespace


namespace {

__global__ void fill_f64_kernel(double* __restrict__ p, int64_t count, double value) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

// Empty slices: max() defaults to 0.0, so the scale is 1.0 (quantize.py:67-68).
int fill_scales_one(kh::Device* d, double* scales, int64_t count) {
    fill_f64_kernel<<<(unsigned)((count + 255) / 256), 256, 0, d->stream>>>(scales, count, 1.0);
    return kh::launch_status("fill_f64");
}

// Pass 1 of a per-tensor quantize: per-block absmax bits into library scratch.
int tensor_absmax(kh::Device* d, const float* x, int64_t n, bool vec, unsigned** partials, int* nparts) {
    const int g = grid_for(vec ? (n >> 2) : n, 8, kMaxPartials);
    unsigned* p = static_cast<unsigned*>(kh::scratch_area(d, kMaxPartials * sizeof(unsigned)));
    if (!p) return KH_ERR_OOM;
    if (vec)
        absmax_partials_kernel<true><<<g, 256, 0, d->stream>>>(x, n, p);
    else
        absmax_partials_kernel<false><<<g, 256, 0, d->stream>>>(x, n, p);
    *partials = p;
    *nparts = g;
    return kh::launch_status("absmax_partials");
}

}  // namespace

extern "C" {

int kh_quantize_tensor(const float* x, int64_t n, int8_t* q, double* scale) {
    KH_REQUIRE(n >= 0, "kh_quantize_tensor: negative size");
    KH_REQUIRE(scale, "kh_quantize_tensor: null scale");
    KH_REQUIRE(n == 0 || (x && q), "kh_quantize_tensor: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (n == 0) return fill_scales_one(d, scale, 1);
    const bool vec = kh::aligned(x, 16) && kh::aligned(q, 4);
    if (vec && n <= kSmallTensor) {
        quant_tensor_small_kernel<<<1, kSmallThreads, 0, d->stream>>>(x, n, q, scale, d->fault);
        return kh::launch_status("quant_tensor_small");
    }
    unsigned* partials = nullptr;
    int nparts = 0;
    int rc = tensor_absmax(d, x, n, vec, &partials, &nparts);
    if (rc) return rc;
    const int g = grid_for(vec ? (n >> 2) : n, 8, 8192);
    if (vec)
        quant_tensor_kernel<true><<<g, 256, 0, d->stream>>>(x, n, q, scale, partials, nparts, d->fault);
    else
        quant_tensor_kernel<false><<<g, 256, 0, d->stream>>>(x, n, q, scale, partials, nparts, d->fault);
    return kh::launch_status("quant_tensor");
}

int kh_absmax_parts(const float* x, int64_t n, unsigned* parts, int max_parts, int* nparts) {
    KH_REQUIRE(n >= 0 && max_parts > 0 && parts && nparts, "kh_absmax_parts: bad arguments");
    KH_REQUIRE(n == 0 || x, "kh_absmax_parts: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (n == 0) {
        fill_u32_kernel<<<1, 256, 0, d->stream>>>(parts, 1, 0u);
        *nparts = 1;
        return kh::launch_status("fill_u32");
    }
    const bool vec = kh::aligned(x, 16);
    const int g = grid_for(vec ? (n >> 2) : n, 8, std::min(max_parts, kMaxPartials));
    if (vec)
        absmax_partials_kernel<true><<<g, 256, 0, d->stream>>>(x, n, parts);
    else
        absmax_partials_kernel<false><<<g, 256, 0, d->stream>>>(x, n, parts);
    *nparts = g;
    return kh::launch_status("absmax_partials");
}

int kh_quantize_tensor_parts(const float* x, int64_t n, const unsigned* parts, int nparts, int8_t* q, double* scale) {
    KH_REQUIRE(n >= 0, "kh_quantize_tensor_parts: negative size");
    KH_REQUIRE(scale && parts && nparts > 0, "kh_quantize_tensor_parts: bad partials or scale");
    KH_REQUIRE(n == 0 || (x && q), "kh_quantize_tensor_parts: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (n == 0) return fill_scales_one(d, scale, 1);
    const bool vec = kh::aligned(x, 16) && kh::aligned(q, 4);
    const int g = grid_for(vec ? (n >> 2) : n, 8, 8192);
    if (vec)
        quant_tensor_kernel<true><<<g, 256, 0, d->stream>>>(x, n, q, scale, parts, nparts, d->fault);
    else
        quant_tensor_kernel<false><<<g, 256, 0, d->stream>>>(x, n, q, scale, parts, nparts, d->fault);
    return kh::launch_status("quant_tensor");
}

int kh_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, double* scales) {
    KH_REQUIRE(rows >= 0 && cols >= 0, "kh_quantize_rows: negative shape");
    if (rows == 0) return KH_OK;
    KH_REQUIRE(scales, "kh_quantize_rows: null scales");
    KH_REQUIRE(cols == 0 || (x && q), "kh_quantize_rows: null pointer");
    KH_REQUIRE(rows <= 0x7FFFFFFFLL, "kh_quantize_rows: too many rows");
    KH_DEVICE_OR_RETURN(d);
    if (cols == 0) return fill_scales_one(d, scales, rows);
    const bool vec = (cols % 4 == 0) && kh::aligned(x, 16) && kh::aligned(q, 4);
    const unsigned per_row = (unsigned)rows;
    const unsigned four_rows = (unsigned)((rows + 3) / 4);
    const unsigned two_rows = (unsigned)((rows + 1) / 2);
    // The smallest row slot (threads x float4 per thread) that holds the row:
    // slots past the row's end still cost their loads' issue.
    if (vec && cols <= 256)
        quant_rows_reg_kernel<1, 1><<<four_rows, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 512)
        quant_rows_reg_kernel<1, 2><<<four_rows, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 1024)
        quant_rows_reg_kernel<1, 4><<<four_rows, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 1536)
        quant_rows_reg_kernel<2, 3><<<two_rows, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 2048)
        quant_rows_reg_kernel<2, 4><<<two_rows, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 4096)
        quant_rows_reg_kernel<4, 4><<<per_row, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 16384)
        quant_rows_reg_kernel<4, 16><<<per_row, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else if (vec && cols <= 32768)
        quant_rows_reg_kernel<4, 32><<<per_row, 256, 0, d->stream>>>(x, q, scales, rows, cols, d->fault);
    else
        quant_rows_generic_kernel<<<per_row, 256, 0, d->stream>>>(x, q, scales, cols, d->fault);
    return kh::launch_status("quant_rows");
}

static int quantize_packed(const float* w, int64_t k, int64_t n, int8_t* qp, double* scales, bool per_col) {
    KH_DEVICE_OR_RETURN(d);
    const unsigned gx = (unsigned)((n + kTile - 1) / kTile);
    const unsigned gy = (unsigned)((k + kTile - 1) / kTile);
    if (per_col) {
        unsigned* colmax = static_cast<unsigned*>(kh::scratch_area(d, (size_t)n * sizeof(unsigned)));
        if (!colmax) return KH_ERR_OOM;
        fill_u32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, d->stream>>>(colmax, n, 0u);
        dim3 g1((unsigned)((n + 255) / 256), (unsigned)((k + kColRowsPerBlock - 1) / kColRowsPerBlock));
        col_absmax_kernel<<<g1, 256, 0, d->stream>>>(w, k, n, colmax);
        pack_quant_kernel<true><<<dim3(gx, gy), 256, 0, d->stream>>>(w, k, n, colmax, 0, qp, scales, d->fault);
    } else {
        unsigned* partials = nullptr;
        int nparts = 0;
        int rc = tensor_absmax(d, w, k * n, kh::aligned(w, 16), &partials, &nparts);
        if (rc) return rc;
        pack_quant_kernel<false><<<dim3(gx, gy), 256, 0, d->stream>>>(w, k, n, partials, nparts, qp, scales, d->fault);
    }
    return kh::launch_status("pack_quant");
}

int kh_quantize_cols_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scales) {
    KH_REQUIRE(k >= 0 && n >= 0, "kh_quantize_cols_packed: negative shape");
    if (n == 0) return KH_OK;
    KH_REQUIRE(scales, "kh_quantize_cols_packed: null scales");
    if (k == 0) {
        KH_DEVICE_OR_RETURN(d);
        return fill_scales_one(d, scales, n);
    }
    KH_REQUIRE(w && q_packed, "kh_quantize_cols_packed: null pointer");
    KH_REQUIRE(n <= 0x7FFFFFFFLL * 64 && k <= 0xFFFFLL * 64, "kh_quantize_cols_packed: shape too large");
    return quantize_packed(w, k, n, q_packed, scales, true);
}

int kh_quantize_tensor_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scale) {
    KH_REQUIRE(k >= 0 && n >= 0, "kh_quantize_tensor_packed: negative shape");
    KH_REQUIRE(scale, "kh_quantize_tensor_packed: null scale");
    if (k == 0 || n == 0) {
        KH_DEVICE_OR_RETURN(d);
        return fill_scales_one(d, scale, 1);
    }
    KH_REQUIRE(w && q_packed, "kh_quantize_tensor_packed: null pointer");
    KH_REQUIRE(n <= 0x7FFFFFFFLL * 64 && k <= 0xFFFFLL * 64, "kh_quantize_tensor_packed: shape too large");
    return quantize_packed(w, k, n, q_packed, scale, false);
}

static int dequant(const int8_t* q, int64_t rows, int64_t cols, const double* scales, float* out, bool per_row) {
    KH_DEVICE_OR_RETURN(d);
    const bool vec = (cols % 4 == 0) && kh::aligned(q, 4) && kh::aligned(out, 16);
    if (vec && rows <= 0x7FFFFFFFLL && (cols + kDeqPerBlock - 1) / kDeqPerBlock <= 0x7FFFFFFFLL) {
        const int steps = cols > 3072 ? 4 : (int)((cols + 1023) / 1024);
        const unsigned gx = (unsigned)((cols + 1024 * steps - 1) / (1024 * steps));
        auto go = [&](const int8_t* qq, const double* ss, float* oo, unsigned nr) {
            const dim3 g(gx, nr);
            const int pr = per_row ? 1 : 0;
            if (steps == 4) dequant_vec_kernel<4><<<g, 256, 0, d->stream>>>(qq, cols, ss, pr, oo);
            else if (steps == 3) dequant_vec_kernel<3><<<g, 256, 0, d->stream>>>(qq, cols, ss, pr, oo);
            else if (steps == 2) dequant_vec_kernel<2><<<g, 256, 0, d->stream>>>(qq, cols, ss, pr, oo);
            else dequant_vec_kernel<1><<<g, 256, 0, d->stream>>>(qq, cols, ss, pr, oo);
        };
        // grid.y is limited to 65535: walk the rows in slabs.
        for (int64_t r0 = 0; r0 < rows; r0 += 65535)
            go(q + r0 * cols, scales + (per_row ? r0 : 0), out + r0 * cols, (unsigned)min((int64_t)65535, rows - r0));
    } else {
        const int64_t n = rows * cols;
        const int g = grid_for(n, 16, 16384);
        dequant_generic_kernel<<<g, 256, 0, d->stream>>>(q, n, cols, scales, per_row ? 1 : 0, out);
    }
    return kh::launch_status("dequant");
}

int kh_dequantize_tensor(const int8_t* q, int64_t n, const double* scale, float* out) {
    KH_REQUIRE(n >= 0, "kh_dequantize_tensor: negative size");
    if (n == 0) return KH_OK;
    KH_REQUIRE(q && scale && out, "kh_dequantize_tensor: null pointer");
    return dequant(q, 1, n, scale, out, false);
}

int kh_dequantize_rows(const int8_t* q, int64_t rows, int64_t cols, const double* scales, float* out) {
    KH_REQUIRE(rows >= 0 && cols >= 0, "kh_dequantize_rows: negative shape");
    if (rows == 0 || cols == 0) return KH_OK;
    KH_REQUIRE(q && scales && out, "kh_dequantize_rows: null pointer");
    return dequant(q, rows, cols, scales, out, true);
}

int kh_dequantize_packed(const int8_t* q_packed, int64_t k, int64_t n, const double* scales, int64_t scales_n,
                         float* out) {
    KH_REQUIRE(k >= 0 && n >= 0, "kh_dequantize_packed: negative shape");
    if (k == 0 || n == 0) return KH_OK;
    KH_REQUIRE(q_packed && scales && out, "kh_dequantize_packed: null pointer");
    KH_REQUIRE(scales_n == 1 || scales_n == n, "kh_dequantize_packed: scales_n must be 1 or n");
    KH_REQUIRE(n <= 0x7FFFFFFFLL * 64 && k <= 0xFFFFLL * 64, "kh_dequantize_packed: shape too large");
    KH_DEVICE_OR_RETURN(d);
    dim3 g((unsigned)((n + kTile - 1) / kTile), (unsigned)((k + kTile - 1) / kTile));
    dequant_packed_kernel<<<g, 256, 0, d->stream>>>(q_packed, k, n, scales, scales_n, out);
    return kh::launch_status("dequant_packed");
}

}  // extern "C"
