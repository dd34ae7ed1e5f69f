// kh_probe.hip -- measurement utility, not on the int8 path: the int8 MFMA
// rate a gfx950 sustains on given operand bytes, and the shader clock it runs
// at while doing so.  MI355X's published int8 peak (5.0 POP/s) assumes the
// 2.4 GHz peak engine clock; under a dense v_mfma_i32_32x32x32_i8 load on
// random operands the board's power management lowers the clock, and this
// probe measures the rate that is actually attainable (the ceiling a GEMM's
// roofline fraction should be read against), much as a plain copy kernel
// calibrates the HBM ceiling.
//
// Each wave keeps 8 operand registers (16 bytes per lane each, loaded once
// from `operands`) and issues 16 independent MFMAs per iteration into 8
// accumulators; there is no memory traffic inside the loop.  One workgroup
// of 8 waves (2 per SIMD) per CU.  The clock is the ratio of the shader
// cycle counter (s_memtime) to the 100 MHz reference counter
// (s_memrealtime) over each workgroup's loop, summed over workgroups.
#include <hip/hip_runtime.h>

#include "kh_common.h"

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kProbeThreads = 512;

__global__ __launch_bounds__(kProbeThreads) void mfma_probe_kernel(const int8_t* __restrict__ operands,
                                                                   int64_t iters,
                                                                   unsigned long long* __restrict__ clocks,
                                                                   int* __restrict__ sink) {
    const i32x4* p = reinterpret_cast<const i32x4*>(operands) + ((int64_t)blockIdx.x * kProbeThreads + threadIdx.x) * 8;
    i32x4 f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = p[i];
    i32x16 acc[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) acc[a] = i32x16{0};
    const long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int m = 0; m < 16; ++m)
            acc[m & 7] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[m & 7], f[(3 * m + 1) & 7], acc[m & 7], 0, 0, 0);
    }
    if (threadIdx.x == 0) {
        atomicAdd(&clocks[0], (unsigned long long)(__builtin_amdgcn_s_memtime() - t0));
        atomicAdd(&clocks[1], (unsigned long long)(__builtin_amdgcn_s_memrealtime() - r0));
    }
    int s = 0;
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) s ^= acc[a][r];
    if (s == 0x5eed5eed) sink[threadIdx.x & 63] = s;  // keeps the MFMAs live
}

// A plain streaming read, the ceiling of the weight-streaming GEMMs: each
// workgroup of 512 threads issues all of its 64 KiB of 16-byte loads (8 per
// lane, each instruction covering 8 KiB contiguous) before using any, folds
// them into one word and keeps them live through an unreachable store.
// Bytes past `bytes` read as zero (buffer-resource bound).
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const void* __restrict__ p, uint32_t bytes,
                                                                    int* __restrict__ sink) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
    const uint32_t base = (blockIdx.x * 8u * kProbeThreads + threadIdx.x) * 16u;
    i32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, base + i * kProbeThreads * 16u, 0, 0);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (s == 0x5eed5eed) sink[threadIdx.x & 63] = s;
}

}  // namespace

extern "C" {

int kh_probe_stream_read(const void* p, int64_t bytes) {
    KH_REQUIRE(p && bytes > 0 && bytes % 16 == 0 && bytes < (1LL << 31) && kh::aligned(p, 16),
               "kh_probe_stream_read: 16-byte aligned buffer of 16 B .. 2 GiB (a multiple of 16) required");
    KH_DEVICE_OR_RETURN(d);
    int* sink = static_cast<int*>(kh::scratch_area(d, 256));
    if (!sink) return KH_ERR_OOM;
    const int64_t per_block = 8LL * kProbeThreads * 16;
    const unsigned blocks = (unsigned)((bytes + per_block - 1) / per_block);
    stream_read_kernel<<<blocks, kProbeThreads, 0, d->stream>>>(p, (uint32_t)bytes, sink);
    return kh::launch_status("stream_read");
}

int kh_probe_mfma_i8(const int8_t* operands, int64_t bytes, int64_t iters, double* tops, double* clock_mhz) {
    KH_REQUIRE(iters > 0 && tops && clock_mhz, "kh_probe_mfma_i8: bad arguments");
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_probe_mfma_i8");
    const int64_t need = (int64_t)d->cus * kProbeThreads * 8 * 16;
    KH_REQUIRE(operands && bytes >= need && kh::aligned(operands, 16),
               "kh_probe_mfma_i8: operands must be 16-byte aligned and hold cus * 64 KiB");
    unsigned long long* clocks = static_cast<unsigned long long*>(kh::scratch_area(d, 512));
    if (!clocks) return KH_ERR_OOM;
    int rc = kh::hip_status(hipMemsetAsync(clocks, 0, 512, d->stream), "hipMemsetAsync(probe)");
    if (rc) return rc;
    hipEvent_t e0, e1;
    rc = kh::hip_status(hipEventCreate(&e0), "hipEventCreate");
    if (rc) return rc;
    rc = kh::hip_status(hipEventCreate(&e1), "hipEventCreate");
    if (rc) {
        (void)hipEventDestroy(e0);
        return rc;
    }
    rc = kh::hip_status(hipEventRecord(e0, d->stream), "hipEventRecord(probe)");
    if (!rc) {
        mfma_probe_kernel<<<(unsigned)d->cus, kProbeThreads, 0, d->stream>>>(operands, iters, clocks,
                                                                            reinterpret_cast<int*>(clocks + 4));
        rc = kh::launch_status("mfma_probe");
    }
    if (!rc) rc = kh::hip_status(hipEventRecord(e1, d->stream), "hipEventRecord(probe)");
    if (!rc) rc = kh::hip_status(hipEventSynchronize(e1), "hipEventSynchronize(probe)");
    float ms = 0.0f;
    if (!rc) rc = kh::hip_status(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime(probe)");
    unsigned long long h[2] = {0, 0};
    if (!rc) rc = kh::hip_status(hipMemcpy(h, clocks, sizeof h, hipMemcpyDeviceToHost), "read probe clocks");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc) return rc;
    const double ops = (double)d->cus * (kProbeThreads / 64) * (double)iters * 16.0 * 65536.0;
    *tops = ops / (ms * 1e-3) / 1e12;
    *clock_mhz = h[1] ? 100.0 * (double)h[0] / (double)h[1] : 0.0;
    return KH_OK;
}

}  // extern "C"
