// kh_pipeline.h -- pieces shared by the LDS-DMA GEMM pipelines (int8 in
// kh_gemm_i8.hip, fp32 in kh_gemm_f32.hip): raw buffer resources, the XCD-aware
// workgroup-to-tile order, explicit s_waitcnt immediates and 16-byte LDS-DMA.
// Internal header.
#pragma once

#include <hip/hip_runtime.h>

namespace kh {
namespace pipe {

constexpr int kXcds = 8;
constexpr int kBufferFlags = 0x00020000;  // dword 3 of a raw gfx9 buffer resource

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

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

// s_waitcnt immediate (gfx9 encoding): wait until at most `vm` vector-memory
// and `lgkm` LDS operations of this wave are outstanding; exports not waited.
__host__ __device__ constexpr int wait_imm(int vm, int lgkm) {
    return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | (((vm >> 4) & 3) << 14);
}

// Waits until this wave has at most `stages` x `per_stage` LDS-DMA loads in
// flight (stages in 0..3; uniform branch on a wave-uniform value).
template <int per_stage>
__device__ __forceinline__ void wait_loads_beyond(int stages) {
    if (stages >= 3) __builtin_amdgcn_s_waitcnt(wait_imm(3 * per_stage, 15));
    else if (stages == 2) __builtin_amdgcn_s_waitcnt(wait_imm(2 * per_stage, 15));
    else if (stages == 1) __builtin_amdgcn_s_waitcnt(wait_imm(per_stage, 15));
    else __builtin_amdgcn_s_waitcnt(wait_imm(0, 15));
}

// LDS-DMA of 16 bytes per lane: lane l's bytes land at dst + 16 * l (dst is
// wave-uniform; it goes to M0).
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* dst, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

}  // namespace pipe
}  // namespace kh
