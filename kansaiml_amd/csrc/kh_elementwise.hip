// kh_elementwise.hip -- the fp32 elementwise ops a traced Linear graph puts
// around the matmul (bias add, relu, residual add) and the stand-alone
// dequantize epilogue of an unfused int8_matmul.  All are HBM-streaming:
// one read of each operand, one write, 16-byte accesses where aligned.
#include <hip/hip_runtime.h>

#include "kh_common.h"

#pragma clang fp contract(off)

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Ops.cpp:197-199 / Fused.cpp:5-14: v > 0 ? v : 0 (NaN -> 0, -0 -> 0).
__device__ __forceinline__ float relu1(float v) { return v > 0.0f ? v : 0.0f; }

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                  float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void relu_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = relu1(x[i]);
}

template <bool RELU>
__global__ __launch_bounds__(256) void add_bias_kernel(const float* __restrict__ x, const float* __restrict__ bias,
                                                       float* __restrict__ out, int64_t n, int64_t features) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        const float v = x[i] + bias[i % features];
        out[i] = RELU ? relu1(v) : v;
    }
}

// The int8 GEMM epilogue on a stored accumulator (see kh_gemm_i8.hip).
__global__ __launch_bounds__(256) void dequant_acc_kernel(const int32_t* __restrict__ acc, int64_t M, int64_t N,
                                                          const double* __restrict__ sa, int sa_per_row,
                                                          const double* __restrict__ sb, int sb_per_col,
                                                          const float* __restrict__ bias, float* __restrict__ out) {
    const int64_t n = M * N;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += stride) {
        const int64_t i = e / N, j = e % N;
        const double s = sa[sa_per_row ? i : 0] * sb[sb_per_col ? j : 0];
        float y = (float)((double)acc[e] * s);
        if (bias) y = y + bias[j];
        out[e] = y;
    }
}

// Plain device copy, 16 bytes per lane per step.  Keeps device-to-device
// copies on the compute queue (ordered with the kernels around them) and is
// the known-size kernel that calibrates HBM byte counters.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void copy16_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                     int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

unsigned grid_for(int64_t n) {
    int64_t g = (n + 256 * 4 - 1) / (256 * 4);
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

}  // namespace

extern "C" {

int kh_add(const float* a, const float* b, float* out, int64_t n) {
    KH_REQUIRE(n >= 0, "kh_add: negative size");
    if (n == 0) return KH_OK;
    KH_REQUIRE(a && b && out, "kh_add: null pointer");
    KH_DEVICE_OR_RETURN(d);
    add_kernel<<<grid_for(n), 256, 0, d->stream>>>(a, b, out, n);
    return kh::launch_status("add");
}

int kh_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return KH_OK;
    KH_REQUIRE(dst && src, "kh_memcpy_d2d: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (bytes % 16 == 0 && kh::aligned(dst, 16) && kh::aligned(src, 16)) {
        const int64_t n16 = (int64_t)(bytes / 16);
        int64_t g = (n16 + 256 * 8 - 1) / (256 * 8);
        if (g > 8192) g = 8192;
        copy16_kernel<<<(unsigned)g, 256, 0, d->stream>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n16);
        return kh::launch_status("copy16");
    }
    return kh::hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, d->stream), "hipMemcpyAsync(D2D)");
}

int kh_relu(const float* x, float* out, int64_t n) {
    KH_REQUIRE(n >= 0, "kh_relu: negative size");
    if (n == 0) return KH_OK;
    KH_REQUIRE(x && out, "kh_relu: null pointer");
    KH_DEVICE_OR_RETURN(d);
    relu_kernel<<<grid_for(n), 256, 0, d->stream>>>(x, out, n);
    return kh::launch_status("relu");
}

int kh_add_bias(const float* x, const float* bias, float* out, int64_t batch, int64_t features, int relu) {
    KH_REQUIRE(batch >= 0 && features >= 0, "kh_add_bias: negative shape");
    const int64_t n = batch * features;
    if (n == 0) return KH_OK;
    KH_REQUIRE(x && bias && out, "kh_add_bias: null pointer");
    KH_DEVICE_OR_RETURN(d);
    if (relu)
        add_bias_kernel<true><<<grid_for(n), 256, 0, d->stream>>>(x, bias, out, n, features);
    else
        add_bias_kernel<false><<<grid_for(n), 256, 0, d->stream>>>(x, bias, out, n, features);
    return kh::launch_status("add_bias");
}

int kh_dequantize_acc(const int32_t* acc, int64_t M, int64_t N, const double* sa, int sa_per_row, const double* sb,
                      int sb_per_col, const float* bias, float* out) {
    KH_REQUIRE(M >= 0 && N >= 0, "kh_dequantize_acc: negative shape");
    if (M == 0 || N == 0) return KH_OK;
    KH_REQUIRE(acc && sa && sb && out, "kh_dequantize_acc: null pointer");
    KH_DEVICE_OR_RETURN(d);
    dequant_acc_kernel<<<grid_for(M * N), 256, 0, d->stream>>>(acc, M, N, sa, sa_per_row, sb, sb_per_col, bias, out);
    return kh::launch_status("dequant_acc");
}

}  // extern "C"
