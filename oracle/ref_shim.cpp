// ref_shim.cpp -- extern "C" entry points onto the reference's own CPU
// kernels, so tests and bench.py's cpu_baseline leg can call the real
// compiled reference code (backend/cpu/src/Ops.cpp) through ctypes.
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/.
#include "kansai/backend/cpu/Ops.hpp"

extern "C" {

// kan::cpu::matmul, backend/cpu/include/kansai/backend/cpu/Ops.hpp (declared
// there; defined at backend/cpu/src/Ops.cpp:322-339).
void kref_matmul(const float* a, const float* b, float* out, int64_t M, int64_t K, int64_t N) {
    kan::cpu::matmul(a, b, out, M, K, N);
}

// kan::cpu::batched_matmul, backend/cpu/src/Ops.cpp:427-437, for the case
// Tensor::matmul's batched path takes with a [batch, M, K] left operand and a
// shared 2-D right operand (core/src/Tensor.cpp:364-393): a batch shape of
// rank 1 against one of rank 0.
void kref_batched_matmul_shared(const float* a, const float* b, float* out, int64_t batch, int64_t M, int64_t K,
                                int64_t N) {
    const int64_t a_batch[1] = {batch};
    kan::cpu::batched_matmul(a, a_batch, 1, b, nullptr, 0, a_batch, 1, M, K, N, out);
}

// kan::cpu::add_broadcast, backend/cpu/src/Ops.cpp:121-125: the general
// broadcast add Tensor::add takes for [batch, M, N] + [N]
// (core/src/Tensor.cpp:158-166).
void kref_add_broadcast_rank3(const float* x, const float* bias, float* out, int64_t batch, int64_t M, int64_t N) {
    const int64_t xs[3] = {batch, M, N};
    const int64_t bs[1] = {N};
    kan::cpu::add_broadcast(x, xs, 3, bias, bs, 1, xs, 3, out);
}

// kan::cpu::add_bias_broadcast, backend/cpu/src/Ops.cpp:34-38.
void kref_add_bias_broadcast(const float* x, const float* bias, float* out, int64_t batch, int64_t features) {
    kan::cpu::add_bias_broadcast(x, bias, out, batch, features);
}

}
