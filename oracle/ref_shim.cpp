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

// kan::cpu::add_bias_broadcast, backend/cpu/src/Ops.cpp:34-38.
void kref_add_bias_broadcast(const float* x, const float* bias, float* out, int64_t batch, int64_t features) {
    kan::cpu::add_bias_broadcast(x, bias, out, batch, features);
}

}
