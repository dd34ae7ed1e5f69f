// kh_common.h -- shared internals of the gfx950 HIP backend (not part of the
// C ABI; the ABI is include/kansai_hip.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "kansai_hip.h"

namespace kh {

// ---- errors ---------------------------------------------------------------

// Sets the calling thread's last-error text and returns `code`.
int fail(int code, const std::string& msg);
// Maps a HIP error to KH_ERR_HIP / KH_ERR_OOM with context; KH_OK if ok.
int hip_status(hipError_t e, const char* what);
// Checks the launch that just happened (hipGetLastError).
int launch_status(const char* kernel);

// ---- per-device state ------------------------------------------------------

// Bits of the device fault word (set by kernels with a vector atomic OR,
// read and cleared by kh_synchronize).
constexpr unsigned kFaultNonFinite = 1u;
constexpr unsigned kFaultBadIndex = 2u;

// The fixed device array behind the entry points that allocate nothing
// (kh_linear_i8_noalloc): kNoAllocCodeBytes of int8 codes followed by
// kNoAllocRows binary64 scales.  Defined in kh_runtime.hip; every device
// holds its own copy from module load until the process ends.
constexpr size_t kNoAllocCodeBytes = size_t(2) << 20;
constexpr int64_t kNoAllocRows = 2048;
constexpr size_t kNoAllocBytes = kNoAllocCodeBytes + size_t(kNoAllocRows) * sizeof(double);

struct Device {
    int id = -1;
    hipStream_t stream = nullptr;
    unsigned* fault = nullptr;   // device word, see kFaultNonFinite
    int cus = 0;
    // This device's address of the fixed no-alloc array, looked up once by
    // hipGetSymbolAddress when the device is initialised.
    unsigned char* noalloc = nullptr;
};

// The calling thread's current device, initialised on first use (device 0
// unless kh_init chose another).  Returns nullptr and sets the last error
// when no usable gfx950 device exists.
Device* current();

// The calling thread's current device only if it is already initialised
// (by kh_init or any earlier call); otherwise nullptr and the last error.
// Initialising creates a stream and allocates, so entry points that must
// not allocate use this instead of current().
Device* current_initialized();

// A growable device scratch area of at least `bytes`, owned by the library,
// valid until the next scratch_area() call on the same device.  All library
// work is ordered on the device's single library stream, so consecutive
// calls reuse it safely.  Returns nullptr (and sets the last error) on OOM.
void* scratch_area(Device* d, size_t bytes);

// True while a graph capture (kh_graph_capture_begin .. _end) is open on the
// device's library stream: host-synchronous work must refuse to run.
bool capturing(Device* d);

// ---- argument checks ---------------------------------------------------------

__host__ __device__ inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace kh

#define KH_REQUIRE(cond, msg)                                        \
    do {                                                             \
        if (!(cond)) return ::kh::fail(KH_ERR_INVALID_ARG, (msg));   \
    } while (0)

#define KH_DEVICE_OR_RETURN(d)                                       \
    ::kh::Device* d = ::kh::current();                               \
    if (!d) return KH_ERR_NO_DEVICE

// Host-synchronous calls cannot be recorded into a graph.
#define KH_NOT_CAPTURING(d, what) \
    KH_REQUIRE(!::kh::capturing(d), what ": not allowed while a graph is being captured")

// Non-finite detection uses the IEEE bit pattern: for |v| (sign cleared) the
// unsigned order of the bits is the numeric order, and every NaN/inf pattern
// is >= 0x7F800000, so a max over bits finds both the absmax and any NaN.
#define KH_NONFINITE_BITS 0x7F800000u
