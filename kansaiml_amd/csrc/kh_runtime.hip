// kh_runtime.hip -- device selection, errors, the device memory pool, copies,
// events and deferred-error reporting for the gfx950 backend.
//
// Replaces, for device memory, the reference's page-aligned host Storage
// (core/src/Storage.cpp:22-32) and its first-fit StoragePool
// (core/src/StoragePool.cpp:5-24): a graph run repeatedly through the KIR
// memory planner draws its intermediates from here and, after the first
// run, never calls hipMalloc again.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "kh_common.h"

// The fixed scratch array of the allocation-free entry points (see
// kh::kNoAllocBytes).  In host code this name is a host-side stand-in, not a
// device address: host code uses only the per-device address that
// hipGetSymbolAddress returns in init_slot (Device::noalloc).
static __device__ __align__(256) unsigned char scratch[kh::kNoAllocBytes];

namespace kh {

namespace {

thread_local std::string t_last_error;
thread_local int t_device = -1;

constexpr int kMaxDevices = 16;

struct Graph;

struct Pool {
    std::mutex mu;
    std::unordered_map<size_t, std::vector<void*>> free_lists;  // size class -> blocks
    std::unordered_map<void*, size_t> live;                     // block -> size class
    size_t in_use = 0;
    size_t cached = 0;
    size_t driver_allocs = 0;
    size_t requests = 0;  // kh_alloc calls served
    // Graph capture (kh_graph_capture_begin .. _end).  Blocks freed while
    // capturing go to cap_free, not to free_lists: the captured nodes keep
    // using them at every launch, so no later work may be handed them.
    bool capturing = false;
    std::unordered_map<size_t, std::vector<void*>> cap_free;
    std::vector<void*> cap_used;  // every block handed out while capturing
    // Blocks a live graph's nodes use that were still handed out when its
    // capture ended (its output, for one): kh_free gives them to the graph.
    std::unordered_map<void*, Graph*> pinned;
    int graphs_alive = 0;
};

struct DeviceSlot {
    Device dev;
    Pool pool;
    std::mutex scratch_mu;
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    size_t scratch_requests = 0;  // scratch_area calls
    size_t scratch_mallocs = 0;   // hipMalloc calls made for the scratch area
    std::vector<void*> retired_scratch;  // outgrown while graphs that use it were alive
    bool ready = false;
};

// An instantiated capture and the pool blocks its nodes use.
struct Graph {
    hipGraphExec_t exec = nullptr;
    int device = -1;
    std::vector<std::pair<void*, size_t>> owned;  // back to the pool at destroy
    std::vector<void*> pinned;                    // entries of Pool::pinned for this graph
};

std::mutex g_init_mu;
DeviceSlot g_slots[kMaxDevices];

// Size classes: 256-byte granules up to 1 MiB, 64 KiB granules above.  A
// graph replays the same sizes every call, so exact-class reuse converges
// after one run (the reasoning of the reference's plan_memory docstring,
// python/kansai/kir.py:918-925).
size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    const size_t g = bytes <= (1u << 20) ? 256 : (64u << 10);
    return (bytes + g - 1) / g * g;
}

bool is_gfx950(int dev) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

int init_slot(int dev) {
    DeviceSlot& s = g_slots[dev];
    if (s.ready) return KH_OK;
    int rc = hip_status(hipSetDevice(dev), "hipSetDevice");
    if (rc) return rc;
    hipDeviceProp_t p;
    rc = hip_status(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    if (rc) return rc;
    s.dev.id = dev;
    s.dev.cus = p.multiProcessorCount;
    // Default priority on purpose (all streams at one priority).
    rc = hip_status(hipStreamCreateWithFlags(&s.dev.stream, hipStreamNonBlocking), "hipStreamCreate");
    if (rc) return rc;
    rc = hip_status(hipMalloc(reinterpret_cast<void**>(&s.dev.fault), 256), "hipMalloc(fault word)");
    if (rc) return rc;
    rc = hip_status(hipMemset(s.dev.fault, 0, 256), "hipMemset(fault word)");
    if (rc) return rc;
    // With `dev` current: this device's copy of the fixed no-alloc array.
    void* na = nullptr;
    rc = hip_status(hipGetSymbolAddress(&na, HIP_SYMBOL(::scratch)), "hipGetSymbolAddress(no-alloc scratch)");
    if (rc) return rc;
    s.dev.noalloc = static_cast<unsigned char*>(na);
    s.ready = true;
    return KH_OK;
}

}  // namespace

int fail(int code, const std::string& msg) {
    t_last_error = msg;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return KH_OK;
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? KH_ERR_OOM : KH_ERR_HIP;
    return fail(code, std::string(what) + ": " + hipGetErrorString(e));
}

int launch_status(const char* kernel) {
    return hip_status(hipGetLastError(), kernel);
}

Device* current() {
    int dev = t_device < 0 ? 0 : t_device;
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (!g_slots[dev].ready) {
            int n = 0;
            if (hipGetDeviceCount(&n) != hipSuccess || n <= dev) {
                fail(KH_ERR_NO_DEVICE, "kansai_hip: no HIP device available");
                return nullptr;
            }
            if (!is_gfx950(dev)) {
                fail(KH_ERR_NO_DEVICE, "kansai_hip: device is not gfx950 (MI355X); this backend targets gfx950 only");
                return nullptr;
            }
            if (init_slot(dev) != KH_OK) return nullptr;
        }
    }
    if (t_device != dev) {
        if (hipSetDevice(dev) != hipSuccess) {
            fail(KH_ERR_HIP, "hipSetDevice failed");
            return nullptr;
        }
        t_device = dev;
    }
    return &g_slots[dev].dev;
}

Device* current_initialized() {
    const int dev = t_device < 0 ? 0 : t_device;
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (!g_slots[dev].ready) {
            fail(KH_ERR_NO_DEVICE, "device not initialised: call kh_init (or any other entry point) first");
            return nullptr;
        }
    }
    if (t_device != dev) {
        if (hipSetDevice(dev) != hipSuccess) {
            fail(KH_ERR_HIP, "hipSetDevice failed");
            return nullptr;
        }
        t_device = dev;
    }
    return &g_slots[dev].dev;
}

void* scratch_area(Device* d, size_t bytes) {
    DeviceSlot& s = g_slots[d->id];
    std::lock_guard<std::mutex> lk(s.scratch_mu);
    ++s.scratch_requests;
    if (bytes <= s.scratch_bytes) return s.scratch;
    size_t want = bytes < (1u << 20) ? (1u << 20) : size_class(bytes);
    bool capturing, graphs;
    {
        std::lock_guard<std::mutex> plk(s.pool.mu);
        capturing = s.pool.capturing;
        graphs = s.pool.graphs_alive > 0;
    }
    if (capturing) {
        fail(KH_ERR_INVALID_ARG,
             "scratch area would grow during graph capture: run the work once on the stream before capturing it");
        return nullptr;
    }
    if (s.scratch && graphs) {
        // Captured graphs hold the old area's address: keep it until the
        // last of them is destroyed.
        s.retired_scratch.push_back(s.scratch);
        s.scratch = nullptr;
        s.scratch_bytes = 0;
    } else if (s.scratch) {
        // The old area may still be read by queued work.
        if (hipStreamSynchronize(d->stream) != hipSuccess) {
            fail(KH_ERR_HIP, "hipStreamSynchronize before growing scratch");
            return nullptr;
        }
        (void)hipFree(s.scratch);
        s.scratch = nullptr;
        s.scratch_bytes = 0;
    }
    void* p = nullptr;
    ++s.scratch_mallocs;
    if (hip_status(hipMalloc(&p, want), "hipMalloc(scratch)") != KH_OK) return nullptr;
    s.scratch = p;
    s.scratch_bytes = want;
    return p;
}

bool capturing(Device* d) {
    Pool& pool = g_slots[d->id].pool;
    std::lock_guard<std::mutex> lk(pool.mu);
    return pool.capturing;
}

}  // namespace kh

using kh::fail;
using kh::hip_status;


extern "C" {

int kh_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 0;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int kh_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(KH_ERR_NO_DEVICE, "kansai_hip: no HIP device available");
    if (device < 0 || device >= n || device >= kh::kMaxDevices)
        return fail(KH_ERR_INVALID_ARG, "kh_init: device index out of range");
    kh::t_device = device;
    return kh::current() ? KH_OK : KH_ERR_NO_DEVICE;
}

const char* kh_last_error(void) { return kh::t_last_error.c_str(); }

int kh_device_info(char* name, size_t name_len, int* cus, int* clock_khz, int* mem_clock_khz, int* bus_width,
                   size_t* total_mem) {
    KH_DEVICE_OR_RETURN(d);
    hipDeviceProp_t p;
    int rc = hip_status(hipGetDeviceProperties(&p, d->id), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && name_len) {
        std::strncpy(name, p.gcnArchName, name_len - 1);
        name[name_len - 1] = '\0';
    }
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (mem_clock_khz) *mem_clock_khz = p.memoryClockRate;
    if (bus_width) *bus_width = p.memoryBusWidth;
    if (total_mem) *total_mem = p.totalGlobalMem;
    return KH_OK;
}

int kh_synchronize(void) {
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_synchronize");
    int rc = hip_status(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
    if (rc) return rc;
    unsigned fault = 0;
    rc = hip_status(hipMemcpy(&fault, d->fault, sizeof(unsigned), hipMemcpyDeviceToHost), "read fault word");
    if (rc) return rc;
    if (fault) {
        const unsigned zero = 0;
        rc = hip_status(hipMemcpy(d->fault, &zero, sizeof(unsigned), hipMemcpyHostToDevice), "clear fault word");
        if (rc) return rc;
        if (fault & kh::kFaultNonFinite)
            return fail(KH_ERR_NONFINITE, "cannot quantize a non-finite value (NaN or inf)");
        if (fault & kh::kFaultBadIndex)
            return fail(KH_ERR_INVALID_ARG, "embedding: token id out of range");
    }
    return KH_OK;
}

int kh_get_stream(void** stream) {
    KH_REQUIRE(stream, "kh_get_stream: null out pointer");
    KH_DEVICE_OR_RETURN(d);
    *stream = d->stream;
    return KH_OK;
}

// ---- pool -------------------------------------------------------------------

int kh_alloc(size_t bytes, void** dptr) {
    KH_REQUIRE(dptr, "kh_alloc: null out pointer");
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    const size_t cls = kh::size_class(bytes);
    bool capturing;
    {
        std::lock_guard<std::mutex> lk(pool.mu);
        pool.requests += 1;
        capturing = pool.capturing;
        // While capturing, blocks freed by the capture come back first (the
        // same last-freed-first order as outside a capture).
        for (auto* lists : {capturing ? &pool.cap_free : nullptr, &pool.free_lists}) {
            if (!lists) continue;
            auto it = lists->find(cls);
            if (it != lists->end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                pool.live[p] = cls;
                pool.cached -= cls;
                pool.in_use += cls;
                if (capturing) pool.cap_used.push_back(p);
                *dptr = p;
                return KH_OK;
            }
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        kh_pool_trim();  // give cached blocks back and retry once
        e = hipMalloc(&p, cls);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(KH_ERR_OOM, "kh_alloc: out of device memory for " + std::to_string(bytes) + " bytes");
        }
    }
    std::lock_guard<std::mutex> lk(pool.mu);
    pool.live[p] = cls;
    pool.in_use += cls;
    pool.driver_allocs += 1;
    if (pool.capturing) pool.cap_used.push_back(p);
    *dptr = p;
    return KH_OK;
}

int kh_free(void* dptr) {
    if (!dptr) return KH_OK;
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    std::lock_guard<std::mutex> lk(pool.mu);
    auto it = pool.live.find(dptr);
    if (it == pool.live.end()) return fail(KH_ERR_INVALID_ARG, "kh_free: pointer was not allocated by kh_alloc");
    const size_t cls = it->second;
    pool.live.erase(it);
    pool.in_use -= cls;
    pool.cached += cls;
    auto pin = pool.pinned.find(dptr);
    if (pin != pool.pinned.end()) {
        pin->second->owned.emplace_back(dptr, cls);  // the graph still writes it
        pool.pinned.erase(pin);
    } else if (pool.capturing) {
        pool.cap_free[cls].push_back(dptr);
    } else {
        pool.free_lists[cls].push_back(dptr);
    }
    return KH_OK;
}

int kh_pool_trim(void) {
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_pool_trim");
    int rc = hip_status(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
    if (rc) return rc;
    kh::Pool& pool = kh::g_slots[d->id].pool;
    std::lock_guard<std::mutex> lk(pool.mu);
    for (auto& kv : pool.free_lists)
        for (void* p : kv.second) (void)hipFree(p);
    pool.free_lists.clear();
    pool.cached = 0;
    return KH_OK;
}

int kh_pool_stats(size_t* in_use, size_t* cached, size_t* driver_allocs) {
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    std::lock_guard<std::mutex> lk(pool.mu);
    if (in_use) *in_use = pool.in_use;
    if (cached) *cached = pool.cached;
    if (driver_allocs) *driver_allocs = pool.driver_allocs;
    return KH_OK;
}

int kh_pool_requests(size_t* requests) {
    KH_REQUIRE(requests, "kh_pool_requests: null out pointer");
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    std::lock_guard<std::mutex> lk(pool.mu);
    *requests = pool.requests;
    return KH_OK;
}

int kh_scratch_stats(size_t* bytes, size_t* requests, size_t* driver_allocs) {
    KH_DEVICE_OR_RETURN(d);
    kh::DeviceSlot& slot = kh::g_slots[d->id];
    std::lock_guard<std::mutex> lk(slot.scratch_mu);
    if (bytes) *bytes = slot.scratch_bytes;
    if (requests) *requests = slot.scratch_requests;
    if (driver_allocs) *driver_allocs = slot.scratch_mallocs;
    return KH_OK;
}

// ---- copies -------------------------------------------------------------------

int kh_memcpy_h2d(void* dst, const void* host_src, size_t bytes) {
    if (bytes == 0) return KH_OK;
    KH_REQUIRE(dst && host_src, "kh_memcpy_h2d: null pointer");
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_memcpy_h2d");
    int rc = hip_status(hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, d->stream), "hipMemcpyAsync(H2D)");
    if (rc) return rc;
    return hip_status(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
}

int kh_memcpy_d2h(void* host_dst, const void* src, size_t bytes) {
    if (bytes == 0) return KH_OK;
    KH_REQUIRE(host_dst && src, "kh_memcpy_d2h: null pointer");
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_memcpy_d2h");
    int rc = hip_status(hipMemcpyAsync(host_dst, src, bytes, hipMemcpyDeviceToHost, d->stream), "hipMemcpyAsync(D2H)");
    if (rc) return rc;
    return hip_status(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
}

// ---- events -------------------------------------------------------------------

int kh_event_create(void** event) {
    KH_REQUIRE(event, "kh_event_create: null out pointer");
    KH_DEVICE_OR_RETURN(d);
    hipEvent_t e;
    int rc = hip_status(hipEventCreate(&e), "hipEventCreate");
    if (rc) return rc;
    *event = e;
    return KH_OK;
}

int kh_event_record(void* event) {
    KH_REQUIRE(event, "kh_event_record: null event");
    KH_DEVICE_OR_RETURN(d);
    return hip_status(hipEventRecord(static_cast<hipEvent_t>(event), d->stream), "hipEventRecord");
}

int kh_event_elapsed_ms(void* start, void* end, float* ms) {
    KH_REQUIRE(start && end && ms, "kh_event_elapsed_ms: null argument");
    KH_DEVICE_OR_RETURN(d);
    KH_NOT_CAPTURING(d, "kh_event_elapsed_ms");
    int rc = hip_status(hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize");
    if (rc) return rc;
    return hip_status(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
                      "hipEventElapsedTime");
}

int kh_event_destroy(void* event) {
    if (!event) return KH_OK;
    return hip_status(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

// ---- graphs ---------------------------------------------------------------------

int kh_graph_capture_begin(void) {
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    {
        std::lock_guard<std::mutex> lk(pool.mu);
        KH_REQUIRE(!pool.capturing, "kh_graph_capture_begin: a capture is already in progress");
        pool.capturing = true;
        pool.cap_used.clear();
    }
    int rc = hip_status(hipStreamBeginCapture(d->stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    if (rc) {
        std::lock_guard<std::mutex> lk(pool.mu);
        pool.capturing = false;
    }
    return rc;
}

int kh_graph_capture_end(void** graph) {
    KH_DEVICE_OR_RETURN(d);
    kh::Pool& pool = kh::g_slots[d->id].pool;
    {
        std::lock_guard<std::mutex> lk(pool.mu);
        KH_REQUIRE(pool.capturing, "kh_graph_capture_end: no capture in progress");
    }
    if (graph) *graph = nullptr;
    hipGraph_t g = nullptr;
    int rc = hip_status(hipStreamEndCapture(d->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    if (!rc && graph) rc = hip_status(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (g) (void)hipGraphDestroy(g);
    std::lock_guard<std::mutex> lk(pool.mu);
    pool.capturing = false;
    if (rc || !graph) {
        // Nothing captured will run: the capture's blocks are ordinary again.
        for (auto& kv : pool.cap_free)
            for (void* p : kv.second) pool.free_lists[kv.first].push_back(p);
        pool.cap_free.clear();
        pool.cap_used.clear();
        if (exec) (void)hipGraphExecDestroy(exec);
        return rc;
    }
    auto* gr = new kh::Graph;
    gr->exec = exec;
    gr->device = d->id;
    for (auto& kv : pool.cap_free)
        for (void* p : kv.second) gr->owned.emplace_back(p, kv.first);
    pool.cap_free.clear();
    for (void* p : pool.cap_used)
        if (pool.live.count(p) && !pool.pinned.count(p)) {
            pool.pinned[p] = gr;
            gr->pinned.push_back(p);
        }
    pool.cap_used.clear();
    pool.graphs_alive += 1;
    *graph = gr;
    return KH_OK;
}

int kh_graph_launch(void* graph) {
    KH_REQUIRE(graph, "kh_graph_launch: null graph");
    KH_DEVICE_OR_RETURN(d);
    auto* gr = static_cast<kh::Graph*>(graph);
    KH_REQUIRE(gr->device == d->id, "kh_graph_launch: graph was captured on another device");
    KH_NOT_CAPTURING(d, "kh_graph_launch");
    return hip_status(hipGraphLaunch(gr->exec, d->stream), "hipGraphLaunch");
}

int kh_graph_destroy(void* graph) {
    if (!graph) return KH_OK;
    KH_DEVICE_OR_RETURN(d);
    auto* gr = static_cast<kh::Graph*>(graph);
    KH_REQUIRE(gr->device == d->id, "kh_graph_destroy: graph was captured on another device");
    KH_NOT_CAPTURING(d, "kh_graph_destroy");
    // A launch may still be running.
    int rc = hip_status(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
    if (rc) return rc;
    (void)hipGraphExecDestroy(gr->exec);
    kh::DeviceSlot& slot = kh::g_slots[d->id];
    bool last;
    {
        std::lock_guard<std::mutex> lk(slot.pool.mu);
        for (auto& b : gr->owned) slot.pool.free_lists[b.second].push_back(b.first);
        for (void* p : gr->pinned) {
            auto it = slot.pool.pinned.find(p);
            if (it != slot.pool.pinned.end() && it->second == gr) slot.pool.pinned.erase(it);
        }
        last = --slot.pool.graphs_alive == 0;
    }
    delete gr;
    if (last) {
        std::lock_guard<std::mutex> lk(slot.scratch_mu);
        for (void* p : slot.retired_scratch) (void)hipFree(p);
        slot.retired_scratch.clear();
    }
    return KH_OK;
}

}  // extern "C"
