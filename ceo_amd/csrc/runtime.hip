// HIP device layer (include/efla_runtime.h), the launch profiler and the
// cached per-device workspace.
#include <hip/hip_runtime.h>
#include <string.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "../../include/efla_runtime.h"
#include "common.hpp"
#include "internal.hpp"

namespace efla {

// ---------------------------------------------------------------------------
// fill kernels
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) fill_kernel(T* __restrict__ p, float value, size_t n) {
    const T v = from_f<T>(value);
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ void __launch_bounds__(256) fill_f16_kernel(_Float16* __restrict__ p, float value,
                                                       size_t n) {
    const _Float16 v = (_Float16)value;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// Zeroes [p, p + bytes): head bytes up to 16-byte alignment, 16-byte words,
// then the tail bytes.
__global__ void __launch_bounds__(256) zero_kernel(uint8_t* __restrict__ p, size_t head,
                                                   size_t nwords, size_t tail) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4* w = reinterpret_cast<uint4*>(p + head);
    for (size_t i = i0; i < nwords; i += stride) w[i] = uint4{0u, 0u, 0u, 0u};
    if (i0 < head) p[i0] = 0;
    if (i0 < tail) p[head + nwords * 16 + i0] = 0;
}

static unsigned grid_for(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 8192) g = 8192;
    if (g == 0) g = 1;
    return (unsigned)g;
}

int fill_zero(void* ptr, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return kSuccess;
    size_t head = (16 - ((uintptr_t)ptr & 15u)) & 15u;
    if (head > bytes) head = bytes;
    const size_t nwords = (bytes - head) / 16;
    const size_t tail = bytes - head - nwords * 16;
    EFLA_LAUNCH("fill_zero", zero_kernel, dim3(grid_for(nwords)), dim3(256), stream,
                (uint8_t*)ptr, head, nwords, tail);
    return (int)hipPeekAtLastError();
}

// ---------------------------------------------------------------------------
// profiler
// ---------------------------------------------------------------------------
namespace {
struct ProfRec {
    const char* name;
    hipEvent_t e0, e1;
};
struct ProfState {
    std::mutex mu;
    bool on = false;
    std::vector<ProfRec> pending;
    std::vector<hipEvent_t> pool;
    std::map<std::string, std::pair<long long, double>> totals;
    std::vector<std::string> order;
};
ProfState& prof() {
    static ProfState s;
    return s;
}
hipEvent_t take_event(ProfState& s) {
    if (!s.pool.empty()) {
        hipEvent_t e = s.pool.back();
        s.pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace

bool prof_enabled() { return prof().on; }

void prof_begin(const char* name, hipStream_t stream, void** token) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    hipEvent_t e0 = take_event(s), e1 = take_event(s);
    if (!e0 || !e1) return;
    (void)hipEventRecord(e0, stream);
    s.pending.push_back(ProfRec{name, e0, e1});
    *token = (void*)(uintptr_t)s.pending.size();  // 1-based index
}

void prof_end(void* token, hipStream_t stream) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    const size_t idx = (size_t)(uintptr_t)token - 1;
    if (idx < s.pending.size()) (void)hipEventRecord(s.pending[idx].e1, stream);
}

}  // namespace efla

using namespace efla;

extern "C" {

void efla_prof_enable(int on) { prof().on = on != 0; }

void efla_prof_reset(void) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    for (auto& r : s.pending) {
        (void)hipEventSynchronize(r.e1);
        s.pool.push_back(r.e0);
        s.pool.push_back(r.e1);
    }
    s.pending.clear();
    s.totals.clear();
    s.order.clear();
}

int efla_prof_collect(void) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    int rc = kSuccess;
    for (auto& r : s.pending) {
        hipError_t e = hipEventSynchronize(r.e1);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.e0, r.e1);
        if (e != hipSuccess) {
            rc = (int)e;
        } else {
            auto it = s.totals.find(r.name);
            if (it == s.totals.end()) {
                s.order.push_back(r.name);
                s.totals[r.name] = {1, (double)ms};
            } else {
                it->second.first += 1;
                it->second.second += ms;
            }
        }
        s.pool.push_back(r.e0);
        s.pool.push_back(r.e1);
    }
    s.pending.clear();
    return rc;
}

int efla_prof_count(void) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    return (int)s.order.size();
}

int efla_prof_entry(int idx, char* name, size_t name_len, long long* launches,
                    double* total_ms) {
    ProfState& s = prof();
    std::lock_guard<std::mutex> g(s.mu);
    if (idx < 0 || (size_t)idx >= s.order.size()) return 1;
    const std::string& n = s.order[idx];
    if (name && name_len) {
        strncpy(name, n.c_str(), name_len - 1);
        name[name_len - 1] = 0;
    }
    auto& t = s.totals[n];
    if (launches) *launches = t.first;
    if (total_ms) *total_ms = t.second;
    return 0;
}

// --- devices ---------------------------------------------------------------
int efla_rt_device_count(int* count) { return (int)hipGetDeviceCount(count); }
int efla_rt_set_device(int device) { return (int)hipSetDevice(device); }
int efla_rt_get_device(int* device) { return (int)hipGetDevice(device); }
int efla_rt_device_synchronize(void) { return (int)hipDeviceSynchronize(); }

int efla_rt_device_info(int device, char* name, size_t name_len, int* compute_units,
                        int* clock_khz, size_t* total_mem, int* lds_per_block,
                        int* warp_size) {
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return (int)e;
    if (name && name_len) {
        strncpy(name, p.gcnArchName, name_len - 1);
        name[name_len - 1] = 0;
    }
    if (compute_units) *compute_units = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (total_mem) *total_mem = p.totalGlobalMem;
    if (lds_per_block) *lds_per_block = (int)p.sharedMemPerBlock;
    if (warp_size) *warp_size = p.warpSize;
    return kSuccess;
}

// --- memory ----------------------------------------------------------------
int efla_rt_malloc(void** ptr, size_t bytes) { return (int)hipMalloc(ptr, bytes); }
int efla_rt_free(void* ptr) { return (int)hipFree(ptr); }
int efla_rt_host_malloc(void** ptr, size_t bytes) {
    return (int)hipHostMalloc(ptr, bytes, hipHostMallocDefault);
}
int efla_rt_host_free(void* ptr) { return (int)hipHostFree(ptr); }

static hipMemcpyKind kind_of(int kind) {
    switch (kind) {
        case 0: return hipMemcpyHostToHost;
        case 1: return hipMemcpyHostToDevice;
        case 2: return hipMemcpyDeviceToHost;
        case 3: return hipMemcpyDeviceToDevice;
        default: return hipMemcpyDefault;
    }
}

int efla_rt_memcpy(void* dst, const void* src, size_t bytes, int kind) {
    return (int)hipMemcpy(dst, src, bytes, kind_of(kind));
}
int efla_rt_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                         hipStream_t stream) {
    return (int)hipMemcpyAsync(dst, src, bytes, kind_of(kind), stream);
}
int efla_rt_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
    return (int)hipMemGetInfo(free_bytes, total_bytes);
}

int efla_rt_fill(void* ptr, float value, size_t numel, int dtype, hipStream_t stream) {
    if (numel == 0) return kSuccess;
    if (ptr == nullptr) return kInvalidValue;
    const dim3 g(grid_for(numel)), b(256);
    switch (dtype) {
        case kDtypeF32:
            EFLA_LAUNCH("fill", fill_kernel<float>, g, b, stream, (float*)ptr, value, numel);
            break;
        case kDtypeBF16:
            EFLA_LAUNCH("fill", fill_kernel<bf16>, g, b, stream, (bf16*)ptr, value, numel);
            break;
        case kDtypeF16:
            EFLA_LAUNCH("fill", fill_f16_kernel, g, b, stream, (_Float16*)ptr, value, numel);
            break;
        default:
            return kInvalidValue;
    }
    return (int)hipPeekAtLastError();
}

// --- streams / events ---------------------------------------------------------
int efla_rt_stream_create(hipStream_t* stream) { return (int)hipStreamCreate(stream); }
int efla_rt_stream_destroy(hipStream_t stream) {
    // the stream's cached workspaces go first, while its handle still names it
    const int rc = efla_rt_workspace_release_stream(stream);
    if (rc != kSuccess) return rc;
    return (int)hipStreamDestroy(stream);
}
int efla_rt_stream_synchronize(hipStream_t stream) { return (int)hipStreamSynchronize(stream); }
int efla_rt_event_create(hipEvent_t* event) { return (int)hipEventCreate(event); }
int efla_rt_event_destroy(hipEvent_t event) { return (int)hipEventDestroy(event); }
int efla_rt_event_record(hipEvent_t event, hipStream_t stream) {
    return (int)hipEventRecord(event, stream);
}
int efla_rt_event_synchronize(hipEvent_t event) { return (int)hipEventSynchronize(event); }
int efla_rt_event_elapsed_ms(float* ms, hipEvent_t start, hipEvent_t stop) {
    return (int)hipEventElapsedTime(ms, start, stop);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------
namespace efla {

struct WsEntry {
    std::mutex mu;  // held by the lease for as long as a caller uses the buffer
    // the thread holding mu (default id when free): only that thread stores
    // its own id here, so it alone can see it and refuse a second lease
    std::atomic<std::thread::id> owner{};
    void* ptr = nullptr;
    size_t bytes = 0;
};

namespace {
typedef std::tuple<int, hipStream_t, int> WsKey;  // (device, stream, slot)
std::mutex g_ws_mu;                                // guards the map, not the entries
std::map<WsKey, std::unique_ptr<WsEntry>> g_ws;

// An entry is erased only by efla_rt_workspace_release_stream, whose caller
// guarantees that no other thread uses that stream meanwhile, so the pointer
// stays valid for as long as its (device, stream) is in use.
WsEntry* ws_entry(int dev, hipStream_t stream, int slot) {
    std::lock_guard<std::mutex> g(g_ws_mu);
    std::unique_ptr<WsEntry>& e = g_ws[WsKey(dev, stream, slot)];
    if (!e) e.reset(new WsEntry);
    return e.get();
}
}  // namespace

void WsLease::release() {
    if (entry) {
        entry->owner.store(std::thread::id());
        entry->mu.unlock();
    }
    entry = nullptr;
}

int workspace_acquire(size_t bytes, hipStream_t stream, void** ptr, WsLease& lease, int slot) {
    if (lease.entry) return kInvalidValue;  // one buffer per lease
    int dev = 0;
    EFLA_CHECK(hipGetDevice(&dev));
    WsEntry* e = ws_entry(dev, stream, slot);
    // a second lease on one (stream, slot) from the holding thread would wait
    // on itself forever: report the misuse instead
    if (e->owner.load() == std::this_thread::get_id()) return kInvalidValue;
    e->mu.lock();
    e->owner.store(std::this_thread::get_id());
    lease.entry = e;
    if (e->bytes < bytes) {
        if (e->ptr) {
            // every earlier user of this buffer queued its work on `stream`
            EFLA_CHECK(hipStreamSynchronize(stream));
            EFLA_CHECK(hipFree(e->ptr));
            e->ptr = nullptr;
            e->bytes = 0;
        }
        // round up to 64 MiB steps so slowly growing problems do not realloc
        const size_t step = (size_t)64 << 20;
        const size_t want = (bytes + step - 1) / step * step;
        EFLA_CHECK(hipMalloc(&e->ptr, want));
        e->bytes = want;
    }
    *ptr = e->ptr;
    return kSuccess;
}

int device_cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64) {
        const int c = cached[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    if (n > 0 && dev < 64) cached[dev].store(n, std::memory_order_relaxed);
    return n;
}
}  // namespace efla

namespace efla {
namespace {
// the current device's entries; the map lock is not held
// while an entry is locked (a lease holder may be waiting for the map lock)
std::vector<WsEntry*> device_entries(int dev) {
    std::vector<WsEntry*> out;
    std::lock_guard<std::mutex> g(g_ws_mu);
    for (auto& kv : g_ws)
        if (std::get<0>(kv.first) == dev) out.push_back(kv.second.get());
    return out;
}
}  // namespace
}  // namespace efla

extern "C" size_t efla_rt_workspace_bytes(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    size_t total = 0;
    for (efla::WsEntry* e : efla::device_entries(dev)) {
        std::lock_guard<std::mutex> ge(e->mu);
        total += e->bytes;
    }
    return total;
}

extern "C" int efla_rt_workspace_release_stream(hipStream_t stream) {
    int dev = 0;
    EFLA_CHECK(hipGetDevice(&dev));
    std::vector<efla::WsKey> keys;
    std::vector<efla::WsEntry*> entries;
    {
        std::lock_guard<std::mutex> g(efla::g_ws_mu);
        for (auto& kv : efla::g_ws)
            if (std::get<0>(kv.first) == dev && std::get<1>(kv.first) == stream) {
                keys.push_back(kv.first);
                entries.push_back(kv.second.get());
            }
    }
    if (keys.empty()) return kSuccess;
    // everything queued on the stream, which may still read these buffers
    EFLA_CHECK(hipStreamSynchronize(stream));
    for (efla::WsEntry* e : entries) {
        std::lock_guard<std::mutex> ge(e->mu);  // a lease still launching finishes first
        if (e->ptr) EFLA_CHECK(hipFree(e->ptr));
        e->ptr = nullptr;
        e->bytes = 0;
    }
    std::lock_guard<std::mutex> g(efla::g_ws_mu);
    for (const efla::WsKey& k : keys) efla::g_ws.erase(k);
    return kSuccess;
}

extern "C" int efla_rt_workspace_release(void) {
    int dev = 0;
    EFLA_CHECK(hipGetDevice(&dev));
    for (efla::WsEntry* ep : efla::device_entries(dev)) {
        efla::WsEntry& e = *ep;
        std::lock_guard<std::mutex> ge(e.mu);  // waits for a caller still launching
        if (e.ptr) {
            // after the lock: work a caller queued while this call waited is
            // done too (the stream itself may since have been destroyed)
            EFLA_CHECK(hipDeviceSynchronize());
            EFLA_CHECK(hipFree(e.ptr));
        }
        e.ptr = nullptr;
        e.bytes = 0;
    }
    return kSuccess;
}
