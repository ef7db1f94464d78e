// Host-side internals shared by the library's translation units: checked size
// arithmetic, the per-launch profiler and the cached per-device workspace.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <limits>

namespace efla {

// Return codes are hipError_t values; the ones the reference ABI uses have the
// same numbers as their cudaError_t counterparts (0, 1, 2, 9).
constexpr int kSuccess = hipSuccess;
constexpr int kInvalidValue = hipErrorInvalidValue;
constexpr int kOutOfMemory = hipErrorOutOfMemory;
constexpr int kInvalidConfiguration = hipErrorInvalidConfiguration;
constexpr int kNotSupported = hipErrorNotSupported;

// dtype codes shared with hipDataType (library_types.h): HIP_R_32F = 0,
// HIP_R_16F = 2, HIP_R_16BF = 14 -- numerically the reference's cudaDataType codes.
constexpr int kDtypeF32 = 0;
constexpr int kDtypeF16 = 2;
constexpr int kDtypeBF16 = 14;

inline bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a) return false;
    *out = a * b;
    return true;
}

inline bool mul_ok(size_t a, size_t b, size_t c, size_t* out) {
    size_t t;
    return mul_ok(a, b, &t) && mul_ok(t, c, out);
}

inline bool mul_ok(size_t a, size_t b, size_t c, size_t d, size_t* out) {
    size_t t;
    return mul_ok(a, b, c, &t) && mul_ok(t, d, out);
}

// --- profiler -------------------------------------------------------------
// When enabled, every kernel launch made through EFLA_LAUNCH is bracketed by
// two hipEvents recorded on the launch stream; prof_collect() waits for them
// and accumulates per-kernel launch counts and total milliseconds.
bool prof_enabled();
void prof_begin(const char* name, hipStream_t stream, void** token);
void prof_end(void* token, hipStream_t stream);

struct ProfScope {
    void* token = nullptr;
    hipStream_t stream;
    ProfScope(const char* name, hipStream_t s) : stream(s) {
        if (prof_enabled()) prof_begin(name, s, &token);
    }
    ~ProfScope() {
        if (token) prof_end(token, stream);
    }
};

#define EFLA_LAUNCH(name, kernel, grid, block, stream, ...)                         \
    do {                                                                             \
        ::efla::ProfScope _efla_ps(name, stream);                                    \
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, __VA_ARGS__);             \
    } while (0)

#define EFLA_CHECK(expr)                      \
    do {                                      \
        hipError_t _e = (expr);               \
        if (_e != hipSuccess) return (int)_e; \
    } while (0)

// --- workspace ------------------------------------------------------------
// The library's cached scratch buffers, one per (device, stream, slot).  A
// call that needs scratch takes a lease on the buffer of its own stream and
// keeps it until its kernels are queued: the lease holds the buffer's lock, so
// two host threads on one stream take turns, and callers on different streams
// never share memory.  A buffer that has to grow is freed only after its
// stream has drained (every earlier user of it queued its work on that
// stream, under the same lock), then reallocated; steady-state calls allocate
// nothing.  Slot 0 is general scratch, slot 1 the GEMM library's workspace.
struct WsEntry;
class WsLease {
   public:
    WsLease() = default;
    WsLease(const WsLease&) = delete;
    WsLease& operator=(const WsLease&) = delete;
    ~WsLease() { release(); }
    void release();
    WsEntry* entry = nullptr;
};

// Returns in *ptr a buffer of at least `bytes` for `stream` on the current
// device, valid while `lease` is held.  A lease covers one buffer; a caller
// never takes a second lease on the same (stream, slot) while holding one.
int workspace_acquire(size_t bytes, hipStream_t stream, void** ptr, WsLease& lease,
                      int slot = 0);

// Zero-fill through a kernel (no hipMemsetAsync, so the call is safe inside
// stream capture).
int fill_zero(void* ptr, size_t bytes, hipStream_t stream);
// y[c] = sum_r x[r][c] for bf16 x [M][N] (fp32 sums in a fixed order, bf16 y)
int colsum_bf16_rows(const __bf16* x, long M, long N, __bf16* y, hipStream_t stream);

// Compute units of the current device (cached per device); 0 if the query fails.
int device_cu_count();

}  // namespace efla
