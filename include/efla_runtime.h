/*
 * efla_runtime.h -- HIP device layer for the EFLA host.
 *
 * Takes the place of the reference's CUDA runtime bindings
 * (src/runtime/cuda.zig: cudart externs 140-172, CudaStream 291-314,
 * CudaEvent 317-351, CudaDevice 354-402, cudaMalloc helper 461-467, and the
 * fill/cast stubs 490-505) so the host can manage devices, memory, streams and
 * events without linking CUDA.  All functions return hipError_t codes as int.
 * Streams are created at the default priority.
 */
#ifndef EFLA_RUNTIME_H
#define EFLA_RUNTIME_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- devices (CudaDevice, cuda.zig:354-402) --- */
int efla_rt_device_count(int* count);
int efla_rt_set_device(int device);
int efla_rt_get_device(int* device);
int efla_rt_device_synchronize(void);
/* name: caller buffer of name_len bytes; any output pointer may be NULL */
int efla_rt_device_info(int device, char* name, size_t name_len, int* compute_units,
                        int* clock_khz, size_t* total_mem, int* lds_per_block,
                        int* warp_size);

/* --- memory (cudaMalloc/cudaFree/cudaMemcpy*, cuda.zig:140-172, 461-467) --- */
int efla_rt_malloc(void** ptr, size_t bytes);
int efla_rt_free(void* ptr);
int efla_rt_host_malloc(void** ptr, size_t bytes); /* pinned host memory */
int efla_rt_host_free(void* ptr);
/* kind: 0 host->host, 1 host->device, 2 device->host, 3 device->device, 4 default */
int efla_rt_memcpy(void* dst, const void* src, size_t bytes, int kind);
int efla_rt_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                         hipStream_t stream);
int efla_rt_mem_get_info(size_t* free_bytes, size_t* total_bytes);

/* Fill numel elements of dtype (EFLA_DTYPE_F32/F16/BF16) with value, through a
 * kernel on `stream`.  Replaces the no-op cudaFill stub (cuda.zig:490-496) and
 * fill_cuda (kernels.h:352-358). */
int efla_rt_fill(void* ptr, float value, size_t numel, int dtype, hipStream_t stream);

/* --- streams (CudaStream, cuda.zig:291-314) --- */
int efla_rt_stream_create(hipStream_t* stream);
/* Releases the stream's cached library workspaces
 * (efla_rt_workspace_release_stream), then destroys it. */
int efla_rt_stream_destroy(hipStream_t stream);
int efla_rt_stream_synchronize(hipStream_t stream);

/* --- events (CudaEvent, cuda.zig:317-351) --- */
int efla_rt_event_create(hipEvent_t* event);
int efla_rt_event_destroy(hipEvent_t event);
int efla_rt_event_record(hipEvent_t event, hipStream_t stream);
int efla_rt_event_synchronize(hipEvent_t event);
int efla_rt_event_elapsed_ms(float* ms, hipEvent_t start, hipEvent_t stop);

/* --- library workspace ---
 * Entry points that need scratch and are given none use buffers the library
 * caches per (device, stream): callers on different streams never share
 * scratch, and calls on one stream from several host threads take turns
 * while they queue their kernels.  A buffer grows (after its stream drains)
 * only when a larger problem arrives. */
/* Bytes currently held by the cached workspaces of the current device. */
size_t efla_rt_workspace_bytes(void);
/* Release the cached workspaces of the current device (synchronises it). */
int efla_rt_workspace_release(void);
/* Release the cached workspaces of one stream on the current device: waits
 * for the stream, frees its buffers and forgets it, so a later stream that
 * receives the same handle value starts with none.  Call it before
 * hipStreamDestroy on any stream the library's entry points were given
 * (efla_rt_stream_destroy does so itself), and not while another thread
 * issues library calls on that stream.  No counterpart in the reference (its
 * entry points allocate and free scratch per call, efla.cu:631-647,
 * 695-696). */
int efla_rt_workspace_release_stream(hipStream_t stream);

/* GEMM backend of the gemm_* entries for this process: 0 (default) the
 * library's hand-written kernels (the large-tile kernel where it takes the
 * problem, else the generic one); 1 the generic hand-written kernel only.
 * Other values -> 1.  No vendor BLAS is linked. */
int efla_rt_set_gemm_backend(int backend);

/* --- launch profiler ---
 * While enabled, each kernel the library launches is bracketed by hipEvents
 * recorded on its stream.  efla_prof_collect() waits for the recorded events
 * and folds them into per-kernel totals; efla_prof_entry() reads them back
 * by index (returns 1 when idx is out of range). */
void efla_prof_enable(int on);
void efla_prof_reset(void);
int efla_prof_collect(void);
int efla_prof_count(void);
int efla_prof_entry(int idx, char* name, size_t name_len, long long* launches,
                    double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* EFLA_RUNTIME_H */
