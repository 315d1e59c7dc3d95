/*
 * musapy_hip_runtime.h -- thin C-ABI HIP runtime layer under the op layer.
 *
 * Replaces the MUSA runtime bindings and the memory/stream plumbing of musapy-core:
 *   rust/musapy-core/src/musa_ffi.rs:25-150      musaMalloc/Free/Memcpy/Stream/Event bindings
 *   rust/musapy-core/src/musa_ffi.rs:369-408     check_musa / check_last_kernel_launch
 *   rust/musapy-core/src/buffer_pool.rs:51-170    size-class cache of device buffers
 *   rust/musapy-core/src/deferred_free.rs:55-138  free-after-sync queue
 *   rust/musapy-core/src/mem_stats.rs:18-114      allocation counters
 * Device memory comes from a stream-aware caching allocator: sizes round up to 8 classes per
 * power of two, a freed block is cached with the stream its free was ordered on, reuse on that
 * stream is immediate and host-only, reuse from another stream is ordered by an event, and a
 * miss calls hipMalloc (after returning the cache to the device when memory runs out).  No call
 * blocks the host on device work except the copies to/from host memory and the synchronizes.
 * All functions return 0 on success or a hipError_t code (negative: a kernel-wrapper error).  A
 * failing call also clears HIP's per-thread "last error", so that code is reported once, by the
 * call that caused it, and not again by the next mpy_rt_check_launch.
 * Streams are always created with the default priority.
 */
#ifndef MUSAPY_HIP_RUNTIME_H
#define MUSAPY_HIP_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;

#ifdef __cplusplus
extern "C" {
#endif

int mpy_rt_device_count(int* count);
int mpy_rt_set_device(int device);
/* name / total HBM bytes / CU count / peak memory clock of a device */
int mpy_rt_device_info(int device, char* name, size_t name_len, size_t* total_mem, int* cu_count, int* arch_major,
                       int* arch_minor);

/* stream-ordered allocation on `device` (cached); `stream` may be NULL (null stream).  The block
 * may be used by work on `stream` right away; a free is ordered after the work queued on the
 * stream it names. */
int mpy_rt_malloc(void** ptr, size_t nbytes, int device, hipStream_t stream);
int mpy_rt_free(void* ptr, hipStream_t stream);
/* returns the cached (freed, unused) blocks of `device` (all devices when < 0) to the device;
 * synchronizes the device first */
int mpy_rt_empty_cache(int device);
/* bytes held in the cache of `device` (all devices when < 0) */
size_t mpy_rt_mem_cached(int device);

int mpy_rt_memcpy_h2d(void* dst, const void* src, size_t nbytes, hipStream_t stream);
int mpy_rt_memcpy_d2h(void* dst, const void* src, size_t nbytes, hipStream_t stream);
int mpy_rt_memcpy_d2d(void* dst, const void* src, size_t nbytes, hipStream_t stream);

int mpy_rt_stream_create(hipStream_t* stream, int device);
int mpy_rt_stream_destroy(hipStream_t stream);
int mpy_rt_stream_synchronize(hipStream_t stream);
int mpy_rt_device_synchronize(void);

int mpy_rt_event_create(hipEvent_t* event, int timing);
int mpy_rt_event_destroy(hipEvent_t event);
int mpy_rt_event_record(hipEvent_t event, hipStream_t stream);
int mpy_rt_stream_wait_event(hipStream_t stream, hipEvent_t event);
int mpy_rt_event_synchronize(hipEvent_t event);
int mpy_rt_event_elapsed_ms(float* ms, hipEvent_t start, hipEvent_t stop);

/* After a kernel-ABI call: returns the pending launch error (hipGetLastError) or, if none, the
 * kernel library's own wrapper error negated (musapy_kernels_take_error: -1 cumsum scratch,
 * -2 reduction tile too long, -3 bad rank or axis, -4 cumsum extent past 32 bits, -5 no-alloc
 * scratch too small). */
int mpy_rt_check_launch(void);
const char* mpy_rt_error_string(int code);

/* allocation statistics of this process: live bytes, high-water mark, allocation count */
void mpy_rt_mem_stats(size_t* live_bytes, size_t* peak_bytes, size_t* num_allocs);

/* Writes `nbytes` of a pattern to `ptr` with a kernel (graph-capture safe, unlike memset). */
int mpy_rt_fill_u32(void* ptr, uint32_t value, size_t nbytes, hipStream_t stream);

/* The wait-fault word of a workspace given to the kernel library (musapy_kernels_take_fault_ws),
 * read on `stream` through the runtime so that tests can inject it: 0, a fault bit set (the
 * workspace has been zeroed again), or -1. */
int mpy_rt_take_fault_ws(void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- test hooks (counterpart of the reference's mock runtime, musa_ffi.rs:154-355) ----
 * mpy_rt_set_backend(MPY_RT_BACKEND_HOST) swaps every HIP call of this layer for a host fake:
 * one device, memory from the C heap, copies as memcpy, streams and events as tokens,
 * synchronizes immediate, kernel launches without effect (their results are meaningless).  It
 * lets CPU-only tests drive the op layer's error paths.  It is refused (hipErrorNotSupported) on
 * a machine with a HIP device, where the kernels would be handed host pointers, and while memory
 * of the other backend is held.
 * mpy_rt_inject(call, code, skip, count): after `skip` more calls of the class, the next `count`
 * calls fail with `code` (a hipError_t; for MPY_RT_CALL_FAULT the fault bits to report), on
 * either backend.  count 0 disarms it. */
enum { MPY_RT_BACKEND_HIP = 0, MPY_RT_BACKEND_HOST = 1 };
enum {
  MPY_RT_CALL_MALLOC = 0, /* device allocation misses (hipMalloc) */
  MPY_RT_CALL_MEMCPY,     /* host<->device and device copies */
  MPY_RT_CALL_SYNC,       /* stream, device and event synchronizes */
  MPY_RT_CALL_LAUNCH,     /* the launch-error check after a kernel-ABI call */
  MPY_RT_CALL_FAULT,      /* a workspace's wait-fault word read after a synchronize */
  MPY_RT_CALL_EVENT,      /* event create / record / stream wait */
  MPY_RT_CALL_STREAM,     /* stream create */
  MPY_RT_CALL_COUNT
};
int mpy_rt_set_backend(int backend);
int mpy_rt_inject(int call, int code, int skip, int count);

#ifdef __cplusplus
}
#endif
#endif /* MUSAPY_HIP_RUNTIME_H */
