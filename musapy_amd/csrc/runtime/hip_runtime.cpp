// hip_runtime.cpp -- the C-ABI HIP runtime layer (include/musapy_hip_runtime.h).
//
// Stands in for rust/musapy-core/src/{musa_ffi,buffer_pool,deferred_free,mem_stats}.rs.
// Allocation is stream-ordered (hipMallocAsync) from the device's default pool whose release
// threshold is raised to "never", so freed blocks stay cached for reuse the way the reference's
// buffer pool keeps them (buffer_pool.rs:74-148), but reuse is ordered by the stream instead of
// by events.  If a device reports no memory-pool support, plain hipMalloc/hipFree are used.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "../../../include/musapy_hip_runtime.h"

extern "C" int musapy_kernels_take_error(void);

namespace {

std::atomic<size_t> g_live{0}, g_peak{0}, g_count{0};
std::mutex g_mu;
std::unordered_map<void*, size_t> g_sizes;  // live allocation sizes (for the counters)
int g_pool_state[64] = {0};                 // 0 unknown, 1 pool configured, 2 no pool support

int ensure_pool(int device) {
  if (device < 0 || device >= 64) return int(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_pool_state[device] != 0) return 0;
  int supported = 0;
  hipError_t e = hipDeviceGetAttribute(&supported, hipDeviceAttributeMemoryPoolsSupported, device);
  if (e != hipSuccess || !supported) {
    g_pool_state[device] = 2;
    return 0;
  }
  hipMemPool_t pool;
  e = hipDeviceGetDefaultMemPool(&pool, device);
  if (e != hipSuccess) {
    g_pool_state[device] = 2;
    return 0;
  }
  uint64_t threshold = UINT64_MAX;
  e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold);
  g_pool_state[device] = (e == hipSuccess) ? 1 : 2;
  return 0;
}

void note_alloc(void* p, size_t n) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    g_sizes[p] = n;
  }
  size_t live = g_live.fetch_add(n) + n;
  size_t peak = g_peak.load();
  while (live > peak && !g_peak.compare_exchange_weak(peak, live)) {
  }
  g_count.fetch_add(1);
}

void note_free(void* p) {
  size_t n = 0;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_sizes.find(p);
    if (it != g_sizes.end()) {
      n = it->second;
      g_sizes.erase(it);
    }
  }
  g_live.fetch_sub(n);
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = v;
}

}  // namespace

extern "C" {

int mpy_rt_device_count(int* count) { return int(hipGetDeviceCount(count)); }

int mpy_rt_set_device(int device) { return int(hipSetDevice(device)); }

int mpy_rt_device_info(int device, char* name, size_t name_len, size_t* total_mem, int* cu_count, int* arch_major,
                       int* arch_minor) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return int(e);
  if (name && name_len) {
    std::strncpy(name, prop.gcnArchName, name_len - 1);
    name[name_len - 1] = 0;
  }
  if (total_mem) *total_mem = prop.totalGlobalMem;
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (arch_major) *arch_major = prop.major;
  if (arch_minor) *arch_minor = prop.minor;
  return 0;
}

int mpy_rt_malloc(void** ptr, size_t nbytes, int device, hipStream_t stream) {
  *ptr = nullptr;
  if (nbytes == 0) nbytes = 1;  // a valid, unique pointer even for empty arrays
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return int(e);
  ensure_pool(device);
  if (g_pool_state[device] == 1)
    e = hipMallocAsync(ptr, nbytes, stream);
  else
    e = hipMalloc(ptr, nbytes);
  if (e != hipSuccess) {
    *ptr = nullptr;
    return int(e);
  }
  note_alloc(*ptr, nbytes);
  return 0;
}

int mpy_rt_free(void* ptr, hipStream_t stream) {
  if (!ptr) return 0;
  note_free(ptr);
  hipPointerAttribute_t attr;
  int device = 0;
  if (hipPointerGetAttributes(&attr, ptr) == hipSuccess) device = attr.device;
  if (device >= 0 && device < 64 && g_pool_state[device] == 1) return int(hipFreeAsync(ptr, stream));
  return int(hipFree(ptr));
}

int mpy_rt_memcpy_h2d(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return int(e);
  return int(hipStreamSynchronize(s));  // the host buffer may be released right after
}
int mpy_rt_memcpy_d2h(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return int(e);
  return int(hipStreamSynchronize(s));
}
int mpy_rt_memcpy_d2d(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  return int(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, s));
}

int mpy_rt_stream_create(hipStream_t* stream, int device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return int(e);
  return int(hipStreamCreateWithFlags(stream, hipStreamNonBlocking));
}
int mpy_rt_stream_destroy(hipStream_t stream) { return int(hipStreamDestroy(stream)); }
int mpy_rt_stream_synchronize(hipStream_t stream) { return int(hipStreamSynchronize(stream)); }
int mpy_rt_device_synchronize(void) { return int(hipDeviceSynchronize()); }

int mpy_rt_event_create(hipEvent_t* ev, int timing) {
  return int(hipEventCreateWithFlags(ev, timing ? hipEventDefault : hipEventDisableTiming));
}
int mpy_rt_event_destroy(hipEvent_t ev) { return int(hipEventDestroy(ev)); }
int mpy_rt_event_record(hipEvent_t ev, hipStream_t s) { return int(hipEventRecord(ev, s)); }
int mpy_rt_stream_wait_event(hipStream_t s, hipEvent_t ev) { return int(hipStreamWaitEvent(s, ev, 0)); }
int mpy_rt_event_synchronize(hipEvent_t ev) { return int(hipEventSynchronize(ev)); }
int mpy_rt_event_elapsed_ms(float* ms, hipEvent_t a, hipEvent_t b) { return int(hipEventElapsedTime(ms, a, b)); }

int mpy_rt_check_launch(void) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return int(e);
  return musapy_kernels_take_error() ? -1 : 0;
}

const char* mpy_rt_error_string(int code) {
  if (code == -1) return "kernel wrapper error: scratch buffer missing or too small";
  return hipGetErrorString(hipError_t(code));
}

void mpy_rt_mem_stats(size_t* live, size_t* peak, size_t* count) {
  if (live) *live = g_live.load();
  if (peak) *peak = g_peak.load();
  if (count) *count = g_count.load();
}

int mpy_rt_fill_u32(void* ptr, uint32_t value, size_t nbytes, hipStream_t stream) {
  size_t n = nbytes / 4;
  if (n == 0) return 0;
  size_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  k_fill_u32<<<dim3(unsigned(g)), 256, 0, stream>>>(static_cast<uint32_t*>(ptr), value, n);
  return int(hipGetLastError());
}

}  // extern "C"
