// hip_runtime.cpp -- the C-ABI HIP runtime layer (include/musapy_hip_runtime.h).
//
// Stands in for rust/musapy-core/src/{musa_ffi,buffer_pool,deferred_free,mem_stats}.rs.
//
// Device memory comes from a stream-aware caching allocator, the counterpart of the reference's
// size-class buffer pool (buffer_pool.rs:51-170) and its free-after-sync queue
// (deferred_free.rs:55-138):
//   * sizes are rounded up to one of 8 classes per power of two (at most 12.5% slack; 512 B
//     minimum), and a freed block goes to a per-device free list tagged with the stream its free
//     was ordered on;
//   * an allocation on that same stream reuses the block at once -- stream order already puts the
//     new work after every earlier use -- with no HIP call at all; the most recently freed block
//     of the class is taken first;
//   * reuse from another stream first makes the allocating stream wait on an event recorded on
//     the freeing stream;
//   * a miss calls hipMalloc; when that runs out of memory, the cache is returned to the device
//     (after a device synchronize) and the allocation is tried once more.
// hipMallocAsync/hipFreeAsync on the default memory pool were measured to block the host until
// the device drains (host time per op equal to its GPU time), which is what this avoids.
// All functions return 0 on success or a hipError_t code.  Streams are always created with the
// default priority.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../../include/musapy_hip_runtime.h"

extern "C" int musapy_kernels_take_error(void);

namespace {

constexpr int kMaxDevices = 64;

struct Block {
  void* ptr;
  size_t size;         // size class actually allocated
  size_t requested;    // bytes the caller asked for (statistics)
  hipStream_t stream;  // stream the last free was ordered on (or the owner while live)
  bool idle;           // no work can be pending on it (its stream was synchronized and destroyed)
};

struct DevicePool {
  std::multimap<size_t, Block> free;         // size class -> cached blocks
  std::unordered_map<void*, Block> live;     // blocks held by callers
  size_t cached_bytes = 0;
};

std::mutex g_mu;
DevicePool g_pools[kMaxDevices];
std::atomic<size_t> g_live{0}, g_peak{0}, g_count{0};

size_t size_class(size_t n) {
  if (n <= 512) return 512;
  const int lg = 63 - __builtin_clzll(uint64_t(n - 1));  // n - 1 >= 512, so lg >= 9
  const size_t step = size_t(1) << (lg - 3);
  return (n + step - 1) / step * step;
}

void note_alloc(size_t n) {
  size_t live = g_live.fetch_add(n) + n;
  size_t peak = g_peak.load();
  while (live > peak && !g_peak.compare_exchange_weak(peak, live)) {
  }
  g_count.fetch_add(1);
}

// The return value of a runtime call.  A failing HIP call also leaves its code as the thread's
// "last error", which the next launch check would report against an unrelated kernel; the
// caller is told here instead, so the sticky copy is consumed.
int rc(hipError_t e) {
  if (e != hipSuccess) (void)hipGetLastError();
  return int(e);
}

// make `waiter` wait for everything queued so far on `target`
hipError_t order_after(hipStream_t waiter, hipStream_t target) {
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return e;
  e = hipEventRecord(ev, target);
  if (e == hipSuccess) e = hipStreamWaitEvent(waiter, ev, 0);
  hipEventDestroy(ev);
  return e;
}

// returns every cached block of `device` to the device; the caller holds g_mu
hipError_t release_cached_locked(int device) {
  DevicePool& P = g_pools[device];
  if (P.free.empty()) return hipSuccess;
  int prev = 0;
  hipGetDevice(&prev);
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return e;
  e = hipDeviceSynchronize();  // frees were stream-ordered: their work must be done
  for (auto& kv : P.free) hipFree(kv.second.ptr);
  P.free.clear();
  P.cached_bytes = 0;
  hipSetDevice(prev);
  return e;
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = v;
}

}  // namespace

extern "C" {

int mpy_rt_device_count(int* count) { return rc(hipGetDeviceCount(count)); }

int mpy_rt_set_device(int device) { return rc(hipSetDevice(device)); }

int mpy_rt_device_info(int device, char* name, size_t name_len, size_t* total_mem, int* cu_count, int* arch_major,
                       int* arch_minor) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return rc(e);
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
  if (device < 0 || device >= kMaxDevices) return rc(hipErrorInvalidDevice);
  const size_t cls = size_class(nbytes ? nbytes : 1);  // a valid, unique pointer even for empty arrays
  std::lock_guard<std::mutex> lk(g_mu);
  DevicePool& P = g_pools[device];
  auto range = P.free.equal_range(cls);
  if (range.first != range.second) {
    // Prefer the most recently freed block of this stream (or one with nothing pending): frees
    // are appended at the end of their size class, so walk the class backwards.  The latest
    // block is the one most likely still held in the Infinity Cache: an op whose output is freed
    // and allocated again each call then writes the same memory each time.  With no such block,
    // take the oldest one, whose pending work is the most likely to be done.
    auto pick = range.first;
    for (auto it = range.second; it != range.first;) {
      --it;
      if (it->second.idle || it->second.stream == stream) {
        pick = it;
        break;
      }
    }
    Block b = pick->second;
    if (!b.idle && b.stream != stream) {
      hipError_t e = order_after(stream, b.stream);
      if (e != hipSuccess) return rc(e);
    }
    P.free.erase(pick);
    P.cached_bytes -= b.size;
    b.stream = stream;
    b.idle = false;
    b.requested = nbytes;
    P.live[b.ptr] = b;
    note_alloc(nbytes);
    *ptr = b.ptr;
    return 0;
  }
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return rc(e);
  void* p = nullptr;
  e = hipMalloc(&p, cls);
  if (e == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    for (int d = 0; d < kMaxDevices; ++d)
      if (!g_pools[d].free.empty()) release_cached_locked(d);
    hipSetDevice(device);
    e = hipMalloc(&p, cls);
  }
  if (e != hipSuccess) return rc(e);
  P.live[p] = Block{p, cls, nbytes, stream, false};
  note_alloc(nbytes);
  *ptr = p;
  return 0;
}

int mpy_rt_free(void* ptr, hipStream_t stream) {
  if (!ptr) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  for (int d = 0; d < kMaxDevices; ++d) {
    DevicePool& P = g_pools[d];
    auto it = P.live.find(ptr);
    if (it == P.live.end()) continue;
    Block b = it->second;
    P.live.erase(it);
    g_live.fetch_sub(b.requested);
    b.stream = stream;
    b.idle = false;
    P.free.emplace(b.size, b);
    P.cached_bytes += b.size;
    return 0;
  }
  return rc(hipFree(ptr));  // not from this allocator
}

int mpy_rt_empty_cache(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (device >= 0) return device < kMaxDevices ? int(release_cached_locked(device)) : int(hipErrorInvalidDevice);
  hipError_t first = hipSuccess;
  for (int d = 0; d < kMaxDevices; ++d) {
    hipError_t e = release_cached_locked(d);
    if (first == hipSuccess) first = e;
  }
  return rc(first);
}

int mpy_rt_memcpy_h2d(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return rc(e);
  return rc(hipStreamSynchronize(s));  // the host buffer may be released right after
}
int mpy_rt_memcpy_d2h(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return rc(e);
  return rc(hipStreamSynchronize(s));
}
int mpy_rt_memcpy_d2d(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  return rc(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, s));
}

int mpy_rt_stream_create(hipStream_t* stream, int device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return rc(e);
  return rc(hipStreamCreateWithFlags(stream, hipStreamNonBlocking));
}
int mpy_rt_stream_destroy(hipStream_t stream) {
  // cached blocks last freed on this stream outlive it: drain it, then mark them idle so no
  // later reuse records an event on the destroyed handle
  hipError_t e = hipStreamSynchronize(stream);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (int d = 0; d < kMaxDevices; ++d) {
      for (auto& kv : g_pools[d].free)
        if (kv.second.stream == stream) kv.second.idle = true;
      for (auto& kv : g_pools[d].live)
        if (kv.second.stream == stream) kv.second.idle = true;
    }
  }
  hipError_t e2 = hipStreamDestroy(stream);
  return rc(e != hipSuccess ? e : e2);
}
int mpy_rt_stream_synchronize(hipStream_t stream) { return rc(hipStreamSynchronize(stream)); }
int mpy_rt_device_synchronize(void) { return rc(hipDeviceSynchronize()); }

int mpy_rt_event_create(hipEvent_t* ev, int timing) {
  return rc(hipEventCreateWithFlags(ev, timing ? hipEventDefault : hipEventDisableTiming));
}
int mpy_rt_event_destroy(hipEvent_t ev) { return rc(hipEventDestroy(ev)); }
int mpy_rt_event_record(hipEvent_t ev, hipStream_t s) { return rc(hipEventRecord(ev, s)); }
int mpy_rt_stream_wait_event(hipStream_t s, hipEvent_t ev) { return rc(hipStreamWaitEvent(s, ev, 0)); }
int mpy_rt_event_synchronize(hipEvent_t ev) { return rc(hipEventSynchronize(ev)); }
int mpy_rt_event_elapsed_ms(float* ms, hipEvent_t a, hipEvent_t b) { return rc(hipEventElapsedTime(ms, a, b)); }

int mpy_rt_check_launch(void) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return rc(e);
  const int w = musapy_kernels_take_error();
  return w ? -w : 0;
}

const char* mpy_rt_error_string(int code) {
  if (code == -1) return "kernel wrapper error: cumsum scratch buffer missing or too small";
  if (code == -2) return "kernel wrapper error: a reduction tile reaches 2^31 elements (pass more tiles)";
  if (code == -3) return "kernel wrapper error: ndim outside [0, 32] or axis outside [0, ndim)";
  if (code == -4) return "kernel wrapper error: a cumsum with 2^32 or more rows (or a non-axis extent of 2^32 or more)";
  if (code == -5) return "kernel wrapper error: the reduction needs more scratch than the no-alloc entry point holds";
  if (code < 0) return "kernel wrapper error";
  return hipGetErrorString(hipError_t(code));
}

void mpy_rt_mem_stats(size_t* live, size_t* peak, size_t* count) {
  if (live) *live = g_live.load();
  if (peak) *peak = g_peak.load();
  if (count) *count = g_count.load();
}

size_t mpy_rt_mem_cached(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (device >= 0) return device < kMaxDevices ? g_pools[device].cached_bytes : 0;
  size_t t = 0;
  for (int d = 0; d < kMaxDevices; ++d) t += g_pools[d].cached_bytes;
  return t;
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
