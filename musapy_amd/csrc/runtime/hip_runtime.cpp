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
//
// Every HIP call goes through a call table (Calls).  The default table calls HIP.  Tests can
// swap in a host-memory table (mpy_rt_set_backend) that runs the whole op layer on a machine
// without a GPU -- device memory is host memory, copies are memcpy, streams and events are
// tokens, kernel launches do nothing -- and can arm one-shot errors on any call class
// (mpy_rt_inject), on either table.  This is the counterpart of the reference's mock runtime
// (rust/musapy-core/src/musa_ffi.rs:154-355) for testing the error paths: launch errors,
// synchronize errors, device wait faults, allocation failures.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../../include/musapy_hip_runtime.h"
#include "../../../include/musapy_kernels.h"

namespace {

constexpr int kMaxDevices = 64;

// ---------------------------------------------------------------------------------------------
// the call table
struct Calls {
  hipError_t (*device_count)(int*);
  hipError_t (*set_device)(int);
  hipError_t (*get_device)(int*);
  hipError_t (*device_info)(int, char*, size_t, size_t*, int*, int*, int*);
  hipError_t (*malloc)(void**, size_t);
  hipError_t (*free)(void*);
  hipError_t (*memcpy_async)(void*, const void*, size_t, hipMemcpyKind, hipStream_t);
  hipError_t (*stream_create)(hipStream_t*);
  hipError_t (*stream_destroy)(hipStream_t);
  hipError_t (*stream_sync)(hipStream_t);
  hipError_t (*device_sync)();
  hipError_t (*event_create)(hipEvent_t*, unsigned);
  hipError_t (*event_destroy)(hipEvent_t);
  hipError_t (*event_record)(hipEvent_t, hipStream_t);
  hipError_t (*stream_wait_event)(hipStream_t, hipEvent_t);
  hipError_t (*event_sync)(hipEvent_t);
  hipError_t (*event_elapsed)(float*, hipEvent_t, hipEvent_t);
  hipError_t (*last_error)();  // the pending launch error, consumed
  hipError_t (*fill_u32)(void*, uint32_t, size_t, hipStream_t);
  int (*take_fault_ws)(void*, size_t, hipStream_t);  // a workspace's wait-fault word (kernel library)
};

__global__ void k_fill_u32(uint32_t* p, uint32_t v, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = v;
}

hipError_t hip_device_info(int device, char* name, size_t name_len, size_t* total_mem, int* cu_count, int* major,
                           int* minor) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return e;
  if (name && name_len) {
    std::strncpy(name, prop.gcnArchName, name_len - 1);
    name[name_len - 1] = 0;
  }
  if (total_mem) *total_mem = prop.totalGlobalMem;
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (major) *major = prop.major;
  if (minor) *minor = prop.minor;
  return hipSuccess;
}

const Calls kHipCalls = {
    [](int* n) { return hipGetDeviceCount(n); },
    [](int d) { return hipSetDevice(d); },
    [](int* d) { return hipGetDevice(d); },
    hip_device_info,
    [](void** p, size_t n) { return hipMalloc(p, n); },
    [](void* p) { return hipFree(p); },
    [](void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t st) { return hipMemcpyAsync(d, s, n, k, st); },
    [](hipStream_t* s) { return hipStreamCreateWithFlags(s, hipStreamNonBlocking); },
    [](hipStream_t s) { return hipStreamDestroy(s); },
    [](hipStream_t s) { return hipStreamSynchronize(s); },
    []() { return hipDeviceSynchronize(); },
    [](hipEvent_t* e, unsigned f) { return hipEventCreateWithFlags(e, f); },
    [](hipEvent_t e) { return hipEventDestroy(e); },
    [](hipEvent_t e, hipStream_t s) { return hipEventRecord(e, s); },
    [](hipStream_t s, hipEvent_t e) { return hipStreamWaitEvent(s, e, 0); },
    [](hipEvent_t e) { return hipEventSynchronize(e); },
    [](float* ms, hipEvent_t a, hipEvent_t b) { return hipEventElapsedTime(ms, a, b); },
    []() { return hipGetLastError(); },
    [](void* p, uint32_t v, size_t nbytes, hipStream_t st) {
      const size_t n = nbytes / 4;
      if (n == 0) return hipSuccess;
      size_t g = (n + 255) / 256;
      if (g > 65536) g = 65536;
      k_fill_u32<<<dim3(unsigned(g)), 256, 0, st>>>(static_cast<uint32_t*>(p), v, n);
      return hipGetLastError();
    },
    [](void* ws, size_t n, hipStream_t st) { return musapy_kernels_take_fault_ws(ws, n, st); },
};

// The host-memory table: one fake device, memory from the C heap, streams and events as tokens,
// every synchronize immediate, kernel launches without effect (the pending HIP error of a launch
// that found no device is consumed and not reported).
std::atomic<uintptr_t> g_fake_token{0x1000};
const Calls kHostCalls = {
    [](int* n) { *n = 1; return hipSuccess; },
    [](int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; },
    [](int* d) { *d = 0; return hipSuccess; },
    [](int d, char* name, size_t len, size_t* mem, int* cus, int* major, int* minor) {
      if (d != 0) return hipErrorInvalidDevice;
      if (name && len) {
        std::strncpy(name, "host-fake", len - 1);
        name[len - 1] = 0;
      }
      if (mem) *mem = size_t(1) << 34;
      if (cus) *cus = 1;
      if (major) *major = 9;
      if (minor) *minor = 5;
      return hipSuccess;
    },
    [](void** p, size_t n) {
      *p = std::aligned_alloc(256, (n + 255) / 256 * 256);
      return *p ? hipSuccess : hipErrorOutOfMemory;
    },
    [](void* p) { std::free(p); return hipSuccess; },
    [](void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) { std::memmove(d, s, n); return hipSuccess; },
    [](hipStream_t* s) { *s = reinterpret_cast<hipStream_t>(g_fake_token.fetch_add(16)); return hipSuccess; },
    [](hipStream_t) { return hipSuccess; },
    [](hipStream_t) { return hipSuccess; },
    []() { return hipSuccess; },
    [](hipEvent_t* e, unsigned) { *e = reinterpret_cast<hipEvent_t>(g_fake_token.fetch_add(16)); return hipSuccess; },
    [](hipEvent_t) { return hipSuccess; },
    [](hipEvent_t, hipStream_t) { return hipSuccess; },
    [](hipStream_t, hipEvent_t) { return hipSuccess; },
    [](hipEvent_t) { return hipSuccess; },
    [](float* ms, hipEvent_t, hipEvent_t) { *ms = 0.0f; return hipSuccess; },
    []() { (void)hipGetLastError(); return hipSuccess; },
    [](void* p, uint32_t v, size_t nbytes, hipStream_t) {
      uint32_t* q = static_cast<uint32_t*>(p);
      for (size_t i = 0; i < nbytes / 4; ++i) q[i] = v;
      return hipSuccess;
    },
    [](void*, size_t, hipStream_t) { return 0; },
};

std::atomic<const Calls*> g_calls{&kHipCalls};
inline const Calls& H() { return *g_calls.load(std::memory_order_acquire); }

// one-shot error injection: after `skip` more calls of the class, the next `count` calls return
// `code` (for MPY_RT_CALL_FAULT: report `code` as the fault word) instead of doing their work
struct Injection {
  std::atomic<int> code{0}, skip{0}, count{0};
};
Injection g_inject[MPY_RT_CALL_COUNT];

// true (and the code in *code) when this call of `cls` is to fail
bool injected(int cls, int* code) {
  Injection& in = g_inject[cls];
  if (in.count.load(std::memory_order_relaxed) <= 0) return false;
  if (in.skip.load(std::memory_order_relaxed) > 0) {
    in.skip.fetch_sub(1);
    return false;
  }
  if (in.count.fetch_sub(1) <= 0) return false;
  *code = in.code.load();
  return true;
}

#define MPY_INJECT(CLS)                                      \
  do {                                                       \
    int code_ = 0;                                           \
    if (injected(CLS, &code_)) return rc(hipError_t(code_)); \
  } while (0)

// ---------------------------------------------------------------------------------------------
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
  if (e != hipSuccess) (void)H().last_error();
  return int(e);
}

// make `waiter` wait for everything queued so far on `target`
hipError_t order_after(hipStream_t waiter, hipStream_t target) {
  hipEvent_t ev = nullptr;
  hipError_t e = H().event_create(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return e;
  e = H().event_record(ev, target);
  if (e == hipSuccess) e = H().stream_wait_event(waiter, ev);
  (void)H().event_destroy(ev);  // the wait holds what it needs; a failed destroy only leaks the event
  return e;
}

// returns every cached block of `device` to the device; the caller holds g_mu
hipError_t release_cached_locked(int device) {
  DevicePool& P = g_pools[device];
  if (P.free.empty()) return hipSuccess;
  int prev = 0;
  if (H().get_device(&prev) != hipSuccess) prev = device;
  hipError_t e = H().set_device(device);
  if (e != hipSuccess) return e;
  e = H().device_sync();  // frees were stream-ordered: their work must be done
  for (auto& kv : P.free) {
    const hipError_t fe = H().free(kv.second.ptr);
    if (e == hipSuccess) e = fe;  // the block leaves the cache either way
  }
  P.free.clear();
  P.cached_bytes = 0;
  (void)H().set_device(prev);
  return e;
}

}  // namespace

extern "C" {

int mpy_rt_device_count(int* count) { return rc(H().device_count(count)); }

int mpy_rt_set_device(int device) { return rc(H().set_device(device)); }

int mpy_rt_device_info(int device, char* name, size_t name_len, size_t* total_mem, int* cu_count, int* arch_major,
                       int* arch_minor) {
  return rc(H().device_info(device, name, name_len, total_mem, cu_count, arch_major, arch_minor));
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
  hipError_t e = H().set_device(device);
  if (e != hipSuccess) return rc(e);
  void* p = nullptr;
  int code = 0;
  e = injected(MPY_RT_CALL_MALLOC, &code) ? hipError_t(code) : H().malloc(&p, cls);
  if (e == hipErrorOutOfMemory) {
    (void)H().last_error();
    for (int d = 0; d < kMaxDevices; ++d)  // best effort: whatever was released helps the retry
      if (!g_pools[d].free.empty()) (void)release_cached_locked(d);
    e = H().set_device(device);
    if (e != hipSuccess) return rc(e);
    e = injected(MPY_RT_CALL_MALLOC, &code) ? hipError_t(code) : H().malloc(&p, cls);
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
  return rc(H().free(ptr));  // not from this allocator
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
  MPY_INJECT(MPY_RT_CALL_MEMCPY);
  hipError_t e = H().memcpy_async(dst, src, n, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return rc(e);
  return rc(H().stream_sync(s));  // the host buffer may be released right after
}
int mpy_rt_memcpy_d2h(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  MPY_INJECT(MPY_RT_CALL_MEMCPY);
  hipError_t e = H().memcpy_async(dst, src, n, hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return rc(e);
  return rc(H().stream_sync(s));
}
int mpy_rt_memcpy_d2d(void* dst, const void* src, size_t n, hipStream_t s) {
  if (n == 0) return 0;
  MPY_INJECT(MPY_RT_CALL_MEMCPY);
  return rc(H().memcpy_async(dst, src, n, hipMemcpyDeviceToDevice, s));
}

int mpy_rt_stream_create(hipStream_t* stream, int device) {
  MPY_INJECT(MPY_RT_CALL_STREAM);
  hipError_t e = H().set_device(device);
  if (e != hipSuccess) return rc(e);
  return rc(H().stream_create(stream));
}
int mpy_rt_stream_destroy(hipStream_t stream) {
  // cached blocks last freed on this stream outlive it: drain it, then mark them idle so no
  // later reuse records an event on the destroyed handle
  hipError_t e = H().stream_sync(stream);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (int d = 0; d < kMaxDevices; ++d) {
      for (auto& kv : g_pools[d].free)
        if (kv.second.stream == stream) kv.second.idle = true;
      for (auto& kv : g_pools[d].live)
        if (kv.second.stream == stream) kv.second.idle = true;
    }
  }
  hipError_t e2 = H().stream_destroy(stream);
  return rc(e != hipSuccess ? e : e2);
}
int mpy_rt_stream_synchronize(hipStream_t stream) {
  MPY_INJECT(MPY_RT_CALL_SYNC);
  return rc(H().stream_sync(stream));
}
int mpy_rt_device_synchronize(void) {
  MPY_INJECT(MPY_RT_CALL_SYNC);
  return rc(H().device_sync());
}

int mpy_rt_event_create(hipEvent_t* ev, int timing) {
  MPY_INJECT(MPY_RT_CALL_EVENT);
  return rc(H().event_create(ev, timing ? hipEventDefault : hipEventDisableTiming));
}
int mpy_rt_event_destroy(hipEvent_t ev) { return rc(H().event_destroy(ev)); }
int mpy_rt_event_record(hipEvent_t ev, hipStream_t s) {
  MPY_INJECT(MPY_RT_CALL_EVENT);
  return rc(H().event_record(ev, s));
}
int mpy_rt_stream_wait_event(hipStream_t s, hipEvent_t ev) {
  MPY_INJECT(MPY_RT_CALL_EVENT);
  return rc(H().stream_wait_event(s, ev));
}
int mpy_rt_event_synchronize(hipEvent_t ev) {
  MPY_INJECT(MPY_RT_CALL_SYNC);
  return rc(H().event_sync(ev));
}
int mpy_rt_event_elapsed_ms(float* ms, hipEvent_t a, hipEvent_t b) { return rc(H().event_elapsed(ms, a, b)); }

int mpy_rt_check_launch(void) {
  hipError_t e = H().last_error();
  int code = 0;
  if (injected(MPY_RT_CALL_LAUNCH, &code)) e = hipError_t(code);
  if (e != hipSuccess) return int(e);
  const int w = musapy_kernels_take_error();
  return w ? -w : 0;
}

int mpy_rt_take_fault_ws(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int code = 0;
  if (injected(MPY_RT_CALL_FAULT, &code)) return code;
  return H().take_fault_ws(workspace, workspace_bytes, stream);
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
  return rc(H().fill_u32(ptr, value, nbytes, stream));
}

int mpy_rt_set_backend(int backend) {
  if (backend != MPY_RT_BACKEND_HIP && backend != MPY_RT_BACKEND_HOST) return int(hipErrorInvalidValue);
  if (backend == MPY_RT_BACKEND_HOST) {
    // kernels still launch under the fake (they find no device and do nothing); with a real GPU
    // they would be handed host pointers, so the fake is refused wherever a device exists
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    (void)hipGetLastError();
    if (e == hipSuccess && n > 0) return int(hipErrorNotSupported);
  }
  std::lock_guard<std::mutex> lk(g_mu);
  for (int d = 0; d < kMaxDevices; ++d)
    if (!g_pools[d].live.empty() || !g_pools[d].free.empty()) return int(hipErrorNotSupported);  // memory of the other backend
  g_calls.store(backend == MPY_RT_BACKEND_HOST ? &kHostCalls : &kHipCalls, std::memory_order_release);
  return 0;
}

int mpy_rt_inject(int call, int code, int skip, int count) {
  if (call < 0 || call >= MPY_RT_CALL_COUNT || count < 0 || skip < 0) return int(hipErrorInvalidValue);
  Injection& in = g_inject[call];
  in.count.store(0);
  in.code.store(code);
  in.skip.store(skip);
  in.count.store(count);
  return 0;
}

}  // extern "C"
