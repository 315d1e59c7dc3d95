// kcommon.hpp -- device/host helpers shared by the gfx950 kernels.
//
// Replaces kernels/include/common.h of the reference (offset_nd / reduce_input_offset,
// common.h:42-79), which recomputes a 64-bit div/mod per dimension, per operand, per element.
// Here the host coalesces dimensions first and the device divides with precomputed 32-bit
// magic numbers, once per row rather than once per element.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
#include <stddef.h>
#include <sys/types.h>

#include "plan.hpp"
#include "../../../include/musapy_kernels.h"

namespace mpy {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------------------------------------
// device side of the magic-number division of plan.hpp (FastDiv)
__device__ inline uint32_t fd_div(const FastDiv& f, uint32_t n) {
  uint32_t t = __umulhi(n, f.m);
  return uint32_t((uint64_t(t) + n) >> f.s);
}

// ---------------------------------------------------------------------------------------------
// Offsets of the outer (non-innermost) coordinates of a row, for up to NOPS operands.
// Dims are stored innermost-first; dim sizes < 2^32, row index < 2^32 (host checks).
template <int NOPS>
struct RowIndexer {
  int nd;                       // number of outer dims
  FastDiv div[kMaxDims];
  int64_t stride[NOPS][kMaxDims];
};

template <int NOPS>
__device__ inline void row_offsets(const RowIndexer<NOPS>& ix, uint32_t row, int64_t (&off)[NOPS]) {
#pragma unroll
  for (int o = 0; o < NOPS; ++o) off[o] = 0;
  for (int i = 0; i < ix.nd; ++i) {
    uint32_t q = fd_div(ix.div[i], row);
    uint32_t c = row - q * ix.div[i].d;
    row = q;
#pragma unroll
    for (int o = 0; o < NOPS; ++o) off[o] += int64_t(c) * ix.stride[o][i];
  }
}

template <int NOPS>
inline RowIndexer<NOPS> make_row_indexer(const Plan& p) {
  RowIndexer<NOPS> ix{};
  ix.nd = p.ndim - 1;
  for (int i = 0; i < ix.nd; ++i) {
    int dim = p.ndim - 2 - i;  // innermost outer dim first
    ix.div[i] = make_fastdiv(uint32_t(p.shape[dim]));
    for (int o = 0; o < NOPS; ++o) ix.stride[o][i] = p.stride[o][dim];
  }
  return ix;
}

// ---------------------------------------------------------------------------------------------
// Aligned vector of N elements: one global_load_dwordx4 per 16 bytes.
template <typename T, int N>
struct alignas(sizeof(T) * N >= 16 ? 16 : sizeof(T) * N) Vec {
  T v[N];
};

template <typename T, int N>
__device__ inline Vec<T, N> vload(const T* p) {
  return *reinterpret_cast<const Vec<T, N>*>(p);
}
template <typename T, int N>
__device__ inline void vstore(T* p, const Vec<T, N>& v) {
  *reinterpret_cast<Vec<T, N>*>(p) = v;
}

// Streaming (nontemporal) accesses: global_load/store ... nt.  Data read or written once per
// launch is marked so the L2 and the Infinity Cache do not keep it at the expense of other
// lines; measured on MI355X, a 64M f32 row reduction streams at 6.8 TB/s this way against 6.1
// with default loads.  The access goes through an integer vector of the same size, because the
// builtin takes scalar and vector types only.
template <int B> struct NtWord;
template <> struct NtWord<16> { typedef unsigned int type __attribute__((ext_vector_type(4))); };
template <> struct NtWord<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
template <> struct NtWord<4> { using type = unsigned int; };
template <> struct NtWord<2> { using type = unsigned short; };
template <> struct NtWord<1> { using type = unsigned char; };

// vectors wider than 16 bytes (the wider side of a cast) move as several 16-byte words
template <typename T, int N>
__device__ inline Vec<T, N> vload_nt(const T* p) {
  constexpr int kB = int(sizeof(Vec<T, N>));
  constexpr int kW = kB > 16 ? 16 : kB;
  using W = typename NtWord<kW>::type;
  static_assert(sizeof(W) == kW && kB % kW == 0, "streaming load width");
  W w[kB / kW];
#pragma unroll
  for (int i = 0; i < kB / kW; ++i) w[i] = __builtin_nontemporal_load(reinterpret_cast<const W*>(p) + i);
  Vec<T, N> v;
  __builtin_memcpy(&v, w, sizeof(v));
  return v;
}
template <typename T, int N>
__device__ inline void vstore_nt(T* p, const Vec<T, N>& v) {
  constexpr int kB = int(sizeof(Vec<T, N>));
  constexpr int kW = kB > 16 ? 16 : kB;
  using W = typename NtWord<kW>::type;
  static_assert(sizeof(W) == kW && kB % kW == 0, "streaming store width");
  W w[kB / kW];
  __builtin_memcpy(w, &v, sizeof(v));
#pragma unroll
  for (int i = 0; i < kB / kW; ++i) __builtin_nontemporal_store(w[i], reinterpret_cast<W*>(p) + i);
}

// Load policy of the elementwise kernels by volume: a launch that streams at least this many
// input bytes uses streaming loads; below it, default loads (small inputs are often read again
// and are worth keeping in the caches).  Measured on MI355X with outputs rotated over 4 buffers,
// so that each launch's writes reach HBM: 16M f32 add (128 MB of input) 31.7-32.0 us with
// streaming loads against 35.7-36.2 with default loads, C3's i64 + f64 75 vs 82 us, f64 -> f32
// 33.8 vs 35.2 us.  (Writing the same output buffer every launch, the Infinity Cache absorbs the
// writes and favours default loads below 192 MB; that is not what a pipeline of ops sees.)
// Reductions always stream (they write next to nothing).
constexpr uint64_t kStreamLoadBytes = uint64_t(32) << 20;

template <typename T, int N>
__device__ inline Vec<T, N> vload_pol(const T* p, bool nt) {
  return nt ? vload_nt<T, N>(p) : vload<T, N>(p);
}

// Store policy by volume: an output of at least this many bytes is written with streaming
// stores (binary ops and scans; unary ops and casts from kStreamStoreBytesUnary).  Such an output
// does not stay in the 256 MB Infinity Cache for its consumer anyway.  Measured on MI355X with
// inputs and outputs rotated over 4 buffers, against default stores: 64M f32 add 130 -> 120 us,
// the i64 + f64 add of 16M 66.5 -> 61.5, c128 mul 129 -> 121, the (8192, 8192) f32 transpose
// 113 -> 107, a flip 97.5 -> 91.5, the c128 transpose 110.5 -> 102.5, C5's cumsum 195 -> 188,
// C2's broadcast add 24.7 -> 23.1, 16M f32 add 33.6 -> 32.3 us (with 128-lane blocks).  Unary
// ops and casts stream from 32 MB: with every launch writing lines that the Infinity Cache no
// longer holds (outputs rotated over 512 MB or more), f64 -> f32 of 16M 35.7-35.8 -> 34.3 us, c64
// abs 35.7-36.3 -> 34.2-34.4, f32 -> bf16 18.8 -> 18.4, f32 -> f16 18.8-19.0 -> 18.5 (clamp of 16M
// f64 level).  With outputs rotated over fewer buffers, whose writes the cache absorbed, a 64 MB
// unary output had measured slower streamed.
constexpr uint64_t kStreamStoreBytes = uint64_t(64) << 20;
constexpr uint64_t kStreamStoreBytesUnary = uint64_t(32) << 20;
// The store policy is a template parameter, not a runtime flag: the compiler merges a runtime
// choice between a streaming and a default store of the same value to the same address into one
// default store (the two branches are combined and the nontemporal hint is dropped), which left
// every kernel of this library without streaming stores until the policy was made static.
template <bool NT, typename T, int N>
__device__ inline void vstore_as(T* p, const Vec<T, N>& v) {
  if constexpr (NT) vstore_nt<T, N>(p, v); else vstore<T, N>(p, v);
}

// Calls fn(std::integral_constant<int, 0>{}) .. fn(std::integral_constant<int, N - 1>{}) as
// straight-line code.  For loops around streaming stores: the compiler promotes a store out of a
// one-trip loop (N = 1) and drops its nontemporal hint on the way.
template <int N, int I = 0, class Fn>
__device__ inline void static_for(Fn&& fn) {
  if constexpr (I < N) {
    fn(std::integral_constant<int, I>{});
    static_for<N, I + 1>(fn);
  }
}

// Calls `launch` with std::true_type or std::false_type: a kernel template's store policy from
// the launcher's runtime decision.
template <class L>
inline void with_store_policy(bool nt, L&& launch) {
  if (nt) launch(std::true_type{}); else launch(std::false_type{});
}

// Block-wide barrier that orders LDS accesses only.  __syncthreads() also waits until every
// global load and store the wave has issued is complete (s_waitcnt vmcnt(0) before s_barrier),
// so a barrier that follows a hand-over store would hold the whole block for that store's round
// trip; where the barrier only publishes LDS values, this one lets such stores stay in flight.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------------------------
// Wavefront-64 butterfly helpers (ds_swizzle/dpp are chosen by the compiler for __shfl_xor).
template <typename T>
__device__ inline T shfl_xor(T v, int m) {
  return __shfl_xor(v, m, kWave);
}

// Wrapper-level error of the calling thread (read and cleared by musapy_kernels_take_error):
// 1 = cumsum scratch missing or too small, 2 = a reduction tile longer than 2^31 elements,
// 3 = ndim outside [0, 32] or axis outside [0, ndim), 4 = a scan with 2^32 or more rows (or a
// non-axis extent of 2^32 or more), 5 = a no-alloc reduction that needs more than the static
// scratch holds.
inline thread_local int g_wrapper_error = 0;

// ---------------------------------------------------------------------------------------------
// Bounded device waits.  The kernels that wait for another workgroup's result (the combiner of a
// single-launch reduction, the look-back of a row scan) poll at most `wait_spin_limit()` times.
// When that runs out they stop waiting, OR their fault code into the fault word of the workspace
// (or scratch) the launch was given, skip or finish their work, and exit normally -- so a grid
// always drains.  The host reads and clears that word after synchronizing the stream
// (musapy_kernels_take_fault_ws), so a fault is reported to the stream whose launch gave up.
enum : uint32_t { kFaultReduceWait = 1u, kFaultScanWait = 2u };
// polls a bounded wait may make (default 2^24; musapy_kernels_set_spin_limit)
uint32_t wait_spin_limit();

// A caller's workspace: its last 8-byte word holds the fault word (in its first 4 bytes), and
// everything before that word is the launch's payload (slots, counters, prefixes).  false when
// the workspace is missing, not 8-byte aligned, or too small to hold both.
struct WsSplit {
  uint64_t* payload;
  size_t payload_bytes;
  uint32_t* fault;
};
inline bool ws_split(void* ws, size_t bytes, WsSplit& s) {
  if (ws == nullptr || bytes < 16 || (reinterpret_cast<uintptr_t>(ws) & 7)) return false;
  const size_t last = (bytes - 8) & ~size_t(7);
  s.payload = static_cast<uint64_t*>(ws);
  s.payload_bytes = last;
  s.fault = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + last);
  return true;
}

// The ranks and axes the planners accept: 0 <= ndim <= kMaxDims (the reference's
// MUSAPY_MAX_NDIM, elementwise.mu:16) and, for a reduction or scan of a non-scalar, 0 <= axis <
// ndim.  A wrapper called outside them launches nothing and reports error 3.
inline bool args_ok(int ndim, int axis = 0) {
  if (ndim >= 0 && ndim <= kMaxDims && (ndim == 0 || (axis >= 0 && axis < ndim))) return true;
  g_wrapper_error = 3;
  return false;
}

// interleaved complex elements, the ABI types themselves
using c64 = musapy_c64_t;
using c128 = musapy_c128_t;

}  // namespace mpy
