// scan.hip -- cumsum (inclusive prefix sum along one axis), for gfx950.
//
// Drop-in for the reference's musapy_cumsum_{i64,f32,f64}_v3 (kernels/reduction.mu:557-820,
// 1723-1776), which runs a 3-5 launch Blelloch hierarchy and writes the output twice.  Here:
//   row   the scanned axis is unit-stride in input and output: a single pass over the data with
//         a decoupled look-back (Merrill & Garland, "Single-pass Parallel Prefix Scan with
//         Decoupled Look-back", 2016).  Each block scans one TILE of one row, publishes the
//         tile aggregate, then folds predecessor state into its exclusive prefix.  Tiles are
//         claimed from an atomic counter in chunk-major order (all rows' chunk 0, then chunk 1,
//         ...), so a tile's predecessor was always claimed earlier and is running or done.
//         Determinism: a tile's inclusive prefix is defined as P(c) = P(c-1) + A(c); the
//         look-back starts from the nearest published P(j) and re-folds A(j+1..c-1) left to
//         right, which reproduces P(c-1) bit for bit whichever j it found.
//   col   the axis is strided but the innermost other dim is unit-stride: lanes walk adjacent
//         columns, each carrying a running sum down the axis (coalesced, sequential order).
//   generic  one lane per row, sequential along the axis (any strides).
// col and generic add in exactly the reference CPU order (acc = 0; acc += x[k]).
#include "kcommon.hpp"
#include "publish.hpp"
#include "../../../include/musapy_kernels.h"

namespace mpy {

constexpr int kSBlock = 256;

template <class T> struct ScanAcc { using A = T; };
template <> struct ScanAcc<int64_t> { using A = uint64_t; };  // wrapping adds

template <class T> constexpr int scan_items() { return sizeof(T) == 4 ? 16 : 8; }
// Shape of the block-per-row kernel: 1024 lanes with one 16-byte vector each (16 KB tiles).  On
// MI355X a block-per-row stream of (1024, 65536) f64 moved 5.35 TB/s in this shape against 4.82
// with 256 lanes x 64 bytes and 4.31 with 256 x 128 bytes: many waves with short per-lane
// tiles hide the per-tile barrier best.
constexpr int kSeqBlock = 1024;
template <class T> constexpr int seq_items() { return int(16 / sizeof(T)); }

__device__ inline uint64_t bits_of(double v) { return uint64_t(__double_as_longlong(v)); }
__device__ inline uint64_t bits_of(float v) { return uint64_t(__float_as_uint(v)); }
__device__ inline uint64_t bits_of(uint64_t v) { return v; }
template <class A> __device__ inline A from_bits(uint64_t b);
template <> __device__ inline double from_bits<double>(uint64_t b) { return __longlong_as_double((long long)b); }
template <> __device__ inline float from_bits<float>(uint64_t b) { return __uint_as_float(uint32_t(b)); }
template <> __device__ inline uint64_t from_bits<uint64_t>(uint64_t b) { return b; }

// Published look-back values (publish.hpp): each status word is written once per launch after
// k_scan_clear zeroed it, so a reader that sees the tag on every word holds the final value.

__global__ void k_scan_clear(uint64_t* w, uint64_t n) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
    w[i] = 0;
}

struct RowScanArgs {
  RowIndexer<2> ix;     // non-axis dims: [0] input strides, [1] output strides
  uint64_t L;
  uint32_t rows;
  uint32_t tiles;       // tiles per row
  uint32_t* counter;    // tile claim counter; nullptr when tiles == 1 (no look-back)
  uint64_t* status;     // per row: inclusive prefixes of tiles 0..T-2, aggregates of 1..T-2
  uint32_t* fault;      // the device's fault word (kcommon.hpp): a look-back wait ran out
  uint32_t spin_limit;  // polls a look-back may make
  bool vec;             // 16-byte aligned rows
};

__device__ inline float shfl_up_acc(float v, int d) { return __shfl_up(v, d, kWave); }
__device__ inline double shfl_up_acc(double v, int d) { return __shfl_up(v, d, kWave); }
__device__ inline uint64_t shfl_up_acc(uint64_t v, int d) {
  return (uint64_t)__shfl_up((unsigned long long)v, d, kWave);
}

// wave-64 inclusive scan (Hillis-Steele over shuffles, fixed order)
template <class A>
__device__ inline A wave_incl_scan(A v, int lane) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    A u = shfl_up_acc(v, d);
    if (lane >= d) v = u + v;
  }
  return v;
}

template <class T>
__global__ __launch_bounds__(kSBlock) void k_scan_rows(const T* __restrict__ a, T* __restrict__ c, RowScanArgs sa) {
  using A = typename ScanAcc<T>::A;
  constexpr int N = scan_items<T>();
  constexpr uint64_t TILE = uint64_t(kSBlock) * N;
  constexpr int kWaves = kSBlock / kWave;
  __shared__ uint32_t s_id;
  __shared__ A s_wave[kWaves];
  __shared__ A s_prefix;
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;

  uint32_t id = blockIdx.x;
  if (sa.counter) {
    if (tid == 0) s_id = atomicAdd(sa.counter, 1u);
    __syncthreads();
    id = s_id;
  }
  const uint32_t chunk = id / sa.rows;
  const uint32_t row = id - chunk * sa.rows;
  int64_t off[2];
  row_offsets<2>(sa.ix, row, off);
  const T* ain = a + off[0];
  T* cout = c + off[1];
  const uint64_t k0 = uint64_t(chunk) * TILE + uint64_t(tid) * N;

  // load N consecutive elements and scan them in registers
  A x[N];
  if (sa.vec && k0 + N <= sa.L) {
    constexpr int VV = int(16 / sizeof(T));
#pragma unroll
    for (int j = 0; j < N; j += VV) {
      Vec<T, VV> v = vload<T, VV>(ain + k0 + j);
#pragma unroll
      for (int q = 0; q < VV; ++q) x[j + q] = A(v.v[q]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = (k0 + j < sa.L) ? A(ain[k0 + j]) : A(0);
  }
#pragma unroll
  for (int j = 1; j < N; ++j) x[j] = x[j - 1] + x[j];

  // block-wide exclusive prefix of the per-lane totals
  A tot = x[N - 1];
  A incl = wave_incl_scan(tot, lane);
  if (lane == kWave - 1) s_wave[wv] = incl;
  __syncthreads();
  A wave_off = A(0);
  A agg = A(0);
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    if (i < wv) wave_off = wave_off + s_wave[i];
    agg = agg + s_wave[i];
  }
  A lane_excl = shfl_up_acc(incl, 1);
  if (lane == 0) lane_excl = A(0);
  // the exclusive prefix inside the tile: wave offset + lane offset (fixed association)
  A local = wave_off + lane_excl;

  // tile prefix from the look-back (one lane; the rest of the block waits at the barrier)
  if (tid == 0) {
    A P = A(0);
    if (sa.counter) {
      constexpr int W = sizeof(A) == 4 ? 1 : 2;
      const uint32_t NT = sa.tiles;  // >= 2 here; the last tile publishes nothing
      uint64_t* rowp = sa.status + uint64_t(row) * (2 * NT - 3) * W;
      auto incl_of = [&](uint32_t c) { return rowp + uint64_t(c) * W; };            // tiles 0..T-2
      auto agg_of = [&](uint32_t c) { return rowp + uint64_t(NT - 1 + c - 1) * W; };  // tiles 1..T-2
      if (chunk == 0) {
        publish_value<W>(incl_of(0), bits_of(agg));
      } else {
        if (chunk <= NT - 2) publish_value<W>(agg_of(chunk), bits_of(agg));
        // walk back to the nearest tile whose inclusive prefix is published
        uint32_t j = chunk - 1;
        uint32_t spins = 0;
        bool ok = true;
        uint64_t b = 0;
        for (;;) {
          if (spins++ >= sa.spin_limit) {  // a limit of 0 gives up before the first poll
            ok = false;
            break;
          }
          if (read_value<W>(incl_of(j), b)) {
            P = from_bits<A>(b);
            break;
          }
          if (j > 0 && read_value<W>(agg_of(j), b)) {  // tile 0 only ever publishes an inclusive prefix
            --j;
            continue;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) {
          atomicOr(sa.fault, kFaultScanWait);  // the prefix stays 0: the host reports the fault
        } else {
          // re-fold the aggregates after j in order: P(m) = P(m-1) + A(m)
          for (uint32_t m = j + 1; m < chunk; ++m) {
            read_value<W>(agg_of(m), b);  // seen published during the walk back
            P = P + from_bits<A>(b);
          }
        }
        if (chunk <= NT - 2) publish_value<W>(incl_of(chunk), bits_of(P + agg));
      }
    }
    s_prefix = P;
  }
  __syncthreads();
  const A P = s_prefix;

  // out = P + (local exclusive + in-lane inclusive)
  if (sa.vec && k0 + N <= sa.L) {
    constexpr int VV = int(16 / sizeof(T));
#pragma unroll
    for (int j = 0; j < N; j += VV) {
      Vec<T, VV> v;
#pragma unroll
      for (int q = 0; q < VV; ++q) v.v[q] = T(P + (local + x[j + q]));
      vstore<T, VV>(cout + k0 + j, v);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (k0 + j < sa.L) cout[k0 + j] = T(P + (local + x[j]));
  }
}

// Row scan without look-back, for many rows: block b walks row b tile by tile, keeping the
// running prefix P in registers and prefetching the next tile while it scans the current one.
// The association is fixed by the shape (lane, wave, tile), so results are identical run to
// run; they differ from k_scan_rows' only by the rounding of a different tile shape.
template <class T>
__device__ inline void load_tile(const T* ain, uint64_t k0, uint64_t L, bool vec, typename ScanAcc<T>::A (&x)[seq_items<T>()]) {
  using A = typename ScanAcc<T>::A;
  constexpr int N = seq_items<T>();
  if (vec && k0 + N <= L) {
    constexpr int VV = int(16 / sizeof(T));
#pragma unroll
    for (int j = 0; j < N; j += VV) {
      Vec<T, VV> v = vload<T, VV>(ain + k0 + j);
#pragma unroll
      for (int q = 0; q < VV; ++q) x[j + q] = A(v.v[q]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = (k0 + j < L) ? A(ain[k0 + j]) : A(0);
  }
}

template <class T>
__global__ __launch_bounds__(kSeqBlock) void k_scan_rows_seq(const T* __restrict__ a, T* __restrict__ c, RowScanArgs sa) {
  using A = typename ScanAcc<T>::A;
  constexpr int N = seq_items<T>();
  constexpr uint64_t TILE = uint64_t(kSeqBlock) * N;
  constexpr int kWaves = kSeqBlock / kWave;
  __shared__ A s_wave[2][kWaves];
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const uint32_t row = blockIdx.x;
  int64_t off[2];
  row_offsets<2>(sa.ix, row, off);
  const T* ain = a + off[0];
  T* cout = c + off[1];
  A x[N], y[N];
  load_tile<T>(ain, uint64_t(tid) * N, sa.L, sa.vec, x);
  A P = A(0);
  for (uint32_t t = 0; t < sa.tiles; ++t) {
    const uint64_t k0 = uint64_t(t) * TILE + uint64_t(tid) * N;
    if (t + 1 < sa.tiles) load_tile<T>(ain, k0 + TILE, sa.L, sa.vec, y);
#pragma unroll
    for (int j = 1; j < N; ++j) x[j] = x[j - 1] + x[j];
    A tot = x[N - 1];
    A incl = wave_incl_scan(tot, lane);
    if (lane == kWave - 1) s_wave[t & 1][wv] = incl;  // double-buffered: no barrier needed after use
    __syncthreads();
    A wave_off = A(0), agg = A(0);
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      if (i < wv) wave_off = wave_off + s_wave[t & 1][i];
      agg = agg + s_wave[t & 1][i];
    }
    A lane_excl = shfl_up_acc(incl, 1);
    if (lane == 0) lane_excl = A(0);
    const A local = wave_off + lane_excl;
    if (sa.vec && k0 + N <= sa.L) {
      constexpr int VV = int(16 / sizeof(T));
#pragma unroll
      for (int j = 0; j < N; j += VV) {
        Vec<T, VV> v;
#pragma unroll
        for (int q = 0; q < VV; ++q) v.v[q] = T(P + (local + x[j + q]));
        vstore<T, VV>(cout + k0 + j, v);
      }
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j)
        if (k0 + j < sa.L) cout[k0 + j] = T(P + (local + x[j]));
    }
    P = P + agg;
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = y[j];
  }
}

// one lane per column (or per row for the generic case), sequential along the axis
struct SeqScanArgs {
  RowIndexer<2> ix;   // dims enumerated by the lane: [0] input, [1] output strides
  uint64_t L;
  int64_t ls_in, ls_out;
  uint64_t lanes;
};

template <class T>
__global__ __launch_bounds__(kSBlock) void k_scan_seq(const T* __restrict__ a, T* __restrict__ c, SeqScanArgs sa) {
  using A = typename ScanAcc<T>::A;
  const uint64_t g = uint64_t(blockIdx.x) * kSBlock + threadIdx.x;
  if (g >= sa.lanes) return;
  int64_t off[2];
  row_offsets<2>(sa.ix, uint32_t(g), off);
  const T* ain = a + off[0];
  T* cout = c + off[1];
  A acc = A(0);
  uint64_t k = 0;
  for (; k + 4 <= sa.L; k += 4) {
    T x0 = ain[int64_t(k) * sa.ls_in], x1 = ain[int64_t(k + 1) * sa.ls_in];
    T x2 = ain[int64_t(k + 2) * sa.ls_in], x3 = ain[int64_t(k + 3) * sa.ls_in];
    acc = acc + A(x0); cout[int64_t(k) * sa.ls_out] = T(acc);
    acc = acc + A(x1); cout[int64_t(k + 1) * sa.ls_out] = T(acc);
    acc = acc + A(x2); cout[int64_t(k + 2) * sa.ls_out] = T(acc);
    acc = acc + A(x3); cout[int64_t(k + 3) * sa.ls_out] = T(acc);
  }
  for (; k < sa.L; ++k) {
    acc = acc + A(ain[int64_t(k) * sa.ls_in]);
    cout[int64_t(k) * sa.ls_out] = T(acc);
  }
}

// ---------------------------------------------------------------------------------------------

template <class T>
void launch_cumsum(const T* a, T* c, T* tmp, int ndim, const size_t* shape, const ssize_t* strides, int axis,
                   size_t axis_len, size_t out_size, hipStream_t st) {
  if (out_size == 0 || axis_len == 0) return;
  if (!args_ok(ndim, axis)) return;
  ScanPlan p;
  plan_scan(p, ndim, shape, strides, axis);
  // rows and the non-axis extents are decoded in 32 bits (row_offsets, the lane index of
  // k_scan_seq): refuse shapes past that instead of aliasing rows
  bool fits = p.rows < (uint64_t(1) << 32);
  for (int d = 0; d < p.ond; ++d) fits = fits && p.oshape[d] < (uint64_t(1) << 32);
  if (!fits) {
    g_wrapper_error = 4;
    return;
  }
  constexpr uint64_t TILE = uint64_t(kSBlock) * scan_items<T>();
  if (p.kind == kRowScan && p.L > 16) {
    RowScanArgs sa{};
    // non-axis dims, innermost first
    sa.ix.nd = p.ond;
    for (int i = 0; i < p.ond; ++i) {
      int d = p.ond - 1 - i;
      sa.ix.div[i] = make_fastdiv(uint32_t(p.oshape[d]));
      sa.ix.stride[0][i] = p.istride[d];
      sa.ix.stride[1][i] = p.ostride[d];
    }
    if (p.ond == 1 && p.oshape[0] == 1) sa.ix.nd = 0;
    sa.L = p.L;
    sa.rows = uint32_t(p.rows);
    sa.tiles = uint32_t((p.L + TILE - 1) / TILE);
    bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c)) & 15u) == 0;
    for (int d = 0; d < p.ond; ++d)
      if (((p.istride[d] * int64_t(sizeof(T))) % 16) || ((p.ostride[d] * int64_t(sizeof(T))) % 16)) vec = false;
    sa.vec = vec;
    // enough rows to give every CU two of them: walk each row in one block, no look-back
    if (sa.tiles > 1 && p.rows >= 512) {
      constexpr uint64_t STILE = uint64_t(kSeqBlock) * seq_items<T>();
      RowScanArgs ss = sa;
      ss.tiles = uint32_t((p.L + STILE - 1) / STILE);
      k_scan_rows_seq<T><<<dim3(ss.rows), kSeqBlock, 0, st>>>(a, c, ss);
      return;
    }
    if (sa.tiles > 1) {
      // tmp capacity per the caller's formula: rows * (bpr [+ ceil(bpr/256) if bpr > 256]) elements
      uint64_t bpr = (p.L + 255) / 256;
      uint64_t cap = uint64_t(p.rows) * (bpr + (bpr > 256 ? (bpr + 255) / 256 : 0)) * sizeof(T);
      // word 0: claim counter; then per row (2*tiles-3)*W status words (inclusive prefixes of
      // tiles 0..T-2, aggregates of tiles 1..T-2); one spare word
      const uint64_t W = sizeof(T) == 4 ? 1 : 2;
      uint64_t words = 2 + uint64_t(p.rows) * (2 * uint64_t(sa.tiles) - 3) * W;
      if (uint64_t(p.rows) * sa.tiles >= (uint64_t(1) << 32)) {  // tile ids are 32-bit
        g_wrapper_error = 4;
        return;
      }
      if (tmp == nullptr || words * 8 > cap) {
        g_wrapper_error = 1;
        return;
      }
      uint64_t* w = reinterpret_cast<uint64_t*>(tmp);
      sa.counter = reinterpret_cast<uint32_t*>(w);
      sa.status = w + 1;
      sa.fault = device_fault_word(st);
      sa.spin_limit = wait_spin_limit();
      if (sa.fault == nullptr) {  // a wait that ran out could not be reported: take no waits
        g_wrapper_error = 1;
        return;
      }
      unsigned cg = unsigned(words < 65536 * 256 ? (words + 255) / 256 : 65536);
      k_scan_clear<<<cg, 256, 0, st>>>(w, words);
    }
    k_scan_rows<T><<<dim3(unsigned(uint64_t(sa.rows) * sa.tiles)), kSBlock, 0, st>>>(a, c, sa);
    return;
  }
  SeqScanArgs sq{};
  sq.L = p.L;
  sq.ls_in = p.ls_in;
  sq.ls_out = p.ls_out;
  sq.lanes = p.rows;
  sq.ix.nd = p.ond;
  for (int i = 0; i < p.ond; ++i) {
    int d = p.ond - 1 - i;
    sq.ix.div[i] = make_fastdiv(uint32_t(p.oshape[d]));
    sq.ix.stride[0][i] = p.istride[d];
    sq.ix.stride[1][i] = p.ostride[d];
  }
  unsigned grid = unsigned((sq.lanes + kSBlock - 1) / kSBlock);
  k_scan_seq<T><<<grid, kSBlock, 0, st>>>(a, c, sq);
}

}  // namespace mpy

using namespace mpy;

extern "C" {

// rust/musapy-ops/src/kernels.rs:185-187
void musapy_cumsum_i64_v3(const int64_t* a, int64_t* c, int64_t* tmp, int ndim, const size_t* in_shape,
                          const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t st) {
  launch_cumsum<int64_t>(a, c, tmp, ndim, in_shape, in_strides, axis, axis_len, out_size, st);
}
void musapy_cumsum_f32_v3(const float* a, float* c, float* tmp, int ndim, const size_t* in_shape,
                          const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t st) {
  launch_cumsum<float>(a, c, tmp, ndim, in_shape, in_strides, axis, axis_len, out_size, st);
}
void musapy_cumsum_f64_v3(const double* a, double* c, double* tmp, int ndim, const size_t* in_shape,
                          const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t st) {
  launch_cumsum<double>(a, c, tmp, ndim, in_shape, in_strides, axis, axis_len, out_size, st);
}

// Returns and clears the calling thread's last wrapper-level error (1 = cumsum scratch missing
// or too small for the look-back state, 2 = reduction tile above 2^31 elements).  New: the
// reference wrappers have no such failure mode.
int musapy_kernels_take_error(void) {
  int e = g_wrapper_error;
  g_wrapper_error = 0;
  return e;
}

}  // extern "C"
