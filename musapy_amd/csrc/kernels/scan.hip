// scan.hip -- cumsum (inclusive prefix sum along one axis), for gfx950.
//
// Drop-in for the reference's musapy_cumsum_{i64,f32,f64}_v3 (kernels/reduction.mu:557-820,
// 1723-1776), which runs a 3-5 launch Blelloch hierarchy and writes the output twice.  Every
// path here reads the input once and writes the output once, in one launch (plus a small
// clear of the look-back state):
//   look-back  the scanned axis is unit-stride and the rows are few, or each row is one tile: a
//              single pass with a decoupled look-back (Merrill & Garland, "Single-pass Parallel
//              Prefix Scan with Decoupled Look-back", 2016) over tiles taken in memory order.
//   row walk   unit-stride rows that are many (>= 512) and longer than one tile: one block per
//              row walks it tile by tile, carrying the prefix in registers (no inter-block wait).
//              Measured faster than the look-back on (1024, 65536) f64 (230 vs 260-290 us): with
//              that many rows the look-back's round trip per tile costs more than the walk's
//              one-block-per-row access pattern.
//   col        the axis is strided but the innermost other dim is unit-stride: lanes walk
//              adjacent columns, each carrying a running sum down the axis (coalesced,
//              sequential order).
//   generic    one lane per row, sequential along the axis (any strides).
// col and generic add in exactly the reference CPU order (acc = 0; acc += x[k]).  The tiled
// paths fix their association by the tile shape, so results are the same bits run to run.
#include "kcommon.hpp"
#include "publish.hpp"
#include "../../../include/musapy_kernels.h"

namespace mpy {

constexpr int kSBlock = 256;

template <class T> struct ScanAcc { using A = T; };
template <> struct ScanAcc<int64_t> { using A = uint64_t; };  // wrapping adds

// Shape of the block-per-row kernel: 1024 lanes with one 16-byte vector each (16 KB tiles).  On
// MI355X a block-per-row stream of (1024, 65536) f64 moved 5.35 TB/s in this shape against 4.82
// with 256 lanes x 64 bytes and 4.31 with 256 x 128 bytes: many waves with short per-lane
// tiles hide the per-tile barrier best.  Keeping 2 or 3 tiles of loads in flight instead of 1
// measured no faster (512- and 1024-lane blocks, 223-328 us against 230 us).
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

// ---------------------------------------------------------------------------------------------
// Row scan with a decoupled look-back, tiles taken in memory order.  A block claims a tile id
// from an atomic counter -- so every tile it may wait on was claimed earlier and belongs to a
// running or finished block, whatever order the hardware dispatches blocks in -- and
// id = row * tiles + chunk, so consecutive claims read consecutive memory, the access pattern
// of a plain copy.  (Chunk-major claims, the previous design, streamed many rows at once and
// were slower.)  A tile is kVpt sub-tiles of kLbBlock 16-byte vectors: lane t of sub-tile v
// holds elements (v * kLbBlock + t) * VE .. + VE - 1, so every load instruction is fully
// coalesced, and one barrier exchanges the wave totals of all sub-tiles.
//
// Look-back: the tile publishes its aggregate A(c) (tagged relaxed atomics, publish.hpp), then
// wave 0 reads the status of up to 64 predecessors at once (lane l: tile c - 1 - l; all of a
// lane's status words in one round trip).  Once the nearest tile j with a published inclusive
// prefix P(j) is found and every tile between has its aggregate published,
// P(c - 1) = (((P(j) + A(j+1)) + A(j+2)) + ...) + A(c - 1), folded left to right, and
// P(c) = P(c - 1) + A(c) is published in turn.  Tile 0 publishes P(0) without waiting, so no tile
// waits for another tile's look-back, only for its predecessors' loads.  The fold follows the
// definition P(c) = P(c - 1) + A(c) whichever j is found, so the result is the same bits run to
// run.  A wait is bounded (wait_spin_limit polls): when it runs out the tile records
// kFaultScanWait, takes P = 0 and still publishes, so every block exits.
constexpr int kLbBlock = 512;
constexpr int kVpt = 4;  // 32 KB f64 tiles: measured faster than 16 KB here (fewer look-backs per byte)

struct LbArgs {
  RowIndexer<2> ix;     // non-axis dims: [0] input strides, [1] output strides
  uint64_t L;
  FastDiv tdiv;         // divides a tile id by the tiles per row
  uint32_t tiles;       // tiles per row
  uint32_t* counter;    // tile claim counter; nullptr when tiles == 1 (no look-back)
  uint64_t* status;     // per tile: W words of A(c), then W words of P(c)
  uint32_t* fault;      // the device's fault word (kcommon.hpp)
  uint32_t spin_limit;  // polls a look-back may make
  bool vec;             // 16-byte aligned rows
};

template <class T>
__global__ __launch_bounds__(kLbBlock) void k_scan_lookback(const T* __restrict__ a, T* __restrict__ c, LbArgs sa) {
  using A = typename ScanAcc<T>::A;
  constexpr int VE = int(16 / sizeof(T));
  constexpr int kWaves = kLbBlock / kWave;
  constexpr uint64_t TE = uint64_t(kLbBlock) * kVpt * VE;
  constexpr int W = sizeof(A) == 4 ? 1 : 2;
  __shared__ uint32_t s_id;
  __shared__ A s_wave[kVpt][kWaves];
  __shared__ A s_prefix;
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;

  uint32_t id = blockIdx.x;
  if (sa.counter) {
    if (tid == 0) s_id = atomicAdd(sa.counter, 1u);
    __syncthreads();
    id = s_id;
  }
  const uint32_t row = fd_div(sa.tdiv, id);
  const uint32_t chunk = id - row * sa.tiles;
  int64_t off[2];
  row_offsets<2>(sa.ix, row, off);
  const T* ain = a + off[0];
  T* cout = c + off[1];
  const uint64_t t0 = uint64_t(chunk) * TE;
  const bool full = sa.vec && t0 + TE <= sa.L;

  A x[kVpt][VE];
  if (full) {
    Vec<T, VE> v[kVpt];
#pragma unroll
    for (int u = 0; u < kVpt; ++u) v[u] = vload<T, VE>(ain + t0 + (uint64_t(u) * kLbBlock + tid) * VE);
#pragma unroll
    for (int u = 0; u < kVpt; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) x[u][e] = A(v[u].v[e]);
  } else {
#pragma unroll
    for (int u = 0; u < kVpt; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const uint64_t k = t0 + (uint64_t(u) * kLbBlock + tid) * VE + e;
        x[u][e] = k < sa.L ? A(ain[k]) : A(0);
      }
  }
  // in-lane inclusive runs, then a wave scan of the run totals per sub-tile
  A incl[kVpt];
#pragma unroll
  for (int u = 0; u < kVpt; ++u) {
#pragma unroll
    for (int e = 1; e < VE; ++e) x[u][e] = x[u][e - 1] + x[u][e];
    incl[u] = wave_incl_scan(x[u][VE - 1], lane);
    if (lane == kWave - 1) s_wave[u][wv] = incl[u];
  }
  __syncthreads();
  // exclusive offset of each lane's run inside the tile, and the tile aggregate (fixed order)
  A lane_off[kVpt];
  A run = A(0);
#pragma unroll
  for (int u = 0; u < kVpt; ++u) {
    A wo = A(0), st = A(0);
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      if (i < wv) wo = wo + s_wave[u][i];
      st = st + s_wave[u][i];
    }
    A le = shfl_up_acc(incl[u], 1);
    if (lane == 0) le = A(0);
    lane_off[u] = run + (wo + le);
    run = run + st;
  }
  const A agg = run;

  if (wv == 0) {
    A P = A(0);
    if (sa.counter) {
      uint64_t* const rowst = sa.status + uint64_t(row) * sa.tiles * (2 * W);
      auto agg_of = [&](uint32_t t) { return rowst + uint64_t(t) * (2 * W); };
      auto inc_of = [&](uint32_t t) { return rowst + uint64_t(t) * (2 * W) + W; };
      const bool last = chunk + 1 == sa.tiles;  // nothing waits on the last tile of a row
      if (chunk == 0) {
        if (lane == 0 && !last) publish_value<W>(inc_of(0), bits_of(agg));
      } else {
        if (lane == 0 && !last) publish_value<W>(agg_of(chunk), bits_of(agg));
        const bool valid = uint32_t(lane) < chunk;  // lane l looks at tile chunk - 1 - l
        const uint32_t j = valid ? chunk - 1 - uint32_t(lane) : 0;
        for (uint32_t spins = 0;; ++spins) {
          if (spins >= sa.spin_limit) {  // a limit of 0 gives up before the first poll
            if (lane == 0) atomicOr(sa.fault, kFaultScanWait);  // the prefix stays 0
            break;
          }
          // all status words of the lane's tile in one round trip: no load waits on another
          uint64_t wi[W], wa[W];
#pragma unroll
          for (int q = 0; q < W; ++q) {
            wi[q] = valid ? ld_relaxed(inc_of(j) + q) : 0;
            wa[q] = valid ? ld_relaxed(agg_of(j) + q) : 0;
          }
          bool has_inc = valid, has_agg = valid;
          uint64_t bi = 0, ba = 0;
#pragma unroll
          for (int q = 0; q < W; ++q) {
            has_inc = has_inc && (wi[q] & kTag);
            has_agg = has_agg && (wa[q] & kTag);
            bi |= (wi[q] & 0xffffffffu) << (32 * q);
            ba |= (wa[q] & 0xffffffffu) << (32 * q);
          }
          const uint64_t incm = __ballot(has_inc);
          const uint64_t okm = __ballot(has_agg || has_inc);
          if (incm != 0) {
            const int li = __builtin_ctzll(incm);  // nearest tile with a published prefix
            const uint64_t below = li == 0 ? 0 : ((uint64_t(1) << li) - 1);
            if ((okm & below) == below) {
              P = from_bits<A>(__shfl((unsigned long long)bi, li, kWave));
              for (int l = li - 1; l >= 0; --l) P = P + from_bits<A>(__shfl((unsigned long long)ba, l, kWave));
              break;
            }
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0 && !last) publish_value<W>(inc_of(chunk), bits_of(P + agg));
      }
    }
    if (lane == 0) s_prefix = P;
  }
  __syncthreads();
  const A P = s_prefix;

  if (full) {
#pragma unroll
    for (int u = 0; u < kVpt; ++u) {
      Vec<T, VE> v;
#pragma unroll
      for (int e = 0; e < VE; ++e) v.v[e] = T(P + (lane_off[u] + x[u][e]));
      vstore<T, VE>(cout + t0 + (uint64_t(u) * kLbBlock + tid) * VE, v);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kVpt; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const uint64_t k = t0 + (uint64_t(u) * kLbBlock + tid) * VE + e;
        if (k < sa.L) cout[k] = T(P + (lane_off[u] + x[u][e]));
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Row walk, for many rows: block b walks row b tile by tile, keeping the running prefix P in
// registers and prefetching the next tile while it scans the current one.  The association is
// fixed by the shape (lane, wave, tile), so results are identical run to run.
struct RowScanArgs {
  RowIndexer<2> ix;     // non-axis dims: [0] input strides, [1] output strides
  uint64_t L;
  uint32_t tiles;       // tiles per row
  bool vec;             // 16-byte aligned rows
};

template <class T>
__device__ inline void load_tile(const T* ain, uint64_t k0, uint64_t L, bool vec,
                                 typename ScanAcc<T>::A (&x)[seq_items<T>()]) {
  using A = typename ScanAcc<T>::A;
  constexpr int N = seq_items<T>();
  if (vec && k0 + N <= L) {
    Vec<T, N> v = vload<T, N>(ain + k0);
#pragma unroll
    for (int q = 0; q < N; ++q) x[q] = A(v.v[q]);
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = (k0 + j < L) ? A(ain[k0 + j]) : A(0);
  }
}

template <class T>
__global__ __launch_bounds__(kSeqBlock) void k_scan_rows_seq(const T* __restrict__ a, T* __restrict__ c,
                                                             RowScanArgs sa) {
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
      Vec<T, N> v;
#pragma unroll
      for (int q = 0; q < N; ++q) v.v[q] = T(P + (local + x[q]));
      vstore<T, N>(cout + k0, v);
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

// ---------------------------------------------------------------------------------------------
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
  if (p.kind == kRowScan && p.L > 16) {
    RowIndexer<2> ix{};  // non-axis dims, innermost first
    ix.nd = p.ond;
    for (int i = 0; i < p.ond; ++i) {
      int d = p.ond - 1 - i;
      ix.div[i] = make_fastdiv(uint32_t(p.oshape[d]));
      ix.stride[0][i] = p.istride[d];
      ix.stride[1][i] = p.ostride[d];
    }
    if (p.ond == 1 && p.oshape[0] == 1) ix.nd = 0;
    bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c)) & 15u) == 0;
    for (int d = 0; d < p.ond; ++d)
      if (((p.istride[d] * int64_t(sizeof(T))) % 16) || ((p.ostride[d] * int64_t(sizeof(T))) % 16)) vec = false;
    constexpr uint64_t TE = uint64_t(kLbBlock) * kVpt * (16 / sizeof(T));
    const uint64_t tiles = (p.L + TE - 1) / TE;
    // many rows of several tiles: walk each row in one block, no look-back
    if (tiles > 1 && p.rows >= 512) {
      RowScanArgs ss{};
      ss.ix = ix;
      ss.L = p.L;
      ss.vec = vec;
      constexpr uint64_t STILE = uint64_t(kSeqBlock) * seq_items<T>();
      ss.tiles = uint32_t((p.L + STILE - 1) / STILE);
      k_scan_rows_seq<T><<<dim3(unsigned(p.rows)), kSeqBlock, 0, st>>>(a, c, ss);
      return;
    }
    if (uint64_t(p.rows) * tiles >= (uint64_t(1) << 32)) {  // tile ids are 32-bit
      g_wrapper_error = 4;
      return;
    }
    LbArgs sa{};
    sa.ix = ix;
    sa.L = p.L;
    sa.vec = vec;
    sa.tiles = uint32_t(tiles);
    sa.tdiv = make_fastdiv(sa.tiles);
    if (tiles > 1) {
      // tmp capacity per the caller's formula: rows * (bpr [+ ceil(bpr/256) if bpr > 256]) elements
      const uint64_t bpr = (p.L + 255) / 256;
      const uint64_t cap = uint64_t(p.rows) * (bpr + (bpr > 256 ? (bpr + 255) / 256 : 0)) * sizeof(T);
      // word 0: the tile claim counter; then 2 * W status words per tile (aggregate, prefix)
      const uint64_t W = sizeof(typename ScanAcc<T>::A) == 4 ? 1 : 2;
      const uint64_t words = 1 + uint64_t(p.rows) * tiles * 2 * W;
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
    k_scan_lookback<T><<<dim3(unsigned(uint64_t(p.rows) * tiles)), kLbBlock, 0, st>>>(a, c, sa);
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
// or too small for the look-back state, 2 = reduction tile above 2^31 elements, 3 = bad rank or
// axis, 4 = a scan extent past 32 bits, 5 = no-alloc scratch too small).  New: the reference
// wrappers have no such failure mode.
int musapy_kernels_take_error(void) {
  int e = g_wrapper_error;
  g_wrapper_error = 0;
  return e;
}

}  // extern "C"
