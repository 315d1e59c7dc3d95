// reduce.hip -- sum / prod / max / min / mean / argmax / argmin over one axis, for gfx950.
//
// Drop-in for the reference's kernels/reduction.mu:1342-2055 (the `_v2` wrappers: naive,
// small_axis, partial, final, mid).  All entry points share two streaming kernels chosen from
// the host plan (plan.hpp):
//   row  the reduced axis is the walk direction: a group of lanes (a whole block, one wave, or a
//        single lane for very short axes) reduces one (output, tile) segment with 16-byte loads
//        when the axis is unit-stride, then combines through wave-64 butterflies and LDS;
//   col  the reduced axis is strided but the innermost output dim is unit-stride (axis=0 of a
//        C-order matrix): 64 lanes x VEC walk adjacent columns, the 4 waves of a block split the
//        rows, and LDS merges the waves -- every load is a coalesced row segment.
// Large reductions are split into tiles: the partial entry points write [out_size][tiles] and
// the final entry points reduce those rows with the same row kernel.  Every combine order is
// fixed, so results are identical from run to run.
#include "kcommon.hpp"
#include "reduce_ops.hpp"
#include "publish.hpp"
#include "../../../include/musapy_kernels.h"

#include <atomic>
#include <type_traits>
#include <mutex>

namespace mpy {

constexpr int kRBlock = 256;
constexpr int kRowBS = 512;  // block size of the block-per-segment row kernel (measured best on MI355X)
// Whole-array reductions: 256-lane blocks, each lane keeping 8 x 16-byte loads in flight (32 KB
// chunks).  At a quarter of the waves of 512-lane blocks with 4 loads per lane, a 64M f32 sum with
// its hand-over measured 40.5 us event-timed against 41.4-41.5 us (a one-round grid of 1024
// blocks; 2048 blocks 40.9 us, 4096 blocks 41.5-42.1 us): the 8192 waves of the previous grid
// took the dispatcher about 3.6 us to start.
constexpr int kAllBS = 256;
constexpr int kAllUnroll = 8;
// Chunks of loads held per lane (walk_chunks): kAllBuffers - 1 chunks in flight at each fold.  With
// the same registers, 4 buffers of 4 loads (12 in flight at each fold) and 3 of 4 measured no faster
// than 2 of 8 (64M f32 sum, argmax and max over (0,1) within 0.5 us, 256M level): the folds are not
// what holds the stream back.
constexpr int kAllBuffers = 2;

// what a kernel writes per (output, tile)
enum : int { kWriteFinal = 0, kWriteVal = 1, kWritePair = 2 };
// which final transform applies to an additive accumulator
enum : int { kFinPlain = 0, kFinMean = 1 };

template <class T>
struct RedOut {
  T* val;            // final values (kWriteFinal of value ops) or partial values
  int64_t* idx;      // arg results (kWriteFinal of arg ops) or partial indices
  double count;      // mean divisor
  int fin;
};

// --------------------------------------------------------------------------------------------
// Writing one finished accumulator.
template <class Op, class T, int WRITE>
__device__ inline void write_result(const RedOut<T>& out, uint64_t slot, typename Op::A acc, int64_t k0 = 0) {
  if constexpr (Op::kOrdered) {
    if constexpr (WRITE == kWritePair) {
      out.val[slot] = acc.idx < 0 ? T(0) : acc.val;
      out.idx[slot] = acc.idx < 0 ? int64_t(-1) : k0 + int64_t(acc.idx);
    } else if constexpr (Op::kArg) {  // final arg result
      out.idx[slot] = acc.idx < 0 ? 0 : k0 + int64_t(acc.idx);
    } else {
      // value max/min: an empty tile writes a marker the next level skips
      if (acc.idx < 0)
        out.val[slot] = Op::better(T(1), T(0)) ? ext_none<T>() : ext_none_min<T>();
      else
        out.val[slot] = acc.val;
    }
  } else {
    if (WRITE == kWriteFinal && out.fin == kFinMean)
      out.val[slot] = mean_of<T>(acc, out.count);
    else
      out.val[slot] = narrow<T>(acc);
  }
}

// NaN at axis position 0 absorbs the whole max/min/arg scan (see reduce_ops.hpp).
template <class Op, class T>
__device__ inline typename Op::A absorb_first(typename Op::A acc, T first) {
  if constexpr (Op::kOrdered) {
    if (is_nan(first)) {
      acc.val = first;
      acc.idx = 0;
    }
  }
  return acc;
}

// --------------------------------------------------------------------------------------------
// f32 max/min accumulators whose indices are below 2^32 - 1 (tile-relative int32, or absolute
// int64 in a whole-array reduction of fewer elements) as one unsigned 64-bit key, so that one
// unsigned max combines two of them instead of Op::comb on (value, index).  The key's high word
// orders the values (sign-magnitude bits mapped to unsigned order, inverted for min) and is never
// 0 for a value; its low word is ~index, so among equal values the lowest index wins, and an empty
// accumulator (key 0) loses to every element.  +0 and -0 compare equal and so share a key (the +0
// bits): whoever decodes a winning zero restores its sign from the element at the winning index.
// Accumulator values are never NaN here (the scan skips NaNs; the NaN-at-position-0 rule is
// applied after the combine), so the result is bit-identical to folding Op::comb.
template <class Op, class I>
__device__ inline uint64_t ext_key_f32(VI<float, I> a) {
  uint32_t u = __builtin_bit_cast(uint32_t, a.val);
  if ((u & 0x7fffffffu) == 0) u = 0;  // -0 -> +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (!Op::kMax) u = ~u;
  return a.idx < 0 ? 0 : (uint64_t(u) << 32) | uint32_t(~uint32_t(a.idx));
}
// the (value, index) of a key; a zero comes back as +0, and key 0 as the empty accumulator
template <class Op, class I>
__device__ inline VI<float, I> ext_unkey_f32(uint64_t key) {
  if (key == 0) return VI<float, I>{0.0f, I(-1)};
  uint32_t v = uint32_t(key >> 32);
  if (!Op::kMax) v = ~v;
  v = (v & 0x80000000u) ? (v & 0x7fffffffu) : ~v;
  return VI<float, I>{__builtin_bit_cast(float, v), I(~uint32_t(key))};
}
// A whole wave's accumulators combined through their keys (one 64-bit max per butterfly step);
// a winning zero takes its sign from the lane that holds the winning index.
template <class Op, class I>
__device__ inline VI<float, I> wave_reduce_ext_f32(VI<float, I> a) {
  uint64_t key = ext_key_f32<Op>(a);
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    const uint64_t o = acc_shfl(key, m);
    key = o > key ? o : key;
  }
  VI<float, I> r = ext_unkey_f32<Op, I>(key);
  if (key != 0 && __builtin_bit_cast(uint32_t, r.val) == 0) {
    // a zero won (the same key on every lane): take its sign from its lane
    const bool neg = a.idx == r.idx && (__builtin_bit_cast(uint32_t, a.val) >> 31);
    if (__ballot(neg) != 0) r.val = -0.0f;
  }
  return r;
}

// Group reduction (GROUP lanes -> lane 0 of the group holds the result).  `idx32`: the caller's
// int64 indices are all below 2^32 - 1 and no lane holds a NaN it must keep, so f32 max/min
// accumulators may take the packed-key wave combine (int32 indices always do).
template <class Op, int GROUP>
__device__ inline typename Op::A group_reduce(typename Op::A acc, bool idx32 = false) {
  using A = typename Op::A;
  constexpr bool kKeyed = GROUP >= kWave && Op::kOrdered;
  if constexpr (kKeyed && std::is_same_v<A, VI<float, int32_t>>) {
    acc = wave_reduce_ext_f32<Op>(acc);
  } else if constexpr (kKeyed && std::is_same_v<A, VI<float, int64_t>>) {
    if (idx32) {
      acc = wave_reduce_ext_f32<Op>(acc);
    } else {
#pragma unroll
      for (int m = kWave / 2; m >= 1; m >>= 1) acc = Op::comb(acc, acc_shfl(acc, m));
    }
  } else if constexpr (GROUP > 1) {
    constexpr int W = GROUP < kWave ? GROUP : kWave;
#pragma unroll
    for (int m = W / 2; m >= 1; m >>= 1) acc = Op::comb(acc, acc_shfl(acc, m));
  }
  if constexpr (GROUP > kWave) {
    __shared__ A part[GROUP / kWave];
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    if (lane == 0) part[w] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 1; i < GROUP / kWave; ++i) acc = Op::comb(acc, part[i]);
    }
  }
  return acc;
}

// --------------------------------------------------------------------------------------------
// row kernel: work item w = o * tiles + t, o = output index, t = tile along the axis
struct RowArgs {
  RowIndexer<1> ix;   // output coordinates -> input offset
  uint64_t R;         // axis length
  int64_t rs;         // axis stride
  uint64_t chunk;     // axis elements per tile (multiple of VEC when VEC > 1)
  uint32_t tiles;
  uint64_t nwork;     // out_size * tiles
  bool nt;            // streaming loads (launch input volume >= kStreamLoadBytes)
};

// One lane's share of a segment: lane l of a GROUP-lane group reduces elements l*VEC, l*VEC +
// GROUP*VEC, ... of the n-element segment at tb (indices relative to tb).  Lane 0 also returns
// the segment's first element in `first` (ordered reductions need it for the NaN-at-0 rule; it
// is kept from the load instead of being read again at the end).  The fold continues `acc`, and
// ordered reductions record indices as base + (index in the segment).
template <class Op, class T, int GROUP, int VEC, int UNROLL>
__device__ inline typename Op::A accumulate_segment(const T* __restrict__ tb, uint32_t n, int l, int64_t rs,
                                                    bool nt, T& first, typename Op::A acc = Op::init(),
                                                    int64_t base = 0) {
  uint32_t k = uint32_t(l) * VEC;
  constexpr uint32_t stepk = uint32_t(GROUP) * VEC;
  const bool lead = l == 0;  // lane 0 starts at element 0
  if (VEC > 1) {
    for (; k + (UNROLL - 1) * stepk + VEC <= n; k += UNROLL * stepk) {
      Vec<T, VEC> x[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) x[u] = vload_pol<T, VEC>(tb + k + u * stepk, nt);
      // all UNROLL loads are issued before the first use (the scheduler would otherwise hoist
      // arithmetic between them and wait on the first load early)
      __builtin_amdgcn_sched_barrier(0);
      T xs[UNROLL][VEC];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
#pragma unroll
        for (int v = 0; v < VEC; ++v) xs[u][v] = x[u].v[v];
      if (Op::kOrdered && lead && k == 0) first = xs[0][0];
      acc = Op::template step_chunk<UNROLL, VEC>(acc, xs, k, stepk, base);
    }
    for (; k + VEC <= n; k += stepk) {  // whole vectors left
      Vec<T, VEC> x = vload_pol<T, VEC>(tb + k, nt);
      if (Op::kOrdered && lead && k == 0) first = x.v[0];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc = Op::step(acc, x.v[v], base + int64_t(k + v));
    }
    if (k < n) {  // the last, partial vector of the tile
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (k + v < n) {
          const T x = tb[k + v];
          if (Op::kOrdered && lead && k + v == 0) first = x;
          acc = Op::step(acc, x, base + int64_t(k + v));
        }
    }
  } else {
    for (; k + (UNROLL - 1) * stepk < n; k += UNROLL * stepk) {
      T x[UNROLL];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) x[u] = tb[int64_t(k + u * stepk) * rs];
      if (Op::kOrdered && lead && k == 0) first = x[0];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) acc = Op::step(acc, x[u], base + int64_t(k + u * stepk));
    }
    for (; k < n; k += stepk) {
      const T x = tb[int64_t(k) * rs];
      if (Op::kOrdered && lead && k == 0) first = x;
      acc = Op::step(acc, x, base + int64_t(k));
    }
  }
  return acc;
}

template <class Op, class T, int BS, int GROUP, int VEC, int UNROLL, int WRITE>
__global__ __launch_bounds__(BS) void k_reduce_row(const T* __restrict__ a, RowArgs ra, RedOut<T> out) {
  using A = typename Op::A;
  constexpr int kPer = BS / GROUP;  // items per block
  const uint64_t w = uint64_t(blockIdx.x) * kPer + threadIdx.x / GROUP;
  const int l = threadIdx.x % GROUP;
  const bool live = w < ra.nwork;
  A acc = Op::init();
  uint64_t o = 0, t = 0, k0 = 0;
  T first{};
  if (live) {
    // one tile per output (every reduction that fills the GPU with its outputs): no 64-bit
    // division in front of the first load
    if (ra.tiles == 1) {
      o = w;
    } else {
      o = w / ra.tiles;
      t = w - o * ra.tiles;
    }
    int64_t off[1];
    row_offsets<1>(ra.ix, uint32_t(o), off);
    k0 = t * ra.chunk;
    const uint64_t k1 = k0 + ra.chunk < ra.R ? k0 + ra.chunk : ra.R;
    const T* tb = a + off[0] + int64_t(k0) * ra.rs;  // indices below are relative to the tile start
    const uint32_t n = k1 > k0 ? uint32_t(k1 - k0) : 0u;
    acc = accumulate_segment<Op, T, GROUP, VEC, UNROLL>(tb, n, l, ra.rs, ra.nt, first);
  }
  acc = group_reduce<Op, GROUP>(acc);
  if (live && (GROUP <= kWave ? l == 0 : threadIdx.x == 0)) {
    if (t == 0 && ra.R > 0) acc = absorb_first<Op, T>(acc, first);
    write_result<Op, T, WRITE>(out, w, acc, int64_t(k0));
  }
}

// --------------------------------------------------------------------------------------------
// Fused partial + final for few outputs.  Blocks 0 .. out_size*tiles-1 are the row kernel's
// (output, tile) blocks; each publishes its tile's accumulator (publish.hpp) and exits.  Blocks
// out_size*tiles + o, the last of the grid, are combiners: the dispatcher hands them out after
// every streaming block, so they poll the slots while the last tiles are still streaming and
// finish right after the last publish.  Lane l of a combiner owns tiles l, l + 512, ... (PER of
// them at most, a template parameter so the slot registers do not inflate the streaming blocks'
// register budget), waits until all of them are published (a bounded poll), folds them in
// ascending order, and the block tree combines the lanes: a fixed order, independent of timing.
// A combiner holds one block slot; with at most kFusedMaxOutputs of them the streaming blocks
// always find room, so the waits end.  Every slot read is cleared again, leaving the workspace
// zero.  Workspace: out_size * tiles * W slot words.
constexpr size_t kFusedMaxOutputs = 64;
constexpr size_t kFusedMaxTiles = 2048;  // <= 8 * kRowBS (the largest PER dispatched)
struct FusedArgs {
  uint64_t* slots;
  uint32_t* fault;      // the fault word of the launch's workspace (kcommon.hpp)
  uint32_t spin_limit;  // polls the combiner may make before it gives up
};

// Gathers the published W-word slots lane, lane + kRowBS, ... (below `count`) into v: all
// outstanding slots' words are loaded together, the ready ones kept, the rest polled again.
// Returns false when the poll budget ran out with slots still unpublished.
template <int W, int PER, int STRIDE = kRowBS>
__device__ inline bool gather_published(const uint64_t* slots, uint32_t count, uint32_t spin_limit,
                                        uint64_t (&v)[PER][W]) {
  uint32_t pending = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (threadIdx.x + j * STRIDE < count) pending |= 1u << j;
#pragma unroll
    for (int i = 0; i < W; ++i) v[j][i] = 0;
  }
  for (uint32_t spins = 0; pending != 0 && spins < spin_limit; ++spins) {
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (pending & (1u << j))
#pragma unroll
        for (int i = 0; i < W; ++i) v[j][i] = ld_relaxed(slots + uint64_t(threadIdx.x + j * STRIDE) * W + i);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      bool ready = true;
#pragma unroll
      for (int i = 0; i < W; ++i) ready = ready && (v[j][i] & kTag);
      if (ready) pending &= ~(1u << j);
    }
    if (pending) __builtin_amdgcn_s_sleep(2);
  }
  return pending == 0;
}

// After a combiner's gather: true when any lane of the block gave up.  Thread 0 then records the
// fault; the block skips its output write (the caller raises an error instead of returning a
// wrong value).
__device__ inline bool combiner_gave_up(bool ok, uint32_t* fault) {
  const bool bad = __syncthreads_or(ok ? 0 : 1) != 0;
  if (bad && threadIdx.x == 0 && fault) atomicOr(fault, kFaultReduceWait);
  return bad;
}

// a tile's accumulator (tile-relative int32 index) as the final's accumulator (absolute index)
template <class Op, class OpF>
__device__ inline typename OpF::A to_final(const typename Op::A& x, int64_t k0) {
  if constexpr (Op::kOrdered) {
    return typename OpF::A{x.val, x.idx < 0 ? int64_t(-1) : k0 + int64_t(x.idx)};
  } else {
    return x;
  }
}

template <class Op, class OpF, class T, int VEC, int UNROLL, int PER>
__global__ __launch_bounds__(kRowBS) void k_reduce_row_fused(const T* __restrict__ a, RowArgs ra, RedOut<T> out,
                                                             FusedArgs fa) {
  using A = typename Op::A;
  using AF = typename OpF::A;
  static_assert(sizeof(A) % 4 == 0, "accumulator must split into 32-bit slices");
  constexpr int W = int(sizeof(A) / 4);
  const uint64_t w = blockIdx.x;
  if (w < ra.nwork) {  // a streaming (output, tile) block
    const uint64_t o = w / ra.tiles;
    const uint64_t t = w - o * ra.tiles;
    int64_t off[1];
    row_offsets<1>(ra.ix, uint32_t(o), off);
    const uint64_t k0 = t * ra.chunk;
    const uint64_t k1 = k0 + ra.chunk < ra.R ? k0 + ra.chunk : ra.R;
    const uint32_t n = k1 > k0 ? uint32_t(k1 - k0) : 0u;
    T first{};
    A acc = accumulate_segment<Op, T, kRowBS, VEC, UNROLL>(a + off[0] + int64_t(k0) * ra.rs, n, threadIdx.x, ra.rs,
                                                           ra.nt, first);
    acc = group_reduce<Op, kRowBS>(acc);
    if (threadIdx.x == 0) {
      if (t == 0 && ra.R > 0) acc = absorb_first<Op, T>(acc, first);
      uint32_t s[W];
      __builtin_memcpy(s, &acc, sizeof(A));
      publish_slices<W>(fa.slots + w * W, s);
    }
    return;
  }
  // combiner of output o
  const uint64_t o = w - ra.nwork;
  uint64_t* row_slots = fa.slots + o * ra.tiles * W;
  uint64_t v[PER][W];
  const bool ok = gather_published<W, PER>(row_slots, ra.tiles, fa.spin_limit, v);
  AF r = OpF::init();
  A first{};
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t tt = threadIdx.x + j * kRowBS;
    if (tt >= ra.tiles) break;
    uint32_t s[W];
#pragma unroll
    for (int i = 0; i < W; ++i) s[i] = uint32_t(v[j][i]);
    A x;
    __builtin_memcpy(&x, s, sizeof(A));
    if (tt == 0) first = x;
    r = OpF::comb(r, to_final<Op, OpF>(x, int64_t(tt) * int64_t(ra.chunk)));
#pragma unroll
    for (int i = 0; i < W; ++i) st_relaxed(row_slots + uint64_t(tt) * W + i, 0);
  }
  if (combiner_gave_up(ok, fa.fault)) return;  // uniform over the block
  r = group_reduce<OpF, kRowBS>(r);
  if (threadIdx.x == 0) {
    if constexpr (Op::kOrdered) {
      // a NaN at axis position 0 absorbed tile 0 and therefore the whole reduction
      if (first.idx >= 0 && is_nan(first.val)) r = to_final<Op, OpF>(first, 0);
    }
    write_result<OpF, T, kWriteFinal>(out, o, r, 0);
  }
}

// --------------------------------------------------------------------------------------------
// Whole-array reduction (one output): block b of G streams chunks b, b+G, b+2G, ... (chunk =
// one round of the block, kAllBS lanes x UNROLL x 16 bytes; G from launch_reduce_all_fused), folding
// each chunk into its lanes' running accumulators in that fixed order; then blocks publish and a
// combiner block (index G) folds the G block results as in k_reduce_row_fused.  Ordered ops fold
// a chunk with tile-relative int32 indices and move it into an int64 running accumulator per lane.
//
// Walks a block's chunks k = 0 .. mine - 1 through NB register buffers: chunk k lives in buffer
// k % NB, and the loads of chunks k + 1 .. k + NB - 1 are in flight while chunk k is folded.  The
// buffer of every load and fold is a compile-time index (the steady loop is unrolled NB times and
// the last NB - 1 .. 2NB - 2 chunks take one of NB straight-line tails), so no registers are copied
// and no prefetch is conditional: a conditional load would make the wait before each later fold
// cover it too.  `last()` runs once, after the last chunk's loads are issued and before the folds
// that follow them.
template <int NB, class B, class Load, class Fold, class Last>
__device__ inline void walk_chunks(uint64_t mine, B (&buf)[NB], Load&& load, Fold&& fold, Last&& last) {
  static_assert(NB >= 2, "at least two buffers");
  if (mine < uint64_t(NB - 1)) {  // fewer chunks than a full prefetch: all loads, then the folds
    static_for<NB - 1>([&](auto J) { if (J.value < mine) load(uint64_t(J.value), buf[J.value]); });
    last();
    static_for<NB - 1>([&](auto J) { if (J.value < mine) fold(uint64_t(J.value), buf[J.value]); });
    return;
  }
  static_for<NB - 1>([&](auto J) { load(uint64_t(J.value), buf[J.value]); });
  uint64_t k = 0;
  for (; k + 2 * NB - 1 <= mine; k += NB) {
    static_for<NB>([&](auto J) {
      load(k + J.value + NB - 1, buf[(J.value + NB - 1) % NB]);
      fold(k + J.value, buf[J.value]);
    });
  }
  // mine - k = NB - 1 + e chunks are left, 0 <= e < NB; chunks k .. k + NB - 2 are loaded
  const uint32_t e = uint32_t(mine - k) - uint32_t(NB - 1);
  static_for<NB>([&](auto E) {
    if (e == E.value) {
      if constexpr (E.value == 0) last();
      static_for<E.value>([&](auto J) {
        load(k + J.value + NB - 1, buf[(J.value + NB - 1) % NB]);
        if constexpr (J.value + 1 == E.value) last();
        fold(k + J.value, buf[J.value]);
      });
      static_for<NB - 1>([&](auto J) { fold(k + E.value + J.value, buf[(E.value + J.value) % NB]); });
    }
  });
}

// One streaming block's lane accumulator (before the block reduction); `first` receives element 0
// on lane 0 of the block that reads it.
template <class OpF, class T, int VEC, int UNROLL, int BS>
__device__ inline typename OpF::A all_stream(const T* __restrict__ a, uint64_t n, uint32_t grid, uint64_t whole_q,
                                             uint32_t whole_r, uint32_t b, T& first) {
  using AF = typename OpF::A;
  constexpr uint64_t kChunk = uint64_t(BS) * UNROLL * VEC;
  AF acc = OpF::init();
  // The lane's running accumulator (absolute int64 indices) continues from chunk to chunk, so
  // an ordered fold searches a chunk only when the chunk beats it.  Whole chunks are software
  // pipelined: the next kAllBuffers - 1 chunks' loads are in flight while one is folded.
  constexpr uint32_t stepk = uint32_t(BS) * VEC;
  const uint64_t whole = n / kChunk;
  Vec<T, VEC> buf[kAllBuffers][UNROLL];
  // the block's k-th chunk is chunk b + k * grid of the array
  auto load = [&](uint64_t k, Vec<T, VEC>(&dst)[UNROLL]) {
    const T* p = a + (b + k * grid) * kChunk + threadIdx.x * VEC;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) dst[u] = vload_nt<T, VEC>(p + u * stepk);
  };
  auto fold = [&](uint64_t k, const Vec<T, VEC>(&src)[UNROLL]) {
    const uint64_t cc = b + k * grid;
    T xs[UNROLL][VEC];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int v = 0; v < VEC; ++v) xs[u][v] = src[u].v[v];
    if (cc == 0) first = xs[0][0];  // lane 0 holds element 0
    acc = OpF::template step_chunk<UNROLL, VEC>(acc, xs, threadIdx.x * VEC, stepk, int64_t(cc * kChunk));
  };
  // whole = whole_q * grid + whole_r (from the host: a 64-bit division here would delay every
  // block's first load)
  const uint64_t mine = whole_q + (b < whole_r ? 1 : 0);  // whole chunks of this block
  walk_chunks(mine, buf, load, fold, [] {});
  const uint64_t c = b + mine * grid;  // the first chunk index past this block's whole chunks
  if (c == whole && whole * kChunk < n) {  // the last, partial chunk
    T f{};
    acc = accumulate_segment<OpF, T, BS, VEC, UNROLL>(a + c * kChunk, uint32_t(n - c * kChunk), threadIdx.x, 1,
                                                      true, f, acc, int64_t(c * kChunk));
    if (c == 0) first = f;
  }
  return acc;
}

template <class Op, class OpF, class T, int VEC, int UNROLL, int PER>
__global__ __launch_bounds__(kAllBS) void k_reduce_all_fused(const T* __restrict__ a, uint64_t n, uint32_t grid,
                                                             uint64_t whole_q, uint32_t whole_r, RedOut<T> out,
                                                             FusedArgs fa) {
  using AF = typename OpF::A;
  static_assert(sizeof(AF) % 4 == 0, "accumulator must split into 32-bit slices");
  constexpr int W = int(sizeof(AF) / 4);
  const uint32_t b = blockIdx.x;
  if (b < grid) {
    T first{};
    AF acc = all_stream<OpF, T, VEC, UNROLL, kAllBS>(a, n, grid, whole_q, whole_r, b, first);
    acc = group_reduce<OpF, kAllBS>(acc, n < 0xffffffffull);
    if (threadIdx.x == 0) {
      if (b == 0 && n > 0) acc = absorb_first<OpF, T>(acc, first);
      uint32_t s[W];
      __builtin_memcpy(s, &acc, sizeof(AF));
      publish_slices<W>(fa.slots + uint64_t(b) * W, s);
    }
    return;
  }
  // combiner: lane l folds block results l, l + kAllBS, ... (PER of them at most)
  uint64_t v[PER][W];
  const bool ok = gather_published<W, PER, kAllBS>(fa.slots, grid, fa.spin_limit, v);
  AF r = OpF::init();
  AF first{};
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t bb = threadIdx.x + j * kAllBS;
    if (bb >= grid) break;
    uint32_t s[W];
#pragma unroll
    for (int i = 0; i < W; ++i) s[i] = uint32_t(v[j][i]);
    AF x;
    __builtin_memcpy(&x, s, sizeof(AF));
    if (bb == 0) first = x;
    r = OpF::comb(r, x);
  }
  if (!combiner_gave_up(ok, fa.fault)) {  // uniform over the block
    r = group_reduce<OpF, kAllBS>(r, n < 0xffffffffull);  // an absorbed NaN is put back below
    if (threadIdx.x == 0) {
      if constexpr (Op::kOrdered) {
        if (first.idx == 0 && is_nan(first.val)) r = first;  // block 0 absorbed a NaN at position 0
      }
      write_result<OpF, T, kWriteFinal>(out, 0, r, 0);
    }
  }
  // The slots go back to zero last: a barrier after these stores would wait for them (on gfx9 a
  // store holds the vector-memory counter that barriers and later loads wait on until it
  // reaches memory), which cost 0.7 us per barrier in the combiner of a 64M argmax.
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t bb = threadIdx.x + j * kAllBS;
    if (bb < grid) {
#pragma unroll
      for (int i = 0; i < W; ++i) st_relaxed(fa.slots + uint64_t(bb) * W + i, 0);
    }
  }
}

// f32 max / min / argmax / argmin over fewer than 2^32 - 1 elements: the same streaming blocks,
// each publishing its result as one key (ext_key_f32, two tagged words), so that the combiner
// folds keys with unsigned maxima.  With the (value, int64 index) accumulator published whole
// (four words), the combiner's gather and fold took 2.8 us after the last block against 0.8 us
// for an f32 sum, and its 8-slot version too many registers for the two-chunk grid.  The NaN at
// position 0 that absorbs the reduction, and the sign of a winning zero, are read back from the
// input by the combiner.
// Keys handed over through one 64-bit word each: the word holds key + 1, so that 0 still means
// "not published" (a key's high word never exceeds 0xff800000, so key + 1 does not wrap) and an
// empty accumulator's key 0 travels as 1.  One word per slot instead of two tagged halves halves
// the combiner's loads and registers: 8 slots per lane at once instead of 4.
__device__ inline void publish_key(uint64_t* slot, uint64_t key) { st_relaxed(slot, key + 1); }

// The largest of `count` published keys (lane l: slots l, l + kRowBS, ...), on thread 0, and
// whether every slot was published within the poll budget (uniform over the block).  The slots go
// back to zero after the block's last barrier, which would otherwise wait for those stores.
template <int PER, int BS = kRowBS>
__device__ inline bool fold_keys(uint64_t* slots, uint64_t count, uint32_t spin_limit, uint32_t* fault,
                                 uint64_t& key) {
  constexpr int kGroup = PER < 8 ? PER : 8;  // slots of a lane gathered at once
  key = 0;
  bool ok = true;
#pragma clang loop unroll(disable)
  for (uint64_t base = 0; base < count; base += uint64_t(kGroup) * BS) {
    uint64_t v[kGroup];
    uint32_t pending = 0;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      v[j] = 0;
      if (base + threadIdx.x + uint64_t(j) * BS < count) pending |= 1u << j;
    }
    for (uint32_t spins = 0; pending != 0 && spins < spin_limit; ++spins) {
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
        if (pending & (1u << j)) v[j] = ld_relaxed(slots + base + threadIdx.x + uint64_t(j) * BS);
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
        if (v[j] != 0) pending &= ~(1u << j);
      if (pending) __builtin_amdgcn_s_sleep(2);
    }
    ok = ok && pending == 0;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const uint64_t k = v[j] == 0 ? 0 : v[j] - 1;
      key = k > key ? k : key;
    }
  }
  const bool good = !combiner_gave_up(ok, fault);
  if (good) {
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) {
      const uint64_t o = acc_shfl(key, m);
      key = o > key ? o : key;
    }
    __shared__ uint64_t part[BS / kWave];
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 1; i < BS / kWave; ++i) key = part[i] > key ? part[i] : key;
    }
  }
  for (uint64_t bb = threadIdx.x; bb < count; bb += BS) st_relaxed(slots + bb, 0);
  return good;
}

template <class Op, class OpF, int UNROLL, int PER>
__global__ __launch_bounds__(kAllBS) void k_reduce_all_keyed(const float* __restrict__ a, uint64_t n, uint32_t grid,
                                                                uint64_t whole_q, uint32_t whole_r, RedOut<float> out,
                                                                FusedArgs fa) {
  using AF = typename OpF::A;
  const uint32_t b = blockIdx.x;
  if (b < grid) {
    float first = 0.0f;
    AF acc = all_stream<OpF, float, 4, UNROLL, kAllBS>(a, n, grid, whole_q, whole_r, b, first);
    acc = group_reduce<OpF, kAllBS>(acc, true);
    if (threadIdx.x == 0) publish_key(fa.slots + b, ext_key_f32<OpF>(acc));
    return;
  }
  const float a0 = a[0];  // loaded while the streaming blocks run
  uint64_t key;
  if (fold_keys<PER, kAllBS>(fa.slots, grid, fa.spin_limit, fa.fault, key) && threadIdx.x == 0) {
    AF r = ext_unkey_f32<OpF, int64_t>(key);
    if (r.idx >= 0 && r.val == 0.0f) r.val = a[r.idx];  // the first zero's own sign
    if (is_nan(a0)) r = AF{a0, 0};  // a NaN at position 0 absorbs the whole reduction
    write_result<OpF, float, kWriteFinal>(out, 0, r, 0);
  }
}

// --------------------------------------------------------------------------------------------
// col kernel: block = (outer, column group, tile); 64 lanes x VEC columns, 4 waves split rows.
struct ColArgs {
  RowIndexer<1> ix;   // outer output dims (all but the innermost one) -> input offset
  uint64_t C;         // innermost output extent (unit stride in the input)
  uint32_t cgroups;   // ceil(C / (64 * VEC))
  uint64_t R;
  int64_t rs;
  uint64_t chunk;
  uint32_t tiles;
  bool nt;            // streaming loads
};

// One (column group, tile) block of a column reduction: lane `lane` of wave 0 ends with the
// block's accumulators r[v] of its VEC columns (indices relative to the tile) and first[v], the
// elements of axis row 0 when the tile starts there.  `part` is the block's LDS for the waves.
template <class Op, class T, int VEC, int UNROLL, int BS = kRBlock>
__device__ inline void col_partial(const T* __restrict__ a, const ColArgs& ca, bool vec_ok, uint32_t t, uint32_t cg,
                                   uint32_t outer, typename Op::A (&part)[BS / kWave - 1][kWave * VEC],
                                   typename Op::A (&acc)[VEC], T (&first)[VEC]) {
  constexpr int kWaves = BS / kWave;
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  int64_t off[1];
  row_offsets<1>(ca.ix, outer, off);
  const uint64_t c0 = uint64_t(cg) * kWave * VEC + uint64_t(lane) * VEC;
  const T* base = a + off[0] + c0;
  const bool full = vec_ok && c0 + VEC <= ca.C;
  const uint64_t k0 = uint64_t(t) * ca.chunk;
  const uint64_t k1 = k0 + ca.chunk < ca.R ? k0 + ca.chunk : ca.R;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    acc[v] = Op::init();
    first[v] = T{};
  }
  if (c0 < ca.C) {
    uint64_t k = k0 + wv;
    if (full) {
      // the axis's row 0 for the NaN-at-0 rule: one extra load by wave 0 of tile 0, kept out of
      // the streaming loop (a capture inside it cost the ordered kernels ~10% on (8192, 8192))
      if (Op::kOrdered && k == 0 && k < k1) {
        const Vec<T, VEC> x = vload_pol<T, VEC>(base, ca.nt);
#pragma unroll
        for (int v = 0; v < VEC; ++v) first[v] = x.v[v];
      }
      // rounds of UNROLL rows (k, k + kWaves, ...).  Ordered ops are software pipelined: the
      // next round's loads are in flight while the current one is folded -- their fold takes
      // its first-index search in most rounds on random data, and with one wave per SIMD nothing
      // else hides it (max over (8192, 8192) axis 0: 50.9 -> 46.2 us).  Sums keep one round in
      // flight (pipelined: 42.9 -> 44.5 us).
      constexpr uint64_t kStep = uint64_t(UNROLL) * kWaves;
      const uint64_t lastu = uint64_t(UNROLL - 1) * kWaves;
      const uint64_t rounds = k + lastu < k1 ? (k1 - k - lastu - 1) / kStep + 1 : 0;
      Vec<T, VEC> x[UNROLL], y[UNROLL];  // ping-pong buffers
      auto load = [&](uint64_t kk, Vec<T, VEC>(&d)[UNROLL]) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) d[u] = vload_pol<T, VEC>(base + int64_t(kk + u * kWaves) * ca.rs, ca.nt);
      };
      auto fold = [&](uint64_t kk, const Vec<T, VEC>(&src)[UNROLL]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          T xs[UNROLL][1];
#pragma unroll
          for (int u = 0; u < UNROLL; ++u) xs[u][0] = src[u].v[v];
          acc[v] = Op::template step_chunk<UNROLL, 1>(acc[v], xs, uint32_t(kk - k0), uint32_t(kWaves));
        }
      };
      if (!Op::kOrdered) {
        for (uint64_t i = 0; i < rounds; ++i, k += kStep) {
          load(k, x);
          __builtin_amdgcn_sched_barrier(0);
          fold(k, x);
        }
      } else if (rounds > 0) {
        load(k, x);
        uint64_t i = 0;
        for (; i + 2 < rounds; i += 2) {
          load(k + kStep, y);
          fold(k, x);
          load(k + 2 * kStep, x);
          fold(k + kStep, y);
          k += 2 * kStep;
        }
        if (i + 1 < rounds) {
          load(k + kStep, y);
          fold(k, x);
          fold(k + kStep, y);
          k += 2 * kStep;
        } else {
          fold(k, x);
          k += kStep;
        }
      }
      for (; k < k1; k += kWaves) {
        Vec<T, VEC> x = vload_pol<T, VEC>(base + int64_t(k) * ca.rs, ca.nt);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = Op::step(acc[v], x.v[v], int64_t(k - k0));
      }
    } else {
      for (; k < k1; k += kWaves)
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (c0 + v < ca.C) {
            const T x = base[int64_t(k) * ca.rs + v];
            if (Op::kOrdered && k == 0) first[v] = x;
            acc[v] = Op::step(acc[v], x, int64_t(k - k0));
          }
    }
  }
  if (wv > 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) part[wv - 1][lane * VEC + v] = acc[v];
  }
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
#pragma unroll
      for (int i = 0; i < kWaves - 1; ++i) acc[v] = Op::comb(acc[v], part[i][lane * VEC + v]);
  }
}

template <class Op, class T, int VEC, int UNROLL, int WRITE, int BS = kRBlock>
__global__ __launch_bounds__(BS) void k_reduce_col(const T* __restrict__ a, ColArgs ca, RedOut<T> out, bool vec_ok) {
  using A = typename Op::A;
  __shared__ A part[BS / kWave - 1][kWave * VEC];
  const uint32_t b = blockIdx.x;
  const uint32_t t = b % ca.tiles;
  const uint32_t rest = b / ca.tiles;
  const uint32_t cg = rest % ca.cgroups;
  const uint32_t outer = rest / ca.cgroups;
  A acc[VEC];
  T first[VEC];
  col_partial<Op, T, VEC, UNROLL, BS>(a, ca, vec_ok, t, cg, outer, part, acc, first);
  const int lane = threadIdx.x % kWave;
  const uint64_t c0 = uint64_t(cg) * kWave * VEC + uint64_t(lane) * VEC;
  if (threadIdx.x < kWave && c0 < ca.C) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      if (c0 + v >= ca.C) break;
      A r = acc[v];
      if (t == 0 && ca.R > 0) r = absorb_first<Op, T>(r, first[v]);  // wave 0 walked row 0
      const uint64_t o = uint64_t(outer) * ca.C + c0 + v;
      write_result<Op, T, WRITE>(out, o * ca.tiles + t, r, int64_t(t) * int64_t(ca.chunk));
    }
  }
}

// --------------------------------------------------------------------------------------------
// Column sums, products and means in one launch: the (column group, tile) blocks of k_reduce_col
// count themselves in their group's counter as they start and publish wave 0's per-column
// accumulators (tagged relaxed words, publish.hpp) as they finish; the block whose increment
// completed the count folds the group's tiles in tile order, writes the outputs and returns the
// slots and the counter to zero.  Nobody waits but that block, the last of its group to start,
// for blocks already running (combiner blocks polling from the start of the launch measured
// slower than partial + final; counting at the end instead of the start cost 0.35 us more).
template <class Op, class T, int VEC, int UNROLL, int BS>
__global__ __launch_bounds__(BS) void k_reduce_col_last(const T* __restrict__ a, ColArgs ca, RedOut<T> out,
                                                        bool vec_ok, FusedArgs fa, uint32_t* counters) {
  using A = typename Op::A;
  static_assert(!Op::kOrdered && sizeof(A) % 4 == 0, "value folds of 32-bit slices");
  constexpr int W = int(sizeof(A) / 4);
  __shared__ A part[BS / kWave - 1][kWave * VEC];
  __shared__ uint32_t s_last;
  const uint32_t b = blockIdx.x;
  const uint32_t t = b % ca.tiles;
  const uint32_t group = b / ca.tiles;  // outer * cgroups + column group
  const uint32_t cg = group % ca.cgroups;
  const uint32_t outer = group / ca.cgroups;
  // the block counts itself before it streams, so the atomic's round trip overlaps the loads; the
  // last block to start is the one that folds (it waits, boundedly, for slower blocks' slots)
  uint32_t arrived = 0;
  if (threadIdx.x == 0) arrived = atomicAdd(counters + group, 1u);
  A acc[VEC];
  T first[VEC];
  col_partial<Op, T, VEC, UNROLL, BS>(a, ca, vec_ok, t, cg, outer, part, acc, first);
  const int lane = threadIdx.x % kWave;
  const uint64_t c0 = uint64_t(cg) * kWave * VEC + uint64_t(lane) * VEC;
  auto slot = [&](uint32_t tt, int v) {
    return fa.slots + ((uint64_t(group) * ca.tiles + tt) * (kWave * VEC) + uint64_t(lane) * VEC + v) * W;
  };
  if (threadIdx.x < kWave) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (c0 + v < ca.C) {
        uint32_t sl[W];
        __builtin_memcpy(sl, &acc[v], sizeof(A));
        publish_slices<W>(slot(t, v), sl);
      }
  }
  if (threadIdx.x == 0) s_last = arrived == ca.tiles - 1 ? 1u : 0u;
  __syncthreads();
  if (s_last == 0) return;
  // The group's last block.  Each round, wave w reads tile t0 + w (every lane its VEC columns, all
  // words in one round trip) into LDS and clears it; wave 0 then folds the round's tiles in order.
  constexpr int kWaves = BS / kWave;
  __shared__ A g[kWaves][kWave * VEC];
  const int wv = threadIdx.x / kWave;
  A r[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) r[v] = Op::init();
  bool ok = true;
  for (uint32_t t0 = 0; t0 < ca.tiles; t0 += kWaves) {
    const uint32_t tt = t0 + wv;
    if (tt < ca.tiles && c0 < ca.C) {
      uint64_t w[VEC][W];
      uint32_t pending = 0;
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (c0 + v < ca.C) pending |= 1u << v;
      for (uint32_t spins = 0; pending != 0 && spins < fa.spin_limit; ++spins) {  // a limit of 0: no poll
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (pending & (1u << v))
#pragma unroll
            for (int q = 0; q < W; ++q) w[v][q] = ld_relaxed(slot(tt, v) + q);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          bool ready = true;
#pragma unroll
          for (int q = 0; q < W; ++q) ready = ready && (w[v][q] & kTag);
          if (ready) pending &= ~(1u << v);
        }
        if (pending) __builtin_amdgcn_s_sleep(2);
      }
      ok = ok && pending == 0;
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        if (c0 + v >= ca.C) break;
        A x = Op::init();
        if (!(pending & (1u << v))) {
          uint32_t sl[W];
#pragma unroll
          for (int q = 0; q < W; ++q) sl[q] = uint32_t(w[v][q]);
          __builtin_memcpy(&x, sl, sizeof(A));
        }
        g[wv][lane * VEC + v] = x;
#pragma unroll
        for (int q = 0; q < W; ++q) st_relaxed(slot(tt, v) + q, 0);
      }
    }
    __syncthreads();
    if (wv == 0 && c0 < ca.C) {
      for (int k = 0; k < kWaves && t0 + k < ca.tiles; ++k)
#pragma unroll
        for (int v = 0; v < VEC; ++v) r[v] = Op::comb(r[v], g[k][lane * VEC + v]);
    }
    __syncthreads();
  }
  if (__syncthreads_or(ok ? 0 : 1) != 0) {  // a wait ran out: record it and leave the outputs unwritten
    if (threadIdx.x == 0) atomicOr(fa.fault, kFaultReduceWait);
  } else if (wv == 0 && c0 < ca.C) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (c0 + v < ca.C) write_result<Op, T, kWriteFinal>(out, uint64_t(outer) * ca.C + c0 + v, r[v], 0);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + group, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// --------------------------------------------------------------------------------------------
// max / min over both axes of a C-contiguous (R, C) array in one launch, with the result the
// reference's two passes give (reduce_multi, reduction.rs:118-155: axis 0 with keepdims, then
// axis 1).  Pass 1 keeps, per column, the first row holding the column's extreme, and a column
// whose row-0 element is NaN becomes NaN; pass 2 keeps the first column holding the extreme of
// those columns and skips NaN ones, unless column 0 is NaN, which absorbs everything.  So the
// result is the element of extreme value that comes first in COLUMN-major order, among the
// non-NaN elements of the columns whose row-0 element is not NaN -- or x[0][0] when that is NaN.
// The streaming blocks are the column kernel's (column group, row tile) blocks; wave 0 then folds
// its lanes' columns into one (value, col * R + row) key, skipping columns whose row 0 is NaN,
// and publishes it; the last block of the grid combines the published keys in a fixed order.
template <class Op, class OpF, class T, int VEC, int UNROLL, int BS, int PER>
__global__ __launch_bounds__(BS) void k_reduce_col2d(const T* __restrict__ a, ColArgs ca, uint32_t nblk, bool vec_ok,
                                                     RedOut<T> out, FusedArgs fa) {
  using A = typename Op::A;
  using AF = typename OpF::A;
  static_assert(sizeof(AF) % 4 == 0, "accumulator must split into 32-bit slices");
  constexpr int W = int(sizeof(AF) / 4);
  __shared__ A part[BS / kWave - 1][kWave * VEC];
  const uint32_t b = blockIdx.x;
  const bool idx32 = ca.R * ca.C < 0xffffffffull;
  if (b < nblk) {
    const uint32_t t = b % ca.tiles;
    const uint32_t cg = b / ca.tiles;
    // which of wave 0's columns head with a NaN (pass 2 drops them): read before the stream, so
    // the loads overlap it
    const uint64_t c0 = uint64_t(cg) * kWave * VEC + uint64_t(threadIdx.x % kWave) * VEC;
    uint32_t nan_head = 0;
    if (threadIdx.x < kWave) {
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (c0 + v < ca.C && is_nan(a[c0 + v])) nan_head |= 1u << v;
    }
    A acc[VEC];
    T first[VEC];
    col_partial<Op, T, VEC, UNROLL, BS>(a, ca, vec_ok, t, cg, 0, part, acc, first);
    if (threadIdx.x < kWave) {  // wave 0 holds the block's per-column results
      AF best = OpF::init();
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const uint64_t col = c0 + v;
        if (col < ca.C && acc[v].idx >= 0 && !(nan_head & (1u << v)))
          best = OpF::comb(best, AF{acc[v].val, int64_t(col) * int64_t(ca.R) + int64_t(t) * int64_t(ca.chunk) +
                                                    int64_t(acc[v].idx)});
      }
      best = group_reduce<OpF, kWave>(best, idx32);
      if (threadIdx.x == 0) {
        uint32_t s[W];
        __builtin_memcpy(s, &best, sizeof(AF));
        publish_slices<W>(fa.slots + uint64_t(b) * W, s);
      }
    }
    return;
  }
  // combiner: lane l folds keys l, l + BS, ... (PER at most), then the block tree
  uint64_t vv[PER][W];
  const bool ok = gather_published<W, PER, BS>(fa.slots, nblk, fa.spin_limit, vv);
  AF res = OpF::init();
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t bb = threadIdx.x + j * BS;
    if (bb >= nblk) break;
    uint32_t s[W];
#pragma unroll
    for (int i = 0; i < W; ++i) s[i] = uint32_t(vv[j][i]);
    AF xv;
    __builtin_memcpy(&xv, s, sizeof(AF));
    res = OpF::comb(res, xv);
#pragma unroll
    for (int i = 0; i < W; ++i) st_relaxed(fa.slots + uint64_t(bb) * W + i, 0);
  }
  if (combiner_gave_up(ok, fa.fault)) return;  // uniform over the block
  res = group_reduce<OpF, BS>(res, idx32);
  if (threadIdx.x == 0) {
    const T x00 = a[0];
    if (is_nan(x00)) res = AF{x00, 0};  // column 0 is NaN: it absorbs the second pass
    write_result<OpF, T, kWriteFinal>(out, 0, res, 0);
  }
}

// The same two-axis max / min for f32 with rows of at least 2048 elements (16-byte aligned, fewer
// than 2^32 - 1 elements), as row reductions: block r streams row r with the row kernel's access
// pattern and keeps, over the columns whose row-0 element is not NaN (row 0's values are loaded
// beside the row's, from the cache after the first blocks), the extreme and its first column.
// That is the same element: the two-pass result is the column-major first element of extreme value
// among those columns' non-NaN elements, and a row's extreme at its first column, keyed
// (value, column * R + row) (ext_key_f32), is the candidate of that row in column-major order.  Each
// block publishes its key; the last block folds the R keys with unsigned maxima and reads the
// winning zero's sign, and x[0][0] when it is NaN, back from the input.  (8192, 8192): kernel
// 43.7-43.8 us, against 54.2 us for the column-strip kernel (k_reduce_col2d, still used for f64,
// i64 and short rows).  Two rows per block measured slower (52 us: the two rows'
// registers spill at 8 waves per SIMD).
// One lane's extreme over row `row` of C f32 elements (C a multiple of 4), in the row kernel's
// access pattern; with `masked`, elements of columns whose row-0 element (in `a`) is NaN are
// skipped like NaNs.
// With `check` (and not `masked`), row 0's values are loaded beside the row's as well, the fold
// still takes every column, and `nan_seen` tells whether this lane met a NaN in row 0.
template <class Op, int UNROLL>
__device__ inline typename Op::A row_extreme(const float* __restrict__ row, const float* __restrict__ a, uint32_t C,
                                             bool masked, bool check, bool& nan_seen) {
  constexpr int VEC = 4;
  constexpr uint32_t stepk = uint32_t(kRowBS) * VEC;
  const float qn = qnan<float>();
  const bool need_h = masked || check;
  typename Op::A acc = Op::init();
  bool seen = false;
  uint32_t k = uint32_t(threadIdx.x) * VEC;
  for (; k + (UNROLL - 1) * stepk + VEC <= C; k += UNROLL * stepk) {
    Vec<float, VEC> x[UNROLL], h[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) x[u] = vload_nt<float, VEC>(row + k + u * stepk);
    if (need_h) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) h[u] = vload<float, VEC>(a + k + u * stepk);
    }
    __builtin_amdgcn_sched_barrier(0);
    float xs[UNROLL][VEC];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const bool hn = need_h && is_nan(h[u].v[v]);
        seen = seen || hn;
        xs[u][v] = (masked && hn) ? qn : x[u].v[v];
      }
    acc = Op::template step_chunk<UNROLL, VEC>(acc, xs, k, stepk, 0);
  }
  for (; k < C; k += stepk) {  // the rest of the row, in vectors
    const Vec<float, VEC> xv = vload_nt<float, VEC>(row + k);
    Vec<float, VEC> h{};
    if (need_h) h = vload<float, VEC>(a + k);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const bool hn = need_h && is_nan(h.v[v]);
      seen = seen || hn;
      acc = Op::step(acc, (masked && hn) ? qn : xv.v[v], int64_t(k + v));
    }
  }
  nan_seen = seen;
  return acc;
}

template <class Op, class OpF, int UNROLL, int PER>
__global__ __launch_bounds__(kRowBS, 8) void k_reduce_rows2d_keyed(const float* __restrict__ a, uint64_t R, uint32_t C,
                                                                   RedOut<float> out, FusedArgs fa) {
  using A = typename Op::A;
  using AF = typename OpF::A;
  const uint64_t b = blockIdx.x;
  // published by block 0: 1 + (row 0 holds a NaN), in kFlagCopies copies 256 bytes apart, so that
  // the polls of the other blocks spread over as many memory channels
  constexpr int kFlagCopies = 64;
  // blocks that check row 0 themselves: one resident generation (256 CUs x 4 blocks of 8 waves)
  constexpr uint64_t kSelfCheckBlocks = 1024;
  uint64_t* const flag = fa.slots;
  uint64_t* const keys = fa.slots + kFlagCopies * 32;  // one key word per row
  if (b < R) {
    const float* row = a + b * uint64_t(C);
    __shared__ uint32_t s_nanhead;
    // Which columns count: only those whose row-0 element is not NaN.  The blocks of the first
    // resident generation load row 0 beside their own row (from the cache after the first blocks)
    // and find out themselves whether it holds a NaN; block 0 publishes that.  Later blocks fold
    // their row over every column and read the word at the end (its load is issued first).  Only
    // when row 0 holds a NaN does a block fold its row again, masking with row 0's values.  At
    // (8192, 8192): the first generation waiting for the word instead cost 0.6 us (44.3-44.5 us
    // against 43.7-43.8 us), two generations checking 44.4 us, every block checking 4 us more,
    // and waiting for the word before folding 2.4 us.
    const bool self = b < kSelfCheckBlocks;
    uint64_t f = 0;
    if (!self && threadIdx.x == 0) f = ld_relaxed(flag + (b % kFlagCopies) * 32);
    bool nan_here = false;
    A acc = row_extreme<Op, UNROLL>(row, a, C, false, self, nan_here);
    if (self) {
      f = __syncthreads_or(nan_here ? 1 : 0) != 0 ? 2 : 1;
      if (b == 0 && threadIdx.x < kFlagCopies) st_relaxed(flag + threadIdx.x * 32, f);
      if (threadIdx.x == 0) s_nanhead = uint32_t(f);
    } else if (threadIdx.x == 0) {
      for (uint32_t spins = 1; f == 0 && spins < fa.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(2);
        f = ld_relaxed(flag + (b % kFlagCopies) * 32);
      }
      s_nanhead = uint32_t(f);  // 0 when the wait ran out: the block then masks, which is always right
    }
    acc = group_reduce<Op, kRowBS>(acc);  // the row's extreme; its barrier also hands s_nanhead over
    if (s_nanhead != 1) {  // row 0 holds a NaN (or the wait ran out): fold again over the eligible columns
      __syncthreads();     // thread 0 has read the block reduction's partials
      acc = row_extreme<Op, UNROLL>(row, a, C, true, false, nan_here);
      acc = group_reduce<Op, kRowBS>(acc);  // the row's extreme at its first eligible column
    }
    if (threadIdx.x == 0) {
      const uint64_t key =
          acc.idx < 0 ? 0 : ext_key_f32<OpF>(AF{acc.val, int64_t(acc.idx) * int64_t(R) + int64_t(b)});
      publish_key(keys + b, key);
    }
    return;
  }
  // combiner: the R row keys
  const float a0 = a[0];
  // Block 0's flag copies are read here, early (block 0 published them long before this block
  // started with many rows), and returned to zero below only once seen set: a zero stored without
  // reading the word could land before block 0's flag store (nothing orders that store before
  // block 0's key) and leave the flag set for the next launch on this workspace.
  uint64_t fl = 1;
  if (threadIdx.x < kFlagCopies) fl = ld_relaxed(flag + threadIdx.x * 32);
  uint64_t key;
  if (fold_keys<PER>(keys, R, fa.spin_limit, fa.fault, key) && threadIdx.x == 0) {
    AF r = ext_unkey_f32<OpF, int64_t>(key);
    if (r.idx >= 0 && r.val == 0.0f) {  // the first zero's own sign
      const uint64_t col = uint64_t(r.idx) / R, rw = uint64_t(r.idx) % R;
      r.val = a[rw * uint64_t(C) + col];
    }
    if (is_nan(a0)) r = AF{a0, 0};  // column 0 is NaN: it absorbs the second pass
    write_result<OpF, float, kWriteFinal>(out, 0, r, 0);
  }
  if (threadIdx.x < kFlagCopies) {
    for (uint32_t spins = 1; fl == 0 && spins < fa.spin_limit; ++spins) {
      __builtin_amdgcn_s_sleep(2);
      fl = ld_relaxed(flag + threadIdx.x * 32);
    }
    if (fl == 0) atomicOr(fa.fault, kFaultReduceWait);  // reported: the caller zeroes the workspace again
    st_relaxed(flag + threadIdx.x * 32, 0);
  }
}

// max / min over both axes of a C-contiguous f32 (R, C) array whose rows are whole 32 KB chunks
// (C a multiple of kAllChunk, at most 256 chunks per row), in the whole-array reductions' shape:
// G <= 1024 resident 256-lane blocks, block b taking chunks b, b + G, ... (row-major order, so
// chunk c is row c / cpr), 8 loads in flight per lane, the next chunk's loads issued while one is
// folded, plus a combiner block.  Each lane keeps the best key over its elements (ext_key_f32 of
// (value, column * R + row), so that ties go to the first element in column-major order, which is
// what the reference's axis-0-then-axis-1 passes keep); a chunk is searched for its first extreme
// only when its extreme reaches the lane's best.  Row 0 decides which columns count: the blocks
// that hold its chunks (blocks 0 .. cpr - 1, their first chunk) publish, per wave, whether their
// part held a NaN (in kFlag2Copies copies); every block reads them after its last chunk and, only
// when row 0 holds a NaN, folds its chunks again with those columns masked.
constexpr int kFlag2Copies = 16;
constexpr uint64_t kFlag2Stride = 1024;  // words between copies: up to 256 chunks x 4 waves
constexpr uint64_t kAllChunk = uint64_t(kAllBS) * kAllUnroll * 4;  // f32 elements per chunk

template <class OpF>
__device__ inline uint64_t chunk2d_key(uint64_t best, float (&xs)[kAllUnroll][4], const float* row0,
                                       bool masked, uint32_t col0, uint64_t R, uint32_t r) {
  using Op = OpExt<float, OpF::kMax, false, int32_t>;
  float m = xs[0][0];
  if (masked) {
    // columns whose row-0 element is NaN do not count (row0 holds this chunk's row-0 values)
#pragma unroll
    for (int u = 0; u < kAllUnroll; ++u) {
      const Vec<float, 4> h = vload<float, 4>(row0 + (u * kAllBS + threadIdx.x) * 4);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (is_nan(h.v[v])) xs[u][v] = qnan<float>();
    }
    m = xs[0][0];
  }
#pragma unroll
  for (int u = 0; u < kAllUnroll; ++u)
#pragma unroll
    for (int v = (u == 0 ? 1 : 0); v < 4; ++v) m = Op::pick(m, xs[u][v]);
  if (is_nan(m)) return best;
  // the best key m could have in this chunk (at its lowest column-major index): when it does not
  // beat the lane's best, no element of the chunk can, and the search is skipped
  const uint64_t top = ext_key_f32<OpF>(VI<float, int64_t>{m, int64_t(col0) * int64_t(R) + r});
  if (top <= best) return best;
  typename Op::A c = Op::template step_chunk<kAllUnroll, 4>(Op::init(), xs, threadIdx.x * 4, kAllBS * 4, 0);
  const uint64_t key =
      ext_key_f32<OpF>(VI<float, int64_t>{c.val, int64_t(col0 + uint32_t(c.idx)) * int64_t(R) + r});
  return key > best ? key : best;
}

template <class OpF, int PER>
__global__ __launch_bounds__(kAllBS) void k_reduce_2d_chunks(const float* __restrict__ a, uint64_t R, uint32_t C,
                                                              uint32_t grid, uint64_t whole_q, uint32_t whole_r,
                                                              RedOut<float> out, FusedArgs fa) {
  using AF = typename OpF::A;
  constexpr uint32_t stepk = uint32_t(kAllBS) * 4;
  const uint32_t cpr = C / uint32_t(kAllChunk);
  const uint64_t nch = R * cpr;
  uint64_t* const flags = fa.slots;  // [copy][chunk of row 0][wave]: 1 + (a NaN in that part)
  uint64_t* const keys = fa.slots + kFlag2Copies * kFlag2Stride;
  const uint32_t b = blockIdx.x;
  const int wv = threadIdx.x / kWave;
  if (b < grid) {
    auto rowcol = [&](uint64_t c, uint32_t& r, uint32_t& col0) {
      const uint32_t cc = uint32_t(c);  // R * C < 2^32
      r = cpr == 1 ? cc : cc / cpr;
      col0 = (cc - r * cpr) * uint32_t(kAllChunk);
    };
    Vec<float, 4> buf[kAllBuffers][kAllUnroll];
    auto load = [&](uint64_t c, Vec<float, 4>(&d)[kAllUnroll]) {
      const float* p = a + c * kAllChunk + threadIdx.x * 4;
#pragma unroll
      for (int u = 0; u < kAllUnroll; ++u) d[u] = vload_nt<float, 4>(p + u * stepk);
    };
    uint64_t best = 0;
    auto fold = [&](uint64_t c, const Vec<float, 4>(&d)[kAllUnroll], bool masked) {
      float xs[kAllUnroll][4];
#pragma unroll
      for (int u = 0; u < kAllUnroll; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) xs[u][v] = d[u].v[v];
      uint32_t r, col0;
      rowcol(c, r, col0);
      if (!masked && c == b && b < cpr) {
        // a part of row 0: publish whether it holds a NaN (per wave, no barrier in the stream)
        bool nan = false;
#pragma unroll
        for (int u = 0; u < kAllUnroll; ++u)
#pragma unroll
          for (int v = 0; v < 4; ++v) nan = nan || is_nan(xs[u][v]);
        const bool any = __ballot(nan) != 0;
        if (threadIdx.x % kWave < kFlag2Copies)
          st_relaxed(flags + (threadIdx.x % kWave) * kFlag2Stride + b * (kAllBS / kWave) + wv, any ? 2 : 1);
      }
      best = chunk2d_key<OpF>(best, xs, a + col0, masked, col0, R, r);
    };
    const uint64_t mine = whole_q + (b < whole_r ? 1 : 0);  // nch = whole_q * grid + whole_r (host)
    // row 0's NaN flags: lane l reads flag l of this block's copy.  The first read is issued with
    // the block's last loads, so that its round trip overlaps the last folds (the flags were
    // published at the blocks' first chunks); a flag not yet set is polled (bounded wait; a wait
    // that runs out counts as a NaN, so the block masks, which is always right).
    const uint32_t nflags = cpr * (kAllBS / kWave);
    const uint64_t* fc = flags + (b % kFlag2Copies) * kFlag2Stride;
    uint64_t f0 = 0;  // flag threadIdx.x (the first of the lane's flags)
    auto read_flag = [&]() {
      if (threadIdx.x < nflags && fa.spin_limit > 0) f0 = ld_relaxed(fc + threadIdx.x);
    };
    // the block's k-th chunk is chunk b + k * grid of the array
    walk_chunks(
        mine, buf, [&](uint64_t k, Vec<float, 4>(&d)[kAllUnroll]) { load(b + k * grid, d); },
        [&](uint64_t k, const Vec<float, 4>(&d)[kAllUnroll]) { fold(b + k * grid, d, false); }, read_flag);
    bool nan0 = false;
    for (uint32_t l = threadIdx.x; l < nflags; l += kAllBS) {
      uint64_t f = l == threadIdx.x ? f0 : (fa.spin_limit > 0 ? ld_relaxed(fc + l) : 0);
      for (uint32_t spins = 1; f == 0 && spins < fa.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(2);
        f = ld_relaxed(fc + l);
      }
      nan0 = nan0 || f != 1;
    }
    if (__syncthreads_or(nan0 ? 1 : 0)) {  // row 0 holds a NaN: fold the chunks again, masked
      best = 0;
      for (uint64_t c = b; c < nch; c += grid) {
        load(c, buf[0]);
        fold(c, buf[0], true);
      }
    }
    // block max of the lanes' keys
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) {
      const uint64_t o = acc_shfl(best, m);
      best = o > best ? o : best;
    }
    __shared__ uint64_t part[kAllBS / kWave];
    if (threadIdx.x % kWave == 0) part[wv] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 1; i < kAllBS / kWave; ++i) best = part[i] > best ? part[i] : best;
      publish_key(keys + b, best);
    }
    return;
  }
  // combiner
  const float a0 = a[0];
  // Row 0's NaN flags are set at their blocks' first chunks, long before the last key: they are
  // read here, while the streaming blocks run, and returned to zero with plain stores once every
  // block has read them (after the keys), so no read is left after the result write.  A flag is
  // cleared only once seen set: a zero stored unseen could land before the flag store it clears.
  const uint32_t nflags = cpr * (kAllBS / kWave);
  for (uint32_t i = threadIdx.x; i < nflags * kFlag2Copies; i += kAllBS) {
    const uint64_t* p = flags + (i / nflags) * kFlag2Stride + (i % nflags);
    uint64_t f = ld_relaxed(p);
    for (uint32_t spins = 1; f == 0 && spins < fa.spin_limit; ++spins) {
      __builtin_amdgcn_s_sleep(2);
      f = ld_relaxed(p);
    }
    if (f == 0) atomicOr(fa.fault, kFaultReduceWait);  // reported: the caller zeroes the workspace again
  }
  uint64_t key;
  if (fold_keys<PER, kAllBS>(keys, grid, fa.spin_limit, fa.fault, key) && threadIdx.x == 0) {
    AF r = ext_unkey_f32<OpF, int64_t>(key);
    if (r.idx >= 0 && r.val == 0.0f) {  // the first zero's own sign
      const uint64_t col = uint64_t(r.idx) / R, rw = uint64_t(r.idx) % R;
      r.val = a[rw * uint64_t(C) + col];
    }
    if (is_nan(a0)) r = AF{a0, 0};  // column 0 is NaN: it absorbs the second pass
    write_result<OpF, float, kWriteFinal>(out, 0, r, 0);
  }
  for (uint32_t i = threadIdx.x; i < nflags * kFlag2Copies; i += kAllBS)
    st_relaxed(flags + (i / nflags) * kFlag2Stride + (i % nflags), 0);
}

// --------------------------------------------------------------------------------------------
// pair kernel (arg final / mid): rows of (value, index) partials, contiguous [out][n]
template <class Op, class T, int GROUP, int WRITE>
__global__ __launch_bounds__(kRBlock) void k_reduce_pairs(const T* __restrict__ pv, const int64_t* __restrict__ pi,
                                                          uint64_t n, uint64_t chunk, uint32_t tiles, uint64_t nwork,
                                                          RedOut<T> out) {
  using A = typename Op::A;
  const uint64_t w = uint64_t(blockIdx.x) * (kRBlock / GROUP) + threadIdx.x / GROUP;
  const int l = threadIdx.x % GROUP;
  A acc = Op::init();
  uint64_t o = 0, t = 0;
  const bool live = w < nwork;
  if (live) {
    o = w / tiles;
    t = w - o * tiles;
    uint64_t k0 = t * chunk, k1 = k0 + chunk < n ? k0 + chunk : n;
    const T* vrow = pv + o * n;
    const int64_t* irow = pi + o * n;
    // 8 pairs per lane in flight before they are combined (the combine is order-free)
    constexpr int U = 8;
    uint64_t k = k0 + l;
    for (; k + uint64_t(U - 1) * GROUP < k1; k += uint64_t(U) * GROUP) {
      T v[U];
      int64_t ix[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        v[u] = vrow[k + u * GROUP];
        ix[u] = irow[k + u * GROUP];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc = Op::step_pair(acc, v[u], ix[u]);
    }
    for (; k < k1; k += GROUP) acc = Op::step_pair(acc, vrow[k], irow[k]);
  }
  acc = group_reduce<Op, GROUP>(acc);
  if (live && (GROUP <= kWave ? l == 0 : threadIdx.x == 0)) {
    if (t == 0 && is_nan(pv[o * n]) && pi[o * n] >= 0) {  // the level below was absorbed by x[0]
      acc.val = pv[o * n];
      acc.idx = pi[o * n];
    }
    write_result<Op, T, WRITE>(out, w, acc);
  }
}

// ============================================================================================
// host side
inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

template <class T> constexpr int rvec() { return sizeof(T) >= 16 ? 1 : int(16 / sizeof(T)); }

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline RowIndexer<1> out_indexer(const ReducePlan& p, int ndims) {
  // first `ndims` output dims (outermost first) as a row indexer, innermost first
  RowIndexer<1> ix{};
  ix.nd = ndims;
  for (int i = 0; i < ndims; ++i) {
    int d = ndims - 1 - i;
    ix.div[i] = make_fastdiv(uint32_t(p.oshape[d]));
    ix.stride[0][i] = p.ostride[d];
  }
  return ix;
}

// Recommended tiles per output: enough (output, tile) work items to fill 256 CUs several times
// over while each tile still streams a few tens of KB.
inline size_t tiles_hint(const ReducePlan& p, size_t es) {
  if (p.R <= 1 || p.out_size == 0) return 1;
  if (p.kind == kColReduce) {
    // column tiles: ~256 long-lived blocks (one per CU, 8 loads of 16 bytes in flight per lane)
    // measured best: (8192, 8192) f32 axis 0 at 6.3 TB/s vs 6.0 with 512 blocks of 4 loads;
    // more concurrent row bands lose to HBM row conflicts (32 bands: 4.7-5.6 TB/s); >= 64 rows
    // per tile
    const int vec = int(16 / es) > 0 ? int(16 / es) : 1;
    uint64_t C = p.oshape[p.ond - 1];
    uint64_t blocks = (p.out_size / C) * ceil_div(C, uint64_t(kWave) * vec);
    const uint64_t want_blocks = 256;
    if (blocks >= want_blocks) return 1;
    uint64_t tiles = ceil_div(want_blocks, blocks);
    uint64_t max_tiles = ceil_div(p.R, 64);
    if (tiles > max_tiles) tiles = max_tiles;
    return size_t(tiles < 1 ? 1 : tiles);
  }
  // row segments: one 512-lane block per (output, tile); below ~8K work items a single pass
  // leaves the GPU idle, so large axes are split into tiles of >= 32 KB (one full round of
  // 16-byte loads of the block kernel); reductions of <= 256 KB are not split at all
  const uint64_t want_items = 8192;
  if (p.out_size >= 2048) return 1;
  if (p.out_size * p.R * es <= (uint64_t(256) << 10)) return 1;
  uint64_t tiles = ceil_div(want_items, p.out_size);
  uint64_t max_tiles = ceil_div(p.R * es, 32768);
  if (tiles > max_tiles) tiles = max_tiles;
  return size_t(tiles < 1 ? 1 : tiles);
}

template <class Op, class T, int WRITE>
void launch_reduce(const T* a, RedOut<T> out, int ndim, const size_t* shape, const ssize_t* strides, int axis,
                   size_t axis_len, size_t out_size, size_t tiles, hipStream_t st) {
  if (out_size == 0) return;  // axis_len == 0 still writes the identity (0 for sums, 1 for products)
  if (!args_ok(ndim, axis)) return;
  if (tiles < 1) tiles = 1;
  ReducePlan p;
  plan_reduce(p, ndim, shape, strides, axis, axis_len, out_size);
  if (ceil_div(p.R, tiles) >= (uint64_t(1) << 31)) {  // tile-relative indices are 32-bit
    g_wrapper_error = 2;
    return;
  }
  // `tiles` is the caller's partial layout: every slot is written, tiles past the end of the
  // axis hold the operation's "empty" value
  constexpr int V = rvec<T>();
  // reductions write next to nothing, so streaming loads win at every volume measured (the
  // 128 MB c64 sum: 5.1 TB/s streaming vs 4.6 default), unlike the elementwise kernels
  const bool nt = true;
  if (p.kind == kColReduce && p.oshape[p.ond - 1] < (uint64_t(1) << 31)) {
    ColArgs ca{};
    ca.nt = nt;
    ca.ix = out_indexer(p, p.ond - 1);
    ca.C = p.oshape[p.ond - 1];
    ca.cgroups = uint32_t(ceil_div(ca.C, uint64_t(kWave) * V));
    ca.R = p.R;
    ca.rs = p.rstride;
    ca.chunk = ceil_div(p.R, tiles);
    ca.tiles = uint32_t(tiles);
    bool vec_ok = al16(a) && (ca.C % V == 0) && ((uint64_t(p.rstride < 0 ? -p.rstride : p.rstride) * sizeof(T)) % 16 == 0);
    for (int d = 0; d < p.ond - 1; ++d)
      if ((uint64_t(p.ostride[d] < 0 ? -p.ostride[d] : p.ostride[d]) * sizeof(T)) % 16) vec_ok = false;
    const uint64_t blocks = (p.out_size / ca.C) * ca.cgroups * ca.tiles;
    // sums: 8 waves with 4 rows of loads each (42.4-42.7 us for the (8192, 8192) f32 axis-0
    // partial, against 43.4-43.9 with 4 waves x 8 rows); ordered ops keep 4 waves x 8 rows
    // (46.0 us, against 46.9-47.3 with 8 waves): their pipelined fold wants the registers
    if constexpr (Op::kOrdered)
      k_reduce_col<Op, T, V, 8, WRITE, 256><<<dim3(unsigned(blocks)), 256, 0, st>>>(a, ca, out, vec_ok);
    else
      k_reduce_col<Op, T, V, 4, WRITE, 512><<<dim3(unsigned(blocks)), 512, 0, st>>>(a, ca, out, vec_ok);
    return;
  }
  RowArgs ra{};
  ra.nt = nt;
  ra.ix = out_indexer(p, p.ond);
  ra.R = p.R;
  ra.rs = p.rstride;
  ra.tiles = uint32_t(tiles);
  uint64_t chunk = ceil_div(p.R, tiles);
  bool vec_ok = (p.rstride == 1) && al16(a);
  for (int d = 0; d < p.ond; ++d)
    if ((uint64_t(p.ostride[d] < 0 ? -p.ostride[d] : p.ostride[d]) * sizeof(T)) % 16) vec_ok = false;
  if (vec_ok && V > 1) chunk = ceil_div(chunk, V) * V;
  ra.chunk = chunk;
  ra.nwork = uint64_t(out_size) * tiles;
  const uint64_t seg = chunk;
  if (seg * sizeof(T) >= 16384) {  // >= 16 KB: a 512-lane block per segment
    unsigned grid = unsigned(ra.nwork);
    if (vec_ok)
      k_reduce_row<Op, T, kRowBS, kRowBS, V, 4, WRITE><<<grid, kRowBS, 0, st>>>(a, ra, out);
    else
      k_reduce_row<Op, T, kRowBS, kRowBS, 1, 8, WRITE><<<grid, kRowBS, 0, st>>>(a, ra, out);
  } else if (seg >= 64) {
    unsigned grid = unsigned(ceil_div(ra.nwork, kRBlock / kWave));
    if (vec_ok)
      k_reduce_row<Op, T, kRBlock, kWave, V, 2, WRITE><<<grid, kRBlock, 0, st>>>(a, ra, out);
    else
      k_reduce_row<Op, T, kRBlock, kWave, 1, 4, WRITE><<<grid, kRBlock, 0, st>>>(a, ra, out);
  } else if (seg >= 8 && ra.rs == 1) {
    // short contiguous segments (e.g. the [out][tiles] partials of a final): 16 lanes per
    // output read one coalesced run instead of one lane striding through it
    unsigned grid = unsigned(ceil_div(ra.nwork, kRBlock / 16));
    k_reduce_row<Op, T, kRBlock, 16, 1, 2, WRITE><<<grid, kRBlock, 0, st>>>(a, ra, out);
  } else {
    unsigned grid = unsigned(ceil_div(ra.nwork, kRBlock));
    k_reduce_row<Op, T, kRBlock, 1, 1, 4, WRITE><<<grid, kRBlock, 0, st>>>(a, ra, out);
  }
}

// final over [out_size][num_partials] contiguous partials: the row kernel with unit stride
template <class Op, class T>
void launch_final(const T* partials, RedOut<T> out, size_t num_partials, size_t out_size, hipStream_t st) {
  size_t shape[2] = {out_size, num_partials};
  ssize_t strides[2] = {ssize_t(num_partials), 1};
  launch_reduce<Op, T, kWriteFinal>(partials, out, 2, shape, strides, 1, num_partials, out_size, 1, st);
}

template <class Op, class T, int WRITE>
void launch_pairs(const T* pv, const int64_t* pi, RedOut<T> out, size_t n, size_t out_size, size_t tiles,
                  hipStream_t st) {
  if (out_size == 0 || n == 0) return;
  if (tiles < 1) tiles = 1;
  uint64_t chunk = ceil_div(n, tiles);
  uint64_t nwork = uint64_t(out_size) * tiles;
  if (chunk >= 2048) {  // long segments: a whole block per (output, tile)
    k_reduce_pairs<Op, T, kRBlock, WRITE><<<unsigned(nwork), kRBlock, 0, st>>>(pv, pi, n, chunk, uint32_t(tiles), nwork, out);
  } else {
    unsigned grid = unsigned(ceil_div(nwork, kRBlock / kWave));
    k_reduce_pairs<Op, T, kWave, WRITE><<<grid, kRBlock, 0, st>>>(pv, pi, n, chunk, uint32_t(tiles), nwork, out);
  }
}

// count produced by "+1" repeated axis_len times in T (cpu_mean_typed, op_builder.rs:3608-3612)
template <class T> inline double mean_count(size_t n) {
  if (sizeof(T) == 4) return double(n > (size_t(1) << 24) ? (size_t(1) << 24) : n);
  return double(n > (size_t(1) << 53) ? (size_t(1) << 53) : n);
}

template <class T> inline RedOut<T> vout(T* c) { return RedOut<T>{c, nullptr, 0.0, kFinPlain}; }
template <class T> inline RedOut<T> iout(int64_t* c) { return RedOut<T>{nullptr, c, 0.0, kFinPlain}; }
template <class T> inline RedOut<T> mout(T* c, double cnt) { return RedOut<T>{c, nullptr, cnt, kFinMean}; }

// what a single-launch launcher did
enum : int { kFusedLaunched = 0, kFusedNotCovered = -1, kFusedNoRoom = -2 };

template <class Op, class OpF, class T>
int launch_reduce_all_fused(const T* a, RedOut<T> out, uint64_t n, const WsSplit& w, hipStream_t st);

// Column sums, products and means of `tiles` row tiles in one launch (k_reduce_col_last): the
// slots hold groups x tiles x (64 * VEC) accumulators, then one 32-bit counter per group.
template <class Op, class T>
int launch_reduce_col_last(const T* a, RedOut<T> out, const ReducePlan& p, size_t tiles, const WsSplit& w,
                           hipStream_t st) {
  constexpr int V = rvec<T>();
  constexpr uint64_t W = sizeof(typename Op::A) / 4;
  if (p.oshape[p.ond - 1] >= (uint64_t(1) << 31) || ceil_div(p.R, uint64_t(tiles)) >= (uint64_t(1) << 31))
    return kFusedNotCovered;
  ColArgs ca{};
  ca.nt = true;
  ca.ix = out_indexer(p, p.ond - 1);
  ca.C = p.oshape[p.ond - 1];
  ca.cgroups = uint32_t(ceil_div(ca.C, uint64_t(kWave) * V));
  ca.R = p.R;
  ca.rs = p.rstride;
  ca.chunk = ceil_div(p.R, uint64_t(tiles));
  ca.tiles = uint32_t(tiles);
  bool vec_ok = al16(a) && (ca.C % V == 0) && ((uint64_t(p.rstride < 0 ? -p.rstride : p.rstride) * sizeof(T)) % 16 == 0);
  for (int d = 0; d < p.ond - 1; ++d)
    if ((uint64_t(p.ostride[d] < 0 ? -p.ostride[d] : p.ostride[d]) * sizeof(T)) % 16) vec_ok = false;
  const uint64_t groups = (p.out_size / ca.C) * ca.cgroups;
  const uint64_t blocks = groups * tiles;
  const uint64_t slot_words = groups * tiles * uint64_t(kWave) * V * W;
  if (blocks >= (uint64_t(1) << 31)) return kFusedNotCovered;
  if ((slot_words + ceil_div(groups, uint64_t(2))) * 8 > w.payload_bytes) return kFusedNoRoom;
  FusedArgs fa{};
  fa.slots = w.payload;
  fa.fault = w.fault;
  fa.spin_limit = wait_spin_limit();
  uint32_t* counters = reinterpret_cast<uint32_t*>(fa.slots + slot_words);
  k_reduce_col_last<Op, T, V, 4, 512><<<dim3(unsigned(blocks)), 512, 0, st>>>(a, ca, out, vec_ok, fa, counters);
  return kFusedLaunched;
}

// The fused single launch for a row-kind reduction split into `tiles` tiles.  kFusedNotCovered
// (nothing launched) when the shape does not take the 512-lane block path, kFusedNoRoom when the
// workspace is too small for its slots.
template <class Op, class OpF, class T>
int launch_reduce_fused(const T* a, RedOut<T> out, int ndim, const size_t* shape, const ssize_t* strides, int axis,
                        size_t axis_len, size_t out_size, size_t tiles, void* ws, size_t ws_bytes, hipStream_t st) {
  WsSplit w;
  if (out_size == 0 || axis_len == 0 || tiles < 2 || !ws_split(ws, ws_bytes, w)) return kFusedNotCovered;
  if (!args_ok(ndim, axis)) return kFusedNotCovered;
  ReducePlan p;
  plan_reduce(p, ndim, shape, strides, axis, axis_len, out_size);
  if constexpr (!Op::kOrdered) {
    if (p.kind == kColReduce) return launch_reduce_col_last<Op, T>(a, out, p, tiles, w, st);
  }
  if (out_size > kFusedMaxOutputs) return kFusedNotCovered;
  // 2048 tiles measured best for 64M f32 (a combiner lane then folds 4)
  if (tiles > kFusedMaxTiles) tiles = kFusedMaxTiles;
  if (p.kind != kRowReduce || p.rstride != 1 || !al16(a)) return kFusedNotCovered;
  for (int d = 0; d < p.ond; ++d)
    if ((uint64_t(p.ostride[d] < 0 ? -p.ostride[d] : p.ostride[d]) * sizeof(T)) % 16) return kFusedNotCovered;
  // one output over one contiguous run: the interleaved-chunk grid of launch_reduce_all_fused
  if (out_size == 1) {
    const int r = launch_reduce_all_fused<Op, OpF, T>(a, out, p.R, w, st);
    if (r != kFusedNotCovered) return r;
  }
  constexpr int V = rvec<T>();
  uint64_t chunk = ceil_div(ceil_div(p.R, tiles), uint64_t(V)) * V;
  if (chunk * sizeof(T) < 16384 || chunk >= (uint64_t(1) << 31)) return kFusedNotCovered;
  if (uint64_t(out_size) * tiles >= (uint64_t(1) << 31)) return kFusedNotCovered;
  const uint64_t W = sizeof(typename Op::A) / 4;
  const uint64_t words = uint64_t(out_size) * tiles * W;
  if (words * 8 > w.payload_bytes) return kFusedNoRoom;
  FusedArgs fa{};
  fa.slots = w.payload;
  fa.fault = w.fault;
  fa.spin_limit = wait_spin_limit();
  RowArgs ra{};
  ra.nt = true;
  ra.ix = out_indexer(p, p.ond);
  ra.R = p.R;
  ra.rs = 1;
  ra.tiles = uint32_t(tiles);
  ra.chunk = chunk;
  ra.nwork = uint64_t(out_size) * tiles;
  // streaming blocks first, then one combiner per output
  const dim3 grid(unsigned(ra.nwork + out_size));
  switch (ceil_div(tiles, uint64_t(kRowBS))) {
    case 1: k_reduce_row_fused<Op, OpF, T, V, 4, 1><<<grid, kRowBS, 0, st>>>(a, ra, out, fa); break;
    case 2: k_reduce_row_fused<Op, OpF, T, V, 4, 2><<<grid, kRowBS, 0, st>>>(a, ra, out, fa); break;
    default: k_reduce_row_fused<Op, OpF, T, V, 4, 4><<<grid, kRowBS, 0, st>>>(a, ra, out, fa); break;
  }
  return kFusedLaunched;
}

// Whole-array reduction of `n` contiguous, 16-byte aligned elements: G streaming blocks of kAllBS
// lanes (block b takes chunks b, b + G, ...) plus a combiner block, dispatched after them.  G is
// ceil(chunks / 2), at most 1024: 64M f32 runs one round of resident blocks, 8 chunks each.  The
// sums fit five blocks per CU, so their combiner is resident from the start; the keyed arg kernels
// (four per CU) fill the GPU with the streaming blocks, and their combiner starts when the first
// streaming block ends, long before the last.  The combiner polls every 128 cycles.  With 512-lane blocks of 4
// loads per lane, a one-round grid had measured slower (43.0 us against 40.7 us for two chunks per
// block in 4096 blocks, whose later blocks the dispatcher hands to whichever CUs finish first);
// with 256-lane blocks of 8 loads per lane the one-round grid is the fastest measured (see kAllBS).
constexpr uint64_t kAllMaxBlocks = 1024;  // one round of resident 256-lane blocks
template <class Op, class OpF, class T>
int launch_reduce_all_fused(const T* a, RedOut<T> out, uint64_t n, const WsSplit& w, hipStream_t st) {
  constexpr int V = rvec<T>();
  constexpr uint64_t kChunk = uint64_t(kAllBS) * kAllUnroll * V;
  constexpr uint64_t W = sizeof(typename OpF::A) / 4;
  if (n == 0 || !al16(a)) return kFusedNotCovered;
  const uint64_t nchunks = ceil_div(n, kChunk);
  uint64_t grid = ceil_div(nchunks, uint64_t(2));
  if (grid > kAllMaxBlocks) grid = kAllMaxBlocks;
  if (grid < 2) return kFusedNotCovered;
  if (grid * W * 8 > w.payload_bytes) return kFusedNoRoom;
  FusedArgs fa{};
  fa.slots = w.payload;
  fa.fault = w.fault;
  fa.spin_limit = wait_spin_limit();
  const uint32_t g = uint32_t(grid);
  const dim3 blocks(g + 1);
  const uint64_t q = (n / kChunk) / grid;
  const uint32_t r = uint32_t((n / kChunk) % grid);
  const uint64_t per = ceil_div(grid, uint64_t(kAllBS));  // combiner slots per lane, at most 4
  if constexpr (Op::kOrdered && std::is_same_v<T, float>) {
    if (n < 0xffffffffull) {  // one key per block
      if (per == 1)
        k_reduce_all_keyed<Op, OpF, kAllUnroll, 1><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
      else if (per == 2)
        k_reduce_all_keyed<Op, OpF, kAllUnroll, 2><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
      else
        k_reduce_all_keyed<Op, OpF, kAllUnroll, 4><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
      return kFusedLaunched;
    }
  }
  if (per == 1)
    k_reduce_all_fused<Op, OpF, T, V, kAllUnroll, 1><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
  else if (per == 2)
    k_reduce_all_fused<Op, OpF, T, V, kAllUnroll, 2><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
  else
    k_reduce_all_fused<Op, OpF, T, V, kAllUnroll, 4><<<blocks, kAllBS, 0, st>>>(a, n, g, q, r, out, fa);
  return kFusedLaunched;
}


// max / min over both axes of a C-contiguous (R, C) array in one launch: f32 rows of whole 32 KB
// chunks in the whole-array grid (k_reduce_2d_chunks, at most 1024 + 1 blocks), other f32 rows of
// at least 2048 elements as keyed rows (k_reduce_rows2d_keyed, R + 1 blocks), the rest with the
// column kernel's tiling (k_reduce_col2d, about 256 blocks); kFusedNotCovered when the shape fits
// none of them
template <class Op, class OpF, class T>
int launch_reduce_2d_ordered(const T* a, RedOut<T> out, uint64_t R, uint64_t C, void* ws, size_t ws_bytes,
                             hipStream_t st) {
  constexpr int V = rvec<T>();
  constexpr int BS = 256;
  WsSplit w;
  if (R == 0 || C == 0 || !ws_split(ws, ws_bytes, w) || R >= (uint64_t(1) << 31) || R * C >= (uint64_t(1) << 62))
    return kFusedNotCovered;
  if constexpr (std::is_same_v<T, float>) {
    // rows of whole 32 KB chunks: the chunked kernel in one round of resident blocks
    const uint64_t cpr = C / kAllChunk;
    if (C % kAllChunk == 0 && cpr <= 256 && R * C < 0xffffffffull && al16(a) &&
        (kFlag2Copies * kFlag2Stride + kAllMaxBlocks) * 8 <= w.payload_bytes) {
      FusedArgs fk{};
      fk.slots = w.payload;
      fk.fault = w.fault;
      fk.spin_limit = wait_spin_limit();
      const uint64_t nch = R * cpr;
      const uint32_t grid = uint32_t(nch < kAllMaxBlocks ? nch : kAllMaxBlocks);
      const dim3 g(grid + 1);
      const uint64_t per = ceil_div(grid, uint64_t(kAllBS));
      const uint64_t q = nch / grid;
      const uint32_t rr = uint32_t(nch % grid);
      if (per == 1)
        k_reduce_2d_chunks<OpF, 1><<<g, kAllBS, 0, st>>>(a, R, uint32_t(C), grid, q, rr, out, fk);
      else if (per == 2)
        k_reduce_2d_chunks<OpF, 2><<<g, kAllBS, 0, st>>>(a, R, uint32_t(C), grid, q, rr, out, fk);
      else
        k_reduce_2d_chunks<OpF, 4><<<g, kAllBS, 0, st>>>(a, R, uint32_t(C), grid, q, rr, out, fk);
      return kFusedLaunched;
    }
    // rows of at least one block round: the row-keyed kernel
    if (C >= 2048 && C % 4 == 0 && C < (uint64_t(1) << 31) && R * C < 0xffffffffull && al16(a) &&
        (64 * 32 + R) * 8 <= w.payload_bytes) {
      FusedArgs fk{};
      fk.slots = w.payload;
      fk.fault = w.fault;
      fk.spin_limit = wait_spin_limit();
      const dim3 g(unsigned(R + 1));
      using OpR = OpExt<float, Op::kMax, false, int32_t>;
      const uint64_t per = ceil_div(R, uint64_t(kRowBS));
      if (per == 1)
        k_reduce_rows2d_keyed<OpR, OpF, 4, 1><<<g, kRowBS, 0, st>>>(a, R, uint32_t(C), out, fk);
      else if (per == 2)
        k_reduce_rows2d_keyed<OpR, OpF, 4, 2><<<g, kRowBS, 0, st>>>(a, R, uint32_t(C), out, fk);
      else if (per <= 4)
        k_reduce_rows2d_keyed<OpR, OpF, 4, 4><<<g, kRowBS, 0, st>>>(a, R, uint32_t(C), out, fk);
      else
        k_reduce_rows2d_keyed<OpR, OpF, 4, 8><<<g, kRowBS, 0, st>>>(a, R, uint32_t(C), out, fk);
      return kFusedLaunched;
    }
  }
  ColArgs ca{};
  ca.nt = true;
  ca.ix.nd = 0;
  ca.C = C;
  ca.cgroups = uint32_t(ceil_div(C, uint64_t(kWave) * V));
  ca.R = R;
  ca.rs = int64_t(C);
  // about 256 long-lived blocks, as the column kernel (128: 67 us, 256: 54 us, 512: 53.5 us,
  // 1024: 61 us for (8192, 8192) f32 max)
  uint64_t tiles = ca.cgroups >= 256 ? 1 : ceil_div(256, ca.cgroups);
  const uint64_t max_tiles = ceil_div(R, 64);
  if (tiles > max_tiles) tiles = max_tiles;
  if (tiles < 1) tiles = 1;
  if (uint64_t(ca.cgroups) * tiles > 4 * BS) return kFusedNotCovered;  // the combiner folds up to 1024 keys
  ca.chunk = ceil_div(R, tiles);
  ca.tiles = uint32_t(tiles);
  const uint32_t nblk = uint32_t(uint64_t(ca.cgroups) * tiles);
  const bool vec_ok = al16(a) && (C % V == 0) && (C * sizeof(T)) % 16 == 0;
  const uint64_t W = sizeof(typename OpF::A) / 4;
  if (uint64_t(nblk) * W * 8 > w.payload_bytes) return kFusedNoRoom;
  FusedArgs fa{};
  fa.slots = w.payload;
  fa.fault = w.fault;
  fa.spin_limit = wait_spin_limit();
  const dim3 g(nblk + 1);
  switch (ceil_div(nblk, uint64_t(BS))) {
    case 1: k_reduce_col2d<Op, OpF, T, V, 8, BS, 1><<<g, BS, 0, st>>>(a, ca, nblk, vec_ok, out, fa); break;
    case 2: k_reduce_col2d<Op, OpF, T, V, 8, BS, 2><<<g, BS, 0, st>>>(a, ca, nblk, vec_ok, out, fa); break;
    default: k_reduce_col2d<Op, OpF, T, V, 8, BS, 4><<<g, BS, 0, st>>>(a, ca, nblk, vec_ok, out, fa); break;
  }
  return kFusedLaunched;
}
}  // namespace mpy


// =============================================================================================
// extern "C" surface (rust/musapy-ops/src/kernels.rs:139-183, 222-305)
using namespace mpy;

namespace mpy {
template <class T> using OpMax = OpExt<T, true, false>;
template <class T> using OpMin = OpExt<T, false, false>;
template <class T> using OpArgmax = OpExt<T, true, true>;
template <class T> using OpArgmin = OpExt<T, false, true>;
template <class T> using OpArgmax64 = OpExt<T, true, true, int64_t>;  // over (value, absolute index) partials
template <class T> using OpArgmin64 = OpExt<T, false, true, int64_t>;

// --------------------------------------------------------------------------------------------
// Device-resident state of the library: `scratch`, the workspace of the no-alloc single-launch
// reduction (musapy_reduce_fused_noalloc_v1).  Its payload is 1 MiB; the 256 bytes after it hold
// the scratch's fault word (the workspace rule of kcommon.hpp: the last 8-byte word), on a cache
// line of its own.  Each GPU the library runs on holds its own copy until the process ends,
// zero-filled by the code object loader (static storage).  In host code the name is a host-side
// stand-in, not a device address: kernels and copies are only ever given the address that
// hipGetSymbolAddress returns for the current device (DeviceState).
constexpr size_t kScratchPayloadBytes = size_t(1) << 20;  // out_size * tiles * W <= 131072 words
constexpr size_t kScratchBytes = kScratchPayloadBytes + 256;
static __device__ __align__(256) uint64_t scratch[kScratchBytes / 8];

constexpr int kMaxDevices = 64;
struct DeviceState {
  uint64_t* scratch;               // device address of `scratch` on this device
  std::atomic<bool> dirty{false};  // a fault was taken: zero the scratch before its next use
};
std::mutex g_state_mu;
std::atomic<bool> g_state_ready[kMaxDevices];
DeviceState g_state[kMaxDevices];
std::atomic<uint32_t> g_spin_limit{1u << 24};

__global__ void k_zero_words(uint64_t* w, uint64_t n) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
    w[i] = 0;
}
// zeroes `bytes` (a multiple of 8) at `p` with a kernel on `st`
hipError_t zero_on(void* p, size_t bytes, hipStream_t st) {
  const uint64_t n = bytes / 8;
  if (n == 0) return hipSuccess;
  const unsigned g = unsigned(n < 65536 * 256 ? (n + 255) / 256 : 65536);
  k_zero_words<<<dim3(g), 256, 0, st>>>(static_cast<uint64_t*>(p), n);
  return hipGetLastError();
}

// The current device's state, its scratch address resolved once per device with that device
// current; nullptr when a HIP call fails.
DeviceState* device_state() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (g_state_ready[dev].load(std::memory_order_acquire)) return &g_state[dev];
  std::lock_guard<std::mutex> lk(g_state_mu);
  if (!g_state_ready[dev].load(std::memory_order_relaxed)) {
    void* s = nullptr;
    if (hipGetSymbolAddress(&s, HIP_SYMBOL(scratch)) != hipSuccess || s == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_state[dev].scratch = static_cast<uint64_t*>(s);
    g_state_ready[dev].store(true, std::memory_order_release);
  }
  return &g_state[dev];
}

uint32_t wait_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

// Reads the fault word of the workspace [ws, ws + bytes) after the caller's work on `st`; when it
// is set, zeroes the whole workspace on `st` (a publisher that finished after its combiner gave
// up may have left a tag in it) and waits for that.  Returns the fault bits, or -1.
int take_fault_ws(void* ws, size_t bytes, hipStream_t st) {
  WsSplit w;
  if (!ws_split(ws, bytes, w)) return -1;
  uint32_t v = 0;
  if (hipMemcpyAsync(&v, w.fault, sizeof(v), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  if (v == 0) return 0;
  if (zero_on(ws, w.payload_bytes + 8, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  return int(v);
}

// one single-launch reduction: kFusedLaunched, kFusedNotCovered or kFusedNoRoom
inline int fused_dispatch(int op, int dtype, const void* a, void* c, int ndim, const size_t* in_shape,
                          const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles,
                          void* workspace, size_t workspace_bytes, hipStream_t st) {
#define FUSED_PASS ndim, in_shape, in_strides, axis, axis_len, out_size, tiles, workspace, workspace_bytes, st
#define FUSED_CASE(T)                                                                                              \
  {                                                                                                                \
    const T* x = static_cast<const T*>(a);                                                                         \
    T* cv = static_cast<T*>(c);                                                                                    \
    int64_t* ci = static_cast<int64_t*>(c);                                                                        \
    switch (op) {                                                                                                  \
      case MUSAPY_RED_SUM: return launch_reduce_fused<OpSum<T>, OpSum<T>, T>(x, vout<T>(cv), FUSED_PASS);          \
      case MUSAPY_RED_PROD: return launch_reduce_fused<OpProd<T>, OpProd<T>, T>(x, vout<T>(cv), FUSED_PASS);       \
      case MUSAPY_RED_MAX:                                                                                         \
        return launch_reduce_fused<OpMax<T>, OpExt<T, true, false, int64_t>, T>(x, vout<T>(cv), FUSED_PASS);       \
      case MUSAPY_RED_MIN:                                                                                         \
        return launch_reduce_fused<OpMin<T>, OpExt<T, false, false, int64_t>, T>(x, vout<T>(cv), FUSED_PASS);      \
      case MUSAPY_RED_MEAN:                                                                                        \
        if (sizeof(T) == 8 && T(0.5) == T(0)) return kFusedNotCovered; /* integer means go through f64 */          \
        return launch_reduce_fused<OpSum<T>, OpSum<T>, T>(x, mout<T>(cv, mean_count<T>(axis_len)), FUSED_PASS);    \
      case MUSAPY_RED_ARGMAX: return launch_reduce_fused<OpArgmax<T>, OpArgmax64<T>, T>(x, iout<T>(ci), FUSED_PASS); \
      case MUSAPY_RED_ARGMIN: return launch_reduce_fused<OpArgmin<T>, OpArgmin64<T>, T>(x, iout<T>(ci), FUSED_PASS); \
    }                                                                                                              \
    return kFusedNotCovered;                                                                                       \
  }
  // complex: sum, prod and mean (accumulated in f64 components, narrowed once; the mean divides by
  // the f64 axis length, cpu_reduce_cplx, op_builder.rs:3485-3488)
#define FUSED_CPLX(T)                                                                                              \
  {                                                                                                                \
    const T* x = static_cast<const T*>(a);                                                                         \
    T* cv = static_cast<T*>(c);                                                                                    \
    switch (op) {                                                                                                  \
      case MUSAPY_RED_SUM: return launch_reduce_fused<OpSum<T>, OpSum<T>, T>(x, vout<T>(cv), FUSED_PASS);          \
      case MUSAPY_RED_PROD: return launch_reduce_fused<OpProd<T>, OpProd<T>, T>(x, vout<T>(cv), FUSED_PASS);       \
      case MUSAPY_RED_MEAN:                                                                                        \
        return launch_reduce_fused<OpSum<T>, OpSum<T>, T>(x, mout<T>(cv, double(axis_len)), FUSED_PASS);           \
    }                                                                                                              \
    return kFusedNotCovered;                                                                                       \
  }
  switch (dtype) {
    case MUSAPY_DT_F32: FUSED_CASE(float)
    case MUSAPY_DT_F64: FUSED_CASE(double)
    case MUSAPY_DT_I64: FUSED_CASE(int64_t)
    case MUSAPY_DT_C64: FUSED_CPLX(musapy_c64_t)
    case MUSAPY_DT_C128: FUSED_CPLX(musapy_c128_t)
  }
#undef FUSED_CASE
#undef FUSED_CPLX
#undef FUSED_PASS
  return kFusedNotCovered;
}
}  // namespace mpy

#define RED_ARGS int ndim, const size_t *in_shape, const ssize_t *in_strides, int axis, size_t axis_len, size_t out_size
#define RED_PASS ndim, in_shape, in_strides, axis, axis_len, out_size

extern "C" {

size_t musapy_reduce_tiles_hint(int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis,
                                size_t axis_len, size_t out_size, size_t elem_size) {
  if (out_size == 0 || axis_len == 0) return 1;
  if (ndim < 0 || ndim > kMaxDims || (ndim > 0 && (axis < 0 || axis >= ndim))) return 1;  // the launch reports it
  ReducePlan p;
  plan_reduce(p, ndim, in_shape, in_strides, axis, axis_len, out_size);
  return tiles_hint(p, elem_size);
}

// value reductions whose final step is the plain accumulator (sum/prod/max/min, real + complex)
#define MPY_RED_FAMILY(NAME, OP, SN, T)                                                                     \
  void musapy_##NAME##_##SN##_v2(const T* a, T* c, RED_ARGS, hipStream_t st) {                              \
    launch_reduce<OP<T>, T, kWriteFinal>(a, vout<T>(c), RED_PASS, 1, st);                                   \
  }                                                                                                         \
  void musapy_##NAME##_small_axis_##SN##_v2(const T* a, T* c, RED_ARGS, int group_size, hipStream_t st) {   \
    (void)group_size;                                                                                       \
    launch_reduce<OP<T>, T, kWriteFinal>(a, vout<T>(c), RED_PASS, 1, st);                                   \
  }                                                                                                         \
  void musapy_##NAME##_partial_##SN##_v2(const T* a, T* partials, RED_ARGS, size_t tiles_per_output,        \
                                         hipStream_t st) {                                                  \
    launch_reduce<OP<T>, T, kWriteVal>(a, vout<T>(partials), RED_PASS, tiles_per_output, st);               \
  }

#define MPY_RED_FINAL_REAL(NAME, OP, SN, T)                                                                 \
  void musapy_##NAME##_final_##SN##_v2(const T* partials, T* c, size_t num_partials, size_t out_size,       \
                                       hipStream_t st) {                                                    \
    launch_final<OP<T>, T>(partials, vout<T>(c), num_partials, out_size, st);                               \
  }
#define MPY_RED_FINAL_CPLX(NAME, OP, SN, T)                                                                 \
  void musapy_##NAME##_final_##SN##_v2(const T* partials, T* c, size_t num_partials, size_t out_size,       \
                                       size_t axis_len, hipStream_t st) {                                   \
    (void)axis_len;                                                                                         \
    launch_final<OP<T>, T>(partials, vout<T>(c), num_partials, out_size, st);                               \
  }

#define MPY_RED_REAL(SN, T)                  \
  MPY_RED_FAMILY(sum, OpSum, SN, T)          \
  MPY_RED_FAMILY(prod, OpProd, SN, T)        \
  MPY_RED_FAMILY(max, OpMax, SN, T)          \
  MPY_RED_FAMILY(min, OpMin, SN, T)          \
  MPY_RED_FINAL_REAL(sum, OpSum, SN, T)      \
  MPY_RED_FINAL_REAL(prod, OpProd, SN, T)    \
  MPY_RED_FINAL_REAL(max, OpMax, SN, T)      \
  MPY_RED_FINAL_REAL(min, OpMin, SN, T)
MPY_RED_REAL(i64, int64_t)
MPY_RED_REAL(f32, float)
MPY_RED_REAL(f64, double)

#define MPY_RED_CPLX(SN, T)                  \
  MPY_RED_FAMILY(sum, OpSum, SN, T)          \
  MPY_RED_FAMILY(prod, OpProd, SN, T)        \
  MPY_RED_FINAL_CPLX(sum, OpSum, SN, T)      \
  MPY_RED_FINAL_CPLX(prod, OpProd, SN, T)
MPY_RED_CPLX(c64, musapy_c64_t)
MPY_RED_CPLX(c128, musapy_c128_t)

// mean: sum partials, divide in the final step.  Real means divide by the reference's "+1"
// count in T (cpu_mean_typed, op_builder.rs:3608-3612); complex means by the f64 axis length
// (cpu_reduce_cplx, op_builder.rs:3485-3488).
#define MPY_RED_MEAN(SN, T, COUNT)                                                                          \
  void musapy_mean_##SN##_v2(const T* a, T* c, RED_ARGS, hipStream_t st) {                                  \
    launch_reduce<OpSum<T>, T, kWriteFinal>(a, mout<T>(c, COUNT(axis_len)), RED_PASS, 1, st);               \
  }                                                                                                         \
  void musapy_mean_small_axis_##SN##_v2(const T* a, T* c, RED_ARGS, int group_size, hipStream_t st) {       \
    (void)group_size;                                                                                       \
    launch_reduce<OpSum<T>, T, kWriteFinal>(a, mout<T>(c, COUNT(axis_len)), RED_PASS, 1, st);               \
  }                                                                                                         \
  void musapy_mean_partial_##SN##_v2(const T* a, T* partials, RED_ARGS, size_t tiles_per_output,            \
                                     hipStream_t st) {                                                      \
    launch_reduce<OpSum<T>, T, kWriteVal>(a, vout<T>(partials), RED_PASS, tiles_per_output, st);            \
  }                                                                                                         \
  void musapy_mean_final_##SN##_v2(const T* partials, T* c, size_t num_partials, size_t out_size,           \
                                   size_t axis_len, hipStream_t st) {                                       \
    launch_final<OpSum<T>, T>(partials, mout<T>(c, COUNT(axis_len)), num_partials, out_size, st);           \
  }
#define MPY_COUNT_F32(n) mean_count<float>(n)
#define MPY_COUNT_F64(n) mean_count<double>(n)
#define MPY_COUNT_LEN(n) double(n)
MPY_RED_MEAN(f32, float, MPY_COUNT_F32)
MPY_RED_MEAN(f64, double, MPY_COUNT_F64)
MPY_RED_MEAN(c64, musapy_c64_t, MPY_COUNT_LEN)
MPY_RED_MEAN(c128, musapy_c128_t, MPY_COUNT_LEN)

// argmax / argmin
#define MPY_RED_ARG(NAME, OP, SN, T)                                                                        \
  void musapy_##NAME##_##SN##_v2(const T* a, int64_t* c, RED_ARGS, hipStream_t st) {                        \
    launch_reduce<OP<T>, T, kWriteFinal>(a, iout<T>(c), RED_PASS, 1, st);                                   \
  }                                                                                                         \
  void musapy_##NAME##_partial_##SN##_v2(const T* a, T* partials_val, int64_t* partials_idx, RED_ARGS,      \
                                         size_t tiles_per_output, hipStream_t st) {                         \
    RedOut<T> o{partials_val, partials_idx, 0.0, kFinPlain};                                                \
    launch_reduce<OP<T>, T, kWritePair>(a, o, RED_PASS, tiles_per_output, st);                              \
  }                                                                                                         \
  void musapy_##NAME##_final_##SN##_v2(const T* partials_val, const int64_t* partials_idx, int64_t* c,      \
                                       size_t num_partials, size_t out_size, hipStream_t st) {              \
    launch_pairs<OP##64<T>, T, kWriteFinal>(partials_val, partials_idx, iout<T>(c), num_partials, out_size, \
                                            1, st);                                                         \
  }                                                                                                         \
  void musapy_##NAME##_mid_##SN##_v2(const T* partials_val, const int64_t* partials_idx, T* out_val,        \
                                     int64_t* out_idx, size_t out_size, size_t tiles_per_output,            \
                                     size_t axis_len, hipStream_t st) {                                     \
    RedOut<T> o{out_val, out_idx, 0.0, kFinPlain};                                                          \
    launch_pairs<OP##64<T>, T, kWritePair>(partials_val, partials_idx, o, axis_len, out_size,               \
                                           tiles_per_output, st);                                           \
  }
MPY_RED_ARG(argmax, OpArgmax, i64, int64_t)
MPY_RED_ARG(argmax, OpArgmax, f32, float)
MPY_RED_ARG(argmax, OpArgmax, f64, double)
MPY_RED_ARG(argmin, OpArgmin, i64, int64_t)
MPY_RED_ARG(argmin, OpArgmin, f32, float)
MPY_RED_ARG(argmin, OpArgmin, f64, double)

// partial + final in one launch (new; see musapy_kernels.h)
int musapy_reduce_fused_v1(int op, int dtype, const void* a, void* c, int ndim, const size_t* in_shape,
                           const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles,
                           void* workspace, size_t workspace_bytes, hipStream_t st) {
  const int r = fused_dispatch(op, dtype, a, c, RED_PASS, tiles, workspace, workspace_bytes, st);
  return r == kFusedLaunched ? 0 : -1;
}

// max / min over both axes of a C-contiguous (rows, cols) array in one launch, with the result of
// the reference's two per-axis passes (new; see musapy_kernels.h)
int musapy_reduce_2d_ordered_v1(int op, int dtype, const void* a, void* c, size_t rows, size_t cols,
                                void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (op != MUSAPY_RED_MAX && op != MUSAPY_RED_MIN) return -1;
  const bool mx = op == MUSAPY_RED_MAX;
  int r = kFusedNotCovered;
#define RED2D(T)                                                                                                \
  {                                                                                                             \
    const T* x = static_cast<const T*>(a);                                                                      \
    RedOut<T> o = vout<T>(static_cast<T*>(c));                                                                  \
    r = mx ? launch_reduce_2d_ordered<OpExt<T, true, false>, OpExt<T, true, false, int64_t>, T>(                \
                 x, o, rows, cols, workspace, workspace_bytes, st)                                              \
           : launch_reduce_2d_ordered<OpExt<T, false, false>, OpExt<T, false, false, int64_t>, T>(              \
                 x, o, rows, cols, workspace, workspace_bytes, st);                                             \
  }
  switch (dtype) {
    case MUSAPY_DT_F32: RED2D(float) break;
    case MUSAPY_DT_F64: RED2D(double) break;
    case MUSAPY_DT_I64: RED2D(int64_t) break;
  }
#undef RED2D
  return r == kFusedLaunched ? 0 : -1;
}

// The same single launch with the library's static scratch as its workspace (new; no counterpart
// in kernels.rs): for callers that cannot allocate.  Calls that overlap on one device race.  After
// a fault was taken (musapy_kernels_take_fault) the scratch is zeroed first, on this call's stream.
int musapy_reduce_fused_noalloc_v1(int op, int dtype, const void* a, void* c, int ndim, const size_t* in_shape,
                                   const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size,
                                   size_t tiles, hipStream_t st) {
  DeviceState* ds = device_state();
  if (ds == nullptr) return -1;
  if (ds->dirty.load(std::memory_order_acquire)) {
    if (zero_on(ds->scratch, kScratchBytes, st) != hipSuccess) return -1;
    ds->dirty.store(false, std::memory_order_release);
  }
  const int r = fused_dispatch(op, dtype, a, c, RED_PASS, tiles, ds->scratch, kScratchBytes, st);
  if (r == kFusedNoRoom) {
    g_wrapper_error = 5;
    return -2;
  }
  return r == kFusedLaunched ? 0 : -1;
}

// Returns the fault word of the caller's workspace (kFaultReduceWait | kFaultScanWait), read after
// the caller's work on `st`; a fault zeroes the workspace on `st` before returning.
int musapy_kernels_take_fault_ws(void* workspace, size_t workspace_bytes, hipStream_t st) {
  return take_fault_ws(workspace, workspace_bytes, st);
}

// Returns and clears the fault word of the device's no-alloc scratch, read after the caller has
// synchronized the streams whose no-alloc calls it covers.  The scratch itself is zeroed by the
// next no-alloc call on that device, on that call's stream (a clear issued here would not be
// ordered with another stream's work).
int musapy_kernels_take_fault(int device) {
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return -1;
  if (device != prev && hipSetDevice(device) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  int result = 0;
  DeviceState* ds = device_state();
  if (ds == nullptr) {
    result = -1;
  } else if (!ds->dirty.load(std::memory_order_acquire)) {  // dirty: taken already, no call since
    WsSplit w;
    ws_split(ds->scratch, kScratchBytes, w);
    uint32_t v = 0;
    if (hipMemcpy(&v, w.fault, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) {
      result = -1;
    } else if (v != 0) {
      ds->dirty.store(true, std::memory_order_release);
      result = int(v);
    }
  }
  if (result < 0) (void)hipGetLastError();
  if (device != prev) (void)hipSetDevice(prev);
  return result;
}

// Sets how many polls a bounded device wait makes before it gives up and reports a fault; returns
// the previous limit.  0 makes every wait give up at once (used by tests to force the error path
// while every kernel still exits normally).
uint32_t musapy_kernels_set_spin_limit(uint32_t polls) { return g_spin_limit.exchange(polls); }

}  // extern "C"
