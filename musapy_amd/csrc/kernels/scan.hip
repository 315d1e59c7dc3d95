// scan.hip -- cumsum (inclusive prefix sum along one axis), for gfx950.
//
// Drop-in for the reference's musapy_cumsum_{i64,f32,f64}_v3 (kernels/reduction.mu:557-820,
// 1723-1776), which runs a 3-5 launch Blelloch hierarchy and writes the output twice.  Every
// path here reads the input once and writes the output once, in one launch (plus a small
// clear of the look-back state):
//   look-back  the scanned axis is unit-stride and the rows are few, or each row is one tile: a
//              single pass with a decoupled look-back (Merrill & Garland, "Single-pass Parallel
//              Prefix Scan with Decoupled Look-back", 2016) over tiles taken in memory order.
//   chain      unit-stride rows that are many (>= 512) and longer than one tile: 64 KB tiles
//              (16 KB for rows shorter than two of them) in tile-major order over the rows, each
//              waiting only for its row predecessor's prefix.  On (1024, 65536) f64: 180 us, against
//              188 us with 16 KB tiles and 237 us for one block per row walking it tile by tile (the
//              previous design, whose one-block-per-row access pattern topped out at the rate of a
//              plain copy in that pattern).
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


__device__ inline uint64_t bits_of(double v) { return uint64_t(__double_as_longlong(v)); }
__device__ inline uint64_t bits_of(float v) { return uint64_t(__float_as_uint(v)); }
__device__ inline uint64_t bits_of(uint64_t v) { return v; }
template <class A> __device__ inline A from_bits(uint64_t b);
template <> __device__ inline double from_bits<double>(uint64_t b) { return __longlong_as_double((long long)b); }
template <> __device__ inline float from_bits<float>(uint64_t b) { return __uint_as_float(uint32_t(b)); }
template <> __device__ inline uint64_t from_bits<uint64_t>(uint64_t b) { return b; }

// Published look-back values (publish.hpp): each status word is written once per launch after
// k_scan_clear zeroed it, so a reader that sees the tag on every word holds the final value.
// `also`, when given, is one more word to zero: the private fault word of a reference-signature
// call, which sits at the end of its scratch, past the words the scan uses.
__global__ void k_scan_clear(uint64_t* w, uint64_t n, uint32_t* also) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
    w[i] = 0;
  if (also != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *also = 0;
}

// Wave-64 inclusive scan with DPP lane moves (gfx9 DPP: row_shr within rows of 16 lanes, then
// row_bcast:15 / row_bcast:31 across rows).  Against a Hillis-Steele scan over LDS shuffles it
// makes no LDS round trips, so the scans of several sub-tiles need not be interleaved to hide
// latency: the look-back kernel went from 111 to 55 VGPRs (f64), from 4 to 8 waves per SIMD.
// Lanes without a source keep 0; adding +0 changes no value the scan can produce here (every
// output is formed as +0 + ..., so a -0 input reads back as +0 either way, as in the reference's
// acc = 0; acc += x).  A fixed association.
template <int CTRL, int ROW_MASK>
__device__ inline uint32_t dpp_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ inline float dpp_move(float v) { return __uint_as_float(dpp_u32<CTRL, ROW_MASK>(__float_as_uint(v))); }
template <int CTRL, int ROW_MASK = 0xf>
__device__ inline uint64_t dpp_move(uint64_t v) {
  return uint64_t(dpp_u32<CTRL, ROW_MASK>(uint32_t(v))) | (uint64_t(dpp_u32<CTRL, ROW_MASK>(uint32_t(v >> 32))) << 32);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ inline double dpp_move(double v) {
  return __longlong_as_double((long long)dpp_move<CTRL, ROW_MASK>(uint64_t(__double_as_longlong(v))));
}
template <class A>
__device__ inline A wave_incl_scan_dpp(A v) {
  v = v + dpp_move<0x111>(v);       // row_shr:1
  v = v + dpp_move<0x112>(v);       // row_shr:2
  v = v + dpp_move<0x114>(v);       // row_shr:4
  v = v + dpp_move<0x118>(v);       // row_shr:8
  v = v + dpp_move<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = v + dpp_move<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
template <class A>
__device__ inline A wave_shr1(A v) { return dpp_move<0x138>(v); }  // wave_shr:1, lane 0 gets 0
// the value of lane `l` (uniform), through scalar registers
__device__ inline uint32_t read_lane(uint32_t v, int l) { return uint32_t(__builtin_amdgcn_readlane(int(v), l)); }
__device__ inline float read_lane(float v, int l) { return __uint_as_float(read_lane(__float_as_uint(v), l)); }
__device__ inline uint64_t read_lane(uint64_t v, int l) {
  return uint64_t(read_lane(uint32_t(v), l)) | (uint64_t(read_lane(uint32_t(v >> 32), l)) << 32);
}
__device__ inline double read_lane(double v, int l) {
  return __longlong_as_double((long long)read_lane(uint64_t(__double_as_longlong(v)), l));
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
constexpr uint64_t kChainMinRows = 512;  // rows from which the chained scan is used
// Chained-scan tiles: 1024 lanes x 4 vectors (64 KB, two blocks per CU) for rows of at least two
// such tiles, else 512 lanes x 2 vectors (16 KB).  The rate falls with the number of rows one XCD
// streams at once, which in the chain's order is the number of blocks resident on it: at equal
// bytes in flight per CU, 64 rows of 64 KB tiles beat 128 rows of 32 KB tiles (512 x 4: 196 us
// against 180 us for (1024, 65536) f64), and 16 KB tiles took 188 us.  One 128 KB tile per CU
// (1024 x 8) took 205 us: the CU idles at the block's barriers.  Rows of one 64 KB tile or less
// keep the 16 KB tiles, which give them a chain ((2048, 8192) f64: 48 us against 67 us without).
constexpr int kChainBigBlock = 1024;
constexpr int kChainBigVpt = 4;
constexpr int kChainBlock = 512;
constexpr int kChainVpt = 2;
template <class T, int BS, int VPT>
constexpr uint64_t chain_te() { return uint64_t(BS) * VPT * (16 / sizeof(T)); }

struct LbArgs {
  RowIndexer<2> ix;     // non-axis dims: [0] input strides, [1] output strides
  uint64_t L;
  FastDiv tdiv;         // divides a tile id by the tiles per row
  uint32_t tiles;       // tiles per row
  uint32_t* counter;    // tile claim counter; nullptr when tiles == 1 (no look-back)
  uint64_t* status;     // per tile: W words of A(c), then W words of P(c)
  uint32_t* fault;      // the fault word of the launch's workspace or scratch (kcommon.hpp)
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
    incl[u] = wave_incl_scan_dpp(x[u][VE - 1]);
    if (lane == kWave - 1) s_wave[u][wv] = incl[u];
    incl[u] = wave_shr1(incl[u]);  // from here on: the lane's exclusive offset in its wave
  }
  __syncthreads();
  // exclusive offset of each lane's run inside the tile, and the tile aggregate (fixed order):
  // lanes 0 .. kWaves-1 read the sub-tile's wave totals and scan them, and every lane takes its
  // wave's exclusive offset and the sub-tile total from that scan (one LDS read per lane)
  A lane_off[kVpt];
  A run = A(0);
#pragma unroll
  for (int u = 0; u < kVpt; ++u) {
    const A ws = wave_incl_scan_dpp(lane < kWaves ? s_wave[u][lane] : A(0));
    const A st = read_lane(ws, kWaves - 1);
    const A wo = wv > 0 ? read_lane(ws, wv - 1) : A(0);
    lane_off[u] = run + (wo + incl[u]);
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
  lds_barrier();  // the prefix is in LDS; the publish stores stay in flight
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
// Chained row scan, for many rows of several tiles: tile t of row r is block t * R8 + r (R8 =
// rows rounded up to a multiple of 8, the blocks past the last row exit at once), so the grid
// streams tile 0 of every row, then tile 1 of every row, ...  The tile layout and in-tile scan are
// k_scan_lookback's, with BS lanes x VPT vectors per tile (see kChainBigBlock); a tile's prefix is
// always P(t) = P(t - 1) + A(t), a fixed association.  Block (r, t) waits only for P(r, t - 1),
// published by block (r, t - 1): R8 blocks earlier, and on the same XCD (blocks go to the 8 XCDs
// round-robin by index, and R8 is a multiple of 8), whose workgroups are dispatched in index
// order -- so the block it waits on is resident or finished, and no atomic tile counter is
// needed.  The predecessor's prefix is read together with the tile's own loads, and a timing copy
// that skipped the wait ran as fast: the chain costs nothing measurable at C5, and so does the
// in-tile scan (a copy in the same block shape took as long).  The tile shape sets the rate; with
// default stores, (1024, 65536) f64: 512 x 2 vectors 198 us, 512 x 4 205 us, 512 x 1 206 us,
// 256 x 4 215 us, 256 x 2 249 us (the smaller tiles lengthen the per-row chain); with streaming
// stores see kChainBigBlock.  A wait is bounded
// (wait_spin_limit polls): when it runs out the tile records kFaultScanWait, takes P = 0 and
// still publishes, so every block exits.
struct ChainArgs {
  RowIndexer<2> ix;     // non-axis dims: [0] input strides, [1] output strides
  uint64_t L;
  FastDiv rdiv;         // divides a block id by R8
  uint32_t R8;          // rows rounded up to a multiple of 8
  uint32_t rows;
  uint32_t tiles;       // tiles per row
  uint64_t* prefix;     // per (row, tile): W words of P(row, tile)
  uint32_t* fault;      // the fault word of the launch's workspace or scratch (kcommon.hpp)
  uint32_t spin_limit;  // polls a wait may make
  bool vec;             // 16-byte aligned rows
  bool nt_load;
};

template <class T, int BS, int VPT, bool NTS>
__global__ __launch_bounds__(BS) void k_scan_chain(const T* __restrict__ a, T* __restrict__ c, ChainArgs sa) {
  using A = typename ScanAcc<T>::A;
  constexpr int VE = int(16 / sizeof(T));
  constexpr int kWaves = BS / kWave;
  constexpr uint64_t TE = uint64_t(BS) * VPT * VE;
  constexpr int W = sizeof(A) == 4 ? 1 : 2;
  __shared__ A s_wave[VPT][kWaves];
  __shared__ A s_prefix;
  const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
  const uint32_t chunk = fd_div(sa.rdiv, blockIdx.x);
  const uint32_t row = blockIdx.x - chunk * sa.R8;
  if (row >= sa.rows) return;
  int64_t off[2];
  row_offsets<2>(sa.ix, row, off);
  const T* ain = a + off[0];
  T* cout = c + off[1];
  const uint64_t t0 = uint64_t(chunk) * TE;
  const bool full = sa.vec && t0 + TE <= sa.L;

  A x[VPT][VE];
  if (full) {
    // The tile's loads and its output stores are issued at a raised wave priority (s_setprio), so
    // that a block starting or finishing on the CU is not held behind the other block's in-tile
    // scan: (1024, 65536) f64 180.8-182.2 -> 180.1-181.2 us event-timed over three A/B runs.
    Vec<T, VE> v[VPT];
    __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int u = 0; u < VPT; ++u) v[u] = vload_pol<T, VE>(ain + t0 + (uint64_t(u) * BS + tid) * VE, sa.nt_load);
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int u = 0; u < VPT; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) x[u][e] = A(v[u].v[e]);
  } else {
#pragma unroll
    for (int u = 0; u < VPT; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const uint64_t k = t0 + (uint64_t(u) * BS + tid) * VE + e;
        x[u][e] = k < sa.L ? A(ain[k]) : A(0);
      }
  }
  // the predecessor's prefix is read now, so that this round trip overlaps the tile's loads
  // instead of following the in-tile scan (it is usually published by then)
  uint64_t* const rowp = sa.prefix + uint64_t(row) * sa.tiles * W;
  uint64_t pw[W];
#pragma unroll
  for (int q = 0; q < W; ++q) pw[q] = 0;
  if (tid == 0 && chunk > 0) {
#pragma unroll
    for (int q = 0; q < W; ++q) pw[q] = ld_relaxed(rowp + uint64_t(chunk - 1) * W + q);
  }
  // in-lane inclusive runs, then a wave scan of the run totals per sub-tile
  A incl[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
#pragma unroll
    for (int e = 1; e < VE; ++e) x[u][e] = x[u][e - 1] + x[u][e];
    incl[u] = wave_incl_scan_dpp(x[u][VE - 1]);
    if (lane == kWave - 1) s_wave[u][wv] = incl[u];
    incl[u] = wave_shr1(incl[u]);  // from here on: the lane's exclusive offset in its wave
  }
  lds_barrier();  // thread 0's load of the predecessor's prefix stays in flight
  // exclusive offset of each lane's run inside the tile, and the tile aggregate (fixed order):
  // lanes 0 .. kWaves-1 read the sub-tile's wave totals and scan them, and every lane takes its
  // wave's exclusive offset and the sub-tile total from that scan (one LDS read per lane)
  A lane_off[VPT];
  A run = A(0);
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const A ws = wave_incl_scan_dpp(lane < kWaves ? s_wave[u][lane] : A(0));
    const A st = read_lane(ws, kWaves - 1);
    const A wo = wv > 0 ? read_lane(ws, wv - 1) : A(0);
    lane_off[u] = run + (wo + incl[u]);
    run = run + st;
  }
  const A agg = run;

  if (tid == 0) {
    A P = A(0);
    if (chunk > 0) {
      bool got = sa.spin_limit > 0;  // a limit of 0 gives up before the first poll
      uint64_t bits = 0;
#pragma unroll
      for (int q = 0; q < W; ++q) {
        got = got && (pw[q] & kTag);
        bits |= (pw[q] & 0xffffffffu) << (32 * q);
      }
      for (uint32_t spins = 1; !got && spins < sa.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(1);
        got = read_value<W>(rowp + uint64_t(chunk - 1) * W, bits);
      }
      if (got) {
        P = from_bits<A>(bits);
        // nothing else reads the predecessor's prefix: return its words to zero, so that the
        // launch leaves the prefix area as it found it (the last tile of a row publishes nothing)
#pragma unroll
        for (int q = 0; q < W; ++q) st_relaxed(rowp + uint64_t(chunk - 1) * W + q, 0);
      } else {
        atomicOr(sa.fault, kFaultScanWait);  // the prefix stays 0
      }
    }
    if (chunk + 1 < sa.tiles) publish_value<W>(rowp + uint64_t(chunk) * W, bits_of(A(P + agg)));
    s_prefix = P;
  }
  // LDS only: with __syncthreads() every lane's output stores waited for thread 0's publish and
  // clear stores to complete, a store round trip per tile
  lds_barrier();
  const A P = s_prefix;

  if (full) {
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      Vec<T, VE> v;
#pragma unroll
      for (int e = 0; e < VE; ++e) v.v[e] = T(P + (lane_off[u] + x[u][e]));
      vstore_as<NTS, T, VE>(cout + t0 + (uint64_t(u) * BS + tid) * VE, v);
    }
  } else {
#pragma unroll
    for (int u = 0; u < VPT; ++u)
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const uint64_t k = t0 + (uint64_t(u) * BS + tid) * VE + e;
        if (k < sa.L) cout[k] = T(P + (lane_off[u] + x[u][e]));
      }
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

// What a cumsum call resolves to, shared by the reference-signature entry points (scratch
// `tmp` of the reference's size, arbitrary contents) and musapy_cumsum_ws_v1 (a zeroed workspace).
struct ScanShape {
  ScanPlan p;
  RowIndexer<2> ix;  // non-axis dims, innermost first (row scans)
  bool vec = false;  // 16-byte aligned rows
};

// Plans the call; false (with the wrapper error set when it is one) when nothing is to be done.
template <class T>
bool plan_cumsum(ScanShape& sh, const T* a, const T* c, int ndim, const size_t* shape, const ssize_t* strides,
                 int axis, size_t axis_len, size_t out_size) {
  if (out_size == 0 || axis_len == 0) return false;
  if (!args_ok(ndim, axis)) return false;
  ScanPlan& p = sh.p;
  plan_scan(p, ndim, shape, strides, axis);
  // rows and the non-axis extents are decoded in 32 bits (row_offsets, the lane index of
  // k_scan_seq): refuse shapes past that instead of aliasing rows
  bool fits = p.rows < (uint64_t(1) << 32);
  for (int d = 0; d < p.ond; ++d) fits = fits && p.oshape[d] < (uint64_t(1) << 32);
  if (!fits) {
    g_wrapper_error = 4;
    return false;
  }
  if (p.kind == kRowScan) {
    sh.ix = RowIndexer<2>{};
    sh.ix.nd = p.ond;
    for (int i = 0; i < p.ond; ++i) {
      int d = p.ond - 1 - i;
      sh.ix.div[i] = make_fastdiv(uint32_t(p.oshape[d]));
      sh.ix.stride[0][i] = p.istride[d];
      sh.ix.stride[1][i] = p.ostride[d];
    }
    if (p.ond == 1 && p.oshape[0] == 1) sh.ix.nd = 0;
    sh.vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c)) & 15u) == 0;
    for (int d = 0; d < p.ond; ++d)
      if (((p.istride[d] * int64_t(sizeof(T))) % 16) || ((p.ostride[d] * int64_t(sizeof(T))) % 16)) sh.vec = false;
  }
  return true;
}

// whether the chained scan takes the 64 KB tiles: rows of at least two of them
template <class T>
bool chain_big(const ScanShape& sh) {
  return sh.p.L >= 2 * chain_te<T, kChainBigBlock, kChainBigVpt>();
}

// tiles of the chained scan per row, 0 when the call does not take it
template <class T>
uint64_t chain_tiles(const ScanShape& sh) {
  if (sh.p.kind != kRowScan || sh.p.L <= 16 || sh.p.rows < kChainMinRows) return 0;
  const uint64_t CTE =
      chain_big<T>(sh) ? chain_te<T, kChainBigBlock, kChainBigVpt>() : chain_te<T, kChainBlock, kChainVpt>();
  const uint64_t tiles = (sh.p.L + CTE - 1) / CTE;
  return tiles > 1 ? tiles : 0;
}

// The chained scan over `prefix` (rows * tiles * W words); an expired wait is reported in
// `fault`.  With `clear` the words (and `fault` too with `clear_fault`) are zeroed first; without,
// they must be zero already (the launch leaves them zero).
template <class T>
void launch_chain(const T* a, T* c, const ScanShape& sh, uint64_t tiles, uint64_t* prefix, bool clear,
                  uint32_t* fault, bool clear_fault, hipStream_t st) {
  const ScanPlan& p = sh.p;
  const uint64_t R8 = (uint64_t(p.rows) + 7) / 8 * 8;
  if (R8 * tiles >= (uint64_t(1) << 31)) {  // block ids
    g_wrapper_error = 4;
    return;
  }
  const uint64_t W = sizeof(typename ScanAcc<T>::A) == 4 ? 1 : 2;
  const uint64_t words = uint64_t(p.rows) * tiles * W;
  ChainArgs ca{};
  ca.ix = sh.ix;
  ca.L = p.L;
  ca.R8 = uint32_t(R8);
  ca.rdiv = make_fastdiv(ca.R8);
  ca.rows = uint32_t(p.rows);
  ca.tiles = uint32_t(tiles);
  ca.prefix = prefix;
  ca.fault = fault;
  ca.spin_limit = wait_spin_limit();
  ca.vec = sh.vec;
  const uint64_t bytes = uint64_t(p.rows) * p.L * sizeof(T);
  ca.nt_load = bytes >= kStreamLoadBytes;
  if (clear) {
    unsigned cg = unsigned(words < 65536 * 256 ? (words + 255) / 256 : 65536);
    k_scan_clear<<<cg, 256, 0, st>>>(ca.prefix, words, clear_fault ? fault : nullptr);
  }
  const bool big = chain_big<T>(sh);
  with_store_policy(bytes >= kStreamStoreBytes, [&](auto NT) {
    if (big)
      k_scan_chain<T, kChainBigBlock, kChainBigVpt, NT.value>
          <<<dim3(unsigned(R8 * tiles)), kChainBigBlock, 0, st>>>(a, c, ca);
    else
      k_scan_chain<T, kChainBlock, kChainVpt, NT.value><<<dim3(unsigned(R8 * tiles)), kChainBlock, 0, st>>>(a, c, ca);
  });
}

// Where a cumsum launch keeps its state: the chained scan's prefixes (`chain`, zero on entry
// unless `chain_clear`), the look-back's claim counter and status words (`lb`, cleared by the
// launch), and the fault word its waits report to.  `clear_fault`: the word is private to this
// call (a reference-signature scratch) and is zeroed with the launch's state; a workspace's word
// is never zeroed here, since it keeps faults until their owner takes them.
struct ScanScratch {
  uint64_t* chain = nullptr;
  size_t chain_bytes = 0;
  bool chain_clear = true;
  uint64_t* lb = nullptr;
  size_t lb_bytes = 0;
  uint32_t* fault = nullptr;
  bool clear_fault = false;
};

// One cumsum: the chained scan for many rows of several tiles, the look-back for the other row
// scans of several tiles, the sequential scan otherwise.  Returns false (wrapper error 1, nothing
// launched) when the path taken needs state that `sc` does not hold.
template <class T>
bool run_cumsum(const T* a, T* c, const ScanShape& sh, const ScanScratch& sc, hipStream_t st) {
  const ScanPlan& p = sh.p;
  const uint64_t W = sizeof(typename ScanAcc<T>::A) == 4 ? 1 : 2;
  if (p.kind == kRowScan && p.L > 16) {
    // many rows of several tiles: the chained scan, tile-major over the rows
    if (const uint64_t ct = chain_tiles<T>(sh)) {
      if (sc.chain == nullptr || sc.fault == nullptr || uint64_t(p.rows) * ct * W * 8 > sc.chain_bytes) {
        g_wrapper_error = 1;
        return false;
      }
      launch_chain<T>(a, c, sh, ct, sc.chain, sc.chain_clear, sc.fault, sc.clear_fault, st);
      return true;
    }
    constexpr uint64_t TE = uint64_t(kLbBlock) * kVpt * (16 / sizeof(T));
    const uint64_t tiles = (p.L + TE - 1) / TE;
    if (uint64_t(p.rows) * tiles >= (uint64_t(1) << 32)) {  // tile ids are 32-bit
      g_wrapper_error = 4;
      return false;
    }
    LbArgs sa{};
    sa.ix = sh.ix;
    sa.L = p.L;
    sa.vec = sh.vec;
    sa.tiles = uint32_t(tiles);
    sa.tdiv = make_fastdiv(sa.tiles);
    if (tiles > 1) {
      // word 0: the tile claim counter; then 2 * W status words per tile (aggregate, prefix)
      const uint64_t words = 1 + uint64_t(p.rows) * tiles * 2 * W;
      if (sc.lb == nullptr || sc.fault == nullptr || words * 8 > sc.lb_bytes) {
        g_wrapper_error = 1;
        return false;
      }
      uint64_t* w = sc.lb;
      sa.counter = reinterpret_cast<uint32_t*>(w);
      sa.status = w + 1;
      sa.fault = sc.fault;
      sa.spin_limit = wait_spin_limit();
      unsigned cg = unsigned(words < 65536 * 256 ? (words + 255) / 256 : 65536);
      k_scan_clear<<<cg, 256, 0, st>>>(w, words, sc.clear_fault ? sc.fault : nullptr);
    }
    k_scan_lookback<T><<<dim3(unsigned(uint64_t(p.rows) * tiles)), kLbBlock, 0, st>>>(a, c, sa);
    return true;
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
  return true;
}

// The reference-signature entry (musapy_cumsum_*_v3): every piece of state lives in `tmp`, whose
// capacity is the caller's formula, rows * (bpr [+ ceil(bpr/256) if bpr > 256]) elements
// (op_builder.rs:3315-3321).  Its last 8-byte word is the fault word (kcommon.hpp), zeroed by
// the launch that can wait, together with the words it clears.
template <class T>
void launch_cumsum(const T* a, T* c, T* tmp, int ndim, const size_t* shape, const ssize_t* strides, int axis,
                   size_t axis_len, size_t out_size, hipStream_t st) {
  ScanShape sh;
  if (!plan_cumsum<T>(sh, a, c, ndim, shape, strides, axis, axis_len, out_size)) return;
  const ScanPlan& p = sh.p;
  const uint64_t bpr = (p.L + 255) / 256;
  const uint64_t cap = uint64_t(p.rows) * (bpr + (bpr > 256 ? (bpr + 255) / 256 : 0)) * sizeof(T);
  ScanScratch sc;
  WsSplit w;
  if (ws_split(tmp, cap, w)) {
    sc.chain = sc.lb = w.payload;
    sc.chain_bytes = sc.lb_bytes = w.payload_bytes;
    sc.fault = w.fault;
    sc.clear_fault = true;  // zeroed by the clear of the prefixes or status words
  }
  run_cumsum<T>(a, c, sh, sc, st);
}

// musapy_cumsum_ws_v2 / _v1: the chained scan on the zeroed payload of `ws` (no clearing launch),
// the look-back on `tmp` (tmp_bytes of it; may be NULL when the shape does not take it), the
// fault word in `ws`.  -1 when nothing was launched: `chain_only` and another path, or state
// missing (wrapper error 1).
template <class T>
int launch_cumsum_ws(const T* a, T* c, void* tmp, size_t tmp_bytes, int ndim, const size_t* shape,
                     const ssize_t* strides, int axis, size_t axis_len, size_t out_size, void* ws, size_t ws_bytes,
                     bool chain_only, hipStream_t st) {
  ScanShape sh;
  WsSplit w;
  if (!ws_split(ws, ws_bytes, w) || out_size == 0 || axis_len == 0 || !args_ok(ndim, axis)) return -1;
  if (!plan_cumsum<T>(sh, a, c, ndim, shape, strides, axis, axis_len, out_size)) return -1;
  const uint64_t ct = chain_tiles<T>(sh);
  const uint64_t W = sizeof(typename ScanAcc<T>::A) == 4 ? 1 : 2;
  const bool chain = ct != 0 && uint64_t(sh.p.rows) * ct * W * 8 <= w.payload_bytes;
  if (chain_only && !chain) return -1;
  ScanScratch sc;
  sc.fault = w.fault;
  if (chain) {
    sc.chain = w.payload;
    sc.chain_bytes = w.payload_bytes;
    sc.chain_clear = false;
  } else if (tmp != nullptr && (reinterpret_cast<uintptr_t>(tmp) & 7) == 0) {
    // a chained scan too large for the workspace runs on tmp, cleared first
    sc.chain = sc.lb = static_cast<uint64_t*>(tmp);
    sc.chain_bytes = sc.lb_bytes = tmp_bytes & ~size_t(7);
  }
  return run_cumsum<T>(a, c, sh, sc, st) ? 0 : -1;
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

// The chained scan with a zeroed workspace instead of the reference's scratch (new; no
// counterpart in kernels.rs): 0 when launched, -1 when the call does not take the chained path
// or the workspace is too small (nothing launched; use musapy_cumsum_ws_v2 or _v3).
#define CUMSUM_WS_DISPATCH(TMP, TMPB, CHAIN_ONLY)                                                                   \
  switch (dtype) {                                                                                                \
    case MUSAPY_DT_I64:                                                                                           \
      return launch_cumsum_ws<int64_t>(static_cast<const int64_t*>(a), static_cast<int64_t*>(c), TMP, TMPB, ndim, \
                                       in_shape, in_strides, axis, axis_len, out_size, workspace,                 \
                                       workspace_bytes, CHAIN_ONLY, st);                                          \
    case MUSAPY_DT_F32:                                                                                           \
      return launch_cumsum_ws<float>(static_cast<const float*>(a), static_cast<float*>(c), TMP, TMPB, ndim,       \
                                     in_shape, in_strides, axis, axis_len, out_size, workspace, workspace_bytes,  \
                                     CHAIN_ONLY, st);                                                             \
    case MUSAPY_DT_F64:                                                                                           \
      return launch_cumsum_ws<double>(static_cast<const double*>(a), static_cast<double*>(c), TMP, TMPB, ndim,    \
                                      in_shape, in_strides, axis, axis_len, out_size, workspace, workspace_bytes, \
                                      CHAIN_ONLY, st);                                                            \
    default:                                                                                                      \
      return -1;                                                                                                  \
  }
int musapy_cumsum_ws_v1(int dtype, const void* a, void* c, int ndim, const size_t* in_shape,
                        const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, void* workspace,
                        size_t workspace_bytes, hipStream_t st) {
  CUMSUM_WS_DISPATCH(nullptr, 0, true)
}

// Any cumsum with its waits reported in the workspace's fault word (new; no counterpart in
// kernels.rs): the chained scan on the zeroed workspace when it fits, else on `tmp`; the
// look-back on `tmp`; the sequential scan needs neither.  0 when launched, -1 when not (wrapper
// error 1: `tmp` missing or too small for the path taken).
int musapy_cumsum_ws_v2(int dtype, const void* a, void* c, void* tmp, size_t tmp_bytes, int ndim,
                        const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size,
                        void* workspace, size_t workspace_bytes, hipStream_t st) {
  CUMSUM_WS_DISPATCH(tmp, tmp_bytes, false)
}
#undef CUMSUM_WS_DISPATCH

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
