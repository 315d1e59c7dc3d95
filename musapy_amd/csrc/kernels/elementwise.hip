// elementwise.hip -- binary / unary / clamp / cast over N-d broadcast strides, for gfx950.
//
// Drop-in for the reference's kernels/elementwise.mu:577-828 (wrappers) and its nd / flat /
// vec4 / scalar kernels (elementwise.mu:35-208, 295-394, 451-536).  Instead of one thread per
// element decoding every dimension with 64-bit div/mod, the wrapper coalesces dimensions on the
// host (plan.hpp) and picks one of four variants:
//   flat       every operand contiguous or a broadcast scalar: one 16-byte vector per operand
//              per lane, many short blocks;
//   tiles      (binary, long rows) column tiles that walk down the rows: an operand broadcast
//              along the rows stays in registers, a per-row scalar costs one load per row;
//   rows       output rows of the innermost dim; the outer coordinates of a row are decoded
//              once with 32-bit magic division, the inner dim is streamed per operand as
//              vector (stride 1), broadcast (stride 0) or gather (any other stride);
//   transpose  single-input ops whose input is unit-stride along some other dim (a transposed
//              or permuted view): 64 x (32*VEC) tiles staged through LDS so that both the read
//              and the write are 16-byte coalesced accesses;
//   generic    64-bit per-element decode, only for shapes beyond the 32-bit limits above.
#include "kcommon.hpp"
#include "ew_ops.hpp"
#include "../../../include/musapy_kernels.h"

namespace mpy {

constexpr int kBlock = 256;
// Lanes per block of the flat kernels (unit-stride operands, one vector per lane).  Measured on
// MI355X with streaming stores: binary ops run faster in 128-lane blocks than in 256 (64M f32 add
// 124.2 -> 119.4 us, c128 mul 124.4 -> 119.7, the i64 + f64 add 62.5 -> 60.1, 16M f32 add 33.4
// -> 32.9), unary ops and casts slower (clamp of 16M f64 43.3 -> 44.1, f64 -> f32 34.1 -> 34.6).
// Same-type binary ops run faster still in 64-lane blocks (event-timed, one A/B run: 16M f32 add
// 32.7-32.8 -> 32.1-32.3 us, 64M 123.6-124.0 -> 122.4-122.6, c128 mul 123.9-124.4 -> 122.8-123.0),
// the fused-promotion kernel slower (the i64 + f64 add 61.9-62.0 -> 62.7-63.4), so it keeps 128.
constexpr int kFlatBlockUnary = 256;
constexpr int kFlatBlockBinary = 64;
constexpr int kFlatBlockMixed = 128;

// ---------------------------------------------------------------------------------------------
// operand access modes
// kModeRev: stride -1 (a flipped row), read as vectors ending at the item and reversed in registers
enum : int { kModeScalar = 0, kModeUnit = 1, kModeStrided = 2, kModeRev = 3 };

template <class T>
struct In {
  const T* p;
  int mode;
  bool nt = false;  // streaming loads (set by the launcher from the launch's input volume)
};

// ---------------------------------------------------------------------------------------------
// flat: 1-D, every input contiguous (mode 1) or scalar (mode 0).  Full tiles use VEC-wide
// vector accesses; the final partial tile falls back to one element per lane.
template <int VEC, int UNROLL, bool NTS, class F, class TO, class TA>
__global__ __launch_bounds__(kFlatBlockUnary) void k_unary_flat(In<TA> a, TO* __restrict__ c, uint64_t n, F f) {
  constexpr uint64_t kTile = uint64_t(kFlatBlockUnary) * VEC * UNROLL;
  const uint64_t base = uint64_t(blockIdx.x) * kTile;
  const int t = threadIdx.x;
  if (base + kTile <= n) {
    Vec<TA, VEC> va[UNROLL];
    if (a.mode == kModeScalar) {
      const TA s = a.p[0];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
#pragma unroll
        for (int k = 0; k < VEC; ++k) va[u].v[k] = s;
    } else {
      static_for<UNROLL>(
          [&](auto u) { va[u] = vload_pol<TA, VEC>(a.p + base + uint64_t(u * kFlatBlockUnary + t) * VEC, a.nt); });
    }
    static_for<UNROLL>([&](auto u) {
      Vec<TO, VEC> vc;
#pragma unroll
      for (int k = 0; k < VEC; ++k) vc.v[k] = f(va[u].v[k]);
      vstore_as<NTS, TO, VEC>(c + base + uint64_t(u * kFlatBlockUnary + t) * VEC, vc);
    });
  } else {
    for (uint64_t i = base + t; i < n; i += kFlatBlockUnary) c[i] = f(a.mode == kModeScalar ? a.p[0] : a.p[i]);
  }
}

// TO: the output element type (T for arithmetic, uint8_t for comparisons)
template <int VEC, int UNROLL, bool NTS, class F, class T, class TO = T>
__global__ __launch_bounds__(kFlatBlockBinary) void k_binary_flat(In<T> a, In<T> b, TO* __restrict__ c, uint64_t n,
                                                                  F f) {
  constexpr uint64_t kTile = uint64_t(kFlatBlockBinary) * VEC * UNROLL;
  const uint64_t base = uint64_t(blockIdx.x) * kTile;
  const int t = threadIdx.x;
  if (base + kTile <= n) {
    Vec<T, VEC> va[UNROLL], vb[UNROLL];
    if (a.mode == kModeScalar) {
      const T s = a.p[0];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
#pragma unroll
        for (int k = 0; k < VEC; ++k) va[u].v[k] = s;
    } else {
      static_for<UNROLL>(
          [&](auto u) { va[u] = vload_pol<T, VEC>(a.p + base + uint64_t(u * kFlatBlockBinary + t) * VEC, a.nt); });
    }
    if (b.mode == kModeScalar) {
      const T s = b.p[0];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u)
#pragma unroll
        for (int k = 0; k < VEC; ++k) vb[u].v[k] = s;
    } else {
      static_for<UNROLL>(
          [&](auto u) { vb[u] = vload_pol<T, VEC>(b.p + base + uint64_t(u * kFlatBlockBinary + t) * VEC, b.nt); });
    }
    static_for<UNROLL>([&](auto u) {
      Vec<TO, VEC> vc;
#pragma unroll
      for (int k = 0; k < VEC; ++k) vc.v[k] = f(va[u].v[k], vb[u].v[k]);
      vstore_as<NTS, TO, VEC>(c + base + uint64_t(u * kFlatBlockBinary + t) * VEC, vc);
    });
  } else {
    for (uint64_t i = base + t; i < n; i += kFlatBlockBinary)
      c[i] = f(a.mode == kModeScalar ? a.p[0] : a.p[i], b.mode == kModeScalar ? b.p[0] : b.p[i]);
  }
}

// ---------------------------------------------------------------------------------------------
// rows: output rows of length L (the innermost coalesced dim).  A work item is VEC consecutive
// elements of one row; `aligned` (host-checked) guarantees every item is full and every
// unit-stride operand is 16-byte aligned at the item start.
// nt: streaming loads; false for operands that every block re-reads (broadcast rows).
template <int VEC, class T>
__device__ inline void load_item(const T* base, int mode, int64_t s, uint32_t col, uint32_t L, bool full, bool nt,
                                 T (&x)[VEC]) {
  if (mode == kModeScalar) {
    const T v = base[0];
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = v;
  } else if (mode == kModeUnit && full) {
    Vec<T, VEC> v = vload_pol<T, VEC>(base + col, nt);
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = v.v[k];
  } else if (mode == kModeRev && full) {
    // elements col .. col+VEC-1 of the row sit at base-col-(VEC-1) .. base-col
    Vec<T, VEC> v = vload_pol<T, VEC>(base - (int64_t(col) + (VEC - 1)), nt);
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = v.v[VEC - 1 - k];
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      if (col + k < L) x[k] = base[int64_t(col + k) * s];
  }
}

// Block of the unary rows kernel: 128 lanes x 4 items.  Measured on MI355X, flip of (8192, 8192)
// f32 along its rows (kernel time): 86.7-87.0 us, against 90.3 for 256 lanes x 4 items; 512 x 4
// 89.0, 256 x 2 87.0, 256 x 1 87.8, 1024 x 1 86.5.
constexpr int kRowsBlock = 128;
constexpr int kRowsUnroll = 4;
template <int VEC, int UNROLL, bool NTS, class F, class TO, class TA>
__global__ __launch_bounds__(kRowsBlock) void k_unary_rows(In<TA> a, int64_t sa, TO* __restrict__ c, RowIndexer<2> ix,
                                                           FastDiv gpr, uint32_t L, uint32_t items, bool aligned, F f) {
  const uint32_t first = blockIdx.x * (kRowsBlock * UNROLL) + threadIdx.x;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const uint32_t g = first + u * kRowsBlock;
    if (g >= items) break;
    const uint32_t row = fd_div(gpr, g);
    const uint32_t col = (g - row * gpr.d) * VEC;
    int64_t off[2];
    row_offsets<2>(ix, row, off);
    const bool full = aligned || (col + VEC <= L);
    TA x[VEC];
    load_item<VEC, TA>(a.p + off[1], a.mode, sa, col, L, full && aligned, a.nt, x);
    TO* cp = c + off[0] + col;
    if (full && aligned) {
      Vec<TO, VEC> v;
#pragma unroll
      for (int k = 0; k < VEC; ++k) v.v[k] = f(x[k]);
      vstore_as<NTS, TO, VEC>(cp, v);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (col + k < L) cp[k] = f(x[k]);
    }
  }
}

template <int VEC, int UNROLL, bool NTS, class F, class T, class TO = T>
__global__ __launch_bounds__(kBlock) void k_binary_rows(In<T> a, int64_t sa, In<T> b, int64_t sb, TO* __restrict__ c,
                                                        RowIndexer<3> ix, FastDiv gpr, uint32_t L, uint32_t items,
                                                        bool aligned, F f) {
  const uint32_t first = blockIdx.x * (kBlock * UNROLL) + threadIdx.x;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const uint32_t g = first + u * kBlock;
    if (g >= items) break;
    const uint32_t row = fd_div(gpr, g);
    const uint32_t col = (g - row * gpr.d) * VEC;
    int64_t off[3];
    row_offsets<3>(ix, row, off);
    const bool full = aligned || (col + VEC <= L);
    T x[VEC], y[VEC];
    load_item<VEC, T>(a.p + off[1], a.mode, sa, col, L, full && aligned, a.nt, x);
    load_item<VEC, T>(b.p + off[2], b.mode, sb, col, L, full && aligned, b.nt, y);
    TO* cp = c + off[0] + col;
    if (full && aligned) {
      Vec<TO, VEC> v;
#pragma unroll
      for (int k = 0; k < VEC; ++k) v.v[k] = f(x[k], y[k]);
      vstore_as<NTS, TO, VEC>(cp, v);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (col + k < L) cp[k] = f(x[k], y[k]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// mixed dtypes: c = f(TC(a), TC(b)) with the cast functors of the cast kernels, i.e. exactly the
// reference's cast-then-compute (op_builder.rs:410-417) without materialising the cast.
template <int VEC, bool NTS, class F, class TC, class TA, class TB>
__global__ __launch_bounds__(kFlatBlockMixed) void k_binary_flat_mixed(const TA* __restrict__ a,
                                                                        const TB* __restrict__ b,
                                                              TC* __restrict__ c, uint64_t n, bool nt, F f) {
  const uint64_t i0 = (uint64_t(blockIdx.x) * kFlatBlockMixed + threadIdx.x) * VEC;
  const CastF<TA, TC> ca{};
  const CastF<TB, TC> cb{};
  if (i0 + VEC <= n) {
    Vec<TA, VEC> x = vload_pol<TA, VEC>(a + i0, nt);
    Vec<TB, VEC> y = vload_pol<TB, VEC>(b + i0, nt);
    Vec<TC, VEC> z;
#pragma unroll
    for (int k = 0; k < VEC; ++k) z.v[k] = f(ca(x.v[k]), cb(y.v[k]));
    vstore_as<NTS, TC, VEC>(c + i0, z);
  } else {
    for (uint64_t i = i0; i < n; ++i) c[i] = f(ca(a[i]), cb(b[i]));
  }
}

// ---------------------------------------------------------------------------------------------
// row pieces: long output rows (broadcast operands, or operands whose outer strides do not
// merge).  A block writes U consecutive pieces of kPieceBlock*VEC elements of one row, so
// neighbouring blocks write neighbouring memory (column tiles that walk 8 rows each, whose blocks
// write 4 KB pieces 32 KB apart, measured 23.0-23.3 us for C2's (4096,1)+(8192,) against 21.1-21.3
// us).  A lane loads its U items of both operands first (an operand that is row-invariant or one
// value per row hits the cache), then computes and stores them.  Block shape, measured on MI355X
// for C2 with streaming stores (kernel time): 512 lanes x 2 pieces 22.4 us, 256 x 2 23.4, 128 x 2
// 22.7, 1024 x 2 24.8, 256 x 4 23.8, one piece per block 27.5; event-timed in a later A/B, 512 x 2
// 21.5-21.7 us, 64 x 4 22.8, 128 x 4 24.3-24.5, 64 x 8 25.2-25.4.
constexpr int kPieceBlock = 512;  // lanes per row-pieces block
constexpr int kPieces = 2;        // consecutive pieces per block
struct RowPieceArgs {
  RowIndexer<3> ix;   // outer dims: [0] out, [1] a, [2] b strides
  uint32_t L;         // row length (innermost output dim)
  FastDiv groups;     // blocks per row
  bool aligned;       // every item full and 16-byte aligned (host-checked)
};

template <int VEC, int U, bool NTS, class F, class T, class TO = T>
__global__ __launch_bounds__(kPieceBlock) void k_binary_rowpieces(In<T> a, int64_t sa, In<T> b, int64_t sb,
                                                             TO* __restrict__ c, RowPieceArgs ra, F f) {
  const uint32_t row = fd_div(ra.groups, blockIdx.x);
  const uint32_t g = blockIdx.x - row * ra.groups.d;
  int64_t off[3];
  row_offsets<3>(ra.ix, row, off);
  T xa[U][VEC], xb[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t col = ((g * U + u) * kPieceBlock + threadIdx.x) * VEC;
    if (col >= ra.L) break;
    const bool full = ra.aligned || col + VEC <= ra.L;
    load_item<VEC, T>(a.p + off[1], a.mode, sa, col, ra.L, full && ra.aligned, a.nt, xa[u]);
    load_item<VEC, T>(b.p + off[2], b.mode, sb, col, ra.L, full && ra.aligned, b.nt, xb[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t col = ((g * U + u) * kPieceBlock + threadIdx.x) * VEC;
    if (col >= ra.L) break;
    TO* cp = c + off[0] + col;
    if (ra.aligned) {
      Vec<TO, VEC> v;
#pragma unroll
      for (int k = 0; k < VEC; ++k) v.v[k] = f(xa[u][k], xb[u][k]);
      vstore_as<NTS, TO, VEC>(cp, v);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (col + k < ra.L) cp[k] = f(xa[u][k], xb[u][k]);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// transpose: single input that is unit-stride along dim P while the output is unit-stride along
// the innermost dim L.  A block moves a kTP x kTL tile through LDS.  Remaining dims are batch.
struct TransposeArgs {
  uint64_t P, L;           // extents of the two tiled dims
  int64_t in_sL;           // input stride along L (input stride along P is 1)
  int64_t out_sP;          // output stride along P (output stride along L is 1)
  FastDiv tilesL, tilesP;  // tile counts
  RowIndexer<2> batch;     // batch dims: [0] output strides, [1] input strides
  bool vec_in, vec_out;    // 16-byte aligned vector access possible on each side
  bool nt;                 // streaming loads
  bool pmajor;             // consecutive blocks take consecutive tiles along P (else along L)
};

// Tile geometry: PL lanes x VI elements along P (input-contiguous) by TL along L
// (output-contiguous); VI / VO = elements per vector: 16 bytes, 8 for 1-byte types (which keeps
// a u8 -> f64 tile inside LDS).  A pass of the read phase covers kTrBlock / PL rows of L, a pass
// of the write phase kTrBlock / (TL / VO) rows of P.
template <class T> constexpr int tr_vec() { return sizeof(T) >= 16 ? 1 : (sizeof(T) == 1 ? 8 : int(16 / sizeof(T))); }
template <class TI, int PL> constexpr int tr_tp() { return PL * tr_vec<TI>(); }
// Block shapes, measured on MI355X with streaming loads and stores and rotated outputs:
//  * copies and casts, 32 lanes along P: 1024-lane blocks over 128-row tiles (512-byte runs on
//    both sides for 4-byte types; about 66 KB of LDS, two blocks per CU).  (8192, 8192) f32
//    transposed: 91.5 us, against 106.6-107.5 us for the previous 64-row tiles in 256 lanes and
//    97.4-97.9 us in 512 lanes; the c128 transpose 94.8 against 102.5 us;
//  * other functors (exp of a transposed view): 512 lanes over 64-row tiles, 50.0-50.3 us for
//    C2's exp against 52.9 us with the copy shape (the functor's work favours more, smaller tiles);
//  * 16 or 8 lanes along P (small P): 1024 lanes over 128- or 256-row tiles (the (8192, 128, 64)
//    permute: 91.0-92.1 us, against 95.1 us over 256 rows).
// The rows are halved until the tile's LDS fits in 68 KB (wide outputs of narrow inputs).
// Block order: consecutive blocks take consecutive tiles along L (the output rows), so the blocks
// in flight write whole output rows, except when the output rows are longer than the input rows
// (then along P, launch_transpose).  Groups of 1-16 L tiles taken along P first measured slower
// for the (8192, 8192) f32 X^T (93.5-97.8 us against 90.0-90.3), level for c128 and exp, and only
// the (8192, 128, 64) permute gained (89.8-91.0 against 92.4-92.5 us).  Also measured for C2's
// (8192, 4096) view and not kept: the functor applied on the store side (LDS holding the input),
// exp 52.6 against 51.6 us; software-pipelined blocks of 2-4 tiles (next tile's loads in flight,
// LDS-only barriers), 52.3-56 us; the block -> tile map grouped by XCD, level; 16 lanes x 256 rows
// (50.3 us, but X^T 97.3 us) and 8 x 512, 16 x 256 in 512 lanes, 32 x 128 in 512 lanes (53-55 us);
// XOR-swizzled tile columns, free of LDS bank conflicts (which take 3/4 of this tile's LDS-active
// cycles), 50.7-53.7 against 50.0 us, X^T 94-104 against 91.7 us.
template <class F> struct tr_moves_only : std::false_type {};  // copies and casts
template <> struct tr_moves_only<IdentityF> : std::true_type {};
template <class S, class D> struct tr_moves_only<CastF<S, D>> : std::true_type {};
template <> struct tr_moves_only<ToBf16F> : std::true_type {};
template <> struct tr_moves_only<ToF16F> : std::true_type {};
template <class TO, class TI, int PL, int BS, int ROWS>
constexpr int tr_tl() {
  constexpr uint64_t TP = tr_tp<TI, PL>();
  int tl = ROWS;
  while (tl > BS / PL && uint64_t(tl) * (TP + 1) * sizeof(TO) > 68 * 1024) tl /= 2;
  return tl;
}

template <class F, class TO, class TI, int PL, int TL, int BS, bool NTS>
__global__ __launch_bounds__(BS) void k_unary_transpose(const TI* __restrict__ a, TO* __restrict__ c,
                                                            TransposeArgs ta, F f) {
  constexpr int VI = tr_vec<TI>(), VO = tr_vec<TO>();
  constexpr int TP = tr_tp<TI, PL>();
  constexpr int RP = BS / PL;  // L rows per read pass
  static_assert(BS % PL == 0 && TL % RP == 0, "read passes must tile TL");
  constexpr int NRP = TL / RP;
  constexpr int LPW = TL / VO;     // lanes along one output row
  static_assert(BS % LPW == 0 && TP % (BS / LPW) == 0, "write passes must tile TP");
  __shared__ TO tile[TL][TP + 1];
  const uint32_t id = blockIdx.x;
  uint32_t tl, tp, batch;
  if (ta.pmajor) {
    const uint32_t bq = fd_div(ta.tilesP, id);
    tp = id - bq * ta.tilesP.d;
    batch = fd_div(ta.tilesL, bq);
    tl = bq - batch * ta.tilesL.d;
  } else {
    const uint32_t bq = fd_div(ta.tilesL, id);
    tl = id - bq * ta.tilesL.d;
    batch = fd_div(ta.tilesP, bq);
    tp = bq - batch * ta.tilesP.d;
  }
  int64_t off[2];
  row_offsets<2>(ta.batch, batch, off);
  const uint64_t p0 = uint64_t(tp) * TP, l0 = uint64_t(tl) * TL;
  const TI* ab = a + off[1];
  TO* cb = c + off[0];
  const int t = threadIdx.x;
  // read: PL lanes x VI elements along P (unit stride in the input), RP rows of L per pass
  {
    const int pp = (t % PL) * VI;
    const int lr = t / PL;
    const uint64_t p = p0 + pp;
    if (ta.vec_in && l0 + TL <= ta.L && p0 + TP <= ta.P) {
      // interior tile: every pass's load is issued before the first LDS store
      Vec<TI, VI> v[NRP];
#pragma unroll
      for (int k = 0; k < NRP; ++k)
        v[k] = vload_pol<TI, VI>(ab + int64_t(l0 + lr + k * RP) * ta.in_sL + int64_t(p), ta.nt);
#pragma unroll
      for (int k = 0; k < NRP; ++k)
#pragma unroll
        for (int q = 0; q < VI; ++q) tile[lr + k * RP][pp + q] = f(v[k].v[q]);
    } else {
      for (int ll = lr; ll < TL; ll += RP) {
        const uint64_t l = l0 + ll;
        if (l >= ta.L) break;
        const TI* src = ab + int64_t(l) * ta.in_sL + int64_t(p);
        if (ta.vec_in && p + VI <= ta.P) {
          Vec<TI, VI> v = vload_pol<TI, VI>(src, ta.nt);
#pragma unroll
          for (int q = 0; q < VI; ++q) tile[ll][pp + q] = f(v.v[q]);
        } else {
#pragma unroll
          for (int q = 0; q < VI; ++q)
            if (p + q < ta.P) tile[ll][pp + q] = f(src[q]);
        }
      }
    }
  }
  __syncthreads();
  // write: LPW lanes x VO elements along L (unit stride in the output)
  {
    const int ll = (t % LPW) * VO;
    const uint64_t l = l0 + ll;
    for (int pp = t / LPW; pp < TP; pp += BS / LPW) {
      const uint64_t p = p0 + pp;
      if (p >= ta.P) break;
      TO* dst = cb + int64_t(p) * ta.out_sP + int64_t(l);
      if (ta.vec_out && l + VO <= ta.L) {
        Vec<TO, VO> v;
#pragma unroll
        for (int q = 0; q < VO; ++q) v.v[q] = tile[ll + q][pp];
        vstore_as<NTS, TO, VO>(dst, v);
      } else {
#pragma unroll
        for (int q = 0; q < VO; ++q)
          if (l + q < ta.L) dst[q] = tile[ll + q][pp];
      }
    }
  }
}

// Launches the tiled transpose with tile (PL lanes along P) x TL; the tile is narrowed along P
// (and lengthened along L, same LDS bytes) when P is small, so that no tile is mostly empty.
template <class F, class TO, class TI, int PL, int BS, int ROWS>
bool launch_transpose_tiles(const TI* a, TO* c, TransposeArgs ta, uint64_t nb, bool nts, hipStream_t st, F f) {
  constexpr uint64_t TP = tr_tp<TI, PL>();
  constexpr int TL = tr_tl<TO, TI, PL, BS, ROWS>();
  const uint64_t tL = (ta.L + TL - 1) / TL, tP = (ta.P + TP - 1) / TP;
  if (tL * tP * nb >= (uint64_t(1) << 31)) return false;
  ta.tilesL = make_fastdiv(uint32_t(tL));
  ta.tilesP = make_fastdiv(uint32_t(tP));
  with_store_policy(nts, [&](auto NT) {
    k_unary_transpose<F, TO, TI, PL, TL, BS, NT.value><<<dim3(unsigned(tL * tP * nb)), BS, 0, st>>>(a, c, ta, f);
  });
  return true;
}

template <class F, class TO, class TI>
bool launch_transpose(const TI* a, TO* c, TransposeArgs ta, uint64_t nb, bool nts, hipStream_t st, F f) {
  // LDS per tile: TL x (PL*VI + 1) elements of TO (tr_tl); 32 lanes x 128 rows is 66 KB for f32
  if (ta.P * 4 <= uint64_t(tr_tp<TI, 32>()))
    return launch_transpose_tiles<F, TO, TI, 8, 1024, 256>(a, c, ta, nb, nts, st, f);
  if (ta.P * 2 <= uint64_t(tr_tp<TI, 32>()))
    return launch_transpose_tiles<F, TO, TI, 16, 1024, 128>(a, c, ta, nb, nts, st, f);
  // Output rows longer than the input rows: tiles taken along P first, so that the blocks in flight
  // read whole input rows, each functor in the copy's 1024-lane tile.  (8192, 4096) f32 transposed
  // (C2's view, L = 8192 > P = 4096), event-timed: copy 50.5-51.9 -> 48.5-49.4 us, exp
  // 51.5-51.9 -> 49.6-49.9 us.  Square shapes keep the L order (X^T f32 at (8192, 8192): 91.7-92.2
  // us against 96.1-96.7 us taken along P).
  // 16-byte elements (c128 copies) move in 64 x 64 tiles, 1 KB runs on both sides, rather than 32
  // along P (512-byte reads, 2 KB writes): the (4096, 4096) c128 transpose 95.2-95.5 -> 90.7-90.9 us
  // event-timed in one A/B run.
  constexpr bool k16 = sizeof(TI) == 16 && sizeof(TO) == 16;
  if (ta.L > ta.P) {
    ta.pmajor = true;
    if constexpr (k16)
      if (ta.P >= 64) return launch_transpose_tiles<F, TO, TI, 64, 1024, 128>(a, c, ta, nb, nts, st, f);
    return launch_transpose_tiles<F, TO, TI, 32, 1024, 128>(a, c, ta, nb, nts, st, f);
  }
  if constexpr (tr_moves_only<F>::value) {
    if constexpr (k16)
      if (ta.P >= 64) return launch_transpose_tiles<F, TO, TI, 64, 1024, 128>(a, c, ta, nb, nts, st, f);
    return launch_transpose_tiles<F, TO, TI, 32, 1024, 128>(a, c, ta, nb, nts, st, f);
  } else {
    return launch_transpose_tiles<F, TO, TI, 32, 512, 64>(a, c, ta, nb, nts, st, f);
  }
}

// ---------------------------------------------------------------------------------------------
// generic fallback: 64-bit decode per element (shapes beyond the 32-bit row limits).
struct NdMeta64 {
  int nd;
  uint64_t shape[kMaxDims];
  int64_t stride[3][kMaxDims];
};

__device__ inline void nd_offsets(const NdMeta64& m, uint64_t i, int nops, int64_t (&off)[3]) {
  off[0] = off[1] = off[2] = 0;
  for (int d = m.nd - 1; d >= 0; --d) {
    uint64_t q = i / m.shape[d];
    int64_t cd = int64_t(i - q * m.shape[d]);
    i = q;
    for (int o = 0; o < nops; ++o) off[o] += cd * m.stride[o][d];
  }
}

template <class F, class TO, class TA>
__global__ __launch_bounds__(kBlock) void k_unary_generic(const TA* __restrict__ a, TO* __restrict__ c, NdMeta64 m,
                                                          uint64_t n, F f) {
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += uint64_t(gridDim.x) * kBlock) {
    int64_t off[3];
    nd_offsets(m, i, 2, off);
    c[off[0]] = f(a[off[1]]);
  }
}

template <class F, class T, class TO = T>
__global__ __launch_bounds__(kBlock) void k_binary_generic(const T* __restrict__ a, const T* __restrict__ b,
                                                           TO* __restrict__ c, NdMeta64 m, uint64_t n, F f) {
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += uint64_t(gridDim.x) * kBlock) {
    int64_t off[3];
    nd_offsets(m, i, 3, off);
    c[off[0]] = f(a[off[1]], b[off[2]]);
  }
}

template <class F, class TC, class TA, class TB>
__global__ __launch_bounds__(kBlock) void k_binary_generic_mixed(const TA* __restrict__ a, const TB* __restrict__ b,
                                                                 TC* __restrict__ c, NdMeta64 m, uint64_t n, F f) {
  const CastF<TA, TC> ca{};
  const CastF<TB, TC> cb{};
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += uint64_t(gridDim.x) * kBlock) {
    int64_t off[3];
    nd_offsets(m, i, 3, off);
    c[off[0]] = f(ca(a[off[1]]), cb(b[off[2]]));
  }
}

// ---------------------------------------------------------------------------------------------
// host side: variant selection
// vectors per thread: one 16-byte vector per operand per thread (many short blocks) measured best
// for the flat path on MI355X (6.7 TB/s add at 16M elements; 2 vectors per lane in the 64-lane binary
// blocks ran slower, 16M f64 == 42.6 -> 44.6 us, and unary ops and casts with 2 or 4 vectors per lane
// ran 1-5% slower, f32 -> bf16 of 16M elements 18.7 -> 19.1 / 19.9 us); the rows path keeps 4 items
constexpr int kFlatUnroll = 1;
constexpr int kUnroll = 4;

// Elements per work item, measured on MI355X (flat kernels, 16M-64M elements):
//  * binary: one 16-byte load per input (c128 mul at 32 bytes per lane: 5.8 TB/s, at 16: 6.8;
//    comparisons with wider loads lose: lt f32 at 16 B 6.3 TB/s, 32 B 5.7);
//  * unary / casts: one 16-byte store per lane, with loads of up to 32 bytes (f32->c64 6.4 vs
//    5.9 TB/s with 32-byte stores; f64->f32 6.7 with 32-byte loads vs 5.9 with 8-byte stores);
//    a 1- or 2-byte input is read at least 8 bytes at a time (u8->f32 5.7 vs 5.5 TB/s).
template <class T>
constexpr int vec_of() {
  return sizeof(T) >= 16 ? 1 : (sizeof(T) >= 8 ? 2 : (sizeof(T) == 4 ? 4 : 8));
}
template <class TA, class TO>
constexpr int ew_vec() {
  constexpr int vo = sizeof(TO) >= 16 ? 1 : int(16 / sizeof(TO));
  return (sizeof(TA) <= 2 && sizeof(TA) * vo < 8) ? 2 * vo : vo;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int mode_of(int64_t s) {
  return s == 0 ? kModeScalar : (s == 1 ? kModeUnit : (s == -1 ? kModeRev : kModeStrided));
}

inline NdMeta64 make_meta64(const Plan& p) {
  NdMeta64 m{};
  m.nd = p.ndim;
  for (int d = 0; d < p.ndim; ++d) {
    m.shape[d] = p.shape[d];
    for (int o = 0; o < p.nops && o < 3; ++o) m.stride[o][d] = p.stride[o][d];
  }
  return m;
}

// distinct elements operand `o` of a plan reads (broadcast dims, stride 0, count once)
inline uint64_t operand_elems(const Plan& p, int o) {
  uint64_t n = 1;
  for (int d = 0; d < p.ndim; ++d)
    if (p.stride[o][d] != 0) n *= p.shape[d];
  return n;
}

inline unsigned grid_generic(uint64_t n) {
  uint64_t g = (n + kBlock - 1) / kBlock;
  return unsigned(g > 65536 ? 65536 : g);
}

// rows path limits: row count and items must fit 32 bits
inline bool rows_ok(const Plan& p, int vec) {
  uint64_t L = p.shape[p.ndim - 1];
  uint64_t rows = p.numel / L;
  uint64_t items = rows * ((L + vec - 1) / vec);
  if (L >= (uint64_t(1) << 31) || items >= (uint64_t(1) << 31)) return false;
  for (int d = 0; d < p.ndim - 1; ++d)
    if (p.shape[d] >= (uint64_t(1) << 32)) return false;
  return true;
}

// true when every unit-stride (or reversed, stride -1) operand has each VEC item of every row
// on one aligned vector: 16 bytes, or the item's size when that is smaller
template <class T0, class T1, class T2 = T1>
inline bool rows_aligned(const Plan& p, int vec, const void* c, const void* a, const void* b = nullptr) {
  uint64_t L = p.shape[p.ndim - 1];
  if (L % vec) return false;
  const void* ptr[3] = {c, a, b};
  const size_t es[3] = {sizeof(T0), sizeof(T1), sizeof(T2)};
  for (int o = 0; o < p.nops; ++o) {
    int64_t s = p.stride[o][p.ndim - 1];
    if (s != 1 && s != -1) continue;
    // a reversed row's first item ends at the row start: its vector starts vec-1 elements lower
    const uintptr_t q = reinterpret_cast<uintptr_t>(ptr[o]) - (s == -1 ? (vec - 1) * es[o] : 0);
    if (es[o] * vec < 16 ? (q % (es[o] * vec)) : (q % 16)) return false;
    for (int d = 0; d < p.ndim - 1; ++d) {
      uint64_t bytes = uint64_t(p.stride[o][d] < 0 ? -p.stride[o][d] : p.stride[o][d]) * es[o];
      if (bytes % (es[o] * vec < 16 ? es[o] * vec : 16)) return false;
    }
  }
  return true;
}

template <class F, class TO, class TA>
void launch_unary(const TA* a, TO* c, int ndim, const size_t* shape, const ssize_t* as, hipStream_t st, F f) {
  Plan p;
  const ssize_t* ins[1] = {as};
  if (!args_ok(ndim) || !plan_elementwise(p, ndim, shape, 1, ins)) return;
  // the narrower type moves 16 bytes per item, the wider one 16-32 (e.g. f64->f32: 4 elements)
  constexpr int V = ew_vec<TA, TO>();
  const bool nt = operand_elems(p, 1) * sizeof(TA) >= kStreamLoadBytes;
  const bool nts = p.numel * sizeof(TO) >= kStreamStoreBytesUnary;
  if (p.ndim == 1 && p.stride[0][0] == 1 && (p.stride[1][0] == 0 || p.stride[1][0] == 1)) {
    In<TA> ia{a, mode_of(p.stride[1][0]), nt};
    bool vec_ok = aligned16(c) && (ia.mode == kModeScalar || aligned16(a));
    if (vec_ok) {
      constexpr uint64_t kTile = uint64_t(kFlatBlockUnary) * V * kFlatUnroll;
      const uint64_t tiles = (p.numel + kTile - 1) / kTile;
      with_store_policy(nts, [&](auto NT) {
        k_unary_flat<V, kFlatUnroll, NT.value, F, TO, TA><<<dim3(unsigned(tiles)), kFlatBlockUnary, 0, st>>>(
            ia, c, p.numel, f);
      });
    } else {
      uint64_t tiles = (p.numel + uint64_t(kFlatBlockUnary) * kUnroll - 1) / (uint64_t(kFlatBlockUnary) * kUnroll);
      k_unary_flat<1, kUnroll, false, F, TO, TA><<<dim3(unsigned(tiles)), kFlatBlockUnary, 0, st>>>(ia, c, p.numel, f);
    }
    return;
  }
  // transposed input: unit stride along some dim other than the innermost one
  const int nd = p.ndim;
  const int64_t sL = p.stride[1][nd - 1];
  if (nd >= 2 && sL != 0 && sL != 1) {
    int P = -1;
    for (int d = nd - 2; d >= 0; --d)
      if (p.stride[1][d] == 1) { P = d; break; }
    if (P >= 0 && p.shape[P] < (uint64_t(1) << 32) && p.shape[nd - 1] < (uint64_t(1) << 32)) {
      TransposeArgs ta{};
      ta.P = p.shape[P];
      ta.L = p.shape[nd - 1];
      ta.in_sL = sL;
      ta.out_sP = p.stride[0][P];
      uint64_t nb = p.numel / (ta.P * ta.L);
      {
        // batch dims: all dims but P and nd-1, innermost first
        ta.batch.nd = 0;
        ta.vec_in = aligned16(a) && (uint64_t(sL < 0 ? -sL : sL) * sizeof(TA)) % 16 == 0;
        ta.vec_out = aligned16(c) && (uint64_t(ta.out_sP) * sizeof(TO)) % 16 == 0;
        // tiles read across many rows at once: streaming won at 128 MB too (5.1 vs 4.9 TB/s), and with
        // the 1024-lane tiles default loads ran 2-8% slower (f32 X^T 98.1 vs 91.2 us, c128 98.9 vs 91.4)
        ta.nt = true;
        for (int d = nd - 2; d >= 0; --d) {
          if (d == P) continue;
          int k = ta.batch.nd++;
          ta.batch.div[k] = make_fastdiv(uint32_t(p.shape[d]));
          ta.batch.stride[0][k] = p.stride[0][d];
          ta.batch.stride[1][k] = p.stride[1][d];
          if ((uint64_t(p.stride[1][d] < 0 ? -p.stride[1][d] : p.stride[1][d]) * sizeof(TA)) % 16) ta.vec_in = false;
          if ((uint64_t(p.stride[0][d]) * sizeof(TO)) % 16) ta.vec_out = false;
        }
        if (launch_transpose<F, TO, TA>(a, c, ta, nb, nts, st, f)) return;
      }
    }
  }
  if ((nd >= 2 || sL == -1) && rows_ok(p, V)) {
    const uint32_t L = uint32_t(p.shape[nd - 1]);
    In<TA> ia{a, mode_of(sL), nt};
    bool al = rows_aligned<TO, TA>(p, V, c, a);
    uint32_t gpr = (L + V - 1) / V;
    uint32_t items = uint32_t(p.numel / L) * gpr;
    RowIndexer<2> ix = make_row_indexer<2>(p);
    unsigned grid = (items + kRowsBlock * kRowsUnroll - 1) / (kRowsBlock * kRowsUnroll);
    with_store_policy(nts, [&](auto NT) {
      k_unary_rows<V, kRowsUnroll, NT.value, F, TO, TA><<<grid, kRowsBlock, 0, st>>>(ia, sL, c, ix, make_fastdiv(gpr),
                                                                                   L, items, al, f);
    });
    return;
  }
  k_unary_generic<F, TO, TA><<<grid_generic(p.numel), kBlock, 0, st>>>(a, c, make_meta64(p), p.numel, f);
}

template <class F, class T, class TO = T>
void launch_binary(const T* a, const T* b, TO* c, int ndim, const size_t* shape, const ssize_t* as, const ssize_t* bs,
                   hipStream_t st, F f) {
  Plan p;
  const ssize_t* ins[2] = {as, bs};
  if (!args_ok(ndim) || !plan_elementwise(p, ndim, shape, 2, ins)) return;
  constexpr int V = vec_of<T>();
  const int nd = p.ndim;
  const bool nt = (operand_elems(p, 1) + operand_elems(p, 2)) * sizeof(T) >= kStreamLoadBytes;
  const bool nts = p.numel * sizeof(TO) >= kStreamStoreBytes;
  if (nd == 1 && (p.stride[1][0] == 0 || p.stride[1][0] == 1) && (p.stride[2][0] == 0 || p.stride[2][0] == 1)) {
    In<T> ia{a, mode_of(p.stride[1][0]), nt}, ib{b, mode_of(p.stride[2][0]), nt};
    constexpr uintptr_t kOutAlign = sizeof(TO) * V < 16 ? sizeof(TO) * V : 16;  // one output vector
    bool vec_ok = (reinterpret_cast<uintptr_t>(c) % kOutAlign) == 0 && (ia.mode == kModeScalar || aligned16(a)) &&
                  (ib.mode == kModeScalar || aligned16(b));
    if (vec_ok) {
      constexpr uint64_t kTile = uint64_t(kFlatBlockBinary) * V * kFlatUnroll;
      const uint64_t tiles = (p.numel + kTile - 1) / kTile;
      with_store_policy(nts, [&](auto NT) {
        k_binary_flat<V, kFlatUnroll, NT.value, F, T, TO><<<dim3(unsigned(tiles)), kFlatBlockBinary, 0, st>>>(
            ia, ib, c, p.numel, f);
      });
    } else {
      uint64_t tiles = (p.numel + uint64_t(kFlatBlockBinary) * kUnroll - 1) / (uint64_t(kFlatBlockBinary) * kUnroll);
      k_binary_flat<1, kUnroll, false, F, T, TO><<<dim3(unsigned(tiles)), kFlatBlockBinary, 0, st>>>(ia, ib, c,
                                                                                                     p.numel, f);
    }
    return;
  }
  if (rows_ok(p, V)) {
    const uint32_t L = uint32_t(p.shape[nd - 1]);
    const int64_t sa = p.stride[1][nd - 1], sb = p.stride[2][nd - 1];
    In<T> ia{a, mode_of(sa), nt}, ib{b, mode_of(sb), nt};
    bool al = rows_aligned<TO, T, T>(p, V, c, a, b);
    uint32_t gpr = (L + V - 1) / V;
    uint32_t items = uint32_t(p.numel / L) * gpr;
    RowIndexer<3> ix = make_row_indexer<3>(p);
    if (L >= uint32_t(kPieceBlock) * V / 2) {
      // long rows: blocks of U consecutive row pieces
      constexpr int U = kPieces;
      RowPieceArgs ra{};
      ra.ix = ix;
      ra.L = L;
      ra.aligned = al;
      const uint32_t groups = (L + uint32_t(kPieceBlock) * V * U - 1) / (uint32_t(kPieceBlock) * V * U);
      ra.groups = make_fastdiv(groups);
      const uint64_t blocks = uint64_t(p.numel / L) * groups;
      if (blocks < (uint64_t(1) << 31)) {
        with_store_policy(nts, [&](auto NT) {
          k_binary_rowpieces<V, U, NT.value, F, T, TO><<<dim3(unsigned(blocks)), kPieceBlock, 0, st>>>(ia, sa, ib, sb,
                                                                                                       c, ra, f);
        });
        return;
      }
    }
    unsigned grid = (items + kBlock * kUnroll - 1) / (kBlock * kUnroll);
    with_store_policy(nts, [&](auto NT) {
      k_binary_rows<V, kUnroll, NT.value, F, T, TO><<<grid, kBlock, 0, st>>>(ia, sa, ib, sb, c, ix, make_fastdiv(gpr),
                                                                           L, items, al, f);
    });
    return;
  }
  k_binary_generic<F, T, TO><<<grid_generic(p.numel), kBlock, 0, st>>>(a, b, c, make_meta64(p), p.numel, f);
}

template <class F, class TC, class TA, class TB>
void launch_binary_mixed(const void* a, const void* b, void* c, int ndim, const size_t* shape, const ssize_t* as,
                         const ssize_t* bs, hipStream_t st, F f) {
  Plan p;
  const ssize_t* ins[2] = {as, bs};
  if (!args_ok(ndim) || !plan_elementwise(p, ndim, shape, 2, ins)) return;
  const TA* pa = static_cast<const TA*>(a);
  const TB* pb = static_cast<const TB*>(b);
  TC* pc = static_cast<TC*>(c);
  constexpr int V = 16 / (sizeof(TA) > sizeof(TB) ? (sizeof(TA) > sizeof(TC) ? sizeof(TA) : sizeof(TC))
                                                  : (sizeof(TB) > sizeof(TC) ? sizeof(TB) : sizeof(TC)));
  if (p.ndim == 1 && p.stride[1][0] == 1 && p.stride[2][0] == 1 && aligned16(a) && aligned16(b) && aligned16(c)) {
    const uint64_t blocks = (p.numel + uint64_t(kFlatBlockMixed) * V - 1) / (uint64_t(kFlatBlockMixed) * V);
    const bool nt = p.numel * (sizeof(TA) + sizeof(TB)) >= kStreamLoadBytes;
    const bool nts = p.numel * sizeof(TC) >= kStreamStoreBytes;
    with_store_policy(nts, [&](auto NT) {
      k_binary_flat_mixed<V, NT.value, F, TC, TA, TB><<<dim3(unsigned(blocks)), kFlatBlockMixed, 0, st>>>(
          pa, pb, pc, p.numel, nt, f);
    });
    return;
  }
  k_binary_generic_mixed<F, TC, TA, TB><<<grid_generic(p.numel), kBlock, 0, st>>>(pa, pb, pc, make_meta64(p),
                                                                                   p.numel, f);
}

// the (input, input) -> output dtype triples the fused entry point accepts: one input already
// has the result dtype, the other is int32/int64/f32/f64 (the promotions C3-style data reaches)
template <class F>
bool dispatch_mixed(int ta, int tb, int tc, const void* a, const void* b, void* c, int ndim, const size_t* shape,
                    const ssize_t* as, const ssize_t* bs, hipStream_t st, F f) {
#define MIX(A, B, C, TA_, TB_, TC_) \
  if (ta == A && tb == B && tc == C) { launch_binary_mixed<F, TC_, TA_, TB_>(a, b, c, ndim, shape, as, bs, st, f); return true; }
  MIX(MUSAPY_DT_I64, MUSAPY_DT_F64, MUSAPY_DT_F64, int64_t, double, double)
  MIX(MUSAPY_DT_F64, MUSAPY_DT_I64, MUSAPY_DT_F64, double, int64_t, double)
  MIX(MUSAPY_DT_I32, MUSAPY_DT_F64, MUSAPY_DT_F64, int32_t, double, double)
  MIX(MUSAPY_DT_F64, MUSAPY_DT_I32, MUSAPY_DT_F64, double, int32_t, double)
  MIX(MUSAPY_DT_I64, MUSAPY_DT_F32, MUSAPY_DT_F32, int64_t, float, float)
  MIX(MUSAPY_DT_F32, MUSAPY_DT_I64, MUSAPY_DT_F32, float, int64_t, float)
  MIX(MUSAPY_DT_I32, MUSAPY_DT_F32, MUSAPY_DT_F32, int32_t, float, float)
  MIX(MUSAPY_DT_F32, MUSAPY_DT_I32, MUSAPY_DT_F32, float, int32_t, float)
  MIX(MUSAPY_DT_F64, MUSAPY_DT_F32, MUSAPY_DT_F32, double, float, float)
  MIX(MUSAPY_DT_F32, MUSAPY_DT_F64, MUSAPY_DT_F32, float, double, float)
#undef MIX
  return false;
}

}  // namespace mpy

// =============================================================================================
// extern "C" surface (rust/musapy-ops/src/kernels.rs:19-81; new bf16/f16 casts)
using namespace mpy;

extern "C" {

#define MPY_BINARY(NAME, F)                                                                                 \
  void musapy_##NAME##_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape,      \
                              const ssize_t* as, const ssize_t* bs, hipStream_t st) {                      \
    launch_binary<F, float>(a, b, c, ndim, shape, as, bs, st, F{});                                        \
  }                                                                                                         \
  void musapy_##NAME##_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape,   \
                              const ssize_t* as, const ssize_t* bs, hipStream_t st) {                      \
    launch_binary<F, double>(a, b, c, ndim, shape, as, bs, st, F{});                                       \
  }
MPY_BINARY(add, AddF)
MPY_BINARY(sub, SubF)
MPY_BINARY(mul, MulF)
MPY_BINARY(div, DivF)
MPY_BINARY(pow, PowF)
#undef MPY_BINARY

// comparisons (kernels.rs:84-95, 114-117): the binary kernels with a 0/1-byte output
#define MPY_COMPARE(NAME, F)                                                                                \
  void musapy_##NAME##_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape,    \
                              const ssize_t* as, const ssize_t* bs, hipStream_t st) {                      \
    launch_binary<F, float, uint8_t>(a, b, c, ndim, shape, as, bs, st, F{});                               \
  }                                                                                                         \
  void musapy_##NAME##_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape,  \
                              const ssize_t* as, const ssize_t* bs, hipStream_t st) {                      \
    launch_binary<F, double, uint8_t>(a, b, c, ndim, shape, as, bs, st, F{});                              \
  }
MPY_COMPARE(eq, EqF)
MPY_COMPARE(ne, NeF)
MPY_COMPARE(lt, LtF)
MPY_COMPARE(gt, GtF)
MPY_COMPARE(le, LeF)
MPY_COMPARE(ge, GeF)
#undef MPY_COMPARE
#define MPY_COMPARE_C(NAME, F, SN, C)                                                                       \
  void musapy_##NAME##_##SN##_v2(const C* a, const C* b, uint8_t* c, int ndim, const size_t* shape,         \
                                 const ssize_t* as, const ssize_t* bs, hipStream_t st) {                   \
    launch_binary<F, C, uint8_t>(a, b, c, ndim, shape, as, bs, st, F{});                                   \
  }
MPY_COMPARE_C(eq, CEqF, c64, c64)
MPY_COMPARE_C(eq, CEqF, c128, c128)
MPY_COMPARE_C(ne, CNeF, c64, c64)
MPY_COMPARE_C(ne, CNeF, c128, c128)
#undef MPY_COMPARE_C

// complex arithmetic (kernels.rs:102-113)
#define MPY_BINARY_C(NAME, F)                                                                               \
  void musapy_##NAME##_c64_v2(const c64* a, const c64* b, c64* c, int ndim, const size_t* shape,            \
                              const ssize_t* as, const ssize_t* bs, hipStream_t st) {                      \
    launch_binary<F, c64>(a, b, c, ndim, shape, as, bs, st, F{});                                          \
  }                                                                                                         \
  void musapy_##NAME##_c128_v2(const c128* a, const c128* b, c128* c, int ndim, const size_t* shape,        \
                               const ssize_t* as, const ssize_t* bs, hipStream_t st) {                     \
    launch_binary<F, c128>(a, b, c, ndim, shape, as, bs, st, F{});                                         \
  }
MPY_BINARY_C(add, CAddF)
MPY_BINARY_C(sub, CSubF)
MPY_BINARY_C(mul, CMulF)
MPY_BINARY_C(div, CDivF)
#undef MPY_BINARY_C
void musapy_neg_c64_v2(const c64* a, c64* c, int ndim, const size_t* shape, const ssize_t* as, hipStream_t st) {
  launch_unary<CNegF, c64, c64>(a, c, ndim, shape, as, st, CNegF{});
}
void musapy_neg_c128_v2(const c128* a, c128* c, int ndim, const size_t* shape, const ssize_t* as, hipStream_t st) {
  launch_unary<CNegF, c128, c128>(a, c, ndim, shape, as, st, CNegF{});
}
void musapy_abs_c64_v2(const c64* a, float* c, int ndim, const size_t* shape, const ssize_t* as, hipStream_t st) {
  launch_unary<CAbsF, float, c64>(a, c, ndim, shape, as, st, CAbsF{});
}
void musapy_abs_c128_v2(const c128* a, double* c, int ndim, const size_t* shape, const ssize_t* as,
                        hipStream_t st) {
  launch_unary<CAbsF, double, c128>(a, c, ndim, shape, as, st, CAbsF{});
}

#define MPY_UNARY(NAME, F)                                                                                  \
  void musapy_##NAME##_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* as,   \
                              hipStream_t st) {                                                             \
    launch_unary<F, float, float>(a, c, ndim, shape, as, st, F{});                                         \
  }                                                                                                         \
  void musapy_##NAME##_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* as, \
                              hipStream_t st) {                                                             \
    launch_unary<F, double, double>(a, c, ndim, shape, as, st, F{});                                       \
  }
MPY_UNARY(sin, SinF)
MPY_UNARY(cos, CosF)
MPY_UNARY(exp, ExpF)
MPY_UNARY(log, LogF)
MPY_UNARY(abs, AbsF)
MPY_UNARY(sign, SignF)
MPY_UNARY(neg, NegF)
#undef MPY_UNARY

void musapy_clamp_f32_v2(const float* a, float* c, float lo, float hi, int ndim, const size_t* shape,
                         const ssize_t* as, hipStream_t st) {
  launch_unary<ClampF<float>, float, float>(a, c, ndim, shape, as, st, ClampF<float>{lo, hi});
}
void musapy_clamp_f64_v2(const double* a, double* c, double lo, double hi, int ndim, const size_t* shape,
                         const ssize_t* as, hipStream_t st) {
  launch_unary<ClampF<double>, double, double>(a, c, ndim, shape, as, st, ClampF<double>{lo, hi});
}

#define MPY_CAST(SN, ST, DN, DT)                                                                            \
  void musapy_cast_##SN##_##DN##_v2(const ST* a, DT* c, int ndim, const size_t* shape, const ssize_t* as,   \
                                     hipStream_t st) {                                                      \
    launch_unary<CastF<ST, DT>, DT, ST>(a, c, ndim, shape, as, st, CastF<ST, DT>{});                       \
  }
#define MPY_CAST_FROM_INTS(DN, DT)    \
  MPY_CAST(i8, int8_t, DN, DT)        \
  MPY_CAST(i16, int16_t, DN, DT)      \
  MPY_CAST(i32, int32_t, DN, DT)      \
  MPY_CAST(u8, uint8_t, DN, DT)       \
  MPY_CAST(u16, uint16_t, DN, DT)     \
  MPY_CAST(u32, uint32_t, DN, DT)     \
  MPY_CAST(u64, uint64_t, DN, DT)
MPY_CAST_FROM_INTS(f32, float)
MPY_CAST(i64, int64_t, f32, float)
MPY_CAST(f64, double, f32, float)
MPY_CAST_FROM_INTS(f64, double)
MPY_CAST(i64, int64_t, f64, double)
MPY_CAST(f32, float, f64, double)
MPY_CAST_FROM_INTS(i64, int64_t)
MPY_CAST(f32, float, i64, int64_t)
MPY_CAST(f64, double, i64, int64_t)
// real -> complex and c64 -> c128 (kernels.rs:119-124)
MPY_CAST(f32, float, c64, c64)
MPY_CAST(f32, float, c128, c128)
MPY_CAST(f64, double, c64, c64)
MPY_CAST(f64, double, c128, c128)
MPY_CAST(c64, c64, c128, c128)
#undef MPY_CAST_FROM_INTS
#undef MPY_CAST

void musapy_cast_f32_bf16_v2(const float* a, uint16_t* c, int ndim, const size_t* shape, const ssize_t* as,
                             hipStream_t st) {
  launch_unary<ToBf16F, uint16_t, float>(a, c, ndim, shape, as, st, ToBf16F{});
}
void musapy_cast_f32_f16_v2(const float* a, uint16_t* c, int ndim, const size_t* shape, const ssize_t* as,
                            hipStream_t st) {
  launch_unary<ToF16F, uint16_t, float>(a, c, ndim, shape, as, st, ToF16F{});
}

int musapy_binary_mixed_v2(int op, const void* a, int a_dtype, const void* b, int b_dtype, void* c, int c_dtype,
                           int ndim, const size_t* shape, const ssize_t* as, const ssize_t* bs, hipStream_t st) {
  switch (op) {
    case MUSAPY_OP_ADD: return dispatch_mixed(a_dtype, b_dtype, c_dtype, a, b, c, ndim, shape, as, bs, st, AddF{}) ? 0 : -1;
    case MUSAPY_OP_SUB: return dispatch_mixed(a_dtype, b_dtype, c_dtype, a, b, c, ndim, shape, as, bs, st, SubF{}) ? 0 : -1;
    case MUSAPY_OP_MUL: return dispatch_mixed(a_dtype, b_dtype, c_dtype, a, b, c, ndim, shape, as, bs, st, MulF{}) ? 0 : -1;
    case MUSAPY_OP_DIV: return dispatch_mixed(a_dtype, b_dtype, c_dtype, a, b, c, ndim, shape, as, bs, st, DivF{}) ? 0 : -1;
    case MUSAPY_OP_POW: return dispatch_mixed(a_dtype, b_dtype, c_dtype, a, b, c, ndim, shape, as, bs, st, PowF{}) ? 0 : -1;
  }
  return -1;
}

// stride-aware materialisation of a view (kernels.rs:321-324; u8/u16 are new, for 1- and
// 2-byte dtypes).  A transposed source takes the LDS-tiled path.
#define MPY_COPY(NAME, T)                                                                                    \
  void musapy_copy_##NAME(const T* input, T* output, int ndim, const size_t* shape, const ssize_t* in_strides, \
                          hipStream_t st) {                                                                   \
    launch_unary<IdentityF, T, T>(input, output, ndim, shape, in_strides, st, IdentityF{});                  \
  }
MPY_COPY(f32, float)
MPY_COPY(f64, double)
MPY_COPY(i32, int32_t)
MPY_COPY(i64, int64_t)
MPY_COPY(u8, uint8_t)
MPY_COPY(u16, uint16_t)
MPY_COPY(c128, c128)
#undef MPY_COPY

// 2-D transpose materialisation (kernels.rs:327-330): src is a C-contiguous (cols, rows)
// array, dst[r*cols + c] = src[c*rows + r].  This is the copy of the transposed view
// (shape (rows, cols), strides (1, rows)), which the launcher sends to the LDS-tiled kernel.
#define MPY_COPY_T2D(NAME, T)                                                                                \
  void musapy_copy_transpose2d_##NAME(const T* src, T* dst, size_t rows, size_t cols, hipStream_t st) {      \
    const size_t shape[2] = {rows, cols};                                                                    \
    const ssize_t strides[2] = {1, ssize_t(rows)};                                                           \
    launch_unary<IdentityF, T, T>(src, dst, 2, shape, strides, st, IdentityF{});                             \
  }
MPY_COPY_T2D(f32, float)
MPY_COPY_T2D(f64, double)
MPY_COPY_T2D(i32, int32_t)
MPY_COPY_T2D(i64, int64_t)
#undef MPY_COPY_T2D

}  // extern "C"
