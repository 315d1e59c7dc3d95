// reduce_ops.hpp -- accumulator algebra of the reductions.
//
// The semantics are those of the reference's CPU path (rust/musapy-ops/src/op_builder.rs):
//   sum/prod      cpu_reduce_typed 3516-3541: acc = 0 (1), acc += x[k] for k ascending; i64 wraps
//   max/min       3543-3559: acc = x[0]; acc = x[k] when x[k] > acc (< for min), k = 1..
//   argmax/argmin 3560-3578: same scan, returns the k of the kept element
//   mean          cpu_mean_typed 3585-3619: sum / count, count built by repeated "+1" in T
//   complex       cpu_reduce_cplx 3439-3492: re/im accumulated in f64, narrowed once at the end
//
// A parallel tree reproduces the max/min/arg scans bit-exactly with an (value, index)
// accumulator and these rules:
//   * the scan keeps the FIRST element that attains the maximum (ties, including +0/-0, go to the
//     lowest index) -> combine picks the larger value, equal values pick the lower index;
//   * a NaN at k = 0 makes every later comparison false, so the result is x[0] (index 0)
//     -> the tile that holds k = 0 overrides its result with x[0] when x[0] is NaN;
//   * any later NaN never compares greater, so it is skipped.
// With those rules the combine is associative and commutative, so any reduction tree gives the
// same bits as the sequential scan.  Sums and products are evaluated in a fixed tree order
// (deterministic run to run; within the stated tolerance of the sequential sum).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kcommon.hpp"

namespace mpy {

template <class T> __device__ inline bool is_nan(T v) { return v != v; }
template <> __device__ inline bool is_nan<int64_t>(int64_t) { return false; }

template <class T> __device__ inline T qnan() { return T(__builtin_nan("")); }

// ---- shuffles of accumulator types ----
__device__ inline float acc_shfl(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ inline double acc_shfl(double v, int m) { return __shfl_xor(v, m, kWave); }
__device__ inline uint64_t acc_shfl(uint64_t v, int m) {
  return (uint64_t)__shfl_xor((unsigned long long)v, m, kWave);
}
__device__ inline int64_t acc_shfl(int64_t v, int m) { return (int64_t)__shfl_xor((long long)v, m, kWave); }
__device__ inline c128 acc_shfl(c128 v, int m) {
  return c128{__shfl_xor(v.re, m, kWave), __shfl_xor(v.im, m, kWave)};
}

__device__ inline int32_t acc_shfl(int32_t v, int m) { return __shfl_xor(v, m, kWave); }

template <class T, class I>
struct VI {  // value + index; idx < 0 means "no element yet"
  T val;
  I idx;
};
template <class T, class I> __device__ inline VI<T, I> acc_shfl(VI<T, I> v, int m) {
  return VI<T, I>{acc_shfl(v.val, m), acc_shfl(v.idx, m)};
}

// ---------------------------------------------------------------------------------------------
// Additive family.  `T` is the element type, `A` the accumulator.
template <class T> struct SumAcc { using A = T; };
template <> struct SumAcc<int64_t> { using A = uint64_t; };  // two's-complement wrap like release Rust
template <> struct SumAcc<c64> { using A = c128; };
template <> struct SumAcc<c128> { using A = c128; };

// A chunk of U x V elements one lane loaded together: element (u, v) sits at index
// base + k + u * stepk + v, so (u, v) in lexicographic order is increasing index.  The default
// folds the chunk element by element in that order.
template <class Op, class A, class T, int U, int V>
__device__ inline A fold_chunk(A acc, const T (&x)[U][V], uint32_t k, uint32_t stepk, int64_t base) {
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int v = 0; v < V; ++v) acc = Op::step(acc, x[u][v], base + int64_t(k + u * stepk + v));
  return acc;
}

template <class T>
struct OpSum {
  using A = typename SumAcc<T>::A;
  static constexpr bool kOrdered = false;  // max/min-style first-element rule
  static constexpr bool kArg = false;
  __device__ static A init() { return A(0); }
  __device__ static A step(A acc, T v, int64_t) { return acc + A(v); }
  __device__ static A comb(A a, A b) { return a + b; }
  template <int U, int V>
  __device__ static A step_chunk(A acc, const T (&x)[U][V], uint32_t k, uint32_t stepk, int64_t base = 0) {
    return fold_chunk<OpSum, A, T, U, V>(acc, x, k, stepk, base);
  }
};
template <> __device__ inline c128 OpSum<c64>::init() { return c128{0.0, 0.0}; }
template <> __device__ inline c128 OpSum<c64>::step(c128 acc, c64 v, int64_t) {
  return c128{acc.re + double(v.re), acc.im + double(v.im)};
}
template <> __device__ inline c128 OpSum<c64>::comb(c128 a, c128 b) { return c128{a.re + b.re, a.im + b.im}; }
template <> __device__ inline c128 OpSum<c128>::init() { return c128{0.0, 0.0}; }
template <> __device__ inline c128 OpSum<c128>::step(c128 acc, c128 v, int64_t) {
  return c128{acc.re + v.re, acc.im + v.im};
}
template <> __device__ inline c128 OpSum<c128>::comb(c128 a, c128 b) { return c128{a.re + b.re, a.im + b.im}; }

template <class T>
struct OpProd {
  using A = typename SumAcc<T>::A;
  static constexpr bool kOrdered = false;
  static constexpr bool kArg = false;
  __device__ static A init() { return A(1); }
  __device__ static A step(A acc, T v, int64_t) { return acc * A(v); }
  __device__ static A comb(A a, A b) { return a * b; }
  template <int U, int V>
  __device__ static A step_chunk(A acc, const T (&x)[U][V], uint32_t k, uint32_t stepk, int64_t base = 0) {
    return fold_chunk<OpProd, A, T, U, V>(acc, x, k, stepk, base);
  }
};
__device__ inline c128 cmul(c128 a, c128 b) {
  return c128{a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
template <> __device__ inline c128 OpProd<c64>::init() { return c128{1.0, 0.0}; }
template <> __device__ inline c128 OpProd<c64>::step(c128 acc, c64 v, int64_t) {
  return cmul(acc, c128{double(v.re), double(v.im)});
}
template <> __device__ inline c128 OpProd<c64>::comb(c128 a, c128 b) { return cmul(a, b); }
template <> __device__ inline c128 OpProd<c128>::init() { return c128{1.0, 0.0}; }
template <> __device__ inline c128 OpProd<c128>::step(c128 acc, c128 v, int64_t) { return cmul(acc, v); }
template <> __device__ inline c128 OpProd<c128>::comb(c128 a, c128 b) { return cmul(a, b); }

// ---------------------------------------------------------------------------------------------
// Ordered family (max / min / argmax / argmin share the accumulator).  The streaming kernels
// count I = int32 indices relative to the start of their tile (tiles are < 2^31 elements); the
// kernels that combine earlier partials carry absolute int64 indices.
template <class T, bool MAX, bool ARG, class I = int32_t>
struct OpExt {
  using A = VI<T, I>;
  using Idx = I;
  static constexpr bool kOrdered = true;
  static constexpr bool kArg = ARG;
  static constexpr bool kMax = MAX;
  __device__ static bool better(T a, T b) { return MAX ? (a > b) : (a < b); }
  __device__ static A init() { return A{T(0), -1}; }
  // elements of one lane arrive in increasing k, so a tie never replaces the kept element
  __device__ static A step(A acc, T v, int64_t k) {
    if (!is_nan(v) && (acc.idx < 0 || better(v, acc.val))) return A{v, I(k)};
    return acc;
  }
  __device__ static A comb(A a, A b) {
    if (b.idx < 0) return a;
    if (a.idx < 0) return b;
    if (better(b.val, a.val)) return b;
    if (better(a.val, b.val)) return a;
    return b.idx < a.idx ? b : a;
  }
  // pair input (partials of an earlier level): (v, k) where k < 0 marks an empty tile
  __device__ static A step_pair(A acc, T v, int64_t k) {
    if (k < 0 || is_nan(v)) return acc;
    return comb(acc, A{v, I(k)});
  }
  // Two phases per chunk: m = the chunk's extreme over its non-NaN elements (fmax/fmin drop a
  // NaN operand), then, only when m beats the running result, the first element equal to m.
  // That element is the one the sequential scan keeps: every earlier element is smaller (or
  // NaN), and equality also matches +0 against -0, so the kept bits are the first zero's.  A tie
  // with the running result keeps the running (lower) index.
  template <int U, int V>
  __device__ static A step_chunk(A acc, const T (&x)[U][V], uint32_t k, uint32_t stepk, int64_t base = 0) {
    T m = x[0][0];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = (u == 0 ? 1 : 0); v < V; ++v) m = pick(m, x[u][v]);
    const bool improve = acc.idx < 0 ? !is_nan(m) : better(m, acc.val);
    if (improve) {
      uint32_t off = 0;
#pragma unroll
      for (int u = U - 1; u >= 0; --u)
#pragma unroll
        for (int v = V - 1; v >= 0; --v)
          if (x[u][v] == m) off = u * stepk + v;
      // equal to m means the same bits, except that -0 equals +0: keep the first zero's bits
      T val = m;
      if (m == T(0)) {
#pragma unroll
        for (int u = U - 1; u >= 0; --u)
#pragma unroll
          for (int v = V - 1; v >= 0; --v)
            if (x[u][v] == m) val = x[u][v];
      }
      acc = A{val, I(base + int64_t(k + off))};
    }
    return acc;
  }
  // the extreme of two values, ignoring a NaN operand (for integers: plain max/min)
  __device__ static T pick(T a, T b) {
    if constexpr (sizeof(T) == 4 && T(0.5) != T(0)) return MAX ? __builtin_fmaxf(a, b) : __builtin_fminf(a, b);
    else if constexpr (sizeof(T) == 8 && T(0.5) != T(0)) return MAX ? __builtin_fmax(a, b) : __builtin_fmin(a, b);
    else return MAX ? (b > a ? b : a) : (b < a ? b : a);
  }
};

template <class T> __device__ inline T ext_none();  // value written for an empty max/min tile
template <> __device__ inline float ext_none<float>() { return qnan<float>(); }
template <> __device__ inline double ext_none<double>() { return qnan<double>(); }
template <> __device__ inline int64_t ext_none<int64_t>() { return INT64_MIN; }  // never kept by '>'
template <class T> __device__ inline T ext_none_min();
template <> __device__ inline float ext_none_min<float>() { return qnan<float>(); }
template <> __device__ inline double ext_none_min<double>() { return qnan<double>(); }
template <> __device__ inline int64_t ext_none_min<int64_t>() { return INT64_MAX; }

// ---------------------------------------------------------------------------------------------
// conversions of an accumulator to the values written out
template <class T, class A> __device__ inline T narrow(A a) { return T(a); }
template <> __device__ inline int64_t narrow<int64_t, uint64_t>(uint64_t a) { return int64_t(a); }
template <> __device__ inline c64 narrow<c64, c128>(c128 a) { return c64{float(a.re), float(a.im)}; }
template <> __device__ inline c128 narrow<c128, c128>(c128 a) { return a; }

// mean = sum / count where count is the reference's repeated "+1" in T (exact until 2^24 for
// f32, 2^53 for f64, constant afterwards); complex means divide re and im by the f64 length.
template <class T, class A> __device__ inline T mean_of(A s, double count) { return T(s / A(count)); }
template <> __device__ inline c64 mean_of<c64, c128>(c128 s, double n) { return c64{float(s.re / n), float(s.im / n)}; }
template <> __device__ inline c128 mean_of<c128, c128>(c128 s, double n) { return c128{s.re / n, s.im / n}; }

}  // namespace mpy
