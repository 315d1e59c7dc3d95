// ew_ops.hpp -- per-element functors of the elementwise path.
//
// Semantics follow the reference's CPU path, which is the parity oracle:
//   binary  cpu_binary_op          rust/musapy-ops/src/op_builder.rs:1618-1626
//   unary   cpu_unary_elementwise  op_builder.rs:1868-1896 (sign: v>0 -> 1, v<0 -> -1, else +0)
//   clamp   cpu_clamp_typed        op_builder.rs:2017-2047 (v<lo ? lo : v>hi ? hi : v; NaN passes)
//   cast    cpu_cast_pair!         op_builder.rs:227-243   (Rust `as`)
//   compare cpu_compare_typed/_cplx op_builder.rs:1786-1864
//   complex cpu_binary_cplx / cpu_unary_cplx_abs / cpu_cast_cplx  op_builder.rs:1652-1969, 2099-2167
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../../include/musapy_kernels.h"

namespace mpy {

// ---- binary ----
struct AddF { template <class T> __device__ T operator()(T a, T b) const { return a + b; } };
struct SubF { template <class T> __device__ T operator()(T a, T b) const { return a - b; } };
struct MulF { template <class T> __device__ T operator()(T a, T b) const { return a * b; } };
struct DivF { template <class T> __device__ T operator()(T a, T b) const { return a / b; } };
struct PowF {
  __device__ float operator()(float a, float b) const { return powf(a, b); }
  __device__ double operator()(double a, double b) const { return pow(a, b); }
};

// ---- comparisons: 0/1 bytes (cpu_compare_typed / cpu_compare_cplx, op_builder.rs:1786-1864) ----
// IEEE comparisons: a NaN operand makes every comparison false except !=, and +0 == -0.
struct EqF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a == b; } };
struct NeF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a != b; } };
struct LtF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a < b; } };
struct GtF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a > b; } };
struct LeF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a <= b; } };
struct GeF { template <class T> __device__ uint8_t operator()(T a, T b) const { return a >= b; } };
// complex: equal when both parts are equal
struct CEqF {
  template <class C> __device__ uint8_t operator()(C a, C b) const { return a.re == b.re && a.im == b.im; }
};
struct CNeF {
  template <class C> __device__ uint8_t operator()(C a, C b) const { return a.re != b.re || a.im != b.im; }
};

// ---- complex arithmetic (cpu_binary_cplx, op_builder.rs:1652-1731) ----
// Both widths evaluate the textbook component formulas in f64 (no fma contraction) and c64
// narrows each component to f32 once at the end, as the reference's CPU path does through
// CplxScalar::cplx_re/cplx_from_parts; division scales by |b|^2 without Smith's rescaling.
struct CParts {
  double re, im;
};
__device__ inline CParts cparts(musapy_c64_t v) { return CParts{double(v.re), double(v.im)}; }
__device__ inline CParts cparts(musapy_c128_t v) { return CParts{v.re, v.im}; }
template <class C> __device__ inline C cfrom(double re, double im);
template <> __device__ inline musapy_c64_t cfrom<musapy_c64_t>(double re, double im) {
  return musapy_c64_t{float(re), float(im)};
}
template <> __device__ inline musapy_c128_t cfrom<musapy_c128_t>(double re, double im) {
  return musapy_c128_t{re, im};
}
struct CAddF {
  template <class C> __device__ C operator()(C a, C b) const {
    CParts x = cparts(a), y = cparts(b);
    return cfrom<C>(x.re + y.re, x.im + y.im);
  }
};
struct CSubF {
  template <class C> __device__ C operator()(C a, C b) const {
    CParts x = cparts(a), y = cparts(b);
    return cfrom<C>(x.re - y.re, x.im - y.im);
  }
};
struct CMulF {
  template <class C> __device__ C operator()(C a, C b) const {
    CParts x = cparts(a), y = cparts(b);
    return cfrom<C>(x.re * y.re - x.im * y.im, x.re * y.im + x.im * y.re);
  }
};
struct CDivF {
  template <class C> __device__ C operator()(C a, C b) const {
    CParts x = cparts(a), y = cparts(b);
    double den = y.re * y.re + y.im * y.im;
    return cfrom<C>((x.re * y.re + x.im * y.im) / den, (x.im * y.re - x.re * y.im) / den);
  }
};
struct CNegF {
  template <class C> __device__ C operator()(C v) const { return C{-v.re, -v.im}; }
};
// |z| = sqrt(re^2 + im^2) in f64, narrowed for c64 (cpu_unary_cplx_abs, op_builder.rs:1944-1969)
struct CAbsF {
  __device__ float operator()(musapy_c64_t v) const {
    CParts x = cparts(v);
    return float(sqrt(x.re * x.re + x.im * x.im));
  }
  __device__ double operator()(musapy_c128_t v) const { return sqrt(v.re * v.re + v.im * v.im); }
};

// ---- unary ----
struct SinF {
  __device__ float operator()(float v) const { return sinf(v); }
  __device__ double operator()(double v) const { return sin(v); }
};
struct CosF {
  __device__ float operator()(float v) const { return cosf(v); }
  __device__ double operator()(double v) const { return cos(v); }
};
struct ExpF {
  __device__ float operator()(float v) const { return expf(v); }
  __device__ double operator()(double v) const { return exp(v); }
};
struct LogF {
  __device__ float operator()(float v) const { return logf(v); }
  __device__ double operator()(double v) const { return log(v); }
};
struct AbsF {
  __device__ float operator()(float v) const { return fabsf(v); }
  __device__ double operator()(double v) const { return fabs(v); }
};
struct SignF {
  template <class T> __device__ T operator()(T v) const {
    return v > T(0) ? T(1) : (v < T(0) ? T(-1) : T(0));
  }
};
struct NegF { template <class T> __device__ T operator()(T v) const { return -v; } };

template <class T>
struct ClampF {
  T lo, hi;
  __device__ T operator()(T v) const { return v < lo ? lo : (v > hi ? hi : v); }
};

struct IdentityF { template <class T> __device__ T operator()(T v) const { return v; } };

// ---- casts (Rust `as`) ----
template <class S, class D>
struct CastF {
  __device__ D operator()(S v) const { return static_cast<D>(v); }
};

// 64-bit integer -> f32, rounded to nearest even, from 32-bit operations only.  The compiler's own
// lowering shifts the value with v_lshlrev_b64 by a count that the instruction just before it
// computes; in instances measured on gfx950 (transpose tiles of 256 rows x 16 lanes and of 64 rows
// x 64 lanes) that shift used a stale count in whole waves, for the second conversion of each
// pair, returning values such as -1.0 for -721.  Here the leading word is formed with a funnel
// shift (v_alignbit_b32) and a sticky bit for the bits below it, and rounded once by
// v_cvt_f32_u32: a 32-bit word whose top bit is set rounds to 24 bits at bit 8, and the sticky
// bit in bit 0 keeps ties and near-ties apart, so the result is the correctly rounded value.
__device__ inline float u64_to_f32(uint64_t m) {
  const uint32_t hi = uint32_t(m >> 32), lo = uint32_t(m);
  if (hi == 0) return __uint2float_rn(lo);
  const uint32_t lz = __clz(hi);  // 0..31: (hi:lo) << lz has its top bit set
  const uint32_t top = lz == 0 ? hi : __builtin_amdgcn_alignbit(hi, lo, 32u - lz);
  const uint32_t below = lo << lz;  // the bits shifted out of the leading word (a 32-bit shift)
  return ldexpf(__uint2float_rn(top | (below != 0 ? 1u : 0u)), int(32 - lz));
}
__device__ inline float i64_to_f32(int64_t x) {
  const uint64_t m = x < 0 ? uint64_t(0) - uint64_t(x) : uint64_t(x);  // |INT64_MIN| = 2^63 fits
  const float r = u64_to_f32(m);
  return x < 0 ? -r : r;
}
template <> struct CastF<int64_t, float> {
  __device__ float operator()(int64_t v) const { return i64_to_f32(v); }
};
template <> struct CastF<uint64_t, float> {
  __device__ float operator()(uint64_t v) const { return u64_to_f32(v); }
};

// float -> i64 saturates at the range ends and maps NaN to 0 (Rust `as`, since 1.45).
template <class S>
__device__ inline int64_t sat_to_i64(S v) {
  if (v != v) return 0;
  if (v >= S(9223372036854775808.0)) return INT64_MAX;
  if (v <= S(-9223372036854775808.0)) return INT64_MIN;
  return static_cast<int64_t>(v);
}
template <> struct CastF<float, int64_t> {
  __device__ int64_t operator()(float v) const { return sat_to_i64(v); }
};
template <> struct CastF<double, int64_t> {
  __device__ int64_t operator()(double v) const { return sat_to_i64(v); }
};
// real -> complex: re = src (through f64), im = +0 (cpu_cast_cplx, op_builder.rs:2127-2167);
// c64 -> c128 widens each component exactly (cpu_cast_c64_c128, op_builder.rs:2099-2125)
template <class S> struct CastF<S, musapy_c64_t> {
  __device__ musapy_c64_t operator()(S v) const { return musapy_c64_t{float(double(v)), 0.0f}; }
};
template <class S> struct CastF<S, musapy_c128_t> {
  __device__ musapy_c128_t operator()(S v) const { return musapy_c128_t{double(v), 0.0}; }
};
template <> struct CastF<musapy_c64_t, musapy_c128_t> {
  __device__ musapy_c128_t operator()(musapy_c64_t v) const { return musapy_c128_t{double(v.re), double(v.im)}; }
};

// f32 -> bfloat16 bits, round to nearest even.  NaN keeps sign and leading payload, quiet bit set.
struct ToBf16F {
  __device__ uint16_t operator()(float v) const {
    const uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);  // NaN: quiet, payload kept
    // v_cvt_pk_bf16_f32: round to nearest even, the same bits as (u + 0x7fff + lsb) >> 16
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  }
};

// f32 -> IEEE binary16 bits, round to nearest even.  Numbers go through v_cvt_f16_f32 (kernels
// run in the default FP mode: round to nearest even, binary16 subnormals kept), which measured
// 15.3 us for C3's 16M elements against 16.6 us for an integer restatement on the bit pattern;
// NaNs are built on the bit pattern.
struct ToF16F {
  __device__ uint16_t operator()(float v) const {
    const uint32_t u = __float_as_uint(v);
    const uint32_t a = u & 0x7fffffffu;
    // NaN: quiet, sign and the top 10 payload bits kept (the hardware conversion does not keep them)
    if (a > 0x7f800000u) return uint16_t(((u >> 16) & 0x8000u) | 0x7e00u | ((a >> 13) & 0x3ffu));
    // everything else: v_cvt_f16_f32, IEEE round-to-nearest-even with binary16 subnormals kept and
    // overflow to infinity -- the same bits as the integer RNE restatement of the oracle
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  }
};

}  // namespace mpy
