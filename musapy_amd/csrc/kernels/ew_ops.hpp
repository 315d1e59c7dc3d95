// ew_ops.hpp -- per-element functors of the elementwise path.
//
// Semantics follow the reference's CPU path, which is the parity oracle:
//   binary  cpu_binary_op          rust/musapy-ops/src/op_builder.rs:1618-1626
//   unary   cpu_unary_elementwise  op_builder.rs:1868-1896 (sign: v>0 -> 1, v<0 -> -1, else +0)
//   clamp   cpu_clamp_typed        op_builder.rs:2017-2047 (v<lo ? lo : v>hi ? hi : v; NaN passes)
//   cast    cpu_cast_pair!         op_builder.rs:227-243   (Rust `as`)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

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

// f32 -> bfloat16 bits, round to nearest even.  NaN keeps sign and leading payload, quiet bit set.
struct ToBf16F {
  __device__ uint16_t operator()(float v) const {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);
    return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
};

// f32 -> IEEE binary16 bits, round to nearest even, computed on the bit pattern so the result
// does not depend on the FP mode registers.
struct ToF16F {
  __device__ uint16_t operator()(float v) const {
    uint32_t u = __float_as_uint(v);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return uint16_t(sign | 0x7e00u | ((a >> 13) & 0x3ffu));  // NaN
    if (a >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // >= 65520 rounds to inf
    if (a >= 0x38800000u) {  // normal binary16 range (>= 2^-14)
      uint32_t r = a - 0x38000000u;  // rebias exponent 127 -> 15
      r = (r + 0xfffu + ((r >> 13) & 1u)) >> 13;
      return uint16_t(sign | r);
    }
    if (a <= 0x33000000u) return uint16_t(sign);  // <= 2^-25: ties-to-even gives 0
    uint32_t e = a >> 23;                      // 103..112
    uint32_t m = (a & 0x7fffffu) | 0x800000u;  // value = m * 2^(e-150)
    uint32_t sh = 126u - e;                    // quantum 2^-24  ->  q = m >> (126 - e)
    uint32_t q = m >> sh;
    uint32_t rem = m & ((1u << sh) - 1u);
    uint32_t half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return uint16_t(sign | q);
  }
};

}  // namespace mpy
