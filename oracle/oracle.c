/*
 * oracle.c -- CPU restatement of musapy's reference CPU path for the elementwise + reduction
 * hot path.  TEST INFRASTRUCTURE ONLY: it is the parity checker (tests/, the smoke check) and
 * the timed CPU baseline of bench.py; the product (musapy_amd) never links or calls it.
 *
 * Every function follows the `Device::Cpu` code of rust/musapy-ops/src/op_builder.rs line for
 * line in semantics (single-threaded, per-element `cpu_offset_nd`, same evaluation order):
 *   oracle_offset_nd       cpu_offset_nd            op_builder.rs:1581-1590
 *   oracle_binary_*        cpu_binary_typed/_op     op_builder.rs:1618-1626, 1734-1760
 *   oracle_unary_*         cpu_unary_elementwise    op_builder.rs:1868-1896, 1971-1993
 *   oracle_clamp_*         cpu_clamp_typed          op_builder.rs:2004-2047
 *   oracle_compare         cpu_comparison_elementwise / cpu_compare_typed / cpu_compare_cplx
 *                                                   op_builder.rs:1765-1864 (PartialEq/PartialOrd)
 *   oracle_binary_cplx     cpu_binary_cplx          op_builder.rs:1652-1731 (components in f64)
 *   oracle_unary_cplx      cpu_unary_elementwise complex arms + cpu_unary_cplx_abs
 *                                                   op_builder.rs:1904-1969
 *   oracle_cast (complex)  cpu_cast_cplx / cpu_cast_c64_c128  op_builder.rs:2080-2167
 *   oracle_copy_bytes      cpu_copy_bytes           rust/musapy-ops/src/indexing.rs:1388-1409
 *                          (contiguous / copy_into, indexing.rs:181-237, 816-916)
 *   oracle_cast            cpu_cast + cpu_cast_pair op_builder.rs:227-243, 2052-2097 (Rust `as`)
 *   oracle_reduce          cpu_reduce_offset/typed  op_builder.rs:3368-3394, 3496-3582
 *                          cpu_mean_typed           op_builder.rs:3585-3619
 *                          cpu_reduce_cplx          op_builder.rs:3439-3492
 *   oracle_cumsum          cpu_cumsum_typed         op_builder.rs:3640-3688 (literal O(L^2) form,
 *                          and the O(L) running sum, which adds in the same order)
 * Transcendentals call the platform libm (glibc), as Rust's f32::sin etc. do on Linux.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 *
 * Not in the reference (it rejects f16/bf16 casts, op_builder.rs:928-945): oracle_f32_to_f16 /
 * oracle_f32_to_bf16, IEEE-754 round-to-nearest-even evaluated in double arithmetic (a method
 * independent of the kernels' integer bit manipulation); pinned by numpy / torch vectors.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

int64_t oracle_offset_nd(size_t idx, const size_t* shape, const int64_t* strides, int ndim) {
  int64_t off = 0;
  for (int i = ndim - 1; i >= 0; --i) {
    size_t coord = idx % shape[i];
    idx /= shape[i];
    off += (int64_t)coord * strides[i];
  }
  return off;
}

static size_t numel(const size_t* shape, int ndim) {
  size_t n = 1;
  for (int i = 0; i < ndim; ++i) n *= shape[i];
  return n;
}

/* ---- binary ---- */
void oracle_binary_f32(int op, const float* a, const float* b, float* c, int ndim, const size_t* shape,
                       const int64_t* as, const int64_t* bs) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    float x = a[oracle_offset_nd(i, shape, as, ndim)], y = b[oracle_offset_nd(i, shape, bs, ndim)];
    float r;
    switch (op) {
      case ORACLE_ADD: r = x + y; break;
      case ORACLE_SUB: r = x - y; break;
      case ORACLE_MUL: r = x * y; break;
      case ORACLE_DIV: r = x / y; break;
      default: r = powf(x, y); break;
    }
    c[i] = r;
  }
}

void oracle_binary_f64(int op, const double* a, const double* b, double* c, int ndim, const size_t* shape,
                       const int64_t* as, const int64_t* bs) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    double x = a[oracle_offset_nd(i, shape, as, ndim)], y = b[oracle_offset_nd(i, shape, bs, ndim)];
    double r;
    switch (op) {
      case ORACLE_ADD: r = x + y; break;
      case ORACLE_SUB: r = x - y; break;
      case ORACLE_MUL: r = x * y; break;
      case ORACLE_DIV: r = x / y; break;
      default: r = pow(x, y); break;
    }
    c[i] = r;
  }
}

/* ---- complex elementwise: interleaved (re, im); CplxScalar reads both widths as f64 and
 * cplx_from_parts narrows with `as f32` (op_builder.rs:1655-1687) ---- */
static void cplx_load(int dtype, const void* p, int64_t off, double* re, double* im) {
  if (dtype == ORACLE_C64) {
    *re = ((const float*)p)[2 * off];
    *im = ((const float*)p)[2 * off + 1];
  } else {
    *re = ((const double*)p)[2 * off];
    *im = ((const double*)p)[2 * off + 1];
  }
}

static void cplx_store(int dtype, void* p, size_t i, double re, double im) {
  if (dtype == ORACLE_C64) {
    ((float*)p)[2 * i] = (float)re;
    ((float*)p)[2 * i + 1] = (float)im;
  } else {
    ((double*)p)[2 * i] = re;
    ((double*)p)[2 * i + 1] = im;
  }
}

void oracle_binary_cplx(int op, int dtype, const void* a, const void* b, void* c, int ndim, const size_t* shape,
                        const int64_t* as, const int64_t* bs) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    double ar, ai, br, bi, re, im;
    cplx_load(dtype, a, oracle_offset_nd(i, shape, as, ndim), &ar, &ai);
    cplx_load(dtype, b, oracle_offset_nd(i, shape, bs, ndim), &br, &bi);
    switch (op) {
      case ORACLE_ADD: re = ar + br; im = ai + bi; break;
      case ORACLE_SUB: re = ar - br; im = ai - bi; break;
      case ORACLE_MUL: re = ar * br - ai * bi; im = ar * bi + ai * br; break;
      default: { /* ORACLE_DIV */
        double den = br * br + bi * bi;
        re = (ar * br + ai * bi) / den;
        im = (ai * br - ar * bi) / den;
      }
    }
    cplx_store(dtype, c, i, re, im);
  }
}

/* op: ORACLE_NEG (complex output) or ORACLE_ABS (real output: f32 for c64, f64 for c128) */
void oracle_unary_cplx(int op, int dtype, const void* a, void* c, int ndim, const size_t* shape,
                       const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    int64_t off = oracle_offset_nd(i, shape, as, ndim);
    if (op == ORACLE_NEG) {
      /* the reference negates the stored components directly (no f64 round trip) */
      if (dtype == ORACLE_C64) {
        ((float*)c)[2 * i] = -((const float*)a)[2 * off];
        ((float*)c)[2 * i + 1] = -((const float*)a)[2 * off + 1];
      } else {
        ((double*)c)[2 * i] = -((const double*)a)[2 * off];
        ((double*)c)[2 * i + 1] = -((const double*)a)[2 * off + 1];
      }
    } else {
      double re, im;
      cplx_load(dtype, a, off, &re, &im);
      double r = sqrt(re * re + im * im);
      if (dtype == ORACLE_C64) ((float*)c)[i] = (float)r;
      else ((double*)c)[i] = r;
    }
  }
}

/* ---- comparisons: one 0/1 byte per element (op_builder.rs:1765-1864) ---- */
static int cmp_real(int op, double x, double y) {
  switch (op) {
    case ORACLE_EQ: return x == y;
    case ORACLE_NE: return x != y;
    case ORACLE_LT: return x < y;
    case ORACLE_GT: return x > y;
    case ORACLE_LE: return x <= y;
    default: return x >= y;
  }
}

void oracle_compare(int op, int dtype, const void* a, const void* b, uint8_t* c, int ndim, const size_t* shape,
                    const int64_t* as, const int64_t* bs) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    int64_t ao = oracle_offset_nd(i, shape, as, ndim), bo = oracle_offset_nd(i, shape, bs, ndim);
    int r;
    if (dtype == ORACLE_F32) {
      /* f32 compared as f32: widening to double is exact, so the order and NaN rules are kept */
      r = cmp_real(op, ((const float*)a)[ao], ((const float*)b)[bo]);
    } else if (dtype == ORACLE_F64) {
      r = cmp_real(op, ((const double*)a)[ao], ((const double*)b)[bo]);
    } else {
      double ar, ai, br, bi;
      if (dtype == ORACLE_C64) {
        ar = ((const float*)a)[2 * ao], ai = ((const float*)a)[2 * ao + 1];
        br = ((const float*)b)[2 * bo], bi = ((const float*)b)[2 * bo + 1];
      } else {
        ar = ((const double*)a)[2 * ao], ai = ((const double*)a)[2 * ao + 1];
        br = ((const double*)b)[2 * bo], bi = ((const double*)b)[2 * bo + 1];
      }
      /* complex: eq / ne only (ordering comparisons are rejected before dispatch) */
      r = op == ORACLE_EQ ? (ar == br && ai == bi) : (ar != br || ai != bi);
    }
    c[i] = (uint8_t)(r ? 1 : 0);
  }
}

/* ---- unary ---- */
void oracle_unary_f32(int op, const float* a, float* c, int ndim, const size_t* shape, const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    float v = a[oracle_offset_nd(i, shape, as, ndim)], r;
    switch (op) {
      case ORACLE_SIN: r = sinf(v); break;
      case ORACLE_COS: r = cosf(v); break;
      case ORACLE_EXP: r = expf(v); break;
      case ORACLE_LOG: r = logf(v); break;
      case ORACLE_ABS: r = fabsf(v); break;
      case ORACLE_SIGN: r = v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); break;
      default: r = -v; break;
    }
    c[i] = r;
  }
}

void oracle_unary_f64(int op, const double* a, double* c, int ndim, const size_t* shape, const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    double v = a[oracle_offset_nd(i, shape, as, ndim)], r;
    switch (op) {
      case ORACLE_SIN: r = sin(v); break;
      case ORACLE_COS: r = cos(v); break;
      case ORACLE_EXP: r = exp(v); break;
      case ORACLE_LOG: r = log(v); break;
      case ORACLE_ABS: r = fabs(v); break;
      case ORACLE_SIGN: r = v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : 0.0); break;
      default: r = -v; break;
    }
    c[i] = r;
  }
}

/* ---- clamp: v < lo ? lo : (v > hi ? hi : v); lo/hi arrive as f64 and are narrowed for f32 ---- */
void oracle_clamp_f32(const float* a, float* c, double lo, double hi, int ndim, const size_t* shape,
                      const int64_t* as) {
  const float l = (float)lo, h = (float)hi;
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    float v = a[oracle_offset_nd(i, shape, as, ndim)];
    c[i] = v < l ? l : (v > h ? h : v);
  }
}

void oracle_clamp_f64(const double* a, double* c, double lo, double hi, int ndim, const size_t* shape,
                      const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    double v = a[oracle_offset_nd(i, shape, as, ndim)];
    c[i] = v < lo ? lo : (v > hi ? hi : v);
  }
}

/* ---- casts: Rust `as` ---- */
static int64_t f64_as_i64(double v) { /* saturating, NaN -> 0 */
  if (v != v) return 0;
  if (v >= 9223372036854775808.0) return INT64_MAX;
  if (v <= -9223372036854775808.0) return INT64_MIN;
  return (int64_t)v;
}

static double load_as_f64(int t, const void* p, int64_t off, int* is_int, int64_t* iv, uint64_t* uv) {
  *is_int = 1;
  switch (t) {
    case ORACLE_I8: *iv = ((const int8_t*)p)[off]; return 0;
    case ORACLE_I16: *iv = ((const int16_t*)p)[off]; return 0;
    case ORACLE_I32: *iv = ((const int32_t*)p)[off]; return 0;
    case ORACLE_I64: *iv = ((const int64_t*)p)[off]; return 0;
    case ORACLE_U8: *is_int = 2; *uv = ((const uint8_t*)p)[off]; return 0;
    case ORACLE_U16: *is_int = 2; *uv = ((const uint16_t*)p)[off]; return 0;
    case ORACLE_U32: *is_int = 2; *uv = ((const uint32_t*)p)[off]; return 0;
    case ORACLE_U64: *is_int = 2; *uv = ((const uint64_t*)p)[off]; return 0;
    case ORACLE_F32: *is_int = 3; return ((const float*)p)[off];
    default: *is_int = 0; return ((const double*)p)[off];
  }
}

void oracle_cast(int src, int dst, const void* a, void* c, int ndim, const size_t* shape, const int64_t* as) {
  size_t n = numel(shape, ndim);
  if (dst == ORACLE_C64 || dst == ORACLE_C128) {
    /* real -> complex: re = src as f64 then narrowed by cplx_from_parts, im = +0;
     * c64 -> c128: each component widened */
    for (size_t i = 0; i < n; ++i) {
      int64_t off = oracle_offset_nd(i, shape, as, ndim);
      double re, im = 0.0;
      if (src == ORACLE_C64) cplx_load(src, a, off, &re, &im);
      else if (src == ORACLE_F32) re = ((const float*)a)[off];
      else re = ((const double*)a)[off];
      cplx_store(dst, c, i, re, im);
    }
    return;
  }
  for (size_t i = 0; i < n; ++i) {
    int64_t off = oracle_offset_nd(i, shape, as, ndim);
    int kind;
    int64_t iv = 0;
    uint64_t uv = 0;
    double fv = load_as_f64(src, a, off, &kind, &iv, &uv);
    if (dst == ORACLE_F32) {
      float r;
      if (kind == 1) r = (float)iv;          /* one rounding, RNE */
      else if (kind == 2) r = (float)uv;
      else if (kind == 3) r = ((const float*)a)[off];
      else r = (float)fv;                    /* f64 -> f32, RNE */
      ((float*)c)[i] = r;
    } else if (dst == ORACLE_F64) {
      double r;
      if (kind == 1) r = (double)iv;
      else if (kind == 2) r = (double)uv;
      else r = fv;
      ((double*)c)[i] = r;
    } else { /* ORACLE_I64 */
      int64_t r;
      if (kind == 1) r = iv;
      else if (kind == 2) r = (int64_t)uv;   /* u64 -> i64 wraps */
      else r = f64_as_i64(fv);               /* f32 values are exact in f64 */
      ((int64_t*)c)[i] = r;
    }
  }
}

/* f32 -> binary16 bits, RNE, evaluated on doubles with rint() (default rounding = to nearest even) */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  double x = fabs((double)f);
  if (f != f) return (uint16_t)(sign | 0x7e00u | ((u >> 13) & 0x3ffu));
  if (x >= 65520.0) return (uint16_t)(sign | 0x7c00u);
  if (x < 6.103515625e-05) { /* below 2^-14: multiples of 2^-24 */
    double q = rint(x * 16777216.0);
    return (uint16_t)(sign | (uint16_t)q);
  }
  int e;
  double m = frexp(x, &e);        /* x = m * 2^e, m in [0.5, 1) */
  double q = rint(m * 2048.0);    /* 11 significant bits */
  if (q == 2048.0) { q = 1024.0; e += 1; }
  int be = e - 1 + 15;            /* biased exponent of 1.f form */
  if (be >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (uint16_t)(be << 10) | (uint16_t)((int)q - 1024));
}

/* f32 -> bfloat16 bits, RNE, same approach (8 significant bits, exponent range of f32) */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  double x = fabs((double)f);
  if (f != f) return (uint16_t)((u >> 16) | 0x0040u);
  if (isinf(x)) return (uint16_t)(sign | 0x7f80u);
  if (x < ldexp(1.0, -126)) { /* subnormal range: multiples of 2^-133 */
    double q = rint(ldexp(x, 133));
    return (uint16_t)(sign | (uint16_t)q);
  }
  int e;
  double m = frexp(x, &e);
  double q = rint(m * 256.0);     /* 8 significant bits */
  if (q == 256.0) { q = 128.0; e += 1; }
  int be = e - 1 + 127;
  if (be >= 255) return (uint16_t)(sign | 0x7f80u);
  return (uint16_t)(sign | (uint16_t)(be << 7) | (uint16_t)((int)q - 128));
}

void oracle_cast_f32_f16(const float* a, uint16_t* c, int ndim, const size_t* shape, const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) c[i] = oracle_f32_to_f16(a[oracle_offset_nd(i, shape, as, ndim)]);
}

void oracle_cast_f32_bf16(const float* a, uint16_t* c, int ndim, const size_t* shape, const int64_t* as) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) c[i] = oracle_f32_to_bf16(a[oracle_offset_nd(i, shape, as, ndim)]);
}

/* ---- reductions ---- */
static size_t reduce_offset(size_t out_idx, const size_t* shape, const int64_t* strides, int ndim, int axis,
                            size_t k) {
  size_t coords[64];
  int ci = 0;
  size_t tmp = out_idx;
  for (int i = ndim - 1; i >= 0; --i) {
    if (i == axis) continue;
    coords[ci++] = tmp % shape[i];
    tmp /= shape[i];
  }
  int64_t off = 0;
  ci = 0;
  for (int i = ndim - 1; i >= 0; --i) {
    size_t coord = (i == axis) ? k : coords[ci++];
    off += (int64_t)coord * strides[i];
  }
  return (size_t)off;
}

#define REDUCE_BODY(T, ACC_T, CNT_T)                                                                        \
  do {                                                                                                      \
    const T* A = (const T*)a;                                                                               \
    for (size_t o = 0; o < out_size; ++o) {                                                                 \
      size_t base = reduce_offset(o, shape, strides, ndim, axis, 0);                                        \
      int64_t as = strides[axis];                                                                           \
      if (kind == ORACLE_SUM || kind == ORACLE_MEAN || kind == ORACLE_PROD) {                               \
        ACC_T acc = (kind == ORACLE_PROD) ? (ACC_T)1 : (ACC_T)0;                                            \
        for (size_t k = 0; k < axis_len; ++k) {                                                             \
          T v = A[(size_t)((int64_t)base + (int64_t)k * as)];                                               \
          acc = (kind == ORACLE_PROD) ? (ACC_T)(acc * (ACC_T)v) : (ACC_T)(acc + (ACC_T)v);                  \
        }                                                                                                   \
        if (kind == ORACLE_MEAN) {                                                                          \
          CNT_T cnt = 0;                                                                                    \
          for (size_t k = 0; k < axis_len; ++k) cnt = cnt + (CNT_T)1;                                       \
          ((T*)c)[o] = (T)(acc / cnt);                                                                      \
        } else {                                                                                            \
          ((T*)c)[o] = (T)acc;                                                                              \
        }                                                                                                   \
      } else {                                                                                              \
        int want_max = (kind == ORACLE_MAX || kind == ORACLE_ARGMAX);                                       \
        T best = A[base];                                                                                   \
        int64_t bi = 0;                                                                                     \
        for (size_t k = 1; k < axis_len; ++k) {                                                             \
          T v = A[(size_t)((int64_t)base + (int64_t)k * as)];                                               \
          if ((want_max && v > best) || (!want_max && v < best)) {                                          \
            best = v;                                                                                       \
            bi = (int64_t)k;                                                                                \
          }                                                                                                 \
        }                                                                                                   \
        if (kind == ORACLE_ARGMAX || kind == ORACLE_ARGMIN) ((int64_t*)c)[o] = bi;                          \
        else ((T*)c)[o] = best;                                                                             \
      }                                                                                                     \
    }                                                                                                       \
  } while (0)

void oracle_reduce(int kind, int dtype, const void* a, void* c, int ndim, const size_t* shape,
                   const int64_t* strides, int axis, size_t axis_len, size_t out_size) {
  if (out_size == 0 || axis_len == 0) return;
  switch (dtype) {
    case ORACLE_F32: REDUCE_BODY(float, float, float); break;
    case ORACLE_F64: REDUCE_BODY(double, double, double); break;
    case ORACLE_I64: {
      /* i64 sums/products wrap like release-mode Rust: evaluate in uint64_t */
      if (kind == ORACLE_SUM || kind == ORACLE_PROD) {
        const int64_t* A = (const int64_t*)a;
        for (size_t o = 0; o < out_size; ++o) {
          size_t base = reduce_offset(o, shape, strides, ndim, axis, 0);
          uint64_t acc = (kind == ORACLE_PROD) ? 1u : 0u;
          for (size_t k = 0; k < axis_len; ++k) {
            uint64_t v = (uint64_t)A[(size_t)((int64_t)base + (int64_t)k * strides[axis])];
            acc = (kind == ORACLE_PROD) ? acc * v : acc + v;
          }
          ((int64_t*)c)[o] = (int64_t)acc;
        }
      } else {
        REDUCE_BODY(int64_t, int64_t, int64_t);
      }
      break;
    }
    case ORACLE_C64:
    case ORACLE_C128: {
      /* cpu_reduce_cplx: f64 accumulation, one narrowing at the end */
      for (size_t o = 0; o < out_size; ++o) {
        size_t base = reduce_offset(o, shape, strides, ndim, axis, 0);
        double re = 0.0, im = 0.0;
        if (kind == ORACLE_PROD) re = 1.0;
        for (size_t k = 0; k < axis_len; ++k) {
          size_t off = (size_t)((int64_t)base + (int64_t)k * strides[axis]);
          double vr, vi;
          if (dtype == ORACLE_C64) {
            vr = ((const float*)a)[2 * off];
            vi = ((const float*)a)[2 * off + 1];
          } else {
            vr = ((const double*)a)[2 * off];
            vi = ((const double*)a)[2 * off + 1];
          }
          if (kind == ORACLE_PROD) {
            double ar = re, ai = im;
            re = ar * vr - ai * vi;
            im = ar * vi + ai * vr;
          } else {
            re += vr;
            im += vi;
          }
        }
        if (kind == ORACLE_MEAN) {
          re /= (double)axis_len;
          im /= (double)axis_len;
        }
        if (dtype == ORACLE_C64) {
          ((float*)c)[2 * o] = (float)re;
          ((float*)c)[2 * o + 1] = (float)im;
        } else {
          ((double*)c)[2 * o] = re;
          ((double*)c)[2 * o + 1] = im;
        }
      }
      break;
    }
  }
}

/* ---- cumsum ---- */
#define CUMSUM_BODY(T, ACC_T)                                                                               \
  do {                                                                                                      \
    const T* A = (const T*)a;                                                                               \
    T* C = (T*)c;                                                                                           \
    for (size_t idx = 0; idx < out_size; ++idx) {                                                           \
      size_t tmp = idx, axis_coord = 0;                                                                     \
      for (int i = ndim - 1; i >= 0; --i) {                                                                 \
        size_t coord = tmp % shape[i];                                                                      \
        tmp /= shape[i];                                                                                    \
        if (i == axis) axis_coord = coord;                                                                  \
      }                                                                                                     \
      int64_t base_off = 0;                                                                                 \
      tmp = idx;                                                                                            \
      for (int i = ndim - 1; i >= 0; --i) {                                                                 \
        size_t coord = tmp % shape[i];                                                                      \
        tmp /= shape[i];                                                                                    \
        if (i != axis) base_off += (int64_t)coord * strides[i];                                             \
      }                                                                                                     \
      if (literal) {                                                                                        \
        ACC_T acc = 0;                                                                                      \
        for (size_t k = 0; k <= axis_coord; ++k)                                                            \
          acc = acc + (ACC_T)A[(size_t)(base_off + (int64_t)k * strides[axis])];                            \
        C[idx] = (T)acc;                                                                                    \
      } else {                                                                                              \
        /* running sum: the same additions in the same order, reusing the previous prefix */                \
        if (axis_coord == 0) {                                                                              \
          C[idx] = (T)((ACC_T)0 + (ACC_T)A[(size_t)base_off]);                                              \
        } else {                                                                                            \
          C[idx] = (T)((ACC_T)C[idx - out_stride] + (ACC_T)A[(size_t)(base_off + (int64_t)axis_coord * strides[axis])]); \
        }                                                                                                   \
      }                                                                                                     \
    }                                                                                                       \
  } while (0)

void oracle_cumsum(int dtype, int literal, const void* a, void* c, int ndim, const size_t* shape,
                   const int64_t* strides, int axis, size_t out_size) {
  if (out_size == 0) return;
  size_t out_stride = 1; /* output (C-order) stride of the scanned axis */
  for (int i = ndim - 1; i > axis; --i) out_stride *= shape[i];
  switch (dtype) {
    case ORACLE_F32: CUMSUM_BODY(float, float); break;
    case ORACLE_F64: CUMSUM_BODY(double, double); break;
    default: CUMSUM_BODY(int64_t, uint64_t); break;
  }
}

/* ---- view materialisation: byte gather of each element in C order ---- */
void oracle_copy_bytes(const void* in, void* out, int ndim, const size_t* shape, const int64_t* strides,
                       size_t elem_size) {
  size_t n = numel(shape, ndim);
  for (size_t i = 0; i < n; ++i) {
    int64_t off = oracle_offset_nd(i, shape, strides, ndim);
    memcpy((char*)out + i * elem_size, (const char*)in + off * (int64_t)elem_size, elem_size);
  }
}
