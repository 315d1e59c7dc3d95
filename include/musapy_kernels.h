/*
 * musapy_kernels.h -- C ABI of the MI355X (gfx950) elementwise / reduction / scan kernels.
 *
 * This is the drop-in boundary for musapy's stride-aware hot path.  Every symbol below has the
 * exact name and argument list that musapy's Rust op layer binds in
 * rust/musapy-ops/src/kernels.rs (the `unsafe extern "C"` block, lines 16-346); the line of
 * kernels.rs each declaration replaces is given beside it.  `musaStream_t` becomes `hipStream_t`
 * (both are opaque pointers), `muComplex`/`muDoubleComplex` become musapy_c64_t/musapy_c128_t
 * (same #[repr(C)] {re, im} layout, rust/musapy-core/src/musa_x_ffi.rs:74-89).
 *
 * Conventions (rust/musapy-ops/src/kernels.rs:6-9, docs/adr/ADR.md L2-2):
 *  - functions return void and never allocate; launch errors are read with hipGetLastError()
 *    right after the call, execution errors surface at stream synchronisation;
 *  - data pointers are device pointers already advanced by the view offset;
 *  - `shape` / `*_strides` are HOST arrays (elements, strides may be 0 or negative) that are only
 *    read during the call; the output is always C-contiguous and never aliases an input;
 *  - all launches are asynchronous on `stream`.
 * Reduction partial/final/mid contract (rust/musapy-ops/src/op_builder.rs:2239-2301,2523):
 *  partials are laid out [out_size][tiles_per_output]; tile t of output o covers the axis range
 *  [t*ceil(axis_len/tiles), (t+1)*ceil(axis_len/tiles)); any tiles_per_output >= 1 is accepted.
 */
#ifndef MUSAPY_KERNELS_H
#define MUSAPY_KERNELS_H

#include <stddef.h>
#include <stdint.h>
#include <sys/types.h>

/* same typedef as <hip/hip_runtime_api.h>; repeating an identical typedef is valid C11/C++ */
typedef struct ihipStream_t* hipStream_t;

#define MUSAPY_KERNELS_ABI_VERSION 2

#ifdef __cplusplus
extern "C" {
#endif

/* interleaved complex element, layout-identical to muComplex / muDoubleComplex */
typedef struct { float re; float im; } musapy_c64_t;
typedef struct { double re; double im; } musapy_c128_t;


/* ---- binary elementwise over broadcast strides ---- */
/* kernels.rs:19 */ void musapy_add_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:20 */ void musapy_add_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:21 */ void musapy_sub_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:22 */ void musapy_sub_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:23 */ void musapy_mul_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:24 */ void musapy_mul_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:25 */ void musapy_div_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:26 */ void musapy_div_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:27 */ void musapy_pow_f32_v2(const float* a, const float* b, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:28 */ void musapy_pow_f64_v2(const double* a, const double* b, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);

/* ---- unary elementwise ---- */
/* kernels.rs:31 */ void musapy_sin_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:32 */ void musapy_sin_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:33 */ void musapy_cos_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:34 */ void musapy_cos_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:35 */ void musapy_exp_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:36 */ void musapy_exp_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:37 */ void musapy_log_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:38 */ void musapy_log_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:39 */ void musapy_abs_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:40 */ void musapy_abs_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:41 */ void musapy_sign_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:42 */ void musapy_sign_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:43 */ void musapy_neg_f32_v2(const float* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:44 */ void musapy_neg_f64_v2(const double* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);

/* ---- clamp ---- */
/* kernels.rs:47 */ void musapy_clamp_f32_v2(const float* a, float* c, float lo, float hi, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:48 */ void musapy_clamp_f64_v2(const double* a, double* c, double lo, double hi, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);

/* ---- cast (Rust `as` semantics: RNE to float, saturating float->int, NaN->0) ---- */
/* kernels.rs:51 */ void musapy_cast_i8_f32_v2(const int8_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:52 */ void musapy_cast_i16_f32_v2(const int16_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:53 */ void musapy_cast_i32_f32_v2(const int* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:54 */ void musapy_cast_i64_f32_v2(const int64_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:55 */ void musapy_cast_u8_f32_v2(const uint8_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:56 */ void musapy_cast_u16_f32_v2(const uint16_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:57 */ void musapy_cast_u32_f32_v2(const uint32_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:58 */ void musapy_cast_u64_f32_v2(const uint64_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:59 */ void musapy_cast_f64_f32_v2(const double* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:62 */ void musapy_cast_i8_f64_v2(const int8_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:63 */ void musapy_cast_i16_f64_v2(const int16_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:64 */ void musapy_cast_i32_f64_v2(const int* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:65 */ void musapy_cast_i64_f64_v2(const int64_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:66 */ void musapy_cast_u8_f64_v2(const uint8_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:67 */ void musapy_cast_u16_f64_v2(const uint16_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:68 */ void musapy_cast_u32_f64_v2(const uint32_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:69 */ void musapy_cast_u64_f64_v2(const uint64_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:70 */ void musapy_cast_f32_f64_v2(const float* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:73 */ void musapy_cast_i8_i64_v2(const int8_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:74 */ void musapy_cast_i16_i64_v2(const int16_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:75 */ void musapy_cast_i32_i64_v2(const int* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:76 */ void musapy_cast_u8_i64_v2(const uint8_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:77 */ void musapy_cast_u16_i64_v2(const uint16_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:78 */ void musapy_cast_u32_i64_v2(const uint32_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:79 */ void musapy_cast_u64_i64_v2(const uint64_t* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:80 */ void musapy_cast_f32_i64_v2(const float* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:81 */ void musapy_cast_f64_i64_v2(const double* a, int64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);

/* New in this backend (no counterpart in kernels.rs: musapy rejects f16/bf16 casts in
 * validate_cast_pair, rust/musapy-ops/src/op_builder.rs:928-945).  Output is the raw
 * IEEE binary16 / bfloat16 bit pattern, round-to-nearest-even; NaN stays NaN with its sign
 * and leading payload bits and the quiet bit set; overflow rounds to +-inf. */
void musapy_cast_f32_bf16_v2(const float* a, uint16_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
void musapy_cast_f32_f16_v2(const float* a, uint16_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);

/* ---- comparison elementwise: 0/1 bytes over broadcast strides (IEEE: NaN compares unequal) ---- */
/* kernels.rs:84 */ void musapy_eq_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:85 */ void musapy_eq_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:86 */ void musapy_ne_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:87 */ void musapy_ne_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:88 */ void musapy_lt_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:89 */ void musapy_lt_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:90 */ void musapy_gt_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:91 */ void musapy_gt_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:92 */ void musapy_le_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:93 */ void musapy_le_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:94 */ void musapy_ge_f32_v2(const float* a, const float* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:95 */ void musapy_ge_f64_v2(const double* a, const double* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* complex: equal when both the real and the imaginary parts are equal */
/* kernels.rs:114 */ void musapy_eq_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:115 */ void musapy_eq_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:116 */ void musapy_ne_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:117 */ void musapy_ne_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, uint8_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);

/* ---- complex elementwise over interleaved re/im elements ----
 * Component formulas evaluated in f64 without fma contraction; c64 results narrowed once. */
/* kernels.rs:102 */ void musapy_add_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:103 */ void musapy_add_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:104 */ void musapy_sub_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:105 */ void musapy_sub_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:106 */ void musapy_mul_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:107 */ void musapy_mul_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:108 */ void musapy_div_c64_v2(const musapy_c64_t* a, const musapy_c64_t* b, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:109 */ void musapy_div_c128_v2(const musapy_c128_t* a, const musapy_c128_t* b, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);
/* kernels.rs:110 */ void musapy_neg_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:111 */ void musapy_neg_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:112 */ void musapy_abs_c64_v2(const musapy_c64_t* a, float* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:113 */ void musapy_abs_c128_v2(const musapy_c128_t* a, double* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* real -> complex (re = src, im = +0) and c64 -> c128 */
/* kernels.rs:119 */ void musapy_cast_f32_c64_v2(const float* a, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:120 */ void musapy_cast_f32_c128_v2(const float* a, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:121 */ void musapy_cast_f64_c64_v2(const double* a, musapy_c64_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:122 */ void musapy_cast_f64_c128_v2(const double* a, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);
/* kernels.rs:124 */ void musapy_cast_c64_c128_v2(const musapy_c64_t* a, musapy_c128_t* c, int ndim, const size_t* shape, const ssize_t* a_strides, hipStream_t stream);

/* ---- reduction (single pass) ---- */
/* kernels.rs:139 */ void musapy_sum_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:140 */ void musapy_sum_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:141 */ void musapy_sum_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:142 */ void musapy_prod_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:143 */ void musapy_prod_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:144 */ void musapy_prod_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:145 */ void musapy_max_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:146 */ void musapy_max_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:147 */ void musapy_max_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:148 */ void musapy_min_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:149 */ void musapy_min_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:150 */ void musapy_min_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:151 */ void musapy_mean_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:152 */ void musapy_mean_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:154 */ void musapy_sum_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:155 */ void musapy_sum_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:156 */ void musapy_prod_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:157 */ void musapy_prod_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:158 */ void musapy_mean_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:159 */ void musapy_mean_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);

/* ---- small-axis reduction (group_size is a hint) ---- */
/* kernels.rs:161 */ void musapy_sum_small_axis_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:162 */ void musapy_sum_small_axis_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:163 */ void musapy_sum_small_axis_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:164 */ void musapy_prod_small_axis_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:165 */ void musapy_prod_small_axis_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:166 */ void musapy_prod_small_axis_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:167 */ void musapy_max_small_axis_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:168 */ void musapy_max_small_axis_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:169 */ void musapy_max_small_axis_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:170 */ void musapy_min_small_axis_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:171 */ void musapy_min_small_axis_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:172 */ void musapy_min_small_axis_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:173 */ void musapy_mean_small_axis_f32_v2(const float* a, float* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:174 */ void musapy_mean_small_axis_f64_v2(const double* a, double* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);

/* ---- arg reduction (single pass) ---- */
/* kernels.rs:175 */ void musapy_argmax_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:176 */ void musapy_argmax_f32_v2(const float* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:177 */ void musapy_argmax_f64_v2(const double* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:178 */ void musapy_argmin_i64_v2(const int64_t* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:179 */ void musapy_argmin_f32_v2(const float* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:180 */ void musapy_argmin_f64_v2(const double* a, int64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);

/* ---- cumsum (inclusive scan along one axis; tmp = caller scratch of num_rows*(bpr [+ceil(bpr/256) if bpr>256]) elements, bpr=ceil(axis_len/256), may be NULL when bpr<=1) ----
 * A scan whose rows are split into tiles waits on other workgroups; those waits report to the
 * fault word in the last 8 bytes of that scratch capacity (the workspace rule below), which the
 * launch zeroes first: read it with musapy_kernels_take_fault_ws(tmp, capacity_bytes, stream)
 * after synchronizing, before tmp is reused or freed. */
/* kernels.rs:185 */ void musapy_cumsum_i64_v3(const int64_t* a, int64_t* c, int64_t* tmp, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:186 */ void musapy_cumsum_f32_v3(const float* a, float* c, float* tmp, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);
/* kernels.rs:187 */ void musapy_cumsum_f64_v3(const double* a, double* c, double* tmp, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, hipStream_t stream);

/* ---- reduction partial ---- */
/* kernels.rs:222 */ void musapy_sum_partial_i64_v2(const int64_t* a, int64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:223 */ void musapy_sum_partial_f32_v2(const float* a, float* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:224 */ void musapy_sum_partial_f64_v2(const double* a, double* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:225 */ void musapy_prod_partial_i64_v2(const int64_t* a, int64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:226 */ void musapy_prod_partial_f32_v2(const float* a, float* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:227 */ void musapy_prod_partial_f64_v2(const double* a, double* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:228 */ void musapy_max_partial_i64_v2(const int64_t* a, int64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:229 */ void musapy_max_partial_f32_v2(const float* a, float* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:230 */ void musapy_max_partial_f64_v2(const double* a, double* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:231 */ void musapy_min_partial_i64_v2(const int64_t* a, int64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:232 */ void musapy_min_partial_f32_v2(const float* a, float* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:233 */ void musapy_min_partial_f64_v2(const double* a, double* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:235 */ void musapy_mean_partial_f32_v2(const float* a, float* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:236 */ void musapy_mean_partial_f64_v2(const double* a, double* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);

/* ---- reduction final ---- */
/* kernels.rs:240 */ void musapy_sum_final_i64_v2(const int64_t* partials, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:241 */ void musapy_sum_final_f32_v2(const float* partials, float* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:242 */ void musapy_sum_final_f64_v2(const double* partials, double* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:243 */ void musapy_prod_final_i64_v2(const int64_t* partials, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:244 */ void musapy_prod_final_f32_v2(const float* partials, float* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:245 */ void musapy_prod_final_f64_v2(const double* partials, double* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:246 */ void musapy_max_final_i64_v2(const int64_t* partials, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:247 */ void musapy_max_final_f32_v2(const float* partials, float* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:248 */ void musapy_max_final_f64_v2(const double* partials, double* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:249 */ void musapy_min_final_i64_v2(const int64_t* partials, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:250 */ void musapy_min_final_f32_v2(const float* partials, float* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:251 */ void musapy_min_final_f64_v2(const double* partials, double* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:254 */ void musapy_mean_final_f32_v2(const float* partials, float* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:255 */ void musapy_mean_final_f64_v2(const double* partials, double* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);

/* ---- small-axis reduction (group_size is a hint) ---- */
/* kernels.rs:259 */ void musapy_sum_small_axis_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:260 */ void musapy_sum_small_axis_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:261 */ void musapy_prod_small_axis_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:262 */ void musapy_prod_small_axis_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:263 */ void musapy_mean_small_axis_c64_v2(const musapy_c64_t* a, musapy_c64_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);
/* kernels.rs:264 */ void musapy_mean_small_axis_c128_v2(const musapy_c128_t* a, musapy_c128_t* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, int group_size, hipStream_t stream);

/* ---- reduction partial ---- */
/* kernels.rs:265 */ void musapy_sum_partial_c64_v2(const musapy_c64_t* a, musapy_c64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:266 */ void musapy_sum_partial_c128_v2(const musapy_c128_t* a, musapy_c128_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:267 */ void musapy_prod_partial_c64_v2(const musapy_c64_t* a, musapy_c64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:268 */ void musapy_prod_partial_c128_v2(const musapy_c128_t* a, musapy_c128_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:269 */ void musapy_mean_partial_c64_v2(const musapy_c64_t* a, musapy_c64_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:270 */ void musapy_mean_partial_c128_v2(const musapy_c128_t* a, musapy_c128_t* partials, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);

/* ---- reduction final ---- */
/* kernels.rs:271 */ void musapy_sum_final_c64_v2(const musapy_c64_t* partials, musapy_c64_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:272 */ void musapy_sum_final_c128_v2(const musapy_c128_t* partials, musapy_c128_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:273 */ void musapy_prod_final_c64_v2(const musapy_c64_t* partials, musapy_c64_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:274 */ void musapy_prod_final_c128_v2(const musapy_c128_t* partials, musapy_c128_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:275 */ void musapy_mean_final_c64_v2(const musapy_c64_t* partials, musapy_c64_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);
/* kernels.rs:276 */ void musapy_mean_final_c128_v2(const musapy_c128_t* partials, musapy_c128_t* c, size_t num_partials, size_t out_size, size_t axis_len, hipStream_t stream);

/* ---- reduction partial ---- */
/* kernels.rs:280 */ void musapy_argmax_partial_i64_v2(const int64_t* a, int64_t* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:281 */ void musapy_argmax_partial_f32_v2(const float* a, float* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:282 */ void musapy_argmax_partial_f64_v2(const double* a, double* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:283 */ void musapy_argmin_partial_i64_v2(const int64_t* a, int64_t* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:284 */ void musapy_argmin_partial_f32_v2(const float* a, float* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);
/* kernels.rs:285 */ void musapy_argmin_partial_f64_v2(const double* a, double* partials_val, int64_t* partials_idx, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles_per_output, hipStream_t stream);

/* ---- reduction final ---- */
/* kernels.rs:289 */ void musapy_argmax_final_i64_v2(const int64_t* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:290 */ void musapy_argmax_final_f32_v2(const float* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:291 */ void musapy_argmax_final_f64_v2(const double* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:292 */ void musapy_argmin_final_i64_v2(const int64_t* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:293 */ void musapy_argmin_final_f32_v2(const float* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);
/* kernels.rs:294 */ void musapy_argmin_final_f64_v2(const double* partials_val, const int64_t* partials_idx, int64_t* c, size_t num_partials, size_t out_size, hipStream_t stream);

/* ---- arg reduction mid level ---- */
/* kernels.rs:299 */ void musapy_argmax_mid_i64_v2(const int64_t* partials_val, const int64_t* partials_idx, int64_t* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);
/* kernels.rs:300 */ void musapy_argmax_mid_f32_v2(const float* partials_val, const int64_t* partials_idx, float* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);
/* kernels.rs:301 */ void musapy_argmax_mid_f64_v2(const double* partials_val, const int64_t* partials_idx, double* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);
/* kernels.rs:302 */ void musapy_argmin_mid_i64_v2(const int64_t* partials_val, const int64_t* partials_idx, int64_t* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);
/* kernels.rs:303 */ void musapy_argmin_mid_f32_v2(const float* partials_val, const int64_t* partials_idx, float* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);
/* kernels.rs:304 */ void musapy_argmin_mid_f64_v2(const double* partials_val, const int64_t* partials_idx, double* out_val, int64_t* out_idx, size_t out_size, size_t tiles_per_output, size_t axis_len, hipStream_t stream);

/* ---- view materialisation: stride-aware copy into a C-contiguous buffer ---- */
/* kernels.rs:321 */ void musapy_copy_f32(const float* input, float* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
/* kernels.rs:322 */ void musapy_copy_f64(const double* input, double* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
/* kernels.rs:323 */ void musapy_copy_i32(const int32_t* input, int32_t* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
/* kernels.rs:324 */ void musapy_copy_i64(const int64_t* input, int64_t* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
/* new: 1-, 2- and 16-byte element copies (bool/int8/uint8; int16/uint16/float16/bfloat16; complex128) */
void musapy_copy_u8(const uint8_t* input, uint8_t* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
void musapy_copy_u16(const uint16_t* input, uint16_t* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
void musapy_copy_c128(const musapy_c128_t* input, musapy_c128_t* output, int ndim, const size_t* shape, const ssize_t* in_strides, hipStream_t stream);
/* 2-D transpose materialisation: src is C-contiguous (cols, rows); dst[r*cols + c] = src[c*rows + r] */
/* kernels.rs:327 */ void musapy_copy_transpose2d_f32(const float* src, float* dst, size_t rows, size_t cols, hipStream_t stream);
/* kernels.rs:328 */ void musapy_copy_transpose2d_f64(const double* src, double* dst, size_t rows, size_t cols, hipStream_t stream);
/* kernels.rs:329 */ void musapy_copy_transpose2d_i32(const int32_t* src, int32_t* dst, size_t rows, size_t cols, hipStream_t stream);
/* kernels.rs:330 */ void musapy_copy_transpose2d_i64(const int64_t* src, int64_t* dst, size_t rows, size_t cols, hipStream_t stream);

/* ---- fused mixed-dtype binary (new; no counterpart in kernels.rs) ----
 * c = op(C(a), C(b)) where C(x) is the Rust `as` cast to c_dtype used by the cast kernels above:
 * bit-identical to musapy's cast-then-compute promotion path (op_builder.rs:410-417, 1055-1119)
 * in one pass instead of two.  Supported (a, b) -> c triples: one of a/b already has dtype c,
 * the other is int32/int64/float32/float64, c is float32/float64.  Returns 0 when launched,
 * -1 when the triple is not supported (nothing is launched; use the cast + binary symbols). */
enum {
  MUSAPY_DT_BOOL = 0, MUSAPY_DT_I8, MUSAPY_DT_I16, MUSAPY_DT_I32, MUSAPY_DT_I64, MUSAPY_DT_U8, MUSAPY_DT_U16,
  MUSAPY_DT_U32, MUSAPY_DT_U64, MUSAPY_DT_F16, MUSAPY_DT_F32, MUSAPY_DT_F64, MUSAPY_DT_BF16, MUSAPY_DT_C64,
  MUSAPY_DT_C128
};
enum { MUSAPY_OP_ADD = 0, MUSAPY_OP_SUB, MUSAPY_OP_MUL, MUSAPY_OP_DIV, MUSAPY_OP_POW };
int musapy_binary_mixed_v2(int op, const void* a, int a_dtype, const void* b, int b_dtype, void* c, int c_dtype, int ndim, const size_t* shape, const ssize_t* a_strides, const ssize_t* b_strides, hipStream_t stream);

/* ---- workspaces of the entry points below (new; no counterpart in kernels.rs) ----
 * A `workspace` is device memory, 8-byte aligned, of `workspace_bytes` bytes.  Its last 8-byte
 * word is the workspace's fault word (the first 4 bytes of that word, at offset
 * (workspace_bytes - 8) rounded down to a multiple of 8); everything before it is payload (slots,
 * counters, prefixes).  Launches that wait on other workgroups report an expired wait in the
 * fault word of the workspace they were given, so each caller (stream) reads its own faults
 * with musapy_kernels_take_fault_ws.  A workspace must be zero before its first use; the
 * launches leave the payload zero, and the fault word holds faults until they are taken.
 *
 * ---- single-launch reduction (new; no counterpart in kernels.rs) ----
 * The `_partial_` + `_final_` (`_mid_`) pair in one launch, for a reduction split into `tiles`
 * tiles:
 *  - a unit-stride axis with tiles of at least 16 KB and at most 64 outputs: every (output,
 *    tile) block publishes its tile's result into `workspace`, and a combiner block per output,
 *    dispatched after them, folds the results in a fixed order;
 *  - SUM, PROD and MEAN along a strided axis whose outputs are unit-stride (column reductions):
 *    the column kernel's (column group, tile) blocks publish their per-column results and count
 *    themselves per group; the block that completes a group's count folds its tiles in order.
 * Either way the result is independent of block timing.  `c` receives the values (the int64
 * indices for ARGMAX/ARGMIN); `dtype` is the compute dtype (F32, F64 or I64 for every op; C64 and
 * C128 for SUM, PROD and MEAN; MEAN takes a floating or complex dtype).  The payload of
 * `workspace` must hold out_size*tiles*W 64-bit words (W = 1 for f32 sum/prod/mean, 2 for f64/i64 sum/prod/mean and
 * f32 max/min/arg, 4 for f64/i64 max/min/arg and every complex op; column reductions: groups *
 * tiles * 64*V*W words, V columns of 16 bytes per lane, plus one 32-bit counter per group, where
 * groups = out_size / (64*V) rounded up per row of outputs), must be zero before the first call,
 * and is left zero by every call; calls that share a workspace must be ordered (one stream).
 * Returns 0 when launched, -1 when the case is not covered or `workspace` is too small (nothing
 * launched; use the partial + final entry points). */
enum { MUSAPY_RED_SUM = 0, MUSAPY_RED_PROD, MUSAPY_RED_MAX, MUSAPY_RED_MIN, MUSAPY_RED_MEAN, MUSAPY_RED_ARGMAX,
       MUSAPY_RED_ARGMIN };
int musapy_reduce_fused_v1(int op, int dtype, const void* a, void* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- cumsum on a zeroed workspace (new; no counterpart in kernels.rs) ----
 * The chained scan of musapy_cumsum_*_v3 for many (>= 512) unit-stride rows of several tiles,
 * with its per-tile prefixes in `workspace` instead of the reference's scratch `tmp`: the
 * workspace follows the rule above (zero before the call, payload left zero: each prefix is
 * returned to zero by the tile that reads it), so no clearing launch is needed.  Its payload
 * needs rows * tiles * W 64-bit words
 * (W = 1 for f32, 2 for f64/i64; a tile is 64 KB, 16384 f32 or 8192 f64/i64 elements, when a row
 * holds at least two such tiles, else 16 KB, 4096 f32 or 2048 f64/i64 elements).  `dtype` is
 * MUSAPY_DT_I64, _F32 or _F64.  Returns 0 when launched, -1 when the call does not take that path
 * or the workspace is too small (nothing launched: use musapy_cumsum_ws_v2 or _v3).  Calls that
 * share a workspace must be ordered.
 * musapy_cumsum_ws_v2: every cumsum, with its waits reported to the fault word of `workspace`:
 * the chained scan on the workspace's payload when it fits (else on `tmp`, cleared first), the
 * look-back of fewer rows on `tmp` (its claim counter and status words, cleared by the launch),
 * the sequential scan of a strided axis with neither.  `tmp` may be NULL when the shape takes
 * no scratch; a `tmp` of the _v3 formula's capacity always suffices.  Returns 0 when launched, -1
 * when not (wrapper error 1: tmp missing or too small for the path taken; 3 or 4 as for _v3). */
int musapy_cumsum_ws_v1(int dtype, const void* a, void* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, void* workspace, size_t workspace_bytes, hipStream_t stream);
int musapy_cumsum_ws_v2(int dtype, const void* a, void* c, void* tmp, size_t tmp_bytes, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- max / min over both axes of a 2-D array in one launch (new; no counterpart in kernels.rs) ----
 * `a` is a C-contiguous (rows, cols) array of the compute dtype (F32, F64 or I64), and `c`
 * receives one value.  The result is bit for bit what the reference's per-axis
 * passes give (rust/musapy-ops/src/reduction.rs:118-155: axis 0 with keepdims, then axis 1), NaN
 * and signed-zero outcomes included: the first extreme element in column-major order, among the
 * non-NaN elements of the columns whose row-0 element is not NaN, or a[0][0] when that is NaN.
 * `op` is MUSAPY_RED_MAX or MUSAPY_RED_MIN; `workspace` follows the workspace rule above.  f32
 * arrays with cols >= 2048 (a multiple of 4, 16-byte aligned, rows * cols < 2^32 - 1) run as keyed
 * rows and use (2048 + rows) 64-bit words of payload; other
 * shapes use the column tiling and at most 1024 slots of 4 words.  Returns 0 when launched, -1
 * when not covered (more than 1024 groups of 64 16-byte column vectors, or rows >= 2^31): then
 * reduce per axis. */
int musapy_reduce_2d_ordered_v1(int op, int dtype, const void* a, void* c, size_t rows, size_t cols, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- single-launch reduction that allocates nothing (new; no counterpart in kernels.rs) ----
 * For callers that cannot call hipMalloc: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  Same operation, arguments and results as
 * musapy_reduce_fused_v1, without `workspace`: the slots live in a static device array of the
 * library, 1 MiB of payload plus a 256-byte line ending in its fault word (one per GPU, held until
 * the process ends, zero when the code object loads, left zero by every call).  The caller still
 * passes the input and the output.  Returns 0 when launched, -1 when the case is not covered
 * (nothing launched), -2 when its slots need more than the 1 MiB the array holds (out_size *
 * tiles * W words of 8 bytes, or the column layout's words and counters, W as above; nothing
 * launched, wrapper error 5).  Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (concurrent streams or host threads) race and must be ordered by the caller.  Its
 * expired waits are read with musapy_kernels_take_fault(device); after one, the next call zeroes
 * the array first, on that call's stream. */
int musapy_reduce_fused_noalloc_v1(int op, int dtype, const void* a, void* c, int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t tiles, hipStream_t stream);

/* ---- wrapper-level error (new; no counterpart in kernels.rs) ----
 * Returns and clears the calling thread's last wrapper error: 0 none, 1 a cumsum scratch buffer
 * that is NULL or smaller than the reference's scratch formula requires, 2 a reduction whose
 * per-tile length reaches 2^31 elements (pass more tiles), 3 ndim outside [0, 32] or an axis
 * outside [0, ndim) (32 is the reference's MUSAPY_MAX_NDIM), 4 a cumsum with 2^32 or more rows
 * (or a dimension outside the scanned axis of 2^32 or more), 5 a no-alloc reduction whose slots
 * need more than the library's static scratch.  A wrapper that reports an error launches
 * nothing. */
int musapy_kernels_take_error(void);

/* ---- device wait faults (new; no counterpart in kernels.rs) ----
 * Three kernels wait for another workgroup's result: the combiners of the single-launch
 * reductions, the look-back of a cumsum whose rows are split into tiles and the predecessor
 * wait of the chained scan.  Each wait polls a bounded number of times; when that runs out, the
 * kernel records a fault in the fault word of the workspace (or scratch) its launch was given,
 * does not write a result it cannot trust (a reduction skips its output; a scan carries on with
 * a zero prefix), and exits normally.  Results of the work queued on that workspace since the
 * last check are then invalid, as after a failed kernel: the reference surfaces such errors at
 * the synchronisation of the stream that ran the work (rust/musapy-core/src/stream.rs:311-377),
 * and a workspace here belongs to one stream, so a fault is reported to that stream only.
 * musapy_kernels_take_fault_ws(workspace, bytes, stream): call after synchronizing `stream` (the
 * stream the workspace's launches ran on); reads the fault word on `stream` and returns 0 (no
 * fault), a bit set of 1 (a reduction combiner gave up) and 2 (a scan wait gave up), or -1 on a
 * HIP error.  A fault also zeroes the whole workspace (payload and word) on `stream` and waits
 * for that, since a block that published after its combiner gave up may have left a slot
 * behind; the workspace is then ready for reuse.
 * musapy_kernels_take_fault(device): the same for the no-alloc scratch of `device` (returns the
 * bits once; the next no-alloc call zeroes the scratch on its own stream).
 * musapy_kernels_set_spin_limit(polls): sets how many polls a wait makes before it gives up
 * (default 2^24) and returns the previous value; 0 makes every wait give up at once, which lets
 * tests drive the error path while every kernel still exits normally. */
int musapy_kernels_take_fault_ws(void* workspace, size_t workspace_bytes, hipStream_t stream);
int musapy_kernels_take_fault(int device);
uint32_t musapy_kernels_set_spin_limit(uint32_t polls);

/* ---- planning helper (new; no counterpart in kernels.rs) ----
 * Tiles per output that the partial entry points should be given for this reduction on this
 * device: 1 means a single-pass entry point already fills the GPU. */
size_t musapy_reduce_tiles_hint(int ndim, const size_t* in_shape, const ssize_t* in_strides, int axis, size_t axis_len, size_t out_size, size_t elem_size);

#ifdef __cplusplus
}
#endif
#endif /* MUSAPY_KERNELS_H */
