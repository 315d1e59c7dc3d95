/* oracle.h -- CPU restatement of musapy's reference CPU path (see oracle.c).
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline; never by the product.  Strides are in elements and may be negative or zero. */
#ifndef MUSAPY_ORACLE_H
#define MUSAPY_ORACLE_H
#include <stddef.h>
#include <stdint.h>

enum { ORACLE_ADD = 0, ORACLE_SUB, ORACLE_MUL, ORACLE_DIV, ORACLE_POW };
enum { ORACLE_SIN = 0, ORACLE_COS, ORACLE_EXP, ORACLE_LOG, ORACLE_ABS, ORACLE_SIGN, ORACLE_NEG };
enum { ORACLE_EQ = 0, ORACLE_NE, ORACLE_LT, ORACLE_GT, ORACLE_LE, ORACLE_GE };
enum { ORACLE_SUM = 0, ORACLE_PROD, ORACLE_MAX, ORACLE_MIN, ORACLE_MEAN, ORACLE_ARGMAX, ORACLE_ARGMIN };
enum { ORACLE_I8 = 0, ORACLE_I16, ORACLE_I32, ORACLE_I64, ORACLE_U8, ORACLE_U16, ORACLE_U32, ORACLE_U64,
       ORACLE_F32, ORACLE_F64, ORACLE_C64, ORACLE_C128 };

int64_t oracle_offset_nd(size_t idx, const size_t* shape, const int64_t* strides, int ndim);
void oracle_binary_f32(int op, const float* a, const float* b, float* c, int ndim, const size_t* shape,
                       const int64_t* as, const int64_t* bs);
void oracle_binary_f64(int op, const double* a, const double* b, double* c, int ndim, const size_t* shape,
                       const int64_t* as, const int64_t* bs);
void oracle_unary_f32(int op, const float* a, float* c, int ndim, const size_t* shape, const int64_t* as);
void oracle_unary_f64(int op, const double* a, double* c, int ndim, const size_t* shape, const int64_t* as);
void oracle_clamp_f32(const float* a, float* c, double lo, double hi, int ndim, const size_t* shape,
                      const int64_t* as);
void oracle_clamp_f64(const double* a, double* c, double lo, double hi, int ndim, const size_t* shape,
                      const int64_t* as);
void oracle_binary_cplx(int op, int dtype, const void* a, const void* b, void* c, int ndim, const size_t* shape,
                        const int64_t* as, const int64_t* bs);
void oracle_unary_cplx(int op, int dtype, const void* a, void* c, int ndim, const size_t* shape,
                       const int64_t* as);
void oracle_compare(int op, int dtype, const void* a, const void* b, uint8_t* c, int ndim, const size_t* shape,
                    const int64_t* as, const int64_t* bs);
void oracle_cast(int src, int dst, const void* a, void* c, int ndim, const size_t* shape, const int64_t* as);
uint16_t oracle_f32_to_f16(float f);
uint16_t oracle_f32_to_bf16(float f);
void oracle_cast_f32_f16(const float* a, uint16_t* c, int ndim, const size_t* shape, const int64_t* as);
void oracle_cast_f32_bf16(const float* a, uint16_t* c, int ndim, const size_t* shape, const int64_t* as);
void oracle_reduce(int kind, int dtype, const void* a, void* c, int ndim, const size_t* shape,
                   const int64_t* strides, int axis, size_t axis_len, size_t out_size);
void oracle_cumsum(int dtype, int literal, const void* a, void* c, int ndim, const size_t* shape,
                   const int64_t* strides, int axis, size_t out_size);
void oracle_copy_bytes(const void* in, void* out, int ndim, const size_t* shape, const int64_t* strides,
                       size_t elem_size);
#endif
