// ops.cpp -- the op builder: three-phase elementwise / cast / reduction / scan operators.
//
// Ports the control flow of rust/musapy-ops/src/op_builder.rs (binary_elementwise 315-532,
// unary_elementwise 550-732, clamp_elementwise 740-891, validate_cast_pair 904-962,
// cast_array 1055-1119, astype_op 1130-1292, reduction_axis 2310-3139, cumsum_op 3144-3363),
// rust/musapy-ops/src/reduction.rs (axis resolution, reduce_multi, arg_reduce_multi),
// rust/musapy-ops/src/broadcast.rs and rust/musapy-ops/src/indexing.rs (views, contiguous
// 181-237 with copy_into 816-916).  Phase B only calls the C kernel ABI; there is no host
// compute path.  Path selection for reductions differs from the reference (which switches on
// axis_len thresholds, op_builder.rs:2513-2514): the kernel library reports how many tiles per
// output a reduction needs to fill the GPU (musapy_reduce_tiles_hint) and the op layer uses the
// single-pass entry point when that is 1, partial + final otherwise.
#include "ops.hpp"

#include <algorithm>

#include "../../../include/musapy_kernels.h"
#include "../../../include/musapy_hip_runtime.h"

namespace mpy {
namespace ops {

namespace {

const char* bname(BinaryKernel k) {
  static const char* n[] = {"add", "sub", "mul", "div", "pow"};
  return n[int(k)];
}
const char* uname(UnaryKernel k) {
  static const char* n[] = {"sin", "cos", "exp", "log", "abs", "sign", "neg"};
  return n[int(k)];
}
const char* rname(ReduceKernel k) {
  static const char* n[] = {"sum", "prod", "max", "min", "mean", "argmax", "argmin"};
  return n[int(k)];
}

void check_out(const char* op, const Array* out, const Shape& shape, Dtype dtype, const Array& a,
               const char* shape_what, const char* dtype_what) {
  if (!out) return;
  auto fmt = [](const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
  };
  if (out->shape() != shape)
    throw ShapeError(std::string(op) + ": out shape " + fmt(out->shape()) + " != " + shape_what + " " + fmt(shape));
  if (out->dtype != dtype)
    throw DtypeError(std::string(op) + ": out dtype " + dtype_name(out->dtype) + " != " + dtype_what + " " +
                     dtype_name(dtype));
  if (out->device != a.device)
    throw DeviceError(std::string(op) + ": out device hip:" + std::to_string(out->device) + " != input device hip:" +
                      std::to_string(a.device));
}

// Allocates the output (or adopts out=) and runs the alias check (op_builder.rs:420-433).
Array make_output(const Array* out, const Shape& shape, Dtype dtype, int device, const StreamPtr& s,
                  std::initializer_list<const Array*> inputs) {
  if (out) {
    if (!out->layout.has_contiguous_strides()) throw ShapeError("out= must have C-contiguous strides");
    for (const Array* in : inputs)
      if (in && out->data.get() == in->data.get())
        throw MemoryError("alias detected: out= shares its buffer with an input");
    out->data->wait_reads_on(s);
    Array r = *out;
    r.stream = s;
    return r;
  }
  return new_array(shape, dtype, device, s);
}

std::vector<size_t> shape_vec(const Shape& s) { return s; }

}  // namespace

void record_op(const char* name, std::initializer_list<const Array*> inputs, const Array& out) {
  if (!is_debug() || !out.stream) return;
  OpContext ctx;
  ctx.op_name = name;
  for (const Array* x : inputs) {
    ctx.input_shapes.push_back(x->shape());
    ctx.input_devices.push_back(x->device);
    ctx.input_dtypes.push_back(x->dtype);
  }
  ctx.output_shape = out.shape();
  ctx.stream_id = out.stream->id();
  ctx.has_frame = take_debug_frame(ctx.frame);
  out.stream->record_op(std::move(ctx));
}

StreamPtr pick_stream(const Array& a, const Array* out) {
  if (out) return out->stream;
  StreamPtr cur = current_stream();
  return cur ? cur : a.stream;
}

// ---------------------------------------------------------------------------------------------
// broadcast.rs:24-92
Shape broadcast_shape(const std::vector<Shape>& shapes) {
  size_t nd = 0;
  for (auto& s : shapes) nd = std::max(nd, s.size());
  Shape r(nd, 1);
  for (auto& s : shapes) {
    size_t off = nd - s.size();
    for (size_t i = 0; i < s.size(); ++i) {
      size_t o = off + i;
      if (r[o] == 1)
        r[o] = s[i];
      else if (s[i] != 1 && s[i] != r[o])
        throw ShapeError("broadcast: incompatible shapes (dim " + std::to_string(o) + " = " + std::to_string(r[o]) +
                         " vs " + std::to_string(s[i]) + ")");
    }
  }
  return r;
}

Strides broadcast_strides(const Layout& layout, const Shape& target) {
  size_t nd = target.size();
  Strides r(nd, 0);
  size_t off = nd >= layout.ndim() ? nd - layout.ndim() : 0;
  for (size_t i = 0; i < layout.ndim(); ++i) {
    size_t o = off + i;
    if (o >= nd) break;
    if (layout.shape[i] == target[o]) r[o] = layout.strides[i];
  }
  return r;
}

// ---------------------------------------------------------------------------------------------
// casts -- op_builder.rs:904-962 plus the new f32 -> f16 / bf16 pairs
void validate_cast_pair(Dtype src, Dtype dst) {
  bool new_pair = src == Dtype::Float32 && (dst == Dtype::Float16 || dst == Dtype::Bfloat16);
  if (new_pair) return;
  switch (src) {
    case Dtype::Int8: case Dtype::Int16: case Dtype::Int32: case Dtype::Int64:
    case Dtype::Uint8: case Dtype::Uint16: case Dtype::Uint32: case Dtype::Uint64:
    case Dtype::Float32: case Dtype::Float64:
      break;
    case Dtype::Complex64: case Dtype::Complex128:
      // only the c64 -> c128 widening; complex -> real has no kernel
      if (src == Dtype::Complex64 && dst == Dtype::Complex128) return;
      throw DtypeError(std::string("cast: ") + dtype_name(src) + " -> " + dtype_name(dst) +
                       " not supported (complex -> real has no cast kernel)");
    default:
      throw DtypeError(std::string("cast: source dtype ") + dtype_name(src) +
                       " not supported (bool/float16/bfloat16 sources have no cast kernel)");
  }
  switch (dst) {
    case Dtype::Float32: case Dtype::Float64: case Dtype::Int64: case Dtype::Complex64: case Dtype::Complex128:
      break;
    default:
      throw DtypeError(std::string("cast: target dtype ") + dtype_name(dst) +
                       " not supported (only float32/float64/int64/complex64/complex128, and float16/bfloat16 "
                       "from float32)");
  }
  if (is_complex(dst) && src != Dtype::Float32 && src != Dtype::Float64)
    throw DtypeError(std::string("cast: ") + dtype_name(src) + " -> " + dtype_name(dst) +
                     " not supported (complex targets take float32/float64 sources and the c64 -> c128 widening)");
  if (src == dst) throw DtypeError(std::string("cast: source and target dtype are identical (") + dtype_name(src) + ")");
}

namespace {

void launch_cast(const void* a, void* c, const Shape& shape, const Strides& st, Dtype src, Dtype dst,
                 hipStream_t s) {
  if (shape_numel(shape) == 0) return;
  const int nd = int(shape.size());
  const size_t* sh = shape.data();
  const ssize_t* ss = st.data();
#define CAST_CASE(SD, ST, FN, DT) \
  case Dtype::SD: FN((const ST*)a, (DT*)c, nd, sh, ss, s); break;
  if (dst == Dtype::Float32) {
    switch (src) {
      CAST_CASE(Int8, int8_t, musapy_cast_i8_f32_v2, float)
      CAST_CASE(Int16, int16_t, musapy_cast_i16_f32_v2, float)
      CAST_CASE(Int32, int32_t, musapy_cast_i32_f32_v2, float)
      CAST_CASE(Int64, int64_t, musapy_cast_i64_f32_v2, float)
      CAST_CASE(Uint8, uint8_t, musapy_cast_u8_f32_v2, float)
      CAST_CASE(Uint16, uint16_t, musapy_cast_u16_f32_v2, float)
      CAST_CASE(Uint32, uint32_t, musapy_cast_u32_f32_v2, float)
      CAST_CASE(Uint64, uint64_t, musapy_cast_u64_f32_v2, float)
      CAST_CASE(Float64, double, musapy_cast_f64_f32_v2, float)
      default: throw DtypeError("cast pair not validated");
    }
  } else if (dst == Dtype::Float64) {
    switch (src) {
      CAST_CASE(Int8, int8_t, musapy_cast_i8_f64_v2, double)
      CAST_CASE(Int16, int16_t, musapy_cast_i16_f64_v2, double)
      CAST_CASE(Int32, int32_t, musapy_cast_i32_f64_v2, double)
      CAST_CASE(Int64, int64_t, musapy_cast_i64_f64_v2, double)
      CAST_CASE(Uint8, uint8_t, musapy_cast_u8_f64_v2, double)
      CAST_CASE(Uint16, uint16_t, musapy_cast_u16_f64_v2, double)
      CAST_CASE(Uint32, uint32_t, musapy_cast_u32_f64_v2, double)
      CAST_CASE(Uint64, uint64_t, musapy_cast_u64_f64_v2, double)
      CAST_CASE(Float32, float, musapy_cast_f32_f64_v2, double)
      default: throw DtypeError("cast pair not validated");
    }
  } else if (dst == Dtype::Int64) {
    switch (src) {
      CAST_CASE(Int8, int8_t, musapy_cast_i8_i64_v2, int64_t)
      CAST_CASE(Int16, int16_t, musapy_cast_i16_i64_v2, int64_t)
      CAST_CASE(Int32, int32_t, musapy_cast_i32_i64_v2, int64_t)
      CAST_CASE(Uint8, uint8_t, musapy_cast_u8_i64_v2, int64_t)
      CAST_CASE(Uint16, uint16_t, musapy_cast_u16_i64_v2, int64_t)
      CAST_CASE(Uint32, uint32_t, musapy_cast_u32_i64_v2, int64_t)
      CAST_CASE(Uint64, uint64_t, musapy_cast_u64_i64_v2, int64_t)
      CAST_CASE(Float32, float, musapy_cast_f32_i64_v2, int64_t)
      CAST_CASE(Float64, double, musapy_cast_f64_i64_v2, int64_t)
      default: throw DtypeError("cast pair not validated");
    }
  } else if (dst == Dtype::Complex64) {
    switch (src) {
      CAST_CASE(Float32, float, musapy_cast_f32_c64_v2, musapy_c64_t)
      CAST_CASE(Float64, double, musapy_cast_f64_c64_v2, musapy_c64_t)
      default: throw DtypeError("cast pair not validated");
    }
  } else if (dst == Dtype::Complex128) {
    switch (src) {
      CAST_CASE(Float32, float, musapy_cast_f32_c128_v2, musapy_c128_t)
      CAST_CASE(Float64, double, musapy_cast_f64_c128_v2, musapy_c128_t)
      CAST_CASE(Complex64, musapy_c64_t, musapy_cast_c64_c128_v2, musapy_c128_t)
      default: throw DtypeError("cast pair not validated");
    }
  } else if (dst == Dtype::Bfloat16 && src == Dtype::Float32) {
    musapy_cast_f32_bf16_v2((const float*)a, (uint16_t*)c, nd, sh, ss, s);
  } else if (dst == Dtype::Float16 && src == Dtype::Float32) {
    musapy_cast_f32_f16_v2((const float*)a, (uint16_t*)c, nd, sh, ss, s);
  } else {
    throw DtypeError("cast pair not validated");
  }
#undef CAST_CASE
  check_launch("cast");
}

}  // namespace

Array cast_array(const Array& a, Dtype target, const StreamPtr& stream) {
  validate_cast_pair(a.dtype, target);
  Array out = new_array(a.shape(), target, a.device, stream);
  a.data->wait_last_write_on(stream);
  launch_cast(a.data_ptr(), out.data->ptr(), a.shape(), a.layout.strides, a.dtype, target, stream->raw());
  a.data->record_read(stream);
  out.data->record_write(stream);
  return out;
}

Array astype_op(const Array& a, Dtype dtype, const Array* out) {
  if (a.dtype != dtype) validate_cast_pair(a.dtype, dtype);
  check_out("astype", out, a.shape(), dtype, a, "input shape", "target dtype");
  StreamPtr s = pick_stream(a, out);
  Array r = make_output(out, a.shape(), dtype, a.device, s, {&a});
  a.data->wait_last_write_on(s);
  if (a.size() > 0) {
    if (a.dtype == dtype) {
      if (!a.is_contiguous())
        throw DtypeError("astype: same-dtype copy requires contiguous input (reference limitation kept)");
      check_rt(mpy_rt_memcpy_d2d(r.data->ptr(), a.data_ptr(), a.nbytes(), s->raw()), "astype copy");
    } else {
      launch_cast(a.data_ptr(), r.data_ptr(), a.shape(), a.layout.strides, a.dtype, dtype, s->raw());
    }
  }
  a.data->record_read(s);
  r.data->record_write(s);
  return r;
}

// ---------------------------------------------------------------------------------------------
// elementwise
Array binary_elementwise(const Array& a, const Array& b, const Array* out, BinaryKernel k) {
  const char* op = bname(k);
  if (a.device != b.device)
    throw DeviceError(std::string(op) + ": device mismatch hip:" + std::to_string(a.device) + " vs hip:" +
                      std::to_string(b.device));
  Shape out_shape = broadcast_shape({a.shape(), b.shape()});
  Dtype dt = promote(a.dtype, b.dtype, /*all_gpu=*/true);
  if (is_complex(dt) && k == BinaryKernel::Pow)
    throw DtypeError(std::string(op) + ": pow not supported for complex dtype " + dtype_name(dt) +
                     " (complex scope: add/sub/mul/div)");
  if (dt != Dtype::Float32 && dt != Dtype::Float64 && !is_complex(dt))
    throw DtypeError(std::string(op) + ": promoted dtype " + dtype_name(dt) +
                     " not supported (compute whitelist: float32/float64/complex64/complex128)");
  check_out(op, out, out_shape, dt, a, "broadcast output shape", "promoted dtype");
  StreamPtr s = pick_stream(a, out);
  if ((a.dtype != dt || b.dtype != dt) && a.shape() == out_shape && b.shape() == out_shape &&
      shape_numel(out_shape) > 0) {
    // promotion without a materialised cast: one fused pass (same bits as cast, then compute)
    Array r = make_output(out, out_shape, dt, a.device, s, {&a, &b});
    a.data->wait_last_write_on(s);
    b.data->wait_last_write_on(s);
    if (musapy_binary_mixed_v2(int(k), a.data_ptr(), int(a.dtype), b.data_ptr(), int(b.dtype), r.data_ptr(),
                               int(dt), int(out_shape.size()), out_shape.data(), a.layout.strides.data(),
                               b.layout.strides.data(), s->raw()) == 0) {
      check_launch(op);
      a.data->record_read(s);
      b.data->record_read(s);
      r.data->record_write(s);
      return r;
    }
  }
  std::optional<Array> ac, bc;
  if (a.dtype != dt) ac = cast_array(a, dt, s);
  if (b.dtype != dt) bc = cast_array(b, dt, s);
  const Array& aw = ac ? *ac : a;
  const Array& bw = bc ? *bc : b;
  Array r = make_output(out, out_shape, dt, a.device, s, {&aw, &bw});
  aw.data->wait_last_write_on(s);
  bw.data->wait_last_write_on(s);
  if (shape_numel(out_shape) > 0) {
    Strides as = aw.shape() == out_shape ? aw.layout.strides : broadcast_strides(aw.layout, out_shape);
    Strides bs = bw.shape() == out_shape ? bw.layout.strides : broadcast_strides(bw.layout, out_shape);
    const int nd = int(out_shape.size());
#define BIN(T, SFX)                                                                                         \
  {                                                                                                         \
    auto fn = k == BinaryKernel::Add ? musapy_add_##SFX##_v2                                                \
              : k == BinaryKernel::Sub ? musapy_sub_##SFX##_v2                                              \
              : k == BinaryKernel::Mul ? musapy_mul_##SFX##_v2                                              \
              : k == BinaryKernel::Div ? musapy_div_##SFX##_v2                                              \
                                       : musapy_pow_##SFX##_v2;                                             \
    fn((const T*)aw.data_ptr(), (const T*)bw.data_ptr(), (T*)r.data_ptr(), nd, out_shape.data(), as.data(), \
       bs.data(), s->raw());                                                                                \
  }
#define BINC(T, SFX)                                                                                        \
  {                                                                                                         \
    auto fn = k == BinaryKernel::Add ? musapy_add_##SFX##_v2                                                \
              : k == BinaryKernel::Sub ? musapy_sub_##SFX##_v2                                              \
              : k == BinaryKernel::Mul ? musapy_mul_##SFX##_v2                                              \
                                       : musapy_div_##SFX##_v2;                                             \
    fn((const T*)aw.data_ptr(), (const T*)bw.data_ptr(), (T*)r.data_ptr(), nd, out_shape.data(), as.data(), \
       bs.data(), s->raw());                                                                                \
  }
    switch (dt) {
      case Dtype::Float32: BIN(float, f32) break;
      case Dtype::Float64: BIN(double, f64) break;
      case Dtype::Complex64: BINC(musapy_c64_t, c64) break;
      default: BINC(musapy_c128_t, c128) break;
    }
#undef BIN
#undef BINC
    check_launch(op);
  }
  aw.data->record_read(s);
  bw.data->record_read(s);
  r.data->record_write(s);
  return r;
}

// op_builder.rs:1338-1557.  Promotion only picks the kernel; the output is bool.  Complex inputs
// take eq/ne only (no total order).  Mixed dtypes are cast to the promoted dtype first, as in
// the reference (op_builder.rs:1430-1438).
Array comparison_elementwise(const Array& a, const Array& b, const Array* out, CompareKernel k) {
  static const char* names[] = {"eq", "ne", "lt", "gt", "le", "ge"};
  const char* op = names[int(k)];
  if (a.device != b.device)
    throw DeviceError(std::string(op) + ": device mismatch hip:" + std::to_string(a.device) + " vs hip:" +
                      std::to_string(b.device));
  Shape out_shape = broadcast_shape({a.shape(), b.shape()});
  Dtype dt = promote(a.dtype, b.dtype, /*all_gpu=*/true);
  const bool eq_ne = k == CompareKernel::Eq || k == CompareKernel::Ne;
  if (is_complex(dt) && !eq_ne)
    throw DtypeError(std::string(op) + ": " + op + " not supported for complex dtype " + dtype_name(dt) +
                     " (complex has no total order; only eq/ne)");
  if (dt != Dtype::Float32 && dt != Dtype::Float64 && !is_complex(dt))
    throw DtypeError(std::string(op) + ": promoted dtype " + dtype_name(dt) +
                     " not supported (compute whitelist: float32/float64, complex eq/ne)");
  check_out(op, out, out_shape, Dtype::Bool, a, "broadcast output shape", "comparison output dtype");
  StreamPtr s = pick_stream(a, out);
  std::optional<Array> ac, bc;
  if (a.dtype != dt) ac = cast_array(a, dt, s);
  if (b.dtype != dt) bc = cast_array(b, dt, s);
  const Array& aw = ac ? *ac : a;
  const Array& bw = bc ? *bc : b;
  Array r = make_output(out, out_shape, Dtype::Bool, a.device, s, {&aw, &bw});
  aw.data->wait_last_write_on(s);
  bw.data->wait_last_write_on(s);
  if (shape_numel(out_shape) > 0) {
    Strides as = aw.shape() == out_shape ? aw.layout.strides : broadcast_strides(aw.layout, out_shape);
    Strides bs = bw.shape() == out_shape ? bw.layout.strides : broadcast_strides(bw.layout, out_shape);
    const int nd = int(out_shape.size());
    uint8_t* c = (uint8_t*)r.data_ptr();
#define CMP(T, SFX)                                                                                       \
  {                                                                                                       \
    auto fn = k == CompareKernel::Eq   ? musapy_eq_##SFX##_v2                                             \
              : k == CompareKernel::Ne ? musapy_ne_##SFX##_v2                                             \
              : k == CompareKernel::Lt ? musapy_lt_##SFX##_v2                                             \
              : k == CompareKernel::Gt ? musapy_gt_##SFX##_v2                                             \
              : k == CompareKernel::Le ? musapy_le_##SFX##_v2                                             \
                                       : musapy_ge_##SFX##_v2;                                            \
    fn((const T*)aw.data_ptr(), (const T*)bw.data_ptr(), c, nd, out_shape.data(), as.data(), bs.data(), \
       s->raw());                                                                                         \
  }
#define CMPC(T, SFX)                                                                                      \
  {                                                                                                       \
    auto fn = k == CompareKernel::Eq ? musapy_eq_##SFX##_v2 : musapy_ne_##SFX##_v2;                       \
    fn((const T*)aw.data_ptr(), (const T*)bw.data_ptr(), c, nd, out_shape.data(), as.data(), bs.data(), \
       s->raw());                                                                                         \
  }
    switch (dt) {
      case Dtype::Float32: CMP(float, f32) break;
      case Dtype::Float64: CMP(double, f64) break;
      case Dtype::Complex64: CMPC(musapy_c64_t, c64) break;
      default: CMPC(musapy_c128_t, c128) break;
    }
#undef CMP
#undef CMPC
    check_launch(op);
  }
  aw.data->record_read(s);
  bw.data->record_read(s);
  r.data->record_write(s);
  return r;
}

Array unary_elementwise(const Array& a, const Array* out, UnaryKernel k) {
  const char* op = uname(k);
  Dtype dt = a.dtype;
  if (is_complex(dt)) {
    if (k != UnaryKernel::Neg && k != UnaryKernel::Abs)
      throw DtypeError(std::string(op) + ": " + op + " not supported for complex dtype " + dtype_name(dt) +
                       " (complex scope: neg/abs)");
  } else if (dt != Dtype::Float32 && dt != Dtype::Float64) {
    throw DtypeError(std::string(op) + ": dtype " + dtype_name(dt) +
                     " not supported (only float32/float64/complex64/complex128)");
  }
  // abs of a complex array is real (op_builder.rs:585-589)
  Dtype odt = !(is_complex(dt) && k == UnaryKernel::Abs) ? dt
              : dt == Dtype::Complex64                      ? Dtype::Float32
                                                            : Dtype::Float64;
  check_out(op, out, a.shape(), odt, a, "input shape", "expected output dtype");
  StreamPtr s = pick_stream(a, out);
  Array r = make_output(out, a.shape(), odt, a.device, s, {&a});
  a.data->wait_last_write_on(s);
  if (a.size() > 0 && is_complex(dt)) {
    const int nd = int(a.ndim());
    const size_t* sh = a.shape().data();
    const ssize_t* st = a.layout.strides.data();
    if (dt == Dtype::Complex64) {
      if (k == UnaryKernel::Abs)
        musapy_abs_c64_v2((const musapy_c64_t*)a.data_ptr(), (float*)r.data_ptr(), nd, sh, st, s->raw());
      else
        musapy_neg_c64_v2((const musapy_c64_t*)a.data_ptr(), (musapy_c64_t*)r.data_ptr(), nd, sh, st, s->raw());
    } else {
      if (k == UnaryKernel::Abs)
        musapy_abs_c128_v2((const musapy_c128_t*)a.data_ptr(), (double*)r.data_ptr(), nd, sh, st, s->raw());
      else
        musapy_neg_c128_v2((const musapy_c128_t*)a.data_ptr(), (musapy_c128_t*)r.data_ptr(), nd, sh, st,
                           s->raw());
    }
    check_launch(op);
  } else if (a.size() > 0) {
    const int nd = int(a.ndim());
#define UN(T, SFX)                                                                                               \
  {                                                                                                              \
    auto fn = k == UnaryKernel::Sin ? musapy_sin_##SFX##_v2                                                      \
              : k == UnaryKernel::Cos ? musapy_cos_##SFX##_v2                                                    \
              : k == UnaryKernel::Exp ? musapy_exp_##SFX##_v2                                                    \
              : k == UnaryKernel::Log ? musapy_log_##SFX##_v2                                                    \
              : k == UnaryKernel::Abs ? musapy_abs_##SFX##_v2                                                    \
              : k == UnaryKernel::Sign ? musapy_sign_##SFX##_v2                                                  \
                                       : musapy_neg_##SFX##_v2;                                                  \
    fn((const T*)a.data_ptr(), (T*)r.data_ptr(), nd, a.shape().data(), a.layout.strides.data(), s->raw());      \
  }
    if (dt == Dtype::Float32) UN(float, f32) else UN(double, f64)
#undef UN
    check_launch(op);
  }
  a.data->record_read(s);
  r.data->record_write(s);
  return r;
}

Array clamp_elementwise(const Array& a, double lo, double hi, const Array* out) {
  Dtype dt = a.dtype;
  if (dt != Dtype::Float32 && dt != Dtype::Float64)
    throw DtypeError(std::string("clamp: dtype ") + dtype_name(dt) + " not supported (only float32/float64)");
  check_out("clamp", out, a.shape(), dt, a, "input shape", "input dtype");
  StreamPtr s = pick_stream(a, out);
  Array r = make_output(out, a.shape(), dt, a.device, s, {&a});
  a.data->wait_last_write_on(s);
  if (a.size() > 0) {
    const int nd = int(a.ndim());
    if (dt == Dtype::Float32)  // lo/hi narrowed like op_builder.rs:850-853
      musapy_clamp_f32_v2((const float*)a.data_ptr(), (float*)r.data_ptr(), float(lo), float(hi), nd,
                          a.shape().data(), a.layout.strides.data(), s->raw());
    else
      musapy_clamp_f64_v2((const double*)a.data_ptr(), (double*)r.data_ptr(), lo, hi, nd, a.shape().data(),
                          a.layout.strides.data(), s->raw());
    check_launch("clamp");
  }
  a.data->record_read(s);
  r.data->record_write(s);
  return r;
}

// ---------------------------------------------------------------------------------------------
// reductions
namespace {

// op_builder.rs:2209-2225
Dtype reduction_compute_dtype(Dtype in, ReduceKernel k) {
  if (in == Dtype::Float32 || in == Dtype::Float64) return in;
  if (is_complex(in)) return in;
  return k == ReduceKernel::Mean ? Dtype::Float64 : Dtype::Int64;
}

bool is_arg(ReduceKernel k) { return k == ReduceKernel::Argmax || k == ReduceKernel::Argmin; }

struct RedCall {
  const void* a;
  int nd;
  const size_t* shape;
  const ssize_t* strides;
  int axis;
  size_t axis_len, out_size;
  hipStream_t s;
};

#define RED_CALL_ARGS c.nd, c.shape, c.strides, c.axis, c.axis_len, c.out_size

void red_single(ReduceKernel k, Dtype ct, const RedCall& c, void* out) {
#define R1(OP, SFX, T, OT) musapy_##OP##_##SFX##_v2((const T*)c.a, (OT*)out, RED_CALL_ARGS, c.s)
#define RREAL(SFX, T)                                                   \
  switch (k) {                                                          \
    case ReduceKernel::Sum: R1(sum, SFX, T, T); break;                  \
    case ReduceKernel::Prod: R1(prod, SFX, T, T); break;                \
    case ReduceKernel::Max: R1(max, SFX, T, T); break;                  \
    case ReduceKernel::Min: R1(min, SFX, T, T); break;                  \
    case ReduceKernel::Argmax: R1(argmax, SFX, T, int64_t); break;      \
    case ReduceKernel::Argmin: R1(argmin, SFX, T, int64_t); break;      \
    default: throw DtypeError("reduction not available for dtype");     \
  }
  switch (ct) {
    case Dtype::Int64: RREAL(i64, int64_t) break;
    case Dtype::Float32:
      if (k == ReduceKernel::Mean) R1(mean, f32, float, float); else RREAL(f32, float)
      break;
    case Dtype::Float64:
      if (k == ReduceKernel::Mean) R1(mean, f64, double, double); else RREAL(f64, double)
      break;
    case Dtype::Complex64:
      if (k == ReduceKernel::Sum) R1(sum, c64, musapy_c64_t, musapy_c64_t);
      else if (k == ReduceKernel::Prod) R1(prod, c64, musapy_c64_t, musapy_c64_t);
      else R1(mean, c64, musapy_c64_t, musapy_c64_t);
      break;
    case Dtype::Complex128:
      if (k == ReduceKernel::Sum) R1(sum, c128, musapy_c128_t, musapy_c128_t);
      else if (k == ReduceKernel::Prod) R1(prod, c128, musapy_c128_t, musapy_c128_t);
      else R1(mean, c128, musapy_c128_t, musapy_c128_t);
      break;
    default: throw DtypeError("reduction compute dtype not supported");
  }
#undef RREAL
#undef R1
}

// partial + final in one launch (musapy_reduce_fused_v1) with the stream's workspace; false when
// the kernel library does not cover the case (then the two-stage path runs)
bool red_fused(ReduceKernel k, Dtype ct, const RedCall& c, void* out, size_t tiles, Stream& s) {
  int op = 0;
  switch (k) {
    case ReduceKernel::Sum: op = MUSAPY_RED_SUM; break;
    case ReduceKernel::Prod: op = MUSAPY_RED_PROD; break;
    case ReduceKernel::Max: op = MUSAPY_RED_MAX; break;
    case ReduceKernel::Min: op = MUSAPY_RED_MIN; break;
    case ReduceKernel::Mean: op = MUSAPY_RED_MEAN; break;
    case ReduceKernel::Argmax: op = MUSAPY_RED_ARGMAX; break;
    case ReduceKernel::Argmin: op = MUSAPY_RED_ARGMIN; break;
    default: return false;
  }
  int dt = 0;
  switch (ct) {
    case Dtype::Float32: dt = MUSAPY_DT_F32; break;
    case Dtype::Float64: dt = MUSAPY_DT_F64; break;
    case Dtype::Int64: dt = MUSAPY_DT_I64; break;
    case Dtype::Complex64: dt = MUSAPY_DT_C64; break;
    case Dtype::Complex128: dt = MUSAPY_DT_C128; break;
    default: return false;
  }
  if (musapy_reduce_fused_v1(op, dt, c.a, out, c.nd, c.shape, c.strides, c.axis, c.axis_len, c.out_size, tiles,
                             s.reduce_workspace(), Stream::kReduceWorkspaceBytes, c.s) != 0)
    return false;
  s.note_bounded_wait();
  return true;
}

// partial -> final for value reductions (sum/prod/max/min/mean)
void red_two_stage(ReduceKernel k, Dtype ct, const RedCall& c, void* out, size_t tiles, void* partials) {
#define P2(OP, SFX, T) musapy_##OP##_partial_##SFX##_v2((const T*)c.a, (T*)partials, RED_CALL_ARGS, tiles, c.s)
#define F2(OP, SFX, T) musapy_##OP##_final_##SFX##_v2((const T*)partials, (T*)out, tiles, c.out_size, c.s)
#define F2L(OP, SFX, T) musapy_##OP##_final_##SFX##_v2((const T*)partials, (T*)out, tiles, c.out_size, c.axis_len, c.s)
#define V2(SFX, T)                                                       \
  switch (k) {                                                           \
    case ReduceKernel::Sum: P2(sum, SFX, T); F2(sum, SFX, T); break;     \
    case ReduceKernel::Prod: P2(prod, SFX, T); F2(prod, SFX, T); break;  \
    case ReduceKernel::Max: P2(max, SFX, T); F2(max, SFX, T); break;     \
    case ReduceKernel::Min: P2(min, SFX, T); F2(min, SFX, T); break;     \
    default: throw DtypeError("reduction not available for dtype");      \
  }
  switch (ct) {
    case Dtype::Int64: V2(i64, int64_t) break;
    case Dtype::Float32:
      if (k == ReduceKernel::Mean) { P2(mean, f32, float); F2L(mean, f32, float); } else V2(f32, float)
      break;
    case Dtype::Float64:
      if (k == ReduceKernel::Mean) { P2(mean, f64, double); F2L(mean, f64, double); } else V2(f64, double)
      break;
    case Dtype::Complex64:
      if (k == ReduceKernel::Sum) { P2(sum, c64, musapy_c64_t); F2L(sum, c64, musapy_c64_t); }
      else if (k == ReduceKernel::Prod) { P2(prod, c64, musapy_c64_t); F2L(prod, c64, musapy_c64_t); }
      else { P2(mean, c64, musapy_c64_t); F2L(mean, c64, musapy_c64_t); }
      break;
    case Dtype::Complex128:
      if (k == ReduceKernel::Sum) { P2(sum, c128, musapy_c128_t); F2L(sum, c128, musapy_c128_t); }
      else if (k == ReduceKernel::Prod) { P2(prod, c128, musapy_c128_t); F2L(prod, c128, musapy_c128_t); }
      else { P2(mean, c128, musapy_c128_t); F2L(mean, c128, musapy_c128_t); }
      break;
    default: throw DtypeError("reduction compute dtype not supported");
  }
#undef V2
#undef F2L
#undef F2
#undef P2
}

void red_arg_two_stage(ReduceKernel k, Dtype ct, const RedCall& c, int64_t* out, size_t tiles, void* pv,
                       int64_t* pi) {
#define A2(OP, SFX, T)                                                                          \
  musapy_##OP##_partial_##SFX##_v2((const T*)c.a, (T*)pv, pi, RED_CALL_ARGS, tiles, c.s);       \
  musapy_##OP##_final_##SFX##_v2((const T*)pv, pi, out, tiles, c.out_size, c.s);
#define AA(SFX, T) \
  if (k == ReduceKernel::Argmax) { A2(argmax, SFX, T) } else { A2(argmin, SFX, T) }
  switch (ct) {
    case Dtype::Int64: AA(i64, int64_t) break;
    case Dtype::Float32: AA(f32, float) break;
    case Dtype::Float64: AA(f64, double) break;
    default: throw DtypeError("arg reduction compute dtype not supported");
  }
#undef AA
#undef A2
}

}  // namespace

std::optional<size_t> resolve_axis(std::optional<ssize_t> axis, size_t ndim) {
  if (!axis) return std::nullopt;
  ssize_t ax = *axis, n = ssize_t(ndim);
  ssize_t norm = ax < 0 ? ax + n : ax;
  if (norm < 0 || norm >= n)
    throw ShapeError("axis " + std::to_string(ax) + " is out of bounds for array of dimension " + std::to_string(ndim));
  return size_t(norm);
}

std::vector<size_t> resolve_axes(const std::vector<ssize_t>* axes, size_t ndim) {
  std::vector<size_t> r;
  if (!axes) return r;
  for (ssize_t ax : *axes) r.push_back(*resolve_axis(ax, ndim));
  std::sort(r.begin(), r.end());
  for (size_t i = 1; i < r.size(); ++i)
    if (r[i] == r[i - 1]) throw ShapeError("duplicate value in 'axis' argument: " + std::to_string(r[i]));
  return r;
}

Array reduction_axis(const Array& a, std::optional<size_t> axis, bool keepdims, const Array* out, ReduceKernel k) {
  const char* op = rname(k);
  if (is_complex(a.dtype) && (k == ReduceKernel::Max || k == ReduceKernel::Min || is_arg(k)))
    throw DtypeError(std::string(op) + ": ordering reduction not supported for complex dtype " + dtype_name(a.dtype) +
                     " (complex has no total order)");
  const Shape in_shape = a.shape();
  const size_t nd = in_shape.size();
  Shape out_shape;
  if (!axis) {
    if (keepdims) out_shape.assign(nd, 1);
  } else {
    for (size_t i = 0; i < nd; ++i) {
      if (i == *axis) {
        if (keepdims) out_shape.push_back(1);
      } else {
        out_shape.push_back(in_shape[i]);
      }
    }
  }
  Dtype ct = reduction_compute_dtype(a.dtype, k);
  Dtype out_dt = is_arg(k) ? Dtype::Int64 : ct;
  const size_t total = shape_numel(in_shape);
  Shape kshape = axis ? in_shape : Shape{total};
  const int kaxis = axis ? int(*axis) : 0;
  const size_t axis_len = axis ? in_shape[*axis] : total;
  const size_t out_size = std::max<size_t>(shape_numel(out_shape), 1);
  check_out(op, out, out_shape, out_dt, a, "expected output shape", "expected");
  StreamPtr s = pick_stream(a, out);
  std::optional<Array> cast;
  if (a.dtype != ct) cast = cast_array(a, ct, s);
  const Array* aw = cast ? &*cast : &a;
  Array r = make_output(out, out_shape, out_dt, a.device, s, {aw});
  aw->data->wait_last_write_on(s);
  std::optional<Array> flat;
  if (!axis && !aw->layout.has_contiguous_strides()) {
    flat = contiguous(*aw);
    flat->data->wait_last_write_on(s);
    aw = &*flat;
  }
  if (axis_len == 0 && shape_numel(out_shape) > 0 &&
      (k == ReduceKernel::Max || k == ReduceKernel::Min || is_arg(k)))
    throw ShapeError(std::string(op) + ": zero-size reduction has no identity");
  if (out_size > 0 && shape_numel(out_shape.empty() ? Shape{1} : out_shape) > 0) {
    Strides kstrides = axis ? aw->layout.strides : Strides{1};
    RedCall c{aw->data_ptr(), int(kshape.size()), kshape.data(), kstrides.data(), kaxis, axis_len, out_size, s->raw()};
    const size_t es = element_size(ct);
    size_t tiles = axis_len == 0 ? 1
                                 : musapy_reduce_tiles_hint(c.nd, c.shape, c.strides, c.axis, axis_len, out_size, es);
    if (tiles <= 1) {
      red_single(k, ct, c, r.data_ptr());
    } else if (red_fused(k, ct, c, r.data_ptr(), tiles, *s)) {
      // one launch: partials handed over through the stream's workspace
    } else if (is_arg(k)) {
      BufferRef pv = Buffer::alloc(out_size * tiles * es, a.device, s);
      BufferRef pi = Buffer::alloc(out_size * tiles * 8, a.device, s);
      red_arg_two_stage(k, ct, c, (int64_t*)r.data_ptr(), tiles, pv->ptr(), (int64_t*)pi->ptr());
    } else {
      BufferRef pp = Buffer::alloc(out_size * tiles * es, a.device, s);
      red_two_stage(k, ct, c, r.data_ptr(), tiles, pp->ptr());
    }
    check_launch(op);
  }
  aw->data->record_read(s);
  r.data->record_write(s);
  return r;
}

// reduction.rs:118-155
Array reduce_multi(const Array& a, const std::vector<ssize_t>* axes, bool keepdims, const Array* out,
                   ReduceKernel k) {
  std::vector<size_t> ax = resolve_axes(axes, a.ndim());
  if (ax.empty()) return reduction_axis(a, std::nullopt, keepdims, out, k);
  if (ax.size() == 1) return reduction_axis(a, ax[0], keepdims, out, k);
  if (out) throw ShapeError("reduction with multiple axes does not support out= yet");
  if (k == ReduceKernel::Sum || k == ReduceKernel::Prod || k == ReduceKernel::Mean) {
    // Adjacent reduced axes that one stride walks (e.g. (1,2) of a C-order array) are reduced as
    // one axis: a single pass instead of one pass per axis.  Only the association of the
    // floating-point sum/product changes (integer results are identical); max/min/arg keep the
    // per-axis passes because their NaN and +-0 outcomes depend on that order.  Means merge only
    // while the merged count is exact in the compute dtype, like the reference's per-axis counts.
    Dtype ct = reduction_compute_dtype(a.dtype, k);
    const double count_cap = ct == Dtype::Float32 ? 16777216.0 : 9007199254740992.0;
    Layout l;
    l.offset = a.layout.offset;
    std::vector<size_t> merged_axes;
    double run_count = 1;
    for (size_t d = 0; d < a.ndim(); ++d) {
      const bool red = std::find(ax.begin(), ax.end(), d) != ax.end();
      const bool prev_red = d > 0 && std::find(ax.begin(), ax.end(), d - 1) != ax.end();
      const size_t n = a.shape()[d];
      if (red && prev_red && !l.shape.empty() &&
          l.strides.back() == a.layout.strides[d] * ssize_t(n) &&
          (k != ReduceKernel::Mean || run_count * double(n) <= count_cap)) {
        l.shape.back() *= n;
        l.strides.back() = a.layout.strides[d];
        run_count *= double(n);
        continue;
      }
      l.shape.push_back(n);
      l.strides.push_back(a.layout.strides[d]);
      run_count = double(n);
      if (red) merged_axes.push_back(l.shape.size() - 1);
    }
    if (merged_axes.size() < ax.size()) {
      Array v = a.view(l);
      std::optional<Array> cur;
      for (size_t x : merged_axes) cur = reduction_axis(cur ? *cur : v, x, true, nullptr, k);
      Shape target;
      for (size_t d = 0; d < a.ndim(); ++d) {
        const bool red = std::find(ax.begin(), ax.end(), d) != ax.end();
        if (!red) target.push_back(a.shape()[d]);
        else if (keepdims) target.push_back(1);
      }
      return cur->view(Layout::from_shape(target));  // results are C-contiguous
    }
  }
  if ((k == ReduceKernel::Max || k == ReduceKernel::Min) && a.ndim() == 2 && ax.size() == 2 && a.is_contiguous() &&
      a.size() > 0) {
    // both axes of a C-contiguous matrix: one launch with the per-axis passes' result
    int dt = -1;
    if (a.dtype == Dtype::Float32) dt = MUSAPY_DT_F32;
    else if (a.dtype == Dtype::Float64) dt = MUSAPY_DT_F64;
    else if (a.dtype == Dtype::Int64) dt = MUSAPY_DT_I64;
    if (dt >= 0) {
      StreamPtr s = pick_stream(a, nullptr);
      Array r = make_output(nullptr, keepdims ? Shape{1, 1} : Shape{}, a.dtype, a.device, s, {&a});
      a.data->wait_last_write_on(s);
      const int op = k == ReduceKernel::Max ? MUSAPY_RED_MAX : MUSAPY_RED_MIN;
      if (musapy_reduce_2d_ordered_v1(op, dt, a.data_ptr(), r.data_ptr(), a.shape()[0], a.shape()[1],
                                      s->reduce_workspace(), Stream::kReduceWorkspaceBytes, s->raw()) == 0) {
        s->note_bounded_wait();
        check_launch(rname(k));
        a.data->record_read(s);
        r.data->record_write(s);
        return r;
      }
    }
  }
  std::optional<Array> cur;
  for (size_t x : ax) cur = reduction_axis(cur ? *cur : a, x, true, nullptr, k);
  if (keepdims) return *cur;
  Array res = *cur;
  for (size_t i = 0; i < ax.size(); ++i) res = index_select(res, ax[i] - i, 0);
  return res;
}

// reduction.rs:186-226
Array arg_reduce_multi(const Array& a, const std::vector<ssize_t>* axes, bool keepdims, const Array* out,
                       ReduceKernel k) {
  std::vector<size_t> ax = resolve_axes(axes, a.ndim());
  if (ax.empty()) return reduction_axis(a, std::nullopt, keepdims, out, k);
  if (ax.size() == 1) return reduction_axis(a, ax[0], keepdims, out, k);
  const size_t nd = a.ndim();
  std::vector<size_t> perm;
  for (size_t i = 0; i < nd; ++i)
    if (std::find(ax.begin(), ax.end(), i) == ax.end()) perm.push_back(i);
  perm.insert(perm.end(), ax.begin(), ax.end());
  Array t = transpose(a, &perm);
  Array cont = contiguous(t);
  Array merged = reshape_merge_last(cont, ax.size());
  Array res = reduction_axis(merged, merged.ndim() - 1, keepdims, out, k);
  if (!keepdims) return res;
  Array split = reshape_split_last(res, ax.size());
  std::vector<size_t> inv(nd);
  for (size_t i = 0; i < nd; ++i) inv[perm[i]] = i;
  return transpose(split, &inv);
}

// op_builder.rs:3144-3363
Array cumsum_op(const Array& a, std::optional<size_t> axis, const Array* out) {
  const Shape in_shape = a.shape();
  const size_t total = shape_numel(in_shape);
  Shape out_shape = axis ? in_shape : Shape{total};
  Shape kshape = out_shape;
  const int kaxis = axis ? int(*axis) : 0;
  Dtype ct = (a.dtype == Dtype::Float32 || a.dtype == Dtype::Float64) ? a.dtype : Dtype::Int64;
  const size_t out_size = shape_numel(out_shape);
  check_out("cumsum", out, out_shape, ct, a, "expected", "expected");
  StreamPtr s = pick_stream(a, out);
  std::optional<Array> cast;
  if (a.dtype != ct) cast = cast_array(a, ct, s);
  const Array* aw = cast ? &*cast : &a;
  Array r = make_output(out, out_shape, ct, a.device, s, {aw});
  aw->data->wait_last_write_on(s);
  std::optional<Array> flat;
  if (!axis && !aw->layout.has_contiguous_strides()) {
    flat = contiguous(*aw);
    flat->data->wait_last_write_on(s);
    aw = &*flat;
  }
  if (out_size > 0) {
    Strides kstrides = axis ? aw->layout.strides : Strides{1};
    const size_t axis_len = kshape[kaxis];
    const size_t bpr = (axis_len + 255) / 256;
    // capacity limit of the reference's hierarchical scan, kept for API parity (op_builder.rs:3291-3300)
    if (bpr > 65536)
      throw ShapeError("cumsum: axis_len " + std::to_string(axis_len) +
                       " exceeds max supported length 16777216 (256^3)");
    const size_t rows = out_size / std::max<size_t>(axis_len, 1);
    const int nd = int(kshape.size());
    s->note_bounded_wait();  // row scans split into tiles wait on their predecessors
    // Every cumsum reports its waits to the stream's workspace.  Many rows: the chained scan on
    // that zeroed workspace (no scratch, no clear launch); fewer rows of several tiles: the
    // look-back, on scratch of the reference's size (op_builder.rs:3315-3321), taken only when
    // the first call reports that the path needs it.
    const int dt = ct == Dtype::Int64 ? MUSAPY_DT_I64 : ct == Dtype::Float32 ? MUSAPY_DT_F32 : MUSAPY_DT_F64;
    void* ws = s->reduce_workspace();
    BufferRef tmp;
    if (musapy_cumsum_ws_v2(dt, aw->data_ptr(), r.data_ptr(), nullptr, 0, nd, kshape.data(), kstrides.data(), kaxis,
                            axis_len, out_size, ws, Stream::kReduceWorkspaceBytes, s->raw()) != 0) {
      (void)musapy_kernels_take_error();  // 1: the path needs scratch (any other error recurs below)
      const size_t scratch = (bpr > 256 ? rows * (bpr + (bpr + 255) / 256) : rows * bpr) * element_size(ct);
      tmp = Buffer::alloc(std::max<size_t>(scratch, 8), a.device, s);
      (void)musapy_cumsum_ws_v2(dt, aw->data_ptr(), r.data_ptr(), tmp->ptr(), tmp->nbytes(), nd, kshape.data(),
                                kstrides.data(), kaxis, axis_len, out_size, ws, Stream::kReduceWorkspaceBytes,
                                s->raw());
    }
    check_launch("cumsum");
  }
  aw->data->record_read(s);
  r.data->record_write(s);
  return r;
}

// ---------------------------------------------------------------------------------------------
// views (rust/musapy-ops/src/indexing.rs:30-149) and materialisation (181-237)
Array transpose(const Array& a, const std::vector<size_t>* axes) { return a.view(a.layout.transposed(axes)); }

Array flip(const Array& a, size_t axis) { return a.view(a.layout.flipped(axis)); }

Array slice(const Array& a, const std::vector<size_t>& start, const std::vector<size_t>& stop,
            const std::vector<size_t>& step) {
  return a.view(a.layout.sliced(start, stop, step));
}

Array index_select(const Array& a, size_t axis, size_t index) {
  if (axis >= a.ndim()) throw ShapeError("index_select: axis out of bounds");
  if (index >= a.shape()[axis]) throw ShapeError("index_select: index out of bounds");
  Layout l;
  l.offset = size_t(ssize_t(a.layout.offset) + ssize_t(index) * a.layout.strides[axis]);
  for (size_t i = 0; i < a.ndim(); ++i) {
    if (i == axis) continue;
    l.shape.push_back(a.layout.shape[i]);
    l.strides.push_back(a.layout.strides[i]);
  }
  return a.view(l);
}

Array reshape_merge_last(const Array& a, size_t k) {
  if (k == 0 || k > a.ndim()) throw ShapeError("reshape_merge_last: invalid number of dims");
  if (!a.layout.has_contiguous_strides()) throw ShapeError("reshape_merge_last: requires contiguous strides");
  Shape s(a.shape().begin(), a.shape().end() - k);
  size_t m = 1;
  for (size_t i = a.ndim() - k; i < a.ndim(); ++i) m *= a.shape()[i];
  s.push_back(m);
  Layout l = Layout::from_shape(s);
  l.offset = a.layout.offset;
  return a.view(l);
}

Array reshape_split_last(const Array& a, size_t k) {
  if (a.ndim() == 0 || a.shape().back() != 1) throw ShapeError("reshape_split_last: last dim must be 1");
  Shape s(a.shape().begin(), a.shape().end() - 1);
  for (size_t i = 0; i < k; ++i) s.push_back(1);
  Layout l = Layout::from_shape(s);
  l.offset = a.layout.offset;
  return a.view(l);
}

Array contiguous(const Array& a) {
  if (a.is_contiguous()) return a;
  StreamPtr s = current_stream() ? current_stream() : a.stream;
  Array r = new_array(a.shape(), a.dtype, a.device, s);
  a.data->wait_last_write_on(s);
  if (a.size() > 0) {
    const size_t es = element_size(a.dtype);
    Shape sh = a.shape();
    Strides st = a.layout.strides;
    const int nd = int(sh.size());
    // the transposed view of a C-contiguous 2-D array takes the reference's transpose2d entry
    // point (indexing.rs:833-838); everything else the general stride-aware copy
    const bool t2d = nd == 2 && st[0] == 1 && st[1] == ssize_t(sh[0]);
    if (t2d && es == 4) {
      musapy_copy_transpose2d_i32((const int32_t*)a.data_ptr(), (int32_t*)r.data_ptr(), sh[0], sh[1], s->raw());
    } else if (t2d && es == 8) {
      musapy_copy_transpose2d_i64((const int64_t*)a.data_ptr(), (int64_t*)r.data_ptr(), sh[0], sh[1], s->raw());
    } else switch (es) {
      case 1: musapy_copy_u8((const uint8_t*)a.data_ptr(), (uint8_t*)r.data_ptr(), nd, sh.data(), st.data(), s->raw()); break;
      case 2: musapy_copy_u16((const uint16_t*)a.data_ptr(), (uint16_t*)r.data_ptr(), nd, sh.data(), st.data(), s->raw()); break;
      case 4: musapy_copy_i32((const int32_t*)a.data_ptr(), (int32_t*)r.data_ptr(), nd, sh.data(), st.data(), s->raw()); break;
      case 8: musapy_copy_i64((const int64_t*)a.data_ptr(), (int64_t*)r.data_ptr(), nd, sh.data(), st.data(), s->raw()); break;
      default:
        musapy_copy_c128((const musapy_c128_t*)a.data_ptr(), (musapy_c128_t*)r.data_ptr(), nd, sh.data(), st.data(),
                         s->raw());
    }
    check_launch("contiguous");
  }
  a.data->record_read(s);
  r.data->record_write(s);
  return r;
}

}  // namespace ops
}  // namespace mpy
