// ops.hpp -- public operators of the op layer.
//
// C++ counterpart of rust/musapy-ops/src/{elementwise,reduction,op_builder,broadcast,indexing}.rs
// for the stride-aware elementwise + reduction path.  Every operator keeps the reference's
// three phases: A) parse (device, broadcast, promotion, whitelist, out=, stream, internal cast,
// allocation, alias check, stream wait), B) launch through the C kernel ABI
// (include/musapy_kernels.h), C) post (event bookkeeping, output Array).
#pragma once

#include <optional>

#include "core.hpp"

namespace mpy {
namespace ops {

enum class BinaryKernel { Add, Sub, Mul, Div, Pow };
enum class UnaryKernel { Sin, Cos, Exp, Log, Abs, Sign, Neg };
enum class ReduceKernel { Sum, Prod, Max, Min, Mean, Argmax, Argmin };
enum class CompareKernel { Eq, Ne, Lt, Gt, Le, Ge };

// broadcast.rs:24-92
Shape broadcast_shape(const std::vector<Shape>& shapes);
Strides broadcast_strides(const Layout& layout, const Shape& target);

// op_builder.rs:315 / 550 / 740 / 1055 / 1130
Array binary_elementwise(const Array& a, const Array& b, const Array* out, BinaryKernel k);
// op_builder.rs:1338-1557: output dtype is always bool (one 0/1 byte per element)
Array comparison_elementwise(const Array& a, const Array& b, const Array* out, CompareKernel k);
Array unary_elementwise(const Array& a, const Array* out, UnaryKernel k);
Array clamp_elementwise(const Array& a, double lo, double hi, const Array* out);
Array cast_array(const Array& a, Dtype target, const StreamPtr& stream);
Array astype_op(const Array& a, Dtype dtype, const Array* out);
void validate_cast_pair(Dtype src, Dtype dst);

// reduction.rs:21-235 + op_builder.rs:2310 / 3144
std::optional<size_t> resolve_axis(std::optional<ssize_t> axis, size_t ndim);
std::vector<size_t> resolve_axes(const std::vector<ssize_t>* axes, size_t ndim);
Array reduction_axis(const Array& a, std::optional<size_t> axis, bool keepdims, const Array* out, ReduceKernel k);
Array reduce_multi(const Array& a, const std::vector<ssize_t>* axes, bool keepdims, const Array* out,
                   ReduceKernel k);
Array arg_reduce_multi(const Array& a, const std::vector<ssize_t>* axes, bool keepdims, const Array* out,
                       ReduceKernel k);
Array cumsum_op(const Array& a, std::optional<size_t> axis, const Array* out);

// indexing.rs views + materialisation
Array transpose(const Array& a, const std::vector<size_t>* axes);
Array flip(const Array& a, size_t axis);
Array slice(const Array& a, const std::vector<size_t>& start, const std::vector<size_t>& stop,
            const std::vector<size_t>& step);
Array index_select(const Array& a, size_t axis, size_t index);
Array reshape_merge_last(const Array& a, size_t k);
Array reshape_split_last(const Array& a, size_t k);
Array contiguous(const Array& a);

// DLPack exchange (interop.cpp).  export_dlpack returns a DLManagedTensor* (versioned = false)
// or a DLManagedTensorVersioned* (versioned = true) whose deleter keeps the array alive; with
// `sync`, `consumer` waits for the array's last write.  import_dlpack adopts a producer's
// kDLROCM tensor without a copy (ownership of `managed` passes to the returned array).
void* export_dlpack(const Array& a, bool versioned, bool sync, hipStream_t consumer, bool copy);
Array import_dlpack(void* managed, bool versioned);

// stream resolution used by every Phase A (op_builder.rs:402-405, resolution.rs:184)
StreamPtr pick_stream(const Array& a, const Array* out);

// Phase C in debug mode (op_builder.rs:507-521): records the op's OpContext (name, the inputs'
// shapes, devices and dtypes, the output's shape, the caller's Python frame when the binding set
// one) on the output's stream; nothing when debug mode is off.
void record_op(const char* name, std::initializer_list<const Array*> inputs, const Array& out);

}  // namespace ops
}  // namespace mpy
