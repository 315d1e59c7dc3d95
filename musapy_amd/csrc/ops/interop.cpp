// interop.cpp -- zero-copy array exchange over DLPack.
//
// The reference plans this as DLPack export/import on its Array (docs/v0.4-beta-plan-zh.md:42-43,
// 96-125): __dlpack__ hands out the device buffer, kept alive by the capsule's deleter, and
// from_dlpack adopts a producer's device buffer without a copy.  Here the device is a HIP device
// (kDLROCM), so PyTorch-ROCm tensors and this backend's arrays exchange memory directly.
//
// Stream semantics follow the Python array API's __dlpack__(stream=...) contract:
//  * export: the consumer names its stream; that stream waits (on the device, through an event)
//    for the array's last write before the consumer sees the tensor.  When the consumer releases
//    the tensor, this backend's allocation stream waits for the consumer's stream before the
//    memory can be reused, so queued consumer work never reads a recycled block.  stream = -1
//    skips the first wait; the release then waits for the whole device.
//  * import: the producer is asked to order its work before this backend's stream; the adopted
//    buffer is handed back (the producer's deleter) only after every stream that used it here
//    has drained.
#include "dlpack.hpp"

#include <cstring>

#include "ops.hpp"
#include "../../../include/musapy_hip_runtime.h"

namespace mpy {
namespace ops {

namespace {

DLDataType dl_dtype(Dtype d) {
  const uint8_t bits = uint8_t(element_size(d) * 8);
  switch (dtype_category(d)) {
    case 0: return DLDataType{kDLBool, 8, 1};
    case 1: return DLDataType{kDLInt, bits, 1};
    case 2: return DLDataType{kDLUInt, bits, 1};
    case 3: return DLDataType{uint8_t(d == Dtype::Bfloat16 ? kDLBfloat : kDLFloat), bits, 1};
    default: return DLDataType{kDLComplex, bits, 1};
  }
}

Dtype from_dl_dtype(DLDataType t) {
  if (t.lanes != 1) throw InteropError("from_dlpack: vector dtypes (lanes=" + std::to_string(t.lanes) + ") are not supported");
  switch (t.code) {
    case kDLBool:
      if (t.bits == 8) return Dtype::Bool;
      break;
    case kDLInt:
      switch (t.bits) {
        case 8: return Dtype::Int8;
        case 16: return Dtype::Int16;
        case 32: return Dtype::Int32;
        case 64: return Dtype::Int64;
      }
      break;
    case kDLUInt:
      switch (t.bits) {
        case 8: return Dtype::Uint8;
        case 16: return Dtype::Uint16;
        case 32: return Dtype::Uint32;
        case 64: return Dtype::Uint64;
      }
      break;
    case kDLFloat:
      switch (t.bits) {
        case 16: return Dtype::Float16;
        case 32: return Dtype::Float32;
        case 64: return Dtype::Float64;
      }
      break;
    case kDLBfloat:
      if (t.bits == 16) return Dtype::Bfloat16;
      break;
    case kDLComplex:
      if (t.bits == 64) return Dtype::Complex64;
      if (t.bits == 128) return Dtype::Complex128;
      break;
  }
  throw InteropError("from_dlpack: unsupported DLPack dtype (code " + std::to_string(int(t.code)) + ", " +
                     std::to_string(int(t.bits)) + " bits)");
}

// make `waiter` wait for the work queued so far on `target` (device-side; no host block)
void order_after(hipStream_t waiter, hipStream_t target) {
  if (waiter == target) return;
  hipEvent_t ev = nullptr;
  check_rt(mpy_rt_event_create(&ev, 0), "dlpack event");
  int e = mpy_rt_event_record(ev, target);
  if (e == 0) e = mpy_rt_stream_wait_event(waiter, ev);
  mpy_rt_event_destroy(ev);
  check_rt(e, "dlpack stream ordering");
}

struct ExportCtx {
  Array keep;  // holds the buffer until the consumer releases the tensor
  std::vector<int64_t> shape, strides;
  hipStream_t consumer = nullptr;
  bool consumer_known = false;
  DLManagedTensor legacy{};
  DLManagedTensorVersioned versioned{};
};

void release_export(ExportCtx* ctx) {
  // The consumer is done with the tensor on the host side; its queued kernels may still read
  // it.  Order the buffer's allocation stream after them before the block can be recycled.
  const StreamPtr& home = ctx->keep.data->home();
  int e = -1;
  if (ctx->consumer_known && home) {
    hipEvent_t ev = nullptr;
    e = mpy_rt_event_create(&ev, 0);
    if (e == 0) {
      e = mpy_rt_event_record(ev, ctx->consumer);
      if (e == 0 && home->raw() != ctx->consumer) e = mpy_rt_stream_wait_event(home->raw(), ev);
      mpy_rt_event_destroy(ev);
    }
  }
  if (e != 0) (void)mpy_rt_device_synchronize();  // unknown consumer stream (or a failed wait)
  delete ctx;
}

void legacy_deleter(DLManagedTensor* t) { release_export(static_cast<ExportCtx*>(t->manager_ctx)); }
void versioned_deleter(DLManagedTensorVersioned* t) { release_export(static_cast<ExportCtx*>(t->manager_ctx)); }

DLTensor describe(ExportCtx* ctx) {
  const Array& a = ctx->keep;
  ctx->shape.assign(a.shape().begin(), a.shape().end());
  ctx->strides.assign(a.layout.strides.begin(), a.layout.strides.end());
  DLTensor t{};
  t.data = a.data_ptr();
  t.device = DLDevice{kDLROCM, a.device};
  t.ndim = int32_t(a.ndim());
  t.dtype = dl_dtype(a.dtype);
  t.shape = ctx->shape.empty() ? nullptr : ctx->shape.data();
  t.strides = ctx->strides.empty() ? nullptr : ctx->strides.data();
  t.byte_offset = 0;
  return t;
}

}  // namespace

void* export_dlpack(const Array& a, bool versioned, bool sync, hipStream_t consumer, bool copy) {
  Array src = a;
  if (copy) {  // an independent copy the consumer may own and modify
    src = contiguous(a);
    if (src.data.get() == a.data.get()) {
      Array c = new_array(a.shape(), a.dtype, a.device, a.stream);
      a.data->wait_last_write_on(a.stream);
      check_rt(mpy_rt_memcpy_d2d(c.data_ptr(), a.data_ptr(), a.nbytes(), a.stream->raw()), "dlpack copy");
      a.data->record_read(a.stream);
      c.data->record_write(a.stream);
      src = c;
    }
  }
  auto* ctx = new ExportCtx();
  ctx->keep = src;
  ctx->consumer = consumer;
  ctx->consumer_known = sync;
  try {
    if (sync) {
      const StreamPtr& w = src.data->last_writer() ? src.data->last_writer() : src.stream;
      order_after(consumer, w->raw());
    }
  } catch (...) {
    delete ctx;
    throw;
  }
  if (versioned) {
    ctx->versioned.version = DLPackVersion{1, 0};
    ctx->versioned.manager_ctx = ctx;
    ctx->versioned.deleter = versioned_deleter;
    ctx->versioned.flags = copy ? kDLFlagIsCopied : 0;
    ctx->versioned.dl_tensor = describe(ctx);
    return &ctx->versioned;
  }
  ctx->legacy.manager_ctx = ctx;
  ctx->legacy.deleter = legacy_deleter;
  ctx->legacy.dl_tensor = describe(ctx);
  return &ctx->legacy;
}

Array import_dlpack(void* managed, bool versioned) {
  DLTensor* t = versioned ? &static_cast<DLManagedTensorVersioned*>(managed)->dl_tensor
                          : &static_cast<DLManagedTensor*>(managed)->dl_tensor;
  auto release = [managed, versioned]() {
    if (versioned) {
      auto* m = static_cast<DLManagedTensorVersioned*>(managed);
      if (m->deleter) m->deleter(m);
    } else {
      auto* m = static_cast<DLManagedTensor*>(managed);
      if (m->deleter) m->deleter(m);
    }
  };
  try {
    if (t->device.device_type != kDLROCM)
      throw InteropError("from_dlpack: device type " + std::to_string(t->device.device_type) +
                         " is not a HIP device (kDLROCM = 10)");
    if (t->ndim < 0 || t->ndim > 32) throw InteropError("from_dlpack: ndim " + std::to_string(t->ndim) + " out of range");
    const Dtype dt = from_dl_dtype(t->dtype);
    const size_t es = element_size(dt);
    Layout l;
    l.shape.resize(size_t(t->ndim));
    for (int i = 0; i < t->ndim; ++i) {
      if (t->shape[i] < 0) throw InteropError("from_dlpack: negative dimension");
      l.shape[i] = size_t(t->shape[i]);
    }
    if (t->strides) {
      l.strides.assign(t->strides, t->strides + t->ndim);
    } else {
      l.strides = contiguous_strides(l.shape);
    }
    l.offset = 0;
    // extent of the elements the view can touch, for the allocation record
    int64_t lo = 0, hi = 0;
    for (int i = 0; i < t->ndim; ++i) {
      if (l.shape[i] == 0) {
        lo = hi = 0;
        break;
      }
      const int64_t span = int64_t(l.shape[i] - 1) * l.strides[i];
      (span < 0 ? lo : hi) += span;
    }
    char* base = static_cast<char*>(t->data) + t->byte_offset;
    StreamPtr s = current_stream();
    const int device = t->device.device_id;
    if (!s || s->device() != device) s = default_stream(device);
    Array a;
    a.data = Buffer::adopt(base, size_t(hi - lo + 1) * es, device, s, release);
    a.layout = l;
    a.dtype = dt;
    a.stream = s;
    a.device = device;
    return a;
  } catch (...) {
    release();
    throw;
  }
}

}  // namespace ops
}  // namespace mpy
