// core.cpp -- implementation of the op layer's core types (see core.hpp).
#include "core.hpp"

#include <strings.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <unordered_map>

#include "../../../include/musapy_hip_runtime.h"

namespace mpy {
namespace ops {

// ---------------------------------------------------------------------------------------------
// dtypes -- rust/musapy-core/src/dtype.rs:56-150
size_t element_size(Dtype d) {
  switch (d) {
    case Dtype::Bool: case Dtype::Int8: case Dtype::Uint8: return 1;
    case Dtype::Int16: case Dtype::Uint16: case Dtype::Float16: case Dtype::Bfloat16: return 2;
    case Dtype::Int32: case Dtype::Uint32: case Dtype::Float32: return 4;
    case Dtype::Int64: case Dtype::Uint64: case Dtype::Float64: case Dtype::Complex64: return 8;
    case Dtype::Complex128: return 16;
  }
  return 0;
}

const char* dtype_name(Dtype d) {
  static const char* n[] = {"bool", "int8", "int16", "int32", "int64", "uint8", "uint16", "uint32",
                            "uint64", "float16", "float32", "float64", "bfloat16", "complex64", "complex128"};
  return n[int(d)];
}

const char* dtype_short(Dtype d) {
  static const char* n[] = {"bool", "i8", "i16", "i32", "i64", "u8", "u16", "u32",
                            "u64", "f16", "f32", "f64", "bf16", "c64", "c128"};
  return n[int(d)];
}

Dtype parse_dtype(const std::string& s) {
  for (int i = 0; i <= int(Dtype::Complex128); ++i) {
    Dtype d = Dtype(i);
    if (s == dtype_name(d) || s == dtype_short(d)) return d;
  }
  throw DtypeError("unknown dtype '" + s + "'");
}

int dtype_category(Dtype d) {
  switch (d) {
    case Dtype::Bool: return 0;
    case Dtype::Int8: case Dtype::Int16: case Dtype::Int32: case Dtype::Int64: return 1;
    case Dtype::Uint8: case Dtype::Uint16: case Dtype::Uint32: case Dtype::Uint64: return 2;
    case Dtype::Float16: case Dtype::Float32: case Dtype::Float64: case Dtype::Bfloat16: return 3;
    case Dtype::Complex64: case Dtype::Complex128: return 4;
  }
  return 0;
}

int precision_width(Dtype d) {
  switch (d) {
    case Dtype::Bool: case Dtype::Int8: case Dtype::Uint8: return 8;
    case Dtype::Int16: case Dtype::Uint16: case Dtype::Float16: case Dtype::Bfloat16: return 16;
    case Dtype::Int32: case Dtype::Uint32: case Dtype::Float32: case Dtype::Complex64: return 32;
    default: return 64;
  }
}

bool is_complex(Dtype d) { return d == Dtype::Complex64 || d == Dtype::Complex128; }

namespace {
Dtype int_of_width(int w) {
  return w == 8 ? Dtype::Int8 : w == 16 ? Dtype::Int16 : w == 32 ? Dtype::Int32 : Dtype::Int64;
}
Dtype complex_of_width(int w) { return w <= 32 ? Dtype::Complex64 : Dtype::Complex128; }

// JAX promotion table, dtype.rs:206-284
Dtype jax_promote(Dtype a, Dtype b) {
  if (a == b) return a;
  if (a == Dtype::Bool) return b;
  if (b == Dtype::Bool) return a;
  int ca = dtype_category(a), pa = precision_width(a);
  int cb = dtype_category(b), pb = precision_width(b);
  if (ca == cb) {
    if (ca == 3 && pa == pb) return Dtype::Float32;  // f16 + bf16
    return pa >= pb ? a : b;
  }
  if ((ca == 1 && cb == 2) || (ca == 2 && cb == 1)) {
    int iw = ca == 1 ? pa : pb, uw = ca == 1 ? pb : pa;
    return int_of_width(iw > uw ? iw : std::min(uw * 2, 64));
  }
  // exact + float: the float type (an integer never widens the float, dtype.rs:250-268)
  if ((ca == 1 || ca == 2) && cb == 3) return b;
  if ((cb == 1 || cb == 2) && ca == 3) return a;
  if ((ca == 1 || ca == 2) && cb == 4) return complex_of_width(std::max({pa, pb, 32}));
  if ((cb == 1 || cb == 2) && ca == 4) return complex_of_width(std::max({pb, pa, 32}));
  if ((ca == 3 && cb == 4) || (ca == 4 && cb == 3)) return complex_of_width(std::max(pa, pb));
  throw DtypeError(std::string("cannot promote ") + dtype_name(a) + " with " + dtype_name(b));
}
}  // namespace

// dtype.rs:306-334
Dtype promote(Dtype a, Dtype b, bool all_gpu) {
  if (a == b) return a;
  Dtype jax = jax_promote(a, b);
  if (!all_gpu) return jax;
  int ca = dtype_category(a), pa = precision_width(a);
  int cb = dtype_category(b), pb = precision_width(b);
  if (ca != cb) return jax;
  bool conflict = ca == 3 && pa == pb &&
                  ((a == Dtype::Float16 && b == Dtype::Bfloat16) || (a == Dtype::Bfloat16 && b == Dtype::Float16));
  if (conflict) return jax;
  return pa <= pb ? a : b;
}

// ---------------------------------------------------------------------------------------------
// layouts -- rust/musapy-core/src/layout.rs
Strides contiguous_strides(const Shape& shape) {
  Strides s(shape.size());
  ssize_t acc = 1;
  for (size_t i = shape.size(); i-- > 0;) {
    s[i] = acc;
    acc *= ssize_t(shape[i]);
  }
  return s;
}

size_t shape_numel(const Shape& shape) {
  size_t n = 1;
  for (size_t d : shape) n *= d;
  return n;
}

Layout Layout::from_shape(const Shape& s) {
  Layout l;
  l.shape = s;
  l.strides = contiguous_strides(s);
  l.offset = 0;
  return l;
}

bool Layout::has_contiguous_strides() const { return strides == contiguous_strides(shape); }

Layout Layout::transposed(const std::vector<size_t>* axes) const {
  size_t nd = ndim();
  if (nd == 0) return *this;
  std::vector<size_t> perm(nd);
  if (!axes) {
    for (size_t i = 0; i < nd; ++i) perm[i] = nd - 1 - i;
  } else {
    if (axes->size() != nd)
      throw ShapeError("axes length " + std::to_string(axes->size()) + " != ndim " + std::to_string(nd));
    std::vector<bool> seen(nd, false);
    for (size_t a : *axes) {
      if (a >= nd || seen[a])
        throw ShapeError("invalid or duplicate axis " + std::to_string(a) + " for ndim " + std::to_string(nd));
      seen[a] = true;
    }
    perm = *axes;
  }
  Layout r;
  r.offset = offset;
  for (size_t i = 0; i < nd; ++i) {
    r.shape.push_back(shape[perm[i]]);
    r.strides.push_back(strides[perm[i]]);
  }
  return r;
}

Layout Layout::flipped(size_t axis) const {
  if (axis >= ndim())
    throw ShapeError("flip axis " + std::to_string(axis) + " out of bounds for ndim " + std::to_string(ndim()));
  Layout r = *this;
  r.strides[axis] = -strides[axis];
  // the offset moves to the axis' last element (layout.rs:183-205); an empty axis has none, and
  // its view keeps the offset rather than wrapping it below zero as the reference's does
  if (shape[axis] > 0) r.offset = size_t(ssize_t(offset) + (ssize_t(shape[axis]) - 1) * strides[axis]);
  return r;
}

Layout Layout::sliced(const std::vector<size_t>& start, const std::vector<size_t>& stop,
                      const std::vector<size_t>& step) const {
  size_t nd = ndim();
  if (start.size() != nd || stop.size() != nd || step.size() != nd)
    throw ShapeError("slice ranges length " + std::to_string(start.size()) + " != ndim " + std::to_string(nd));
  Layout r;
  ssize_t off = ssize_t(offset);
  for (size_t i = 0; i < nd; ++i) {
    if (step[i] == 0) throw ShapeError("slice step cannot be zero");
    if (start[i] > stop[i] || stop[i] > shape[i])
      throw ShapeError("slice [" + std::to_string(start[i]) + ", " + std::to_string(stop[i]) + ", " +
                       std::to_string(step[i]) + "] out of bounds for dimension " + std::to_string(i) + " (size " +
                       std::to_string(shape[i]) + ")");
    size_t dim = stop[i] > start[i] ? (stop[i] - start[i] + step[i] - 1) / step[i] : 0;
    r.shape.push_back(dim);
    r.strides.push_back(strides[i] * ssize_t(step[i]));
    off += ssize_t(start[i]) * strides[i];
  }
  r.offset = size_t(off);
  return r;
}

// ---------------------------------------------------------------------------------------------
// errors from the runtime layer
void check_rt(int code, const char* what) {
  if (code == 0) return;
  std::string msg = std::string(what) + ": " + mpy_rt_error_string(code);
  if (code == 2 /* hipErrorOutOfMemory */) throw OutOfMemoryError(msg);
  if (code == 100 /* hipErrorNoDevice */ || code == 101 /* hipErrorInvalidDevice */) throw DeviceError(msg);
  throw StreamError(msg);
}

void check_launch(const char* label) {
  int code = mpy_rt_check_launch();
  if (code != 0) throw KernelError(std::string("kernel launch failed (") + label + "): " + mpy_rt_error_string(code));
}

// ---------------------------------------------------------------------------------------------
// debug mode and op contexts (rust/musapy-core/src/debug.rs:20-100, stream.rs:42-101)
namespace {
std::once_flag g_debug_init;
std::atomic<bool> g_debug{false};
thread_local bool t_has_frame = false;
thread_local PythonFrame t_frame;

std::string shape_str(const Shape& s) {
  std::string r = "(";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + (s.size() == 1 ? ",)" : ")");
}
}  // namespace

bool is_debug() {
  std::call_once(g_debug_init, [] {
    const char* v = std::getenv("MUSAPY_DEBUG");
    if (v && (std::strcmp(v, "1") == 0 || strcasecmp(v, "true") == 0)) g_debug.store(true, std::memory_order_relaxed);
  });
  return g_debug.load(std::memory_order_relaxed);
}
void set_debug(bool enabled) {
  is_debug();  // the environment is read first, so a later first query cannot override this
  g_debug.store(enabled, std::memory_order_relaxed);
}
void set_debug_frame(const PythonFrame* frame) {
  t_has_frame = frame != nullptr;
  if (frame) t_frame = *frame;
}
bool take_debug_frame(PythonFrame& out) {
  if (!t_has_frame) return false;
  t_has_frame = false;
  out = std::move(t_frame);
  return true;
}

std::string OpContext::to_string() const {
  std::string r = "op '" + op_name + "' on stream " + std::to_string(stream_id);
  if (!input_shapes.empty()) {
    r += ", inputs=[";
    for (size_t i = 0; i < input_shapes.size(); ++i) {
      r += (i ? ", " : "") + shape_str(input_shapes[i]);
      if (i < input_dtypes.size()) r += std::string(" ") + dtype_short(input_dtypes[i]);
    }
    r += "]";
  }
  if (has_frame) r += " at " + frame.filename + ":" + std::to_string(frame.lineno) + " (" + frame.function + ")";
  return r;
}

// ---------------------------------------------------------------------------------------------
// streams
namespace {
std::atomic<uint64_t> g_stream_ids{1};
std::mutex g_streams_mu;
std::vector<StreamPtr> g_default_streams;
thread_local StreamPtr g_current_stream;
// streams with bounded-wait work queued since their last synchronize, by id (synchronize_device)
std::mutex g_wait_mu;
std::unordered_map<uint64_t, std::weak_ptr<Stream>> g_wait_streams;
void unregister_wait(uint64_t id) {
  std::lock_guard<std::mutex> lk(g_wait_mu);
  g_wait_streams.erase(id);
}
}  // namespace

Stream::Stream(int device, hipStream_t raw, bool owned)
    : device_(device), raw_(raw), owned_(owned), id_(g_stream_ids.fetch_add(1)) {}

Stream::~Stream() {
  if (wait_check_) unregister_wait(id_);
  if (workspace_) mpy_rt_free(workspace_, raw_);
  if (owned_ && raw_) mpy_rt_stream_destroy(raw_);
}

void* Stream::reduce_workspace() {
  if (!workspace_) {
    void* p = nullptr;
    check_rt(mpy_rt_malloc(&p, kReduceWorkspaceBytes, device_, raw_), "reduction workspace");
    int code = mpy_rt_fill_u32(p, 0u, kReduceWorkspaceBytes, raw_);
    if (code != 0) {
      mpy_rt_free(p, raw_);
      check_rt(code, "reduction workspace clear");
    }
    workspace_ = p;
  }
  return workspace_;
}

void Stream::note_bounded_wait() {
  if (wait_check_) return;
  wait_check_ = true;
  std::lock_guard<std::mutex> lk(g_wait_mu);
  g_wait_streams[id_] = weak_from_this();
}

void Stream::record_op(OpContext ctx) {
  std::lock_guard<std::mutex> lk(ops_mu_);
  pending_ops_.push_back(std::move(ctx));
}
size_t Stream::pending_count() const {
  std::lock_guard<std::mutex> lk(ops_mu_);
  return pending_ops_.size();
}
std::string Stream::oldest_op_string() const {
  std::lock_guard<std::mutex> lk(ops_mu_);
  return pending_ops_.empty() ? std::string() : pending_ops_.front().to_string();
}
void Stream::clear_pending_ops() {
  std::lock_guard<std::mutex> lk(ops_mu_);
  pending_ops_.clear();
}
std::string Stream::failed_op_suffix() const {
  const std::string o = oldest_op_string();
  return o.empty() ? o : " | failed op: " + o;
}

void Stream::synchronize() {
  int code = mpy_rt_stream_synchronize(raw_);
  if (code != 0) {
    poisoned_ = true;
    throw StreamError(std::string("stream synchronize failed: ") + mpy_rt_error_string(code) + failed_op_suffix());
  }
  if (wait_check_) {
    wait_check_ = false;
    unregister_wait(id_);
    // the workspace holds the fault word of every bounded wait queued on this stream
    const int fault = workspace_ ? mpy_rt_take_fault_ws(workspace_, kReduceWorkspaceBytes, raw_) : 0;
    if (fault != 0) {
      poisoned_ = true;
      const std::string failed = failed_op_suffix();
      if (fault < 0) {
        mpy_rt_free(workspace_, raw_);  // never reuse slots that may be stale
        workspace_ = nullptr;
        throw StreamError("stream synchronize: the stream's wait-fault word could not be read" + failed);
      }
      std::string what;
      if (fault & 1) what += "a single-launch reduction's combiner";
      if (fault & 2) what += std::string(what.empty() ? "" : " and ") + "a cumsum look-back";
      throw KernelError("device wait expired in " + what + " on stream " + std::to_string(id_) +
                        ": results of the work queued on this stream since its last synchronize are invalid "
                        "(stream poisoned)" + failed);
    }
  }
  clear_pending_ops();
}

void synchronize_device(int device) {
  check_rt(mpy_rt_set_device(device), "set device");
  check_rt(mpy_rt_device_synchronize(), "device synchronize");
  std::vector<StreamPtr> pending{default_stream(device)};
  {
    std::vector<std::weak_ptr<Stream>> ws;
    {
      // the streams are locked outside the mutex: dropping the last reference runs ~Stream,
      // which takes it
      std::lock_guard<std::mutex> lk(g_wait_mu);
      for (auto& kv : g_wait_streams) ws.push_back(kv.second);
    }
    for (auto& w : ws) {
      StreamPtr s = w.lock();
      if (s && s->device() == device && s != pending.front()) pending.push_back(std::move(s));
    }
  }
  std::exception_ptr first;
  for (auto& s : pending) {
    try {
      s->synchronize();
    } catch (...) {
      if (!first) first = std::current_exception();
    }
  }
  if (first) std::rethrow_exception(first);
}

StreamPtr Stream::create(int device) {
  hipStream_t s = nullptr;
  check_rt(mpy_rt_stream_create(&s, device), "stream create");
  return std::make_shared<Stream>(device, s, true);
}

StreamPtr default_stream(int device) {
  std::lock_guard<std::mutex> lk(g_streams_mu);
  if (device < 0) throw DeviceError("invalid device index " + std::to_string(device));
  if (size_t(device) >= g_default_streams.size()) g_default_streams.resize(device + 1);
  if (!g_default_streams[device]) g_default_streams[device] = Stream::create(device);
  return g_default_streams[device];
}

StreamPtr current_stream() { return g_current_stream; }
void set_current_stream(StreamPtr s) { g_current_stream = std::move(s); }

// ---------------------------------------------------------------------------------------------
// buffers
namespace {
// make `waiter` wait for everything submitted so far on `target`
void stream_wait_stream(const StreamPtr& waiter, const StreamPtr& target) {
  if (!waiter || !target || waiter.get() == target.get()) return;
  hipEvent_t ev = nullptr;
  check_rt(mpy_rt_event_create(&ev, 0), "event create");
  int e = mpy_rt_event_record(ev, target->raw());
  if (e == 0) e = mpy_rt_stream_wait_event(waiter->raw(), ev);
  mpy_rt_event_destroy(ev);  // also when the record or the wait failed
  check_rt(e, "stream wait event");
}
}  // namespace

std::shared_ptr<Buffer> Buffer::alloc(size_t nbytes, int device, const StreamPtr& stream) {
  std::shared_ptr<Buffer> b(new Buffer());
  void* p = nullptr;
  int code = mpy_rt_malloc(&p, nbytes, device, stream ? stream->raw() : nullptr);
  if (code != 0) {
    std::string msg = "device allocation of " + std::to_string(nbytes) + " bytes failed: " + mpy_rt_error_string(code);
    if (code == 2) throw OutOfMemoryError(msg);
    throw MemoryError(msg);
  }
  b->ptr_ = p;
  b->nbytes_ = nbytes;
  b->device_ = device;
  b->home_ = stream;
  return b;
}

std::shared_ptr<Buffer> Buffer::adopt(void* ptr, size_t nbytes, int device, const StreamPtr& stream,
                                      std::function<void()> release) {
  std::shared_ptr<Buffer> b(new Buffer());
  b->ptr_ = ptr;
  b->nbytes_ = nbytes;
  b->device_ = device;
  b->home_ = stream;
  b->release_ = std::move(release);
  return b;
}

Buffer::~Buffer() {
  if (release_) {
    // the owner may reuse the memory as soon as it is released: let our queued work finish
    if (last_writer_) mpy_rt_stream_synchronize(last_writer_->raw());
    for (auto& r : readers_) mpy_rt_stream_synchronize(r->raw());
    if (home_) mpy_rt_stream_synchronize(home_->raw());
    try {
      release_();
    } catch (...) {
    }
    return;
  }
  if (!ptr_) return;
  // the free is ordered on the home stream: order it after the other streams' use first, or,
  // where that cannot be done (no home stream, a failing event call), wait for them on the host
  auto order_after = [this](const StreamPtr& s) {
    if (!s || (home_ && s.get() == home_.get())) return;
    try {
      if (!home_) throw StreamError("no home stream");
      stream_wait_stream(home_, s);
    } catch (...) {
      mpy_rt_stream_synchronize(s->raw());
    }
  };
  order_after(last_writer_);
  for (auto& r : readers_) order_after(r);
  mpy_rt_free(ptr_, home_ ? home_->raw() : nullptr);
}

void Buffer::wait_last_write_on(const StreamPtr& s) {
  if (last_writer_ && last_writer_.get() != s.get()) stream_wait_stream(s, last_writer_);
}

void Buffer::wait_reads_on(const StreamPtr& s) {
  for (auto& r : readers_)
    if (r.get() != s.get()) stream_wait_stream(s, r);
}

void Buffer::record_read(const StreamPtr& s) {
  if (home_ && s.get() == home_.get()) return;  // the free is ordered on the home stream anyway
  for (auto& r : readers_)
    if (r.get() == s.get()) return;
  readers_.push_back(s);
}

void Buffer::record_write(const StreamPtr& s) {
  readers_.clear();
  last_writer_ = s;
}

// ---------------------------------------------------------------------------------------------
// arrays
void* Array::data_ptr() const {
  return static_cast<char*>(data->ptr()) + layout.offset * element_size(dtype);
}

Array Array::view(const Layout& l) const {
  Array r = *this;
  r.layout = l;
  return r;
}

Array new_array(const Shape& shape, Dtype dtype, int device, const StreamPtr& stream) {
  // the kernels' rank limit (the reference's MUSAPY_MAX_NDIM, elementwise.mu:16); views and
  // broadcasts never exceed the rank of an array that was created
  if (shape.size() > 32)
    throw ShapeError("arrays have at most 32 dimensions (got " + std::to_string(shape.size()) + ")");
  Array a;
  a.layout = Layout::from_shape(shape);
  a.dtype = dtype;
  a.device = device;
  a.stream = stream;
  a.data = Buffer::alloc(std::max<size_t>(shape_numel(shape) * element_size(dtype), 1), device, stream);
  return a;
}

Array from_host(const void* src, const Shape& shape, Dtype dtype, int device) {
  // inside a stream context on this device the array belongs to that stream (resolution.rs)
  StreamPtr cur = current_stream();
  StreamPtr s = cur && cur->device() == device ? cur : default_stream(device);
  Array a = new_array(shape, dtype, device, s);
  size_t n = shape_numel(shape) * element_size(dtype);
  if (n) check_rt(mpy_rt_memcpy_h2d(a.data->ptr(), src, n, s->raw()), "host-to-device copy");
  return a;
}

std::vector<uint8_t> to_host(const Array& a) {
  const size_t es = element_size(a.dtype);
  const size_t n = a.size();
  std::vector<uint8_t> out(n * es);
  a.stream->synchronize();
  if (n == 0) return out;
  // span of the view in elements relative to the first element
  ssize_t lo = 0, hi = 0;
  for (size_t d = 0; d < a.ndim(); ++d) {
    ssize_t ext = (ssize_t(a.layout.shape[d]) - 1) * a.layout.strides[d];
    if (ext > 0) hi += ext; else lo += ext;
  }
  std::vector<uint8_t> span(size_t(hi - lo + 1) * es);
  const char* first = static_cast<const char*>(a.data_ptr());
  check_rt(mpy_rt_memcpy_d2h(span.data(), first + lo * ssize_t(es), span.size(), a.stream->raw()),
           "device-to-host copy");
  if (a.layout.has_contiguous_strides()) {
    std::memcpy(out.data(), span.data(), out.size());
    return out;
  }
  // host-side strided gather (rust/musapy-python/src/array.rs:588-650)
  std::vector<size_t> idx(a.ndim(), 0);
  for (size_t i = 0; i < n; ++i) {
    ssize_t off = -lo;
    for (size_t d = 0; d < a.ndim(); ++d) off += ssize_t(idx[d]) * a.layout.strides[d];
    std::memcpy(out.data() + i * es, span.data() + size_t(off) * es, es);
    for (size_t d = a.ndim(); d-- > 0;) {
      if (++idx[d] < a.layout.shape[d]) break;
      idx[d] = 0;
    }
  }
  return out;
}

}  // namespace ops
}  // namespace mpy
