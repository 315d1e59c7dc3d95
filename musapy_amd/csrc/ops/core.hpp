// core.hpp -- host-side types of the op layer: dtypes + promotion, layouts + views, streams,
// device buffers and arrays.
//
// C++ counterpart of musapy-core (rust/musapy-core/src): dtype.rs (Dtype, promote), layout.rs
// (Layout and its zero-copy views), stream.rs (Stream / poison flag), buffer.rs (Buffer,
// BufferRef, cross-stream read/write ordering), array.rs (Array) and error.rs (error taxonomy).
// Device memory, streams and events come from the C-ABI HIP runtime layer
// (include/musapy_hip_runtime.h); this file never calls HIP directly.
#pragma once

#include <sys/types.h>

#include <cstddef>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;

namespace mpy {
namespace ops {

// ---- errors (rust/musapy-core/src/error.rs, mapped to Python in the binding) ----
struct MusapyError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct DeviceError : MusapyError { using MusapyError::MusapyError; };
struct DeviceNotConfiguredError : DeviceError { using DeviceError::DeviceError; };
struct DtypeError : MusapyError { using MusapyError::MusapyError; };
struct ShapeError : MusapyError { using MusapyError::MusapyError; };
struct MemoryError : MusapyError { using MusapyError::MusapyError; };
struct OutOfMemoryError : MemoryError { using MemoryError::MemoryError; };
struct StreamError : MusapyError { using MusapyError::MusapyError; };
struct KernelError : MusapyError { using MusapyError::MusapyError; };
struct InteropError : MusapyError { using MusapyError::MusapyError; };

// ---- dtypes (rust/musapy-core/src/dtype.rs:25-150) ----
enum class Dtype : int {
  Bool, Int8, Int16, Int32, Int64, Uint8, Uint16, Uint32, Uint64,
  Float16, Float32, Float64, Bfloat16, Complex64, Complex128
};
size_t element_size(Dtype d);
const char* dtype_name(Dtype d);        // "float32", ...
const char* dtype_short(Dtype d);       // "f32", ... (the strings musapy's Python layer compares with)
Dtype parse_dtype(const std::string& s);
int dtype_category(Dtype d);            // 0 bool, 1 int, 2 uint, 3 float, 4 complex
int precision_width(Dtype d);
bool is_complex(Dtype d);
// promote (dtype.rs:206-334): JAX table; all_gpu=true picks the narrower input within a category
Dtype promote(Dtype a, Dtype b, bool all_gpu);

// ---- layout (rust/musapy-core/src/layout.rs:28-289) ----
using Shape = std::vector<size_t>;
using Strides = std::vector<ssize_t>;
Strides contiguous_strides(const Shape& shape);
size_t shape_numel(const Shape& shape);

struct Layout {
  Shape shape;
  Strides strides;
  size_t offset = 0;
  static Layout from_shape(const Shape& s);
  size_t ndim() const { return shape.size(); }
  size_t size() const { return shape_numel(shape); }
  bool has_contiguous_strides() const;
  bool is_contiguous() const { return offset == 0 && has_contiguous_strides(); }
  Layout transposed(const std::vector<size_t>* axes) const;
  Layout flipped(size_t axis) const;
  Layout sliced(const std::vector<size_t>& start, const std::vector<size_t>& stop,
                const std::vector<size_t>& step) const;
};

// ---- debug mode (rust/musapy-core/src/debug.rs:20-100) ----
// A process-wide flag, off by default, on when MUSAPY_DEBUG is "1" or "true" at first use or after
// set_debug(true).  While it is on, every op records an OpContext on its output stream, and the
// Python binding hands the op its caller's frame (set_debug_frame / take_debug_frame).
bool is_debug();
void set_debug(bool enabled);
struct PythonFrame {
  std::string filename;
  int lineno = 0;
  std::string function;
};
void set_debug_frame(const PythonFrame* frame);  // nullptr clears it
bool take_debug_frame(PythonFrame& out);         // the calling thread's frame, consumed

// One op queued on a stream while debug mode is on (stream.rs:42-101): what a failure of that
// stream is attributed to.
struct OpContext {
  std::string op_name;
  std::vector<Shape> input_shapes;
  std::vector<int> input_devices;
  std::vector<Dtype> input_dtypes;
  Shape output_shape;
  uint64_t stream_id = 0;
  bool has_frame = false;
  PythonFrame frame;
  std::string to_string() const;  // "op 'add' on stream 3, inputs=[(2, 3), (3,)] at f.py:7 (g)"
};

// ---- streams (rust/musapy-core/src/stream.rs:154-416) ----
class Stream : public std::enable_shared_from_this<Stream> {
 public:
  Stream(int device, hipStream_t raw, bool owned);
  ~Stream();
  Stream(const Stream&) = delete;
  Stream& operator=(const Stream&) = delete;
  hipStream_t raw() const { return raw_; }
  int device() const { return device_; }
  uint64_t id() const { return id_; }
  bool is_poisoned() const { return poisoned_; }
  void poison() { poisoned_ = true; }
  // Synchronize (stream.rs:311-377).  A failing synchronize poisons the stream and raises
  // StreamError.  When work with a bounded device wait (note_bounded_wait) was queued since the
  // last synchronize, the fault word of this stream's workspace is read as well: a wait that ran
  // out (in a launch queued on this stream) poisons the stream and raises KernelError; the
  // library has zeroed the workspace again by then.  As in the reference, poison is a mark
  // (is_poisoned), not a refusal of later work.  Both errors name the oldest pending op when
  // debug mode recorded one (stream.rs:392-416); a clean synchronize clears the pending ops.
  void synchronize();
  // the op layer queued a kernel whose waits can run out (single-launch reduction, row scan) and
  // report to this stream's workspace
  void note_bounded_wait();
  static std::shared_ptr<Stream> create(int device);
  // The priority a caller asked for (stream.rs:154-199).  It is recorded, not applied: every
  // stream of this backend runs at the default priority.
  int priority() const { return priority_; }
  void set_priority(int p) { priority_ = p; }
  // Scratch for the single-launch reductions and chained scans queued on this stream: 1 MiB of
  // slots plus 256 bytes whose last word is the stream's fault word (musapy_kernels.h workspace
  // rule).  Zero-filled once when first requested; every such launch leaves it zero again.  Work
  // on one stream is ordered, so its launches never share it concurrently.
  static constexpr size_t kReduceWorkspaceBytes = (size_t(1) << 20) + 256;
  void* reduce_workspace();
  // pending op contexts (stream.rs:379-404): recorded in debug mode, cleared by a clean
  // synchronize
  void record_op(OpContext ctx);
  size_t pending_count() const;
  std::string oldest_op_string() const;  // "" when none
  void clear_pending_ops();

 private:
  // " | failed op: ..." for an error message, or "" (stream.rs:367-373)
  std::string failed_op_suffix() const;
  int device_;
  hipStream_t raw_;
  bool owned_;
  bool poisoned_ = false;
  bool wait_check_ = false;
  uint64_t id_;
  int priority_ = 0;
  void* workspace_ = nullptr;
  mutable std::mutex ops_mu_;
  std::deque<OpContext> pending_ops_;
};
using StreamPtr = std::shared_ptr<Stream>;

// per-device default stream of this backend (one non-blocking stream per device)
StreamPtr default_stream(int device);
// ms.synchronize(device): waits for the whole device, then synchronizes every live stream of
// that device with bounded-wait work pending, so a wait that ran out on any of them poisons
// that stream and raises (the first such error, after all were checked)
void synchronize_device(int device);
// the "current stream" override of resolution.rs:184 (nullptr = none)
StreamPtr current_stream();
void set_current_stream(StreamPtr s);

// ---- device buffers (rust/musapy-core/src/buffer.rs:50-489) ----
class Buffer {
 public:
  static std::shared_ptr<Buffer> alloc(size_t nbytes, int device, const StreamPtr& stream);
  // Device memory owned by someone else (a DLPack producer).  `release` runs when the last
  // reference goes, after every stream that read or wrote the buffer has drained.
  static std::shared_ptr<Buffer> adopt(void* ptr, size_t nbytes, int device, const StreamPtr& stream,
                                       std::function<void()> release);
  ~Buffer();
  Buffer(const Buffer&) = delete;
  Buffer& operator=(const Buffer&) = delete;
  void* ptr() const { return ptr_; }
  size_t nbytes() const { return nbytes_; }
  int device() const { return device_; }
  // ordering across streams (buffer.rs:225-326); all no-ops when a single stream is used
  void wait_last_write_on(const StreamPtr& s);
  void wait_reads_on(const StreamPtr& s);
  void record_read(const StreamPtr& s);
  void record_write(const StreamPtr& s);
  const StreamPtr& home() const { return home_; }                // allocation (and free) stream
  const StreamPtr& last_writer() const { return last_writer_; }  // null until a recorded write

 private:
  Buffer() = default;
  std::function<void()> release_;   // set for adopted memory
  void* ptr_ = nullptr;
  size_t nbytes_ = 0;
  int device_ = 0;
  StreamPtr home_;                   // allocation (and free) stream
  StreamPtr last_writer_;
  std::vector<StreamPtr> readers_;   // streams that read since the last write
};
using BufferRef = std::shared_ptr<Buffer>;

// ---- arrays (rust/musapy-core/src/array.rs:87-219) ----
struct Array {
  BufferRef data;
  Layout layout;
  Dtype dtype = Dtype::Float32;
  StreamPtr stream;
  int device = 0;

  const Shape& shape() const { return layout.shape; }
  size_t ndim() const { return layout.ndim(); }
  size_t size() const { return layout.size(); }
  size_t nbytes() const { return size() * element_size(dtype); }
  bool is_contiguous() const { return layout.is_contiguous(); }
  // device pointer of the logical first element (adjust_ptr_offset, op_builder.rs:1566-1575)
  void* data_ptr() const;
  Array view(const Layout& l) const;
};

Array new_array(const Shape& shape, Dtype dtype, int device, const StreamPtr& stream);
// host <-> device (array.rs readback semantics: sync, then copy, then host-side strided gather)
Array from_host(const void* src, const Shape& shape, Dtype dtype, int device);
std::vector<uint8_t> to_host(const Array& a);  // C-order bytes of the logical array

// raises KernelError when the last kernel-ABI call failed to launch (musa_ffi.rs:397-408)
void check_launch(const char* label);
// raises on a non-zero runtime-layer return code
void check_rt(int code, const char* what);

}  // namespace ops
}  // namespace mpy
