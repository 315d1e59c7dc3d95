// dlpack.hpp -- the DLPack exchange structures (DLPack specification v1.0: dlpack.h of the
// dmlc/dlpack project, Apache-2.0).  They are an ABI shared with every producer and consumer
// (PyTorch, NumPy, CuPy, JAX), so names, field order and widths follow the specification
// exactly.  Only what this backend exchanges is declared: the device and dtype codes it maps,
// the unversioned DLManagedTensor ("dltensor" capsules) and the versioned
// DLManagedTensorVersioned ("dltensor_versioned" capsules, DLPack >= 1.0).
#pragma once

#include <cstddef>
#include <cstdint>

extern "C" {

enum DLDeviceTypeCode : int32_t {
  kDLCPU = 1,
  kDLCUDA = 2,
  kDLCUDAHost = 3,
  kDLROCM = 10,  // AMD GPUs; HIP device ordinal in device_id
  kDLROCMHost = 11,
};

struct DLDevice {
  int32_t device_type;
  int32_t device_id;
};

enum DLDataTypeCode : uint8_t {
  kDLInt = 0,
  kDLUInt = 1,
  kDLFloat = 2,
  kDLOpaqueHandle = 3,
  kDLBfloat = 4,
  kDLComplex = 5,
  kDLBool = 6,
};

struct DLDataType {
  uint8_t code;
  uint8_t bits;
  uint16_t lanes;
};

struct DLTensor {
  void* data;          // device pointer; the first element is at data + byte_offset
  DLDevice device;
  int32_t ndim;
  DLDataType dtype;
  int64_t* shape;
  int64_t* strides;    // in elements; NULL means C-contiguous
  uint64_t byte_offset;
};

struct DLManagedTensor {
  DLTensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(DLManagedTensor* self);
};

struct DLPackVersion {
  uint32_t major;
  uint32_t minor;
};

constexpr uint64_t kDLFlagReadOnly = uint64_t(1) << 0;
constexpr uint64_t kDLFlagIsCopied = uint64_t(1) << 1;

struct DLManagedTensorVersioned {
  DLPackVersion version;
  void* manager_ctx;
  void (*deleter)(DLManagedTensorVersioned* self);
  uint64_t flags;
  DLTensor dl_tensor;
};

}  // extern "C"

// layout checks against the specification (LP64)
static_assert(sizeof(DLDevice) == 8, "DLDevice");
static_assert(sizeof(DLDataType) == 4, "DLDataType");
static_assert(sizeof(DLTensor) == 48 && offsetof(DLTensor, ndim) == 16 && offsetof(DLTensor, shape) == 24 &&
                  offsetof(DLTensor, byte_offset) == 40,
              "DLTensor");
static_assert(sizeof(DLManagedTensor) == 64 && offsetof(DLManagedTensor, deleter) == 56, "DLManagedTensor");
static_assert(sizeof(DLManagedTensorVersioned) == 80 && offsetof(DLManagedTensorVersioned, flags) == 24 &&
                  offsetof(DLManagedTensorVersioned, dl_tensor) == 32,
              "DLManagedTensorVersioned");
