// publish.hpp -- fence-free hand-over of small values between workgroups.
//
// Agent-scope acquire/release would make every publish write back, and every poll invalidate, a
// whole L2 on this multi-XCD part, so there are no fences at all: a value is stored as W 64-bit
// words, each holding a 32-bit slice of its bits next to a "published" tag, with relaxed (but
// coherent, agent-scope) 64-bit atomics.  A reader that sees the tag on every word holds the
// value the writer stored; the data travels inside the atomic itself, so no ordering between
// different locations is needed.  Users keep each word written once per hand-over and return it
// to zero before it is used again.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mpy {

__device__ inline uint64_t ld_relaxed(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_relaxed(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr uint64_t kTag = uint64_t(1) << 32;

// W 32-bit slices
template <int W>
__device__ inline void publish_slices(uint64_t* w, const uint32_t (&s)[W]) {
#pragma unroll
  for (int i = 0; i < W; ++i) st_relaxed(w + i, kTag | s[i]);
}
template <int W>
__device__ inline bool read_slices(const uint64_t* w, uint32_t (&s)[W]) {
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const uint64_t v = ld_relaxed(w + i);
    if (!(v & kTag)) return false;
    s[i] = uint32_t(v);
  }
  return true;
}

// a 32- (W = 1) or 64-bit (W = 2) value given by its bits
template <int W>
__device__ inline void publish_value(uint64_t* w, uint64_t bits) {
  st_relaxed(w, kTag | (bits & 0xffffffffu));
  if (W == 2) st_relaxed(w + 1, kTag | (bits >> 32));
}
template <int W>
__device__ inline bool read_value(const uint64_t* w, uint64_t& bits) {
  uint64_t lo = ld_relaxed(w);
  if (!(lo & kTag)) return false;
  uint64_t hi = 0;
  if (W == 2) {
    hi = ld_relaxed(w + 1);
    if (!(hi & kTag)) return false;
  }
  bits = (lo & 0xffffffffu) | ((hi & 0xffffffffu) << 32);
  return true;
}

}  // namespace mpy
