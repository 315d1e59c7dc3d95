// plan.hpp -- host-side launch planning for the gfx950 kernels (pure C++, no HIP types).
//
// The ABI (rust/musapy-ops/src/kernels.rs:16-346) hands every kernel wrapper the logical shape
// and per-operand element strides.  Before launching anything the wrappers normalise that
// description: size-1 dims are dropped and adjacent dims are merged whenever every operand
// walks them as one (the reference instead decodes every dimension of every element on the
// device, kernels/include/common.h:42-51).  The resulting plans decide which kernel variant runs.
#pragma once

#include <stdint.h>
#include <stddef.h>
#include <sys/types.h>

namespace mpy {

constexpr int kMaxDims = 32;  // same rank limit as the reference (NdMeta, elementwise.mu:16-31)

// Fast unsigned 32-bit division by a runtime-invariant divisor (Granlund & Montgomery 1994,
// "Division by invariant integers using multiplication", round-up variant):
//   s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1, q = (umulhi(n, m) + n) >> s
// The sum is formed in 64 bits, so the identity holds for every n < 2^32 and 1 <= d < 2^32.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  f.s = s;
  f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
  return f;
}

// host evaluation of the same formula (the device uses __umulhi)
inline uint32_t fd_div_host(const FastDiv& f, uint32_t n) {
  uint32_t t = uint32_t((uint64_t(n) * f.m) >> 32);
  return uint32_t((uint64_t(t) + n) >> f.s);
}

// Elementwise plan.  Operand 0 is the (C-contiguous) output, operands 1.. are inputs.
struct Plan {
  int nops;
  int ndim;                          // >= 1 after normalisation
  uint64_t shape[kMaxDims];          // outermost first
  int64_t stride[4][kMaxDims];       // elements
  uint64_t numel;
};

// Returns false when numel == 0 (nothing to launch).
inline bool plan_elementwise(Plan& p, int ndim, const size_t* shape, int nin,
                             const ssize_t* const* in_strides) {
  p.nops = nin + 1;
  uint64_t numel = 1;
  for (int i = 0; i < ndim; ++i) numel *= uint64_t(shape[i]);
  p.numel = numel;
  if (numel == 0) return false;
  // contiguous output strides of the logical shape
  int64_t ostr[kMaxDims];
  {
    int64_t s = 1;
    for (int i = ndim - 1; i >= 0; --i) {
      ostr[i] = s;
      s *= int64_t(shape[i]);
    }
  }
  // walk innermost -> outermost, merging where all operands agree
  uint64_t cs[kMaxDims];
  int64_t cst[4][kMaxDims];
  int n = 0;
  for (int i = ndim - 1; i >= 0; --i) {
    uint64_t sz = shape[i];
    if (sz == 1) continue;
    int64_t st[4];
    st[0] = ostr[i];
    for (int o = 0; o < nin; ++o) st[o + 1] = in_strides[o][i];
    if (n > 0) {
      bool merge = true;
      for (int o = 0; o < p.nops; ++o)
        if (st[o] != cst[o][n - 1] * int64_t(cs[n - 1])) merge = false;
      if (merge) {
        cs[n - 1] *= sz;
        continue;
      }
    }
    cs[n] = sz;
    for (int o = 0; o < p.nops; ++o) cst[o][n] = st[o];
    ++n;
  }
  if (n == 0) {  // a single element
    cs[0] = 1;
    for (int o = 0; o < p.nops; ++o) cst[o][0] = (o == 0) ? 1 : 0;
    n = 1;
  }
  p.ndim = n;
  for (int i = 0; i < n; ++i) {  // store outermost first
    p.shape[i] = cs[n - 1 - i];
    for (int o = 0; o < p.nops; ++o) p.stride[o][i] = cst[o][n - 1 - i];
  }
  return true;
}

// Reduction plan: the input is seen as a set of output coordinates (C-contiguous in the output)
// times one reduced axis of length R.
enum ReduceKind : int { kRowReduce = 0, kColReduce = 1 };

struct ReducePlan {
  int ond;                        // number of (coalesced) output dims, >= 1
  uint64_t oshape[kMaxDims];      // outermost first
  int64_t ostride[kMaxDims];      // input strides of the output dims
  uint64_t R;                     // reduced length
  int64_t rstride;                // input stride along the reduced axis
  uint64_t out_size;
  int kind;
};

inline void plan_reduce(ReducePlan& p, int ndim, const size_t* shape, const ssize_t* strides,
                        int axis, size_t axis_len, size_t out_size) {
  p.R = axis_len;
  p.rstride = (ndim > 0) ? strides[axis] : 1;
  p.out_size = out_size;
  uint64_t cs[kMaxDims];
  int64_t cst[kMaxDims];
  int n = 0;
  for (int i = ndim - 1; i >= 0; --i) {
    if (i == axis || shape[i] == 1) continue;
    if (n > 0 && int64_t(strides[i]) == cst[n - 1] * int64_t(cs[n - 1])) {
      cs[n - 1] *= shape[i];
      continue;
    }
    cs[n] = shape[i];
    cst[n] = strides[i];
    ++n;
  }
  if (n == 0) {
    cs[0] = 1;
    cst[0] = 0;
    n = 1;
  }
  p.ond = n;
  for (int i = 0; i < n; ++i) {
    p.oshape[i] = cs[n - 1 - i];
    p.ostride[i] = cst[n - 1 - i];
  }
  if (p.R == 1) p.rstride = 1;
  // Column mapping pays off when the innermost output dim is unit-stride in the input while the
  // reduced axis is not: lanes then walk adjacent addresses.
  bool inner_unit = p.oshape[n - 1] > 1 && p.ostride[n - 1] == 1;
  p.kind = (p.rstride != 1 && inner_unit) ? kColReduce : kRowReduce;
}

// Scan plan: like the elementwise plan for (out, in) but the scanned axis is never merged.
enum ScanKind : int { kRowScan = 0, kColScan = 1, kGenericScan = 2 };

struct ScanPlan {
  int ond;                       // coalesced non-axis dims (>= 1)
  uint64_t oshape[kMaxDims];
  int64_t istride[kMaxDims];     // input strides of the non-axis dims
  int64_t ostride[kMaxDims];     // output strides of the non-axis dims
  uint64_t L;                    // scanned length
  int64_t ls_in, ls_out;         // strides along the scanned axis
  uint64_t rows;                 // product of non-axis dims
  int kind;
};

inline void plan_scan(ScanPlan& p, int ndim, const size_t* shape, const ssize_t* strides, int axis) {
  int64_t ostr[kMaxDims] = {};  // callers check 0 <= axis < ndim <= kMaxDims
  {
    int64_t s = 1;
    for (int i = ndim - 1; i >= 0; --i) {
      ostr[i] = s;
      s *= int64_t(shape[i]);
    }
  }
  p.L = shape[axis];
  p.ls_in = strides[axis];
  p.ls_out = ostr[axis];
  uint64_t cs[kMaxDims];
  int64_t ci[kMaxDims], co[kMaxDims];
  int n = 0;
  uint64_t rows = 1;
  for (int i = ndim - 1; i >= 0; --i) {
    if (i == axis || shape[i] == 1) continue;
    rows *= shape[i];
    // The output stride check also keeps the scanned axis from being merged across.
    if (n > 0 && int64_t(strides[i]) == ci[n - 1] * int64_t(cs[n - 1]) &&
        ostr[i] == co[n - 1] * int64_t(cs[n - 1])) {
      cs[n - 1] *= shape[i];
      continue;
    }
    cs[n] = shape[i];
    ci[n] = strides[i];
    co[n] = ostr[i];
    ++n;
  }
  if (n == 0) {
    cs[0] = 1;
    ci[0] = 0;
    co[0] = 0;
    n = 1;
  }
  p.ond = n;
  p.rows = rows;
  for (int i = 0; i < n; ++i) {
    p.oshape[i] = cs[n - 1 - i];
    p.istride[i] = ci[n - 1 - i];
    p.ostride[i] = co[n - 1 - i];
  }
  if (p.L == 1) {
    p.ls_in = 1;
    p.ls_out = 1;
  }
  if (p.ls_in == 1 && p.ls_out == 1)
    p.kind = kRowScan;
  else if (p.oshape[n - 1] > 1 && p.istride[n - 1] == 1 && p.ostride[n - 1] == 1)
    p.kind = kColScan;
  else
    p.kind = kGenericScan;
}

}  // namespace mpy
