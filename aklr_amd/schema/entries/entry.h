// What the torch entry points of this library's AKLR kernels share: the stream a call launches on,
// the status check of the C ABI, and per-call device scratch from torch's allocator.
#pragma once

#include <ATen/ATen.h>
#include <ATen/hip/HIPContext.h>
#include <torch/library.h>

#include "include/aklr_amd.h"

namespace aklr_entry {

// The current torch stream of the device that holds t: the stream the caller works on.
inline hipStream_t stream_of(const at::Tensor& t) { return at::hip::getCurrentHIPStream(t.get_device()).stream(); }

inline void check(int status, const char* op) {
  TORCH_CHECK(status == AKLR_OK, op, ": ", aklr_status_string(status));
}

// Scratch for one call on t's device. Its content does not matter to the kernels: split-K arrival
// words are tagged with the launch that wrote them, and partials are written before they are read.
inline at::Tensor scratch(const at::Tensor& t, size_t bytes) {
  return at::empty({static_cast<int64_t>(bytes ? bytes : 1)}, t.options().dtype(at::kByte));
}

inline bool aligned16(const at::Tensor& t) { return reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0; }

}  // namespace aklr_entry
