// kernel-set (MI355X build) -- library-owned device scratch.
//
// Split-K kernels need a float partial buffer; the fused quantize + GEMM entry
// point needs byte staging for quantized activations. The reference ABI has no
// workspace argument, so the library keeps one scratch region per (device,
// stream): calls on one stream are ordered by the stream, and calls on
// different streams never share scratch. The two buffers are separate, so one
// call may use both.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "kernel_set/types.h"

namespace ks {

struct Scratch {
  float* partial = nullptr;  // split-K partial sums
  void* staging = nullptr;   // staged operands (16-byte aligned)
};

// Returns scratch with at least `partial_floats` floats and `staging_bytes`
// bytes for `stream` on the current device. Grows (synchronously) when too
// small.
ks_status_t get_scratch(hipStream_t stream, size_t partial_floats, size_t staging_bytes,
                        Scratch* out, const char* who);

}  // namespace ks
