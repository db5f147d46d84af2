// kernel-set (MI355X build) -- library-owned device scratch.
//
// Split-K kernels need a float partial buffer; the fused quantize + GEMM entry
// point needs byte staging for quantized activations. The reference ABI has no
// workspace argument, so the library keeps one scratch region per (device,
// stream): calls on one stream are ordered by the stream, and calls on
// different streams never share scratch. The two buffers are separate, so one
// call may use both.
//
// Ownership rules:
//  * A region only grows. A buffer it outgrows is retired, not freed: a HIP
//    graph captured earlier may still hold its address, so it stays valid
//    until the process ends. Growth therefore needs no stream sync.
//  * Growth (hipMalloc) is refused while `stream` is being captured; the call
//    returns KS_ERROR_INVALID_ARGUMENT and names the fix (one eager call with
//    the largest shape before capture).
//  * A graph replays with the region of the stream it was captured on, so it
//    must not run concurrently with eager calls on that stream.
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
// bytes for `stream` on the current device, growing the region when it is too
// small (see the ownership rules above).
ks_status_t get_scratch(hipStream_t stream, size_t partial_floats, size_t staging_bytes,
                        Scratch* out, const char* who);

// Caller-provided scratch for the calling thread: while one is installed,
// get_scratch hands out `partial` (capacity `partial_floats`) instead of the
// registry's memory and never allocates; a request beyond the capacity (or
// any staging request beyond `staging_bytes`) fails with
// KS_ERROR_INVALID_ARGUMENT. Used by the entry points that must not allocate.
class ScratchOverride {
 public:
  ScratchOverride(float* partial, size_t partial_floats, void* staging, size_t staging_bytes,
                  const char* limit_text);
  ~ScratchOverride();
  ScratchOverride(const ScratchOverride&) = delete;
  ScratchOverride& operator=(const ScratchOverride&) = delete;
};

}  // namespace ks
