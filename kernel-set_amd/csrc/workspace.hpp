// kernel-set (MI355X build) -- library-owned device scratch.
//
// Split-K kernels need a float partial buffer and per-tile arrival counters.
// The reference ABI has no workspace argument, so the library keeps one
// scratch region per (device, stream): calls on one stream are ordered by the
// stream, and calls on different streams never share scratch. Counters are
// zeroed once at allocation and every kernel that uses them leaves them at
// zero again, so no per-call memset is enqueued.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "kernel_set/types.h"

namespace ks {

struct Scratch {
  float* partial = nullptr;      // split-K partial sums
  unsigned* counters = nullptr;  // per-tile arrival counters, zero between calls
};

// Returns scratch with at least `partial_floats` floats and `counters` counters
// for `stream` on the current device. Grows (synchronously) when too small.
ks_status_t get_scratch(hipStream_t stream, size_t partial_floats, size_t counters,
                        Scratch* out, const char* who);

}  // namespace ks
