// kernel-set (MI355X build) -- per-(device, stream) scratch registry.
#include "workspace.hpp"

#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "ks_common.hpp"

namespace ks {
namespace {

struct Entry {
  float* partial = nullptr;
  size_t partial_cap = 0;
  void* staging = nullptr;
  size_t staging_cap = 0;
};

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, Entry> g_entries;
// Outgrown buffers. Never freed: graphs captured before the growth still
// address them (released with the process).
std::vector<void*> g_retired;

struct Override {
  bool active = false;
  float* partial = nullptr;
  size_t partial_cap = 0;
  void* staging = nullptr;
  size_t staging_cap = 0;
  const char* limit_text = "";
};
thread_local Override t_override;

size_t round_up(size_t v, size_t q) { return (v + q - 1) / q * q; }

// KS_SUCCESS when `stream` is not capturing; otherwise the growth is refused.
ks_status_t refuse_if_capturing(hipStream_t stream, const char* who) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  ks_status_t st = check_hip(hipStreamIsCapturing(stream, &cs), who);
  if (st != KS_SUCCESS) return st;
  if (cs != hipStreamCaptureStatusNone) {
    set_last_error(std::string(who) +
                   ": library scratch must grow, but the stream is being captured; run one "
                   "eager call with the largest shape on this stream before capture");
    return KS_ERROR_INVALID_ARGUMENT;
  }
  return KS_SUCCESS;
}

ks_status_t grow(hipStream_t stream, void** buf, size_t* cap_bytes, size_t need_bytes,
                 const char* who, const char* what) {
  ks_status_t st = refuse_if_capturing(stream, who);
  if (st != KS_SUCCESS) return st;
  const size_t cap = round_up(need_bytes, size_t{4} << 20);
  void* fresh = nullptr;
  if (hipMalloc(&fresh, cap) != hipSuccess) {
    (void)hipGetLastError();
    set_last_error(std::string(who) + ": " + what + " allocation failed");
    return KS_ERROR_OUT_OF_MEMORY;
  }
  if (*buf) g_retired.push_back(*buf);
  *buf = fresh;
  *cap_bytes = cap;
  return KS_SUCCESS;
}

}  // namespace

ScratchOverride::ScratchOverride(float* partial, size_t partial_floats, void* staging,
                                 size_t staging_bytes, const char* limit_text) {
  t_override = Override{true, partial, partial_floats, staging, staging_bytes, limit_text};
}

ScratchOverride::~ScratchOverride() { t_override = Override{}; }

ks_status_t get_scratch(hipStream_t stream, size_t partial_floats, size_t staging_bytes,
                        Scratch* out, const char* who) {
  if (t_override.active) {
    const Override& o = t_override;
    if (partial_floats > o.partial_cap || staging_bytes > o.staging_cap) {
      set_last_error(std::string(who) + ": shape needs more scratch than the fixed " +
                     o.limit_text + " of the no-allocation entry point");
      return KS_ERROR_INVALID_ARGUMENT;
    }
    out->partial = o.partial;
    out->staging = o.staging;
    return KS_SUCCESS;
  }
  int dev = 0;
  ks_status_t st = check_hip(hipGetDevice(&dev), who);
  if (st != KS_SUCCESS) return st;
  std::lock_guard<std::mutex> lock(g_mu);
  Entry& e = g_entries[{dev, stream}];
  if (partial_floats > e.partial_cap) {
    void* buf = e.partial;
    size_t cap = e.partial_cap * sizeof(float);
    st = grow(stream, &buf, &cap, partial_floats * sizeof(float), who, "scratch");
    if (st != KS_SUCCESS) return st;
    e.partial = static_cast<float*>(buf);
    e.partial_cap = cap / sizeof(float);
  }
  if (staging_bytes > e.staging_cap) {
    st = grow(stream, &e.staging, &e.staging_cap, staging_bytes, who, "staging");
    if (st != KS_SUCCESS) return st;
  }
  out->partial = e.partial;
  out->staging = e.staging;
  return KS_SUCCESS;
}

}  // namespace ks
