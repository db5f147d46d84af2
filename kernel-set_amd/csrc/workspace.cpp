// kernel-set (MI355X build) -- per-(device, stream) scratch registry.
#include "workspace.hpp"

#include <map>
#include <mutex>
#include <string>
#include <utility>

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
std::map<std::pair<int, hipStream_t>, Entry> g_entries;  // freed at process exit

size_t round_up(size_t v, size_t q) { return (v + q - 1) / q * q; }

}  // namespace

ks_status_t get_scratch(hipStream_t stream, size_t partial_floats, size_t staging_bytes,
                        Scratch* out, const char* who) {
  int dev = 0;
  ks_status_t st = check_hip(hipGetDevice(&dev), who);
  if (st != KS_SUCCESS) return st;
  std::lock_guard<std::mutex> lock(g_mu);
  Entry& e = g_entries[{dev, stream}];
  if (partial_floats > e.partial_cap) {
    // Growing must not free memory a kernel still reads: wait for the stream.
    if (e.partial) {
      st = check_hip(hipStreamSynchronize(stream), who);
      if (st != KS_SUCCESS) return st;
      (void)hipFree(e.partial);
      e.partial = nullptr;
      e.partial_cap = 0;
    }
    const size_t cap = round_up(partial_floats, size_t{1} << 20);
    if (hipMalloc(&e.partial, cap * sizeof(float)) != hipSuccess) {
      e.partial = nullptr;
      set_last_error(std::string(who) + ": scratch allocation failed");
      return KS_ERROR_OUT_OF_MEMORY;
    }
    e.partial_cap = cap;
  }
  if (staging_bytes > e.staging_cap) {
    if (e.staging) {
      st = check_hip(hipStreamSynchronize(stream), who);
      if (st != KS_SUCCESS) return st;
      (void)hipFree(e.staging);
      e.staging = nullptr;
      e.staging_cap = 0;
    }
    const size_t cap = round_up(staging_bytes, size_t{1} << 20);
    if (hipMalloc(&e.staging, cap) != hipSuccess) {
      e.staging = nullptr;
      set_last_error(std::string(who) + ": staging allocation failed");
      return KS_ERROR_OUT_OF_MEMORY;
    }
    e.staging_cap = cap;
  }
  out->partial = e.partial;
  out->staging = e.staging;
  return KS_SUCCESS;
}

}  // namespace ks
