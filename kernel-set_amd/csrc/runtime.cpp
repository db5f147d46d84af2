// kernel-set (MI355X build) -- runtime.h over the HIP runtime, plus the
// thread-local error string every entry point reports through.
//
// Behaviour follows kernels/src/common/runtime.cu:1-183 of cklxx/kernel-set:
// same status names, same dtype widths/names, same "<func>: <runtime msg>"
// error text, ks_malloc_device failures map to KS_ERROR_OUT_OF_MEMORY.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "kernel_set/runtime.h"
#include "ks_common.hpp"

#ifndef KERNEL_SET_VERSION
#define KERNEL_SET_VERSION "0.2.1"
#endif

namespace ks {
static thread_local std::string g_last_error;
void set_last_error(const std::string& msg) { g_last_error = msg; }
}  // namespace ks

extern "C" {

const char* ks_version(void) { return KERNEL_SET_VERSION; }

const char* ks_backend_name(void) { return "hip"; }

const char* ks_last_error_string(void) { return ks::g_last_error.c_str(); }

const char* ks_status_string(ks_status_t status) {
  switch (status) {
    case KS_SUCCESS: return "KS_SUCCESS";
    case KS_ERROR_INVALID_ARGUMENT: return "KS_ERROR_INVALID_ARGUMENT";
    case KS_ERROR_UNSUPPORTED_DTYPE: return "KS_ERROR_UNSUPPORTED_DTYPE";
    case KS_ERROR_UNSUPPORTED_SHAPE: return "KS_ERROR_UNSUPPORTED_SHAPE";
    case KS_ERROR_CUDA: return "KS_ERROR_CUDA";
    case KS_ERROR_NOT_IMPLEMENTED: return "KS_ERROR_NOT_IMPLEMENTED";
    case KS_ERROR_OUT_OF_MEMORY: return "KS_ERROR_OUT_OF_MEMORY";
    case KS_ERROR_ARCH_UNSUPPORTED: return "KS_ERROR_ARCH_UNSUPPORTED";
    case KS_ERROR_INTERNAL: return "KS_ERROR_INTERNAL";
  }
  return "KS_ERROR_UNKNOWN";
}

int ks_dtype_size_bits(ks_dtype_t dtype) {
  switch (dtype) {
    case KS_DTYPE_F64: case KS_DTYPE_I64: return 64;
    case KS_DTYPE_F32: case KS_DTYPE_I32: return 32;
    case KS_DTYPE_F16: case KS_DTYPE_BF16: return 16;
    case KS_DTYPE_F8E4M3: case KS_DTYPE_F8E5M2:
    case KS_DTYPE_I8: case KS_DTYPE_U8: return 8;
    case KS_DTYPE_I4: return 4;
  }
  return 0;
}

const char* ks_dtype_name(ks_dtype_t dtype) {
  switch (dtype) {
    case KS_DTYPE_F32: return "f32";
    case KS_DTYPE_F16: return "f16";
    case KS_DTYPE_BF16: return "bf16";
    case KS_DTYPE_F8E4M3: return "f8e4m3";
    case KS_DTYPE_F8E5M2: return "f8e5m2";
    case KS_DTYPE_F64: return "f64";
    case KS_DTYPE_I64: return "i64";
    case KS_DTYPE_I32: return "i32";
    case KS_DTYPE_I8: return "i8";
    case KS_DTYPE_U8: return "u8";
    case KS_DTYPE_I4: return "i4";
  }
  return "unknown";
}

ks_status_t ks_device_count(int* out_count) {
  KS_REQUIRE_PTR(out_count);
  return ks::check_hip(hipGetDeviceCount(out_count), "ks_device_count");
}

ks_status_t ks_set_device(int device) {
  return ks::check_hip(hipSetDevice(device), "ks_set_device");
}

ks_status_t ks_get_device(int* out_device) {
  KS_REQUIRE_PTR(out_device);
  return ks::check_hip(hipGetDevice(out_device), "ks_get_device");
}

ks_status_t ks_get_device_properties(int device,
                                     ks_device_properties_t* out_props) {
  KS_REQUIRE_PTR(out_props);
  hipDeviceProp_t prop;
  ks_status_t st = ks::check_hip(hipGetDeviceProperties(&prop, device),
                                 "ks_get_device_properties");
  if (st != KS_SUCCESS) return st;
  std::memset(out_props, 0, sizeof(*out_props));
  std::strncpy(out_props->name, prop.name, sizeof(out_props->name) - 1);
  out_props->compute_major = prop.major;
  out_props->compute_minor = prop.minor;
  out_props->multiprocessor_count = prop.multiProcessorCount;
  out_props->max_threads_per_block = prop.maxThreadsPerBlock;
  out_props->max_shared_memory_per_block = static_cast<int>(prop.sharedMemPerBlock);
  out_props->warp_size = prop.warpSize;
  out_props->total_global_memory = prop.totalGlobalMem;
  const bool cdna3plus = std::strncmp(prop.gcnArchName, "gfx94", 5) == 0 ||
                         std::strncmp(prop.gcnArchName, "gfx95", 5) == 0;
  out_props->supports_bf16 = 1;
  out_props->supports_fp8 = cdna3plus ? 1 : 0;
  out_props->supports_tf32 = 0;  // gfx950 has no xf32 MFMA
  return KS_SUCCESS;
}

ks_status_t ks_stream_create(ks_stream_t* out_stream) {
  KS_REQUIRE_PTR(out_stream);
  hipStream_t s = nullptr;
  ks_status_t st = ks::check_hip(hipStreamCreate(&s), "ks_stream_create");
  if (st != KS_SUCCESS) return st;
  *out_stream = static_cast<ks_stream_t>(s);
  return KS_SUCCESS;
}

ks_status_t ks_stream_destroy(ks_stream_t stream) {
  return ks::check_hip(hipStreamDestroy(ks::to_stream(stream)), "ks_stream_destroy");
}

ks_status_t ks_stream_synchronize(ks_stream_t stream) {
  return ks::check_hip(hipStreamSynchronize(ks::to_stream(stream)),
                       "ks_stream_synchronize");
}

ks_status_t ks_malloc_device(void** out_ptr, size_t bytes) {
  KS_REQUIRE_PTR(out_ptr);
  hipError_t e = hipMalloc(out_ptr, bytes);
  if (e != hipSuccess) {
    ks::set_last_error(std::string("ks_malloc_device: ") + hipGetErrorString(e));
    return KS_ERROR_OUT_OF_MEMORY;
  }
  return KS_SUCCESS;
}

ks_status_t ks_free_device(void* ptr) {
  return ks::check_hip(hipFree(ptr), "ks_free_device");
}

ks_status_t ks_memcpy(void* dst, const void* src, size_t bytes,
                      ks_memcpy_kind_t kind, ks_stream_t stream) {
  KS_REQUIRE_PTR(dst);
  KS_REQUIRE_PTR(src);
  hipMemcpyKind k = hipMemcpyDeviceToDevice;
  if (kind == KS_MEMCPY_HOST_TO_DEVICE) k = hipMemcpyHostToDevice;
  else if (kind == KS_MEMCPY_DEVICE_TO_HOST) k = hipMemcpyDeviceToHost;
  return ks::check_hip(hipMemcpyAsync(dst, src, bytes, k, ks::to_stream(stream)),
                       "ks_memcpy");
}

ks_status_t ks_memset_device(void* dst, int value, size_t bytes,
                             ks_stream_t stream) {
  KS_REQUIRE_PTR(dst);
  return ks::check_hip(hipMemsetAsync(dst, value, bytes, ks::to_stream(stream)),
                       "ks_memset_device");
}

}  // extern "C"
