/*
 * kernel-set (MI355X build) -- ABI types shared by every entry point.
 *
 * Pure C, no HIP includes: every binding (ctypes, cgo, ...) parses it without a
 * GPU toolchain. The enum values are frozen by the reference ABI
 * (include/kernel_set/types.h:21-66 of cklxx/kernel-set) and must not change:
 * bindings pass them as plain ints.
 */
#ifndef KERNEL_SET_TYPES_H_
#define KERNEL_SET_TYPES_H_

#include <stddef.h>
#include <stdint.h>

#include "kernel_set/export.h"

KS_BEGIN_EXTERN_C

/* A hipStream_t passed opaquely; NULL selects the null (default) stream. */
typedef void* ks_stream_t;

/* Return code of every entry point (reference types.h:24-34). */
typedef enum ks_status_t {
  KS_SUCCESS = 0,
  KS_ERROR_INVALID_ARGUMENT = 1,  /* NULL pointer, bad mode, non-positive size */
  KS_ERROR_UNSUPPORTED_DTYPE = 2, /* element type not served by the op        */
  KS_ERROR_UNSUPPORTED_SHAPE = 3, /* shape the op cannot honour               */
  KS_ERROR_CUDA = 4,              /* HIP runtime failure (code kept for ABI)  */
  KS_ERROR_NOT_IMPLEMENTED = 5,
  KS_ERROR_OUT_OF_MEMORY = 6,
  KS_ERROR_ARCH_UNSUPPORTED = 7,
  KS_ERROR_INTERNAL = 8,
} ks_status_t;

/* Element types (reference types.h:37-49). */
typedef enum ks_dtype_t {
  KS_DTYPE_F32 = 0,
  KS_DTYPE_F16 = 1,
  KS_DTYPE_BF16 = 2,
  KS_DTYPE_F8E4M3 = 3, /* OCP e4m3fn: no infinities, max 448          */
  KS_DTYPE_F8E5M2 = 4, /* OCP e5m2: IEEE-like, max finite 57344       */
  KS_DTYPE_F64 = 5,
  KS_DTYPE_I64 = 6,
  KS_DTYPE_I32 = 7,
  KS_DTYPE_I8 = 8,
  KS_DTYPE_U8 = 9,
  KS_DTYPE_I4 = 10, /* two codes per byte */
} ks_dtype_t;

/* Fused-epilogue activation selector (reference types.h:52-58). Kept for ABI
 * completeness; no entry point of this build takes it. */
typedef enum ks_activation_t {
  KS_ACT_NONE = 0,
  KS_ACT_RELU = 1,
  KS_ACT_GELU = 2,
  KS_ACT_GELU_TANH = 3,
  KS_ACT_SILU = 4,
} ks_activation_t;

/* Quantization granularity (reference types.h:61-66). */
typedef enum ks_quant_mode_t {
  KS_QUANT_PER_TENSOR = 0,
  KS_QUANT_PER_TOKEN = 1,
  KS_QUANT_PER_CHANNEL = 2,
  KS_QUANT_GROUPWISE = 3,
} ks_quant_mode_t;

KS_END_EXTERN_C

#endif /* KERNEL_SET_TYPES_H_ */
