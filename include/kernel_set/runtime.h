/*
 * kernel-set (MI355X build) -- runtime / device management.
 *
 * Replaces include/kernel_set/runtime.h:20-80 of cklxx/kernel-set symbol for
 * symbol. Implemented over the HIP runtime; ks_backend_name() returns "hip".
 */
#ifndef KERNEL_SET_RUNTIME_H_
#define KERNEL_SET_RUNTIME_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

/* Library version string (reference runtime.h:20). */
KS_API const char* ks_version(void);
/* Symbolic name of a status code, never NULL (reference runtime.h:23). */
KS_API const char* ks_status_string(ks_status_t status);
/* Element width in bits; 0 for an unknown dtype (reference runtime.h:26). */
KS_API int ks_dtype_size_bits(ks_dtype_t dtype);
/* Short dtype token such as "bf16" (reference runtime.h:29). */
KS_API const char* ks_dtype_name(ks_dtype_t dtype);
/* "hip" for this build (reference runtime.h:32). */
KS_API const char* ks_backend_name(void);

/* Field order frozen by reference runtime.h:36-48. On gfx950 warp_size is 64,
 * compute_major/minor are 9/5 and supports_fp8 is 1. */
typedef struct ks_device_properties_t {
  char name[256];
  int compute_major;
  int compute_minor;
  int multiprocessor_count;
  int max_threads_per_block;
  int max_shared_memory_per_block;
  int warp_size;
  size_t total_global_memory;
  int supports_bf16;
  int supports_fp8;
  int supports_tf32;
} ks_device_properties_t;

KS_API ks_status_t ks_device_count(int* out_count);          /* runtime.h:50 */
KS_API ks_status_t ks_set_device(int device);                /* runtime.h:51 */
KS_API ks_status_t ks_get_device(int* out_device);           /* runtime.h:52 */
KS_API ks_status_t ks_get_device_properties(int device,      /* runtime.h:53 */
                                            ks_device_properties_t* out_props);

/* Thread-local text of the last failure on this thread, never NULL
 * (reference runtime.h:58). */
KS_API const char* ks_last_error_string(void);

KS_API ks_status_t ks_stream_create(ks_stream_t* out_stream);  /* :62 */
KS_API ks_status_t ks_stream_destroy(ks_stream_t stream);       /* :63 */
KS_API ks_status_t ks_stream_synchronize(ks_stream_t stream);   /* :64 */

KS_API ks_status_t ks_malloc_device(void** out_ptr, size_t bytes); /* :68 */
KS_API ks_status_t ks_free_device(void* ptr);                      /* :69 */

typedef enum ks_memcpy_kind_t {
  KS_MEMCPY_HOST_TO_DEVICE = 0,
  KS_MEMCPY_DEVICE_TO_HOST = 1,
  KS_MEMCPY_DEVICE_TO_DEVICE = 2,
} ks_memcpy_kind_t;

KS_API ks_status_t ks_memcpy(void* dst, const void* src, size_t bytes, /* :77 */
                             ks_memcpy_kind_t kind, ks_stream_t stream);
KS_API ks_status_t ks_memset_device(void* dst, int value, size_t bytes, /* :79 */
                                    ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_RUNTIME_H_ */
