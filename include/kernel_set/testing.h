/*
 * kernel-set (MI355X build) -- test hooks. NOT part of the reference ABI.
 *
 * These exist so parity tests can check intermediate values that the public
 * entry points never expose.
 */
#ifndef KERNEL_SET_TESTING_H_
#define KERNEL_SET_TESTING_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

/* The int32 accumulators of ks_gemm_w8a8 before any scaling:
 * acc[M,N] = sum_k A[m,k] * B[k,n], computed by the same MFMA kernel. No
 * reference counterpart; used to check that accumulation is exact. */
KS_API ks_status_t ks_testing_gemm_w8a8_i32(int32_t* acc, const void* a_i8,
                                            const void* b_i8, int64_t m,
                                            int64_t n, int64_t k,
                                            ks_stream_t stream);

/* out[i] = the 16-bit rounding (bf16 or f16, round to nearest even, NaN kept
 * quiet) that every kernel applies to its fp32 results, of the fp32 bit
 * pattern start + i, i < n. No reference counterpart; used to pin the output
 * rounding against the integer definition over whole ranges of inputs. */
KS_API ks_status_t ks_testing_round_bits(void* out, uint32_t start, int64_t n,
                                         ks_dtype_t out_dtype, ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_TESTING_H_ */
