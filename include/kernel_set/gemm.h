/*
 * kernel-set (MI355X build) -- quantized GEMMs.
 *
 * The first four entry points keep the exact prototypes of the reference ABI
 * (include/kernel_set/gemm.h of cklxx/kernel-set) so existing bindings load
 * this library unchanged; ks_gemm_fp8_blockwise_fused_quant is an extension
 * of this build. All matrices are row-major and device resident; every call
 * only enqueues work on `stream` (NULL = null stream).
 *
 * Out of scope for this build (not exported): ks_gemm, ks_gemm_bias_act,
 * ks_gemm_batched, ks_gemm_nvfp4.
 */
#ifndef KERNEL_SET_GEMM_H_
#define KERNEL_SET_GEMM_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

/* Replaces reference gemm.h:39-49 (kernels/src/gemm/gemm_w8a8.cu:166-217).
 * C[M,N] = (float(acc) * a_s) * b_s (+ bias), acc = sum_k A[m,k]*B[k,n] in exact
 * int32. A int8 [M,K], B int8 [K,N]. a_scale fp32 [M] (PER_TOKEN) or [1]
 * (PER_TENSOR); b_scale fp32 [N] (PER_CHANNEL) or [1] (PER_TENSOR). bias is [N]
 * in out_dtype or NULL. out_dtype f32/f16/bf16. Runs on int8 MFMA. */
KS_API ks_status_t ks_gemm_w8a8(void* c, const void* a_i8, const void* b_i8,
                                const float* a_scale, const float* b_scale,
                                const void* bias, int64_t m, int64_t n,
                                int64_t k, ks_quant_mode_t a_mode,
                                ks_quant_mode_t b_mode, ks_dtype_t out_dtype,
                                ks_stream_t stream);

/* Replaces reference gemm.h:51-59 (kernels/src/gemm/gemm_w4a16.cu:151-182).
 * C[M,N] = A[M,K] @ W + bias, W[k,n] = (q[k,n] - zeros[k/gs,n]) * scales[k/gs,n].
 * b_packed uint8 [K/2, N]: byte (k/2)*N+n holds q[k even] in bits 0-3 and
 * q[k odd] in bits 4-7, codes 0..15. scales/zeros/bias/A/C share `dtype`
 * (f16 or bf16); zeros and bias may be NULL (zero). group_size <= 0 means one
 * group over all K. K must be even and a multiple of the group size. */
KS_API ks_status_t ks_gemm_w4a16(void* c, const void* a, const void* b_packed,
                                 const void* scales, const void* zeros,
                                 const void* bias, int64_t m, int64_t n,
                                 int64_t k, int group_size, ks_dtype_t dtype,
                                 ks_stream_t stream);

/* No counterpart in the reference. ks_gemm_w4a16 with the same arguments and
 * the same result bits, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): split-K
 * partials live in a fixed 16 MiB per-device array instead of library-
 * allocated scratch, and the call never allocates. A shape that needs more
 * returns KS_ERROR_INVALID_ARGUMENT. Calls that overlap on one device (other
 * streams, other threads) race on that array. */
KS_API ks_status_t ks_gemm_w4a16_noalloc(void* c, const void* a, const void* b_packed,
                                         const void* scales, const void* zeros,
                                         const void* bias, int64_t m, int64_t n,
                                         int64_t k, int group_size, ks_dtype_t dtype,
                                         ks_stream_t stream);

/* Replaces reference gemm.h:60-77 (kernels/src/gemm/gemm_fp8.cu:206-290).
 * fp8 A [M,K] x fp8 B [K,N] (both e4m3 or both e5m2, fp8_dtype), fp32
 * accumulation over all of K, then C = (acc * a_s) * b_s with a_scale fp32 [M]
 * (KS_QUANT_PER_TOKEN) or [1] (PER_TENSOR) and b_scale fp32 [N]
 * (KS_QUANT_PER_CHANNEL) or [1] (PER_TENSOR). out_dtype f32/f16/bf16. */
KS_API ks_status_t ks_gemm_fp8(void* out, const void* a_fp8, const void* b_fp8,
                               const float* a_scale, const float* b_scale,
                               int64_t m, int64_t n, int64_t k,
                               ks_quant_mode_t a_mode, ks_quant_mode_t b_mode,
                               ks_dtype_t fp8_dtype, ks_dtype_t out_dtype,
                               ks_stream_t stream);

/* Replaces reference gemm.h:79-98 (kernels/src/gemm/gemm_fp8_blockwise.cu:218-302).
 * fp8 A [M,K] x fp8 B [K,N] with a_scale fp32 [M, ceil(K/block_k)] and b_scale
 * fp32 [ceil(K/block_k), ceil(N/block_n)]. For every K-block the fp32 partial
 * sum is promoted into the output accumulator as part * (a_s * b_s). fp8_dtype
 * is e4m3 or e5m2; out_dtype f32/f16/bf16. */
KS_API ks_status_t ks_gemm_fp8_blockwise(void* out, const void* a_fp8,
                                         const void* b_fp8,
                                         const float* a_scale,
                                         const float* b_scale, int64_t m,
                                         int64_t n, int64_t k, int block_n,
                                         int block_k, ks_dtype_t fp8_dtype,
                                         ks_dtype_t out_dtype,
                                         ks_stream_t stream);

/* Extension: no counterpart in the reference. For callers that hold bf16 /
 * f16 / f32 activations and would otherwise call ks_quantize_fp8_group and
 * then ks_gemm_fp8_blockwise (the reference's own 1 x 128 / 128 x 128 recipe,
 * quant.h:35-40 + gemm.h:79-98). Defined as exactly that composition:
 *   (a8, a_scale) = ks_quantize_fp8_group(a, group_size = block_k, fp8_dtype)
 *   out           = ks_gemm_fp8_blockwise(a8, b_fp8, a_scale, b_scale, ...)
 * and returns the same bits. For M <= 8 it runs as one pass (each workgroup
 * quantizes its own K slice into LDS; requires block_k in {32, 64, 128, 256},
 * block_n % 16 == 0, N % 16 == 0, K % 32 == 0 and a 16-byte-aligned `a`);
 * otherwise it quantizes into library staging (per device and stream) and runs
 * the GEMM. a_dtype f32/f16/bf16; fp8_dtype e4m3/e5m2; out_dtype f32/f16/bf16. */
KS_API ks_status_t ks_gemm_fp8_blockwise_fused_quant(void* out, const void* a,
                                                     const void* b_fp8,
                                                     const float* b_scale,
                                                     int64_t m, int64_t n,
                                                     int64_t k, int block_n,
                                                     int block_k,
                                                     ks_dtype_t a_dtype,
                                                     ks_dtype_t fp8_dtype,
                                                     ks_dtype_t out_dtype,
                                                     ks_stream_t stream);

/* Extension: no counterpart in the reference. For callers that hold bf16 /
 * f16 / f32 activations and would otherwise call ks_quantize_int8 and then
 * ks_gemm_w8a8 (the reference's dynamic int8 recipe, quant.h:42-46 +
 * gemm.h:39-49). Defined as exactly that composition:
 *   (a8, a_scale) = ks_quantize_int8(a, rows = m, cols = k, a_dtype, a_mode)
 *   c             = ks_gemm_w8a8(a8, b_i8, a_scale, b_scale, bias, ..., a_mode, b_mode)
 * and returns the same bits. a_mode is PER_TOKEN (one scale per row) or
 * PER_TENSOR. For M <= 4 (N % 16 == 0, K % 32 == 0, 16-byte-aligned `a` and
 * `b_i8`) it runs as one pass: every workgroup reduces the row maxima over the
 * whole of K and quantizes its own K slice into LDS; otherwise it quantizes
 * into library staging (per device and stream) and runs the GEMM.
 * a_dtype f32/f16/bf16; out_dtype f32/f16/bf16; bias [N] in out_dtype or NULL. */
KS_API ks_status_t ks_gemm_w8a8_fused_quant(void* c, const void* a,
                                            const void* b_i8,
                                            const float* b_scale,
                                            const void* bias, int64_t m,
                                            int64_t n, int64_t k,
                                            ks_quant_mode_t a_mode,
                                            ks_quant_mode_t b_mode,
                                            ks_dtype_t a_dtype,
                                            ks_dtype_t out_dtype,
                                            ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_GEMM_H_ */
