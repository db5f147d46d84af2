/*
 * kernel-set (MI355X build) -- activation quantizers and weight-format helpers.
 *
 * Prototypes identical to the reference ABI (include/kernel_set/quant.h of
 * cklxx/kernel-set). Scales are fp32. Dynamic quantizers derive
 *   scale = max(amax / qmax, 1e-12)   (qmax 448 e4m3, 57344 e5m2, 127 int8)
 * and encode x * (1/scale): a correctly rounded reciprocal, then a multiply.
 * fp8 encoding is round-to-nearest-even with saturation to the finite max.
 *
 * Out of scope (not exported): ks_quantize_nvfp4.
 */
#ifndef KERNEL_SET_QUANT_H_
#define KERNEL_SET_QUANT_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

/* Replaces reference quant.h:14-20 (kernels/src/quant/quant_fp8.cu:148-239).
 * mode PER_TOKEN: scale [rows]; PER_TENSOR: scale [1], which is also used as
 * the amax accumulator while the call runs. in_dtype f32/f16/bf16. */
KS_API ks_status_t ks_quantize_fp8(void* out, float* scale, const void* input,
                                   int64_t rows, int64_t cols,
                                   ks_dtype_t in_dtype, ks_dtype_t fp8_dtype,
                                   ks_quant_mode_t mode, ks_stream_t stream);

/* Replaces reference quant.h:22-26 (quant_fp8.cu:241-291): out = fp8 * scale. */
KS_API ks_status_t ks_dequantize_fp8(void* out, const void* input,
                                     const float* scale, int64_t rows,
                                     int64_t cols, ks_dtype_t out_dtype,
                                     ks_dtype_t fp8_dtype, ks_quant_mode_t mode,
                                     ks_stream_t stream);

/* Replaces reference quant.h:28-40 (kernels/src/quant/quant_fp8_group.cu:133-214).
 * One scale per (row, group of group_size columns); the last group of a row
 * may be short. scale is [rows, ceil(cols/group_size)]. */
KS_API ks_status_t ks_quantize_fp8_group(void* out, float* scale,
                                         const void* input, int64_t rows,
                                         int64_t cols, int group_size,
                                         ks_dtype_t in_dtype,
                                         ks_dtype_t fp8_dtype,
                                         ks_stream_t stream);

/* Replaces reference quant.h:42-46 (kernels/src/quant/quant_int8.cu:118-171).
 * q = round_half_even(clamp(x * (1/scale), -127, 127)). */
KS_API ks_status_t ks_quantize_int8(void* out, float* scale, const void* input,
                                    int64_t rows, int64_t cols,
                                    ks_dtype_t in_dtype, ks_quant_mode_t mode,
                                    ks_stream_t stream);

/* Replaces reference quant.h:48-51 (quant_int8.cu:173-199): out = q * scale. */
KS_API ks_status_t ks_dequantize_int8(void* out, const void* input,
                                      const float* scale, int64_t rows,
                                      int64_t cols, ks_dtype_t out_dtype,
                                      ks_quant_mode_t mode, ks_stream_t stream);

/* Replaces reference quant.h:53-58 (kernels/src/quant/dequant_int4.cu:35-112).
 * qweight_packed int32 [K/8, N]: code of row k is (word >> 4*(k%8)) & 0xF.
 * out[k,n] = (code - zeros[k/gs,n]) * scales[k/gs,n] in out_dtype (f16/bf16/f32;
 * scales and zeros share it and are both required). K must be a multiple of 8
 * and of group_size. */
KS_API ks_status_t ks_dequantize_int4(void* out, const void* qweight_packed,
                                      const void* scales, const void* zeros,
                                      int64_t k, int64_t n, int group_size,
                                      ks_dtype_t out_dtype, ks_stream_t stream);

/* Replaces reference quant.h:60-66 (kernels/src/quant/repack_int4.cu:40-71).
 * int32 [K/8, N] (8 codes per word along K) -> uint8 [K/2, N] as consumed by
 * ks_gemm_w4a16. num_bits must be 4. perm == NULL keeps the row order; a
 * non-NULL perm is an int32 [K] act-order permutation: output row k takes the
 * code of input row perm[k] (the reference returns NOT_IMPLEMENTED for it). */
KS_API ks_status_t ks_repack_int4(void* out_packed, const void* qweight,
                                  const void* perm, int64_t size_k, int64_t size_n,
                                  int num_bits, ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_QUANT_H_ */
