/*
 * kernel-set (MI355X build) -- grouped W4A16 GEMM for Mixture-of-Experts.
 *
 * EXTENSION: the reference has no quantized grouped GEMM. This entry point
 * follows the argument conventions of ks_moe_grouped_gemm (reference
 * include/kernel_set/moe.h:57-65, kernels/src/moe/moe_grouped_gemm.cu:136-198)
 * with the weight operand replaced by the ks_gemm_w4a16 format (reference
 * gemm.h:51-59):
 *   for every expert e, rows [off_e, off_{e+1}) of A [total_rows, K] are
 *   multiplied by dequant(B_e), written to the same rows of C [total_rows, N].
 *   b_packed: uint8 [E, K/2, N]; scales/zeros: dtype [E, K/gs, N] (zeros may be
 *   NULL = 0); expert_offsets: int32 [E+1], non-decreasing, offsets[E] ==
 *   total_rows. Rows outside every expert's range are left untouched.
 * Unlike the reference grouped GEMM it allocates nothing and never synchronizes
 * the stream: the schedule is derived on the device from expert_offsets.
 */
#ifndef KERNEL_SET_MOE_W4A16_H_
#define KERNEL_SET_MOE_W4A16_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

KS_API ks_status_t ks_moe_grouped_gemm_w4a16(
    void* c, const void* a, const void* b_packed, const void* scales,
    const void* zeros, const int32_t* expert_offsets, int num_experts,
    int64_t total_rows, int64_t n, int64_t k, int group_size, ks_dtype_t dtype,
    ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_MOE_W4A16_H_ */
