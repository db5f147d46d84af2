/*
 * kernel-set (MI355X build) -- MoE routing around the grouped W4A16 GEMM.
 *
 * Same entry points, argument order and meaning as the reference's
 * include/kernel_set/moe.h:15-65 (gate -> permutation -> permute -> grouped
 * GEMM -> unpermute). The quantized grouped GEMM is the extension
 * ks_moe_grouped_gemm_w4a16 (moe_w4a16.h).
 *
 * Differences from the reference, all on the safe side of its contract:
 *   - ks_moe_compute_permutation is deterministic: inside each expert the pair
 *     ids are in increasing order (the reference leaves that order to atomic
 *     arrival, kernels/src/moe/moe_permute.cu:86-90). It allocates nothing and
 *     never synchronizes the stream (the reference mallocs and syncs).
 *   - ks_moe_unpermute keeps its inverse map in library scratch owned per
 *     (device, stream) instead of a malloc/free per call.
 */
#ifndef KERNEL_SET_MOE_H_
#define KERNEL_SET_MOE_H_

#include "kernel_set/types.h"

KS_BEGIN_EXTERN_C

/* Softmax over experts, then top-k (lowest expert id wins ties).
 * Reference: include/kernel_set/moe.h:15-22, kernels/src/moe/moe_gate.cu:42-117,245-277.
 *   logits [num_tokens, num_experts] (f32/f16/bf16); out_weights fp32 and
 *   out_indices int32 [num_tokens, top_k]; renormalize != 0 divides the chosen
 *   weights by their sum. num_experts <= 1024, top_k <= 32. */
KS_API ks_status_t ks_moe_gate_softmax_topk(
    float* out_weights, int32_t* out_indices, const void* logits,
    int64_t num_tokens, int num_experts, int top_k, int renormalize,
    ks_dtype_t dtype, ks_stream_t stream);

/* Sigmoid scores, group-limited top-k (DeepSeek-V3): groups ranked by the sum
 * of their two best biased scores, top_k experts picked from the topk_group
 * best groups by biased score; weights are the unbiased sigmoid scores,
 * optionally renormalized, times routed_scaling_factor. correction_bias
 * [num_experts] may be NULL.
 * Reference: include/kernel_set/moe.h:24-31, kernels/src/moe/moe_gate.cu:119-236,279-317. */
KS_API ks_status_t ks_moe_gate_sigmoid_group_topk(
    float* out_weights, int32_t* out_indices, const void* logits,
    const void* correction_bias, int64_t num_tokens, int num_experts,
    int n_group, int topk_group, int top_k, int renormalize,
    float routed_scaling_factor, ks_dtype_t dtype, ks_stream_t stream);

/* Group the routed pairs (pair = token * top_k + slot) by expert.
 *   topk_indices [num_tokens, top_k] int32 -> sorted_token_ids
 *   [num_tokens*top_k] int32 and expert_offsets [num_experts+1] int32 (CSR).
 * Pairs whose expert id is out of range are dropped. num_experts <= 2048.
 * Reference: include/kernel_set/moe.h:33-40, kernels/src/moe/moe_permute.cu:58-101,179-248. */
KS_API ks_status_t ks_moe_compute_permutation(
    int32_t* sorted_token_ids, int32_t* expert_offsets,
    const int32_t* topk_indices, int64_t num_tokens, int num_experts,
    int top_k, ks_stream_t stream);

/* permuted[r] = input[sorted_token_ids[r] / top_k] for r < num_tokens*top_k;
 * rows with an out-of-range id are zero-filled.
 * Reference: include/kernel_set/moe.h:42-47, kernels/src/moe/moe_permute.cu:103-129,250-282. */
KS_API ks_status_t ks_moe_permute(void* permuted, const void* input,
                                  const int32_t* sorted_token_ids,
                                  int64_t num_tokens, int top_k, int64_t hidden,
                                  ks_dtype_t dtype, ks_stream_t stream);

/* out[token] = sum_k weight[token,k] * permuted[pos(token,k)] in fp32, slots in
 * increasing k, rounded once to dtype; pairs absent from sorted_token_ids add 0.
 * Reference: include/kernel_set/moe.h:49-55, kernels/src/moe/moe_permute.cu:131-170,284-382. */
KS_API ks_status_t ks_moe_unpermute(void* out, const void* permuted,
                                    const int32_t* sorted_token_ids,
                                    const float* routing_weights,
                                    int64_t num_tokens, int top_k,
                                    int64_t hidden, ks_dtype_t dtype,
                                    ks_stream_t stream);

/* Dense grouped GEMM: for each expert e,
 * C[off_e:off_{e+1}] = A[off_e:off_{e+1}] @ B_e, fp32 accumulation, one
 * rounding to dtype (f32, f16, bf16, f8e4m3, f8e5m2; A, B and C share it).
 *   a [total_rows, k]; b [num_experts, k, n] (n contiguous); expert_offsets
 *   [num_experts+1] int32 row boundaries; c [total_rows, n]. Rows outside
 *   every expert's range are not written.
 * Reference: include/kernel_set/moe.h:57-65, kernels/src/moe/moe_grouped_gemm.cu:136-198. */
KS_API ks_status_t ks_moe_grouped_gemm(
    void* c, const void* a, const void* b, const int32_t* expert_offsets,
    int num_experts, int64_t total_rows, int64_t n, int64_t k,
    ks_dtype_t dtype, ks_stream_t stream);

KS_END_EXTERN_C

#endif /* KERNEL_SET_MOE_H_ */
