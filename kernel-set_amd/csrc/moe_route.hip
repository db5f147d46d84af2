// kernel-set (MI355X build) -- MoE routing: gates, permutation, permute,
// unpermute (include/kernel_set/moe.h; reference kernels/src/moe/moe_gate.cu
// and kernels/src/moe/moe_permute.cu of cklxx/kernel-set).
//
// Gates: one wave64 per token, experts strided over the lanes (lane l holds
// experts l, l+64, ...), so the logits load is coalesced and every reduction
// (max, sum, arg-max for each of the top_k picks, the per-group top-2) is a
// wave butterfly instead of the reference's single-thread selection loops.
// Selection semantics follow the reference exactly: strict ">" scans in
// increasing expert id, i.e. the lowest id wins a tie; a picked expert is
// masked with -FLT_MAX.
//
// Permutation: one 1024-thread workgroup runs a stable counting sort in LDS
// (per-wave expert histograms -> CSR offsets -> ordered scatter), so the
// output is deterministic (pair ids increase inside each expert) and nothing
// is allocated or synchronized.
#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <string>

#include "kernel_set/moe.h"
#include "ks_common.hpp"
#include "workspace.hpp"

namespace ks {
namespace route {

constexpr int kMaxExperts = 1024;   // gates (reference moe_gate.cu:33)
constexpr int kMaxTopK = 32;        // reference moe_gate.cu:35
constexpr int kMaxGroups = 64;      // reference moe_gate.cu:37
constexpr int kPerLane = kMaxExperts / kWave;
constexpr int kGateThreads = 256;   // four tokens per workgroup
constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / kWave;
constexpr int kMaxPermExperts = 2048;
constexpr float kNegMax = -FLT_MAX;

// Wave arg-max: larger value wins, equal values go to the lower index.
__device__ inline void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const int oi = __shfl_xor(i, o, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// Same, carrying a payload of the winner.
__device__ inline void wave_argmax(float& v, int& i, float& w) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const int oi = __shfl_xor(i, o, kWave);
    const float ow = __shfl_xor(w, o, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
      w = ow;
    }
  }
}

// Wave top-2 of a multiset: (m1, m2) = largest and second largest.
__device__ inline void wave_top2(float& m1, float& m2) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float a1 = __shfl_xor(m1, o, kWave);
    const float a2 = __shfl_xor(m2, o, kWave);
    const float hi = fmaxf(m1, a1);
    const float lo = fmaxf(fminf(m1, a1), fmaxf(m2, a2));
    m1 = hi;
    m2 = lo;
  }
}

__device__ inline float sigmoid_f(float x) {
  if (x >= 0.f) return 1.f / (1.f + __expf(-x));
  const float z = __expf(x);
  return z / (1.f + z);
}

// ---------------------------------------------------------------------------
// softmax -> top-k
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kGateThreads)
gate_softmax_topk_kernel(float* __restrict__ out_w, int32_t* __restrict__ out_i,
                         const typename T::storage* __restrict__ logits,
                         int64_t num_tokens, int num_experts, int top_k, int renormalize) {
  const int lane = threadIdx.x % kWave;
  const int64_t token = static_cast<int64_t>(blockIdx.x) * (kGateThreads / kWave) +
                        threadIdx.x / kWave;
  if (token >= num_tokens) return;  // whole wave leaves together
  const auto* row = logits + token * num_experts;
  const int per = (num_experts + kWave - 1) / kWave;

  float p[kPerLane];
  float mx = kNegMax;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = lane + kWave * j;
    p[j] = (j < per && e < num_experts) ? elem<T>::load(row, e) : kNegMax;
    mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = lane + kWave * j;
    if (j < per && e < num_experts) {
      p[j] = __expf(p[j] - mx);
      sum += p[j];
    }
  }
  sum = wave_sum(sum);
  const float inv = 1.f / sum;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = lane + kWave * j;
    p[j] = (j < per && e < num_experts) ? p[j] * inv : kNegMax;
  }

  float chosen_w = 0.f;  // lane k keeps pick k
  int chosen_i = 0;
  float renorm = 0.f;
  for (int k = 0; k < top_k; ++k) {
    float bv = kNegMax;
    int bi = INT32_MAX;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      if (p[j] > bv) {  // ascending ids within the lane: first max kept
        bv = p[j];
        bi = lane + kWave * j;
      }
    }
    wave_argmax(bv, bi);
    if (lane == k) {
      chosen_w = bv;
      chosen_i = bi;
    }
    renorm += bv;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)  // mask the pick
      if (lane + kWave * j == bi) p[j] = kNegMax;
  }
  const float scale = (renormalize && renorm > 0.f) ? 1.f / renorm : 1.f;
  if (lane < top_k) {
    out_w[token * top_k + lane] = chosen_w * scale;
    out_i[token * top_k + lane] = chosen_i;
  }
}

// ---------------------------------------------------------------------------
// sigmoid -> group-limited top-k (DeepSeek-V3)
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kGateThreads)
gate_sigmoid_group_topk_kernel(float* __restrict__ out_w, int32_t* __restrict__ out_i,
                               const typename T::storage* __restrict__ logits,
                               const typename T::storage* __restrict__ bias,
                               int64_t num_tokens, int num_experts, int n_group,
                               int topk_group, int top_k, int renormalize, float rsf) {
  const int lane = threadIdx.x % kWave;
  const int64_t token = static_cast<int64_t>(blockIdx.x) * (kGateThreads / kWave) +
                        threadIdx.x / kWave;
  if (token >= num_tokens) return;
  const auto* row = logits + token * num_experts;
  const int per = (num_experts + kWave - 1) / kWave;
  const int epg = num_experts / n_group;

  float score[kPerLane], sel[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = lane + kWave * j;
    if (j < per && e < num_experts) {
      score[j] = sigmoid_f(elem<T>::load(row, e));
      sel[j] = bias ? score[j] + elem<T>::load(bias, e) : score[j];
    } else {
      score[j] = 0.f;
      sel[j] = kNegMax;
    }
  }

  // 1) group score = sum of the group's two best biased scores (one if the
  //    group has a single expert); 2) keep the topk_group best groups.
  uint64_t keep = 0;  // bit g set: group g survives
  {
    float gsc = kNegMax;  // lane g holds group g's score
    for (int g = 0; g < n_group; ++g) {
      float m1 = kNegMax, m2 = kNegMax;
#pragma unroll
      for (int j = 0; j < kPerLane; ++j) {
        const int e = lane + kWave * j;
        if (j < per && e < num_experts && e / epg == g) {
          const float v = sel[j];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
      }
      wave_top2(m1, m2);
      const float s = epg >= 2 ? m1 + m2 : m1;
      if (lane == g) gsc = s;
    }
    const int kg = topk_group < n_group ? topk_group : n_group;
    for (int t = 0; t < kg; ++t) {
      const bool cand = lane < n_group && !((keep >> lane) & 1ull);
      float bv = cand ? gsc : kNegMax;
      int bi = lane < n_group ? lane : INT32_MAX;
      wave_argmax(bv, bi);
      if (bv == kNegMax) break;  // nothing left above -FLT_MAX (reference: best_g < 0)
      keep |= 1ull << bi;
    }
  }

  // 3) top_k over the surviving experts by biased score; weight = unbiased.
  float chosen_w = 0.f;
  int chosen_i = 0;
  float renorm = 0.f;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int e = lane + kWave * j;
    if (!(j < per && e < num_experts) || !((keep >> (e / epg)) & 1ull)) sel[j] = kNegMax;
  }
  for (int k = 0; k < top_k; ++k) {
    float bv = kNegMax, bw = 0.f;
    int bi = INT32_MAX;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      if (sel[j] > bv) {
        bv = sel[j];
        bi = lane + kWave * j;
        bw = score[j];
      }
    }
    wave_argmax(bv, bi, bw);
    if (bi == INT32_MAX) continue;  // fewer eligible experts than top_k: id 0, weight 0
    if (lane == k) {
      chosen_w = bw;
      chosen_i = bi;
    }
    renorm += bw;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (lane + kWave * j == bi) sel[j] = kNegMax;
  }
  const float norm = (renormalize && renorm > 0.f) ? 1.f / renorm : 1.f;
  if (lane < top_k) {
    out_w[token * top_k + lane] = chosen_w * norm * rsf;
    out_i[token * top_k + lane] = chosen_i;
  }
}

// ---------------------------------------------------------------------------
// stable counting sort of the routed pairs by expert (one workgroup)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kPermThreads)
permutation_kernel(int32_t* __restrict__ sorted, int32_t* __restrict__ offsets,
                   const int32_t* __restrict__ idx, int32_t num_pairs, int num_experts) {
  extern __shared__ int32_t lds[];
  int32_t* cnt = lds;                                   // [kPermWaves][E] -> write bases
  int32_t* wsum = lds + kPermWaves * num_experts;       // [kPermWaves] scan carries
  const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
  const int E = num_experts;
  for (int i = t; i < kPermWaves * E; i += kPermThreads) cnt[i] = 0;
  __syncthreads();

  // Wave w owns the contiguous pair range [p0, p1).
  const int32_t seg = (num_pairs + kPermWaves - 1) / kPermWaves;
  const int32_t p0 = min(num_pairs, w * seg), p1 = min(num_pairs, p0 + seg);
  for (int32_t b = p0; b < p1; b += kWave) {
    const int32_t pr = b + lane;
    if (pr < p1) {
      const int e = idx[pr];
      if (e >= 0 && e < E) atomicAdd(&cnt[w * E + e], 1);
    }
  }
  __syncthreads();

  // Totals per expert, exclusive scan over experts, then per-wave bases:
  // base[w][e] = offsets[e] + sum_{w' < w} cnt[w'][e].
  for (int e0 = 0; e0 < E; e0 += kPermThreads) {
    const int e = e0 + t;
    int total = 0;
    if (e < E)
      for (int ww = 0; ww < kPermWaves; ++ww) total += cnt[ww * E + e];
    // inclusive scan of `total` across the workgroup
    int incl = total;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int y = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += y;
    }
    if (lane == kWave - 1) wsum[w] = incl;
    __syncthreads();
    if (t == 0) {
      int run = (e0 == 0) ? 0 : wsum[kPermWaves];  // carry from previous chunk
      for (int ww = 0; ww < kPermWaves; ++ww) {
        const int v = wsum[ww];
        wsum[ww] = run;
        run += v;
      }
      wsum[kPermWaves] = run;
    }
    __syncthreads();
    if (e < E) {
      int base = wsum[w] + incl - total;  // exclusive prefix = offsets[e]
      offsets[e] = base;
      for (int ww = 0; ww < kPermWaves; ++ww) {
        const int c = cnt[ww * E + e];
        cnt[ww * E + e] = base;
        base += c;
      }
    }
    __syncthreads();
  }
  if (t == 0) offsets[E] = wsum[kPermWaves];

  // Ordered scatter: inside a 64-pair batch a lane's rank among earlier lanes
  // with the same expert is counted by broadcast; batches run in order.
  for (int32_t b = p0; b < p1; b += kWave) {
    const int32_t pr = b + lane;
    const int e = pr < p1 ? idx[pr] : -1;
    const bool ok = e >= 0 && e < E;
    int rank = 0;
    for (int j = 0; j < kWave; ++j) {
      const int ej = __shfl(e, j, kWave);
      rank += (j < lane && ej == e) ? 1 : 0;
    }
    int pos = 0;
    if (ok) pos = cnt[w * E + e] + rank;
    __builtin_amdgcn_wave_barrier();  // every lane has read its base before any update
    if (ok) {
      sorted[pos] = pr;
      atomicAdd(&cnt[w * E + e], 1);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
// permute / unpermute
// ---------------------------------------------------------------------------
constexpr int kRowThreads = 256;

template <typename T>
__global__ void __launch_bounds__(kRowThreads)
permute_kernel(typename T::storage* __restrict__ out, const typename T::storage* __restrict__ in,
               const int32_t* __restrict__ sorted, int top_k, int64_t hidden, int64_t rows,
               bool vec) {
  // one wave per output row
  const int lane = threadIdx.x % kWave;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kRowThreads / kWave) + threadIdx.x / kWave;
  if (r >= rows) return;
  using S = typename T::storage;
  const int32_t pair = sorted[r];
  const bool valid = pair >= 0 && static_cast<int64_t>(pair) < rows;
  S* dst = out + r * hidden;
  const S* src = in + (valid ? static_cast<int64_t>(pair) / top_k : 0) * hidden;
  if (vec) {  // 16-byte chunks
    const int64_t n16 = hidden * static_cast<int64_t>(sizeof(S)) / 16;
    for (int64_t c = lane; c < n16; c += kWave) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (valid) v = reinterpret_cast<const uint4*>(src)[c];
      reinterpret_cast<uint4*>(dst)[c] = v;
    }
  } else {
    for (int64_t i = lane; i < hidden; i += kWave) dst[i] = valid ? src[i] : S(0);
  }
}

// inverse[pair] = permuted row; -1 where no row maps to the pair.
__global__ void __launch_bounds__(kRowThreads)
fill_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void __launch_bounds__(kRowThreads)
inverse_kernel(int32_t* __restrict__ inv, const int32_t* __restrict__ sorted, int64_t rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowThreads + threadIdx.x;
  if (r >= rows) return;
  const int32_t pair = sorted[r];
  if (pair >= 0 && static_cast<int64_t>(pair) < rows) inv[pair] = static_cast<int32_t>(r);
}

template <typename T>
__global__ void __launch_bounds__(kRowThreads)
unpermute_kernel(typename T::storage* __restrict__ out, const typename T::storage* __restrict__ perm,
                 const int32_t* __restrict__ inv, const float* __restrict__ weights,
                 int64_t num_tokens, int top_k, int64_t hidden) {
  // one wave per token; fp32 accumulation over the slots in increasing k
  const int lane = threadIdx.x % kWave;
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * (kRowThreads / kWave) + threadIdx.x / kWave;
  if (tok >= num_tokens) return;
  for (int64_t i = lane; i < hidden; i += kWave) {
    float acc = 0.f;
    for (int k = 0; k < top_k; ++k) {
      const int64_t pair = tok * top_k + k;
      const int32_t pr = inv[pair];
      if (pr < 0) continue;
      acc = fmaf(elem<T>::load(perm, static_cast<int64_t>(pr) * hidden + i), weights[pair], acc);
    }
    out[tok * hidden + i] = elem<T>::from_f32(acc);
  }
}

inline ks_status_t check_pairs(int64_t num_tokens, int top_k, const char* who, int64_t* pairs) {
  if (top_k > 0 && num_tokens > INT32_MAX / top_k)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, std::string(who) + ": num_tokens*top_k exceeds int32 limit");
  *pairs = num_tokens * top_k;
  return KS_SUCCESS;
}

}  // namespace route
}  // namespace ks

using namespace ks;
using namespace ks::route;

extern "C" {

ks_status_t ks_moe_gate_softmax_topk(float* out_weights, int32_t* out_indices, const void* logits,
                                     int64_t num_tokens, int num_experts, int top_k,
                                     int renormalize, ks_dtype_t dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(out_weights);
  KS_REQUIRE_PTR(out_indices);
  KS_REQUIRE_PTR(logits);
  if (num_tokens <= 0 || num_experts <= 0 || top_k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_softmax_topk: bad shape");
  if (top_k > num_experts)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_softmax_topk: top_k > num_experts");
  if (num_experts > kMaxExperts)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_gate_softmax_topk: num_experts exceeds 1024");
  if (top_k > kMaxTopK)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_gate_softmax_topk: top_k exceeds 32");
  const int64_t blocks = (num_tokens + kGateThreads / kWave - 1) / (kGateThreads / kWave);
  if (blocks > INT32_MAX) KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_gate_softmax_topk: too many tokens");
  auto s = to_stream(stream);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kGateThreads);
  switch (dtype) {
    case KS_DTYPE_F32:
      hipLaunchKernelGGL((gate_softmax_topk_kernel<f32_t>), grid, block, 0, s, out_weights, out_indices,
                         static_cast<const float*>(logits), num_tokens, num_experts, top_k, renormalize);
      break;
    case KS_DTYPE_F16:
      hipLaunchKernelGGL((gate_softmax_topk_kernel<f16_t>), grid, block, 0, s, out_weights, out_indices,
                         static_cast<const uint16_t*>(logits), num_tokens, num_experts, top_k, renormalize);
      break;
    case KS_DTYPE_BF16:
      hipLaunchKernelGGL((gate_softmax_topk_kernel<bf16_t>), grid, block, 0, s, out_weights, out_indices,
                         static_cast<const uint16_t*>(logits), num_tokens, num_experts, top_k, renormalize);
      break;
    default:
      KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_gate_softmax_topk: unsupported dtype");
  }
  KS_LAUNCH_STATUS("ks_moe_gate_softmax_topk");
  return KS_SUCCESS;
}

ks_status_t ks_moe_gate_sigmoid_group_topk(float* out_weights, int32_t* out_indices,
                                           const void* logits, const void* correction_bias,
                                           int64_t num_tokens, int num_experts, int n_group,
                                           int topk_group, int top_k, int renormalize,
                                           float routed_scaling_factor, ks_dtype_t dtype,
                                           ks_stream_t stream) {
  KS_REQUIRE_PTR(out_weights);
  KS_REQUIRE_PTR(out_indices);
  KS_REQUIRE_PTR(logits);
  if (num_tokens <= 0 || num_experts <= 0 || top_k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_sigmoid_group_topk: bad shape");
  if (n_group <= 0 || topk_group <= 0 || topk_group > n_group)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_sigmoid_group_topk: bad group config");
  if (num_experts % n_group != 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_sigmoid_group_topk: num_experts % n_group");
  if (top_k > num_experts)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_gate_sigmoid_group_topk: top_k > num_experts");
  if (num_experts > kMaxExperts || top_k > kMaxTopK || n_group > kMaxGroups)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_gate_sigmoid_group_topk: config exceeds limits");
  const int64_t blocks = (num_tokens + kGateThreads / kWave - 1) / (kGateThreads / kWave);
  if (blocks > INT32_MAX)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_gate_sigmoid_group_topk: too many tokens");
  auto s = to_stream(stream);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kGateThreads);
  switch (dtype) {
    case KS_DTYPE_F32:
      hipLaunchKernelGGL((gate_sigmoid_group_topk_kernel<f32_t>), grid, block, 0, s, out_weights,
                         out_indices, static_cast<const float*>(logits),
                         static_cast<const float*>(correction_bias), num_tokens, num_experts,
                         n_group, topk_group, top_k, renormalize, routed_scaling_factor);
      break;
    case KS_DTYPE_F16:
      hipLaunchKernelGGL((gate_sigmoid_group_topk_kernel<f16_t>), grid, block, 0, s, out_weights,
                         out_indices, static_cast<const uint16_t*>(logits),
                         static_cast<const uint16_t*>(correction_bias), num_tokens, num_experts,
                         n_group, topk_group, top_k, renormalize, routed_scaling_factor);
      break;
    case KS_DTYPE_BF16:
      hipLaunchKernelGGL((gate_sigmoid_group_topk_kernel<bf16_t>), grid, block, 0, s, out_weights,
                         out_indices, static_cast<const uint16_t*>(logits),
                         static_cast<const uint16_t*>(correction_bias), num_tokens, num_experts,
                         n_group, topk_group, top_k, renormalize, routed_scaling_factor);
      break;
    default:
      KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_gate_sigmoid_group_topk: unsupported dtype");
  }
  KS_LAUNCH_STATUS("ks_moe_gate_sigmoid_group_topk");
  return KS_SUCCESS;
}

ks_status_t ks_moe_compute_permutation(int32_t* sorted_token_ids, int32_t* expert_offsets,
                                       const int32_t* topk_indices, int64_t num_tokens,
                                       int num_experts, int top_k, ks_stream_t stream) {
  KS_REQUIRE_PTR(sorted_token_ids);
  KS_REQUIRE_PTR(expert_offsets);
  KS_REQUIRE_PTR(topk_indices);
  if (num_tokens <= 0 || num_experts <= 0 || top_k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_compute_permutation: bad shape");
  int64_t pairs = 0;
  ks_status_t r = check_pairs(num_tokens, top_k, "ks_moe_compute_permutation", &pairs);
  if (r != KS_SUCCESS) return r;
  if (num_experts > kMaxPermExperts)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_compute_permutation: num_experts exceeds 2048");
  const size_t lds = (static_cast<size_t>(kPermWaves) * num_experts + kPermWaves + 1) * sizeof(int32_t);
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&permutation_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>((kPermWaves * kMaxPermExperts + kPermWaves + 1) * 4));
    return true;
  }();
  (void)configured;
  auto s = to_stream(stream);
  hipLaunchKernelGGL(permutation_kernel, dim3(1), dim3(kPermThreads), lds, s, sorted_token_ids,
                     expert_offsets, topk_indices, static_cast<int32_t>(pairs), num_experts);
  KS_LAUNCH_STATUS("ks_moe_compute_permutation");
  return KS_SUCCESS;
}

ks_status_t ks_moe_permute(void* permuted, const void* input, const int32_t* sorted_token_ids,
                           int64_t num_tokens, int top_k, int64_t hidden, ks_dtype_t dtype,
                           ks_stream_t stream) {
  KS_REQUIRE_PTR(permuted);
  KS_REQUIRE_PTR(input);
  KS_REQUIRE_PTR(sorted_token_ids);
  if (num_tokens <= 0 || top_k <= 0 || hidden <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_permute: bad shape");
  int64_t rows = 0;
  ks_status_t r = check_pairs(num_tokens, top_k, "ks_moe_permute", &rows);
  if (r != KS_SUCCESS) return r;
  auto s = to_stream(stream);
  const dim3 grid(static_cast<unsigned>((rows + kRowThreads / kWave - 1) / (kRowThreads / kWave)));
  const dim3 block(kRowThreads);
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool vec = a16(permuted) && a16(input);
  switch (dtype) {
    case KS_DTYPE_F32:
      hipLaunchKernelGGL((permute_kernel<f32_t>), grid, block, 0, s, static_cast<float*>(permuted),
                         static_cast<const float*>(input), sorted_token_ids, top_k, hidden, rows,
                         vec && hidden % 4 == 0);
      break;
    case KS_DTYPE_F16:
    case KS_DTYPE_BF16:
      hipLaunchKernelGGL((permute_kernel<bf16_t>), grid, block, 0, s, static_cast<uint16_t*>(permuted),
                         static_cast<const uint16_t*>(input), sorted_token_ids, top_k, hidden, rows,
                         vec && hidden % 8 == 0);
      break;
    default:
      KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_permute: unsupported dtype");
  }
  KS_LAUNCH_STATUS("ks_moe_permute");
  return KS_SUCCESS;
}

ks_status_t ks_moe_unpermute(void* out, const void* permuted, const int32_t* sorted_token_ids,
                             const float* routing_weights, int64_t num_tokens, int top_k,
                             int64_t hidden, ks_dtype_t dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(permuted);
  KS_REQUIRE_PTR(sorted_token_ids);
  KS_REQUIRE_PTR(routing_weights);
  if (num_tokens <= 0 || top_k <= 0 || hidden <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_unpermute: bad shape");
  if (dtype != KS_DTYPE_F32 && dtype != KS_DTYPE_F16 && dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_unpermute: unsupported dtype");
  int64_t rows = 0;
  ks_status_t r = check_pairs(num_tokens, top_k, "ks_moe_unpermute", &rows);
  if (r != KS_SUCCESS) return r;
  auto s = to_stream(stream);
  Scratch sc;
  r = get_scratch(s, static_cast<size_t>(rows), 0, &sc, "ks_moe_unpermute");
  if (r != KS_SUCCESS) return r;
  int32_t* inv = reinterpret_cast<int32_t*>(sc.partial);
  const dim3 block(kRowThreads);
  const dim3 g1(static_cast<unsigned>((rows + kRowThreads - 1) / kRowThreads));
  hipLaunchKernelGGL(fill_kernel, g1, block, 0, s, inv, rows, -1);
  hipLaunchKernelGGL(inverse_kernel, g1, block, 0, s, inv, sorted_token_ids, rows);
  const dim3 g2(static_cast<unsigned>((num_tokens + kRowThreads / kWave - 1) / (kRowThreads / kWave)));
  switch (dtype) {
    case KS_DTYPE_F32:
      hipLaunchKernelGGL((unpermute_kernel<f32_t>), g2, block, 0, s, static_cast<float*>(out),
                         static_cast<const float*>(permuted), inv, routing_weights, num_tokens, top_k, hidden);
      break;
    case KS_DTYPE_F16:
      hipLaunchKernelGGL((unpermute_kernel<f16_t>), g2, block, 0, s, static_cast<uint16_t*>(out),
                         static_cast<const uint16_t*>(permuted), inv, routing_weights, num_tokens, top_k, hidden);
      break;
    default:
      hipLaunchKernelGGL((unpermute_kernel<bf16_t>), g2, block, 0, s, static_cast<uint16_t*>(out),
                         static_cast<const uint16_t*>(permuted), inv, routing_weights, num_tokens, top_k, hidden);
      break;
  }
  KS_LAUNCH_STATUS("ks_moe_unpermute");
  return KS_SUCCESS;
}

}  // extern "C"
