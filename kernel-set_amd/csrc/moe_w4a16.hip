// kernel-set (MI355X build) -- grouped W4A16 GEMM for Mixture-of-Experts.
//
// Extension entry point (the reference has no quantized grouped GEMM): the
// ks_moe_grouped_gemm conventions (kernels/src/moe/moe_grouped_gemm.cu:136-198
// of cklxx/kernel-set: CSR expert_offsets, rows of A/C grouped by expert) with
// the weight operand in the ks_gemm_w4a16 format (gemm_w4a16.cu:1-17).
//
// No schedule buffer, no allocation, no stream synchronization: one workgroup
// per (column tile, expert) reads its expert's row range straight from
// expert_offsets and walks it in 16*MB-row passes, all of K per workgroup, so
// each expert weight byte is read from HBM once per pass; decode-sized experts
// (<= 16*MB rows) need a single pass. The main form is the LDS-ring tile of
// w4a16_pipe.hpp (128-column tiles, moe_pipe_kernel); shapes it does not take
// run the 64-column register tile (moe_mfma_kernel, 4 waves split K) or the
// per-element fallback.
// Row ranges are clamped to [0, total_rows], so malformed offsets cannot make
// the kernel touch memory outside A and C.
#include <algorithm>

#include "kernel_set/moe_w4a16.h"
#include "ks_common.hpp"
#include "w4a16_mfma.hpp"
#include "w4a16_pipe.hpp"

namespace ks {
namespace moe4 {

using w4mma::kThreads;
using w4mma::kTileN;

template <typename T, int MB>
__global__ void __launch_bounds__(kThreads)
moe_mfma_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
                const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
                const uint16_t* __restrict__ zeros, const int32_t* __restrict__ offsets,
                int64_t total_rows, int64_t n, int64_t k, int gs) {
  constexpr int kRows = 16 * MB;
  constexpr int kPlane = kRows * kTileN;
  __shared__ float red[4 * kPlane];
  const int e = blockIdx.y;
  const int64_t r_begin = min<int64_t>(max<int64_t>(offsets[e], 0), total_rows);
  const int64_t r_end = min<int64_t>(max<int64_t>(offsets[e + 1], r_begin), total_rows);
  if (r_end <= r_begin) return;  // uniform across the workgroup
  const int64_t ng = k / gs;
  w4mma::TileArgs p;
  p.a = a;
  p.b = b + static_cast<int64_t>(e) * (k / 2) * n;
  p.s = scales + static_cast<int64_t>(e) * ng * n;
  p.z = zeros ? zeros + static_cast<int64_t>(e) * ng * n : nullptr;
  p.row0 = r_begin;
  p.row1 = r_end;
  p.n = n;
  p.k = k;
  p.gs = gs;
  p.n0 = static_cast<int64_t>(blockIdx.x) * kTileN;
  p.g_begin = 0;
  p.g_end = static_cast<int>(ng);
  const float* res = red + 3 * kPlane;
  for (int64_t r0 = r_begin; r0 < r_end; r0 += kRows) {
    w4mma::tile_partial<T, MB>(p, r0, red);
    for (int i = threadIdx.x; i < kPlane; i += kThreads) {
      const int64_t row = r0 + i / kTileN, col = p.n0 + i % kTileN;
      if (row < r_end && col < n) c[row * n + col] = elem<T>::from_f32(res[i]);
    }
    __syncthreads();  // `red` is rewritten by the next pass
  }
}

// LDS-ring variant (gs % 64 == 0, K % 128 == 0, N % 16 == 0): one workgroup
// per (128-column tile, expert) walks the expert's rows in 16*MB-row passes
// over the whole K of the expert. Workgroup ids are dispatched to the 8 XCDs
// round-robin; id L serves expert (L % 8) + 8 * (L / 8 / tiles_n), so every
// column tile of an expert runs on one XCD and the expert's activation rows
// are fetched from HBM into that XCD's L2 once, not by all eight.
template <typename T, int MB, bool OG>
__global__ void __launch_bounds__(w4pipe::kThreads, 2)
moe_pipe_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
                const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
                const uint16_t* __restrict__ zeros, const int32_t* __restrict__ offsets,
                int num_experts, int tiles_n, int64_t total_rows, int64_t n, int64_t k, int gs) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int L = blockIdx.x;
  const int e = (L & 7) + 8 * ((L >> 3) / tiles_n);
  const int tile = (L >> 3) % tiles_n;
  if (e >= num_experts) return;
  const int64_t r_begin = min<int64_t>(max<int64_t>(offsets[e], 0), total_rows);
  const int64_t r_end = min<int64_t>(max<int64_t>(offsets[e + 1], r_begin), total_rows);
  if (r_end <= r_begin) return;  // uniform across the workgroup
  const int64_t ng = k / gs;
  w4pipe::PipeArgs p;
  p.a = a;
  p.b = b + static_cast<int64_t>(e) * (k / 2) * n;
  p.s = scales + static_cast<int64_t>(e) * ng * n;
  p.z = zeros ? zeros + static_cast<int64_t>(e) * ng * n : nullptr;
  p.n = n; p.k = k; p.gs = gs;
  p.n0 = static_cast<int64_t>(tile) * w4pipe::kTileN;
  const int total = static_cast<int>(k / w4pipe::kStageK);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int li = lane % 16, q = lane / 16;
  for (int64_t r0 = r_begin; r0 < r_end; r0 += 16 * MB) {
    w4mma::f32x4 O[MB][2];
    w4pipe::pipe_tile<T, MB, OG>(p, r0, r_end, 0, total, smem, O);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = p.n0 + 32 * wave + 16 * j + li;
      if (col >= n) continue;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t row = r0 + 16 * mb + 4 * q + r;
          if (row < r_end) c[row * n + col] = elem<T>::from_f32(O[mb][j][r]);
        }
    }
  }
}

template <typename T, int MB, bool OG>
void launch_pipe_og(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                    const uint16_t* z, const int32_t* offs, int E, int64_t rows, int64_t n,
                    int64_t k, int gs, hipStream_t st) {
  constexpr int lds = w4pipe::Ring<MB>::kBytes;
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_pipe_kernel<T, MB, OG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)configured;
  const int tiles_n = static_cast<int>((n + w4pipe::kTileN - 1) / w4pipe::kTileN);
  const unsigned grid = static_cast<unsigned>(tiles_n * ((E + 7) / 8) * 8);
  hipLaunchKernelGGL((moe_pipe_kernel<T, MB, OG>), dim3(grid), dim3(w4pipe::kThreads), lds, st, c,
                     a, b, s, z, offs, E, tiles_n, rows, n, k, gs);
}

// gs == 128: the one-group-per-stage variant of the ring tile.
template <typename T, int MB>
void launch_pipe(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                 const uint16_t* z, const int32_t* offs, int E, int64_t rows, int64_t n,
                 int64_t k, int gs, hipStream_t st) {
  if (gs == w4pipe::kStageK)
    launch_pipe_og<T, MB, true>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
  else
    launch_pipe_og<T, MB, false>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
}

// Any-shape fallback: one thread per (row, column); the expert is found by a
// binary search over the offsets; reference per-element dequant order.
template <typename T>
__global__ void __launch_bounds__(kThreads)
moe_simple_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
                  const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
                  const uint16_t* __restrict__ zeros, const int32_t* __restrict__ offsets,
                  int num_experts, int64_t total_rows, int64_t n, int64_t k, int gs) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total_rows * n) return;
  const int64_t row = idx / n, col = idx % n;
  int lo = 0, hi = num_experts;  // find e with offsets[e] <= row < offsets[e+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (offsets[mid] <= row) lo = mid; else hi = mid;
  }
  if (row < offsets[lo] || row >= offsets[lo + 1]) return;  // row not routed
  const int64_t ng = k / gs;
  const uint8_t* be = b + static_cast<int64_t>(lo) * (k / 2) * n;
  const uint16_t* se = scales + static_cast<int64_t>(lo) * ng * n;
  const uint16_t* ze = zeros ? zeros + static_cast<int64_t>(lo) * ng * n : nullptr;
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; ++kk) {
    const uint8_t byte = be[(kk >> 1) * n + col];
    const int q = (kk & 1) ? (byte >> 4) : (byte & 0xf);
    const int64_t g = (kk / gs) * n + col;
    const float zp = ze ? elem<T>::to_f32(ze[g]) : 0.f;
    const float w = (static_cast<float>(q) - zp) * elem<T>::to_f32(se[g]);
    acc = fmaf(elem<T>::to_f32(a[row * k + kk]), w, acc);
  }
  c[row * n + col] = elem<T>::from_f32(acc);
}

inline bool aligned(const void* p, uintptr_t q) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % q) == 0;
}

template <typename T>
void run(void* c_, const void* a_, const void* b_, const void* s_, const void* z_,
         const int32_t* offs, int E, int64_t rows, int64_t n, int64_t k, int gs, hipStream_t st) {
  auto* c = static_cast<uint16_t*>(c_);
  const auto* a = static_cast<const uint16_t*>(a_);
  const auto* b = static_cast<const uint8_t*>(b_);
  const auto* s = static_cast<const uint16_t*>(s_);
  const auto* z = static_cast<const uint16_t*>(z_);
  const bool mfma = (gs % 32 == 0) && (n % 4 == 0) && aligned(a, 16) && aligned(b, 4) &&
                    aligned(s, 8) && aligned(z, 8);
  if (!mfma) {
    hipLaunchKernelGGL((moe_simple_kernel<T>),
                       dim3(static_cast<unsigned>((rows * n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, st, c, a, b, s, z, offs, E, rows, n, k, gs);
    return;
  }
  const int64_t avg = (rows + E - 1) / E;
  const bool pipe = (gs % 64 == 0) && (k % w4pipe::kStageK == 0) && (n % 16 == 0) && aligned(a, 16) &&
                    n < (int64_t{1} << 26) && rows * k < (int64_t{1} << 31) &&  // 32-bit copy offsets
                    aligned(b, 16) && aligned(s, 4) && aligned(z, 4);
  if (pipe) {
    // Pass height from the average rows per expert: an expert taller than a
    // pass re-reads its weights, a pass taller than the expert multiplies
    // padding rows (the kernel is MFMA-bound at these shapes).
    if (avg <= 16) launch_pipe<T, 1>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
    else if (avg <= 32) launch_pipe<T, 2>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
    else if (avg <= 48) launch_pipe<T, 3>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
    else launch_pipe<T, 4>(c, a, b, s, z, offs, E, rows, n, k, gs, st);
    return;
  }
  const dim3 grid(static_cast<unsigned>((n + kTileN - 1) / kTileN), static_cast<unsigned>(E));
  if (avg <= 16)
    hipLaunchKernelGGL((moe_mfma_kernel<T, 1>), grid, dim3(kThreads), 0, st, c, a, b, s, z, offs, rows, n, k, gs);
  else if (avg <= 32)
    hipLaunchKernelGGL((moe_mfma_kernel<T, 2>), grid, dim3(kThreads), 0, st, c, a, b, s, z, offs, rows, n, k, gs);
  else
    hipLaunchKernelGGL((moe_mfma_kernel<T, 4>), grid, dim3(kThreads), 0, st, c, a, b, s, z, offs, rows, n, k, gs);
}

}  // namespace moe4
}  // namespace ks

extern "C" {

ks_status_t ks_moe_grouped_gemm_w4a16(void* c, const void* a, const void* b_packed,
                                      const void* scales, const void* zeros,
                                      const int32_t* expert_offsets, int num_experts,
                                      int64_t total_rows, int64_t n, int64_t k, int group_size,
                                      ks_dtype_t dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(c);
  KS_REQUIRE_PTR(a);
  KS_REQUIRE_PTR(b_packed);
  KS_REQUIRE_PTR(scales);
  KS_REQUIRE_PTR(expert_offsets);
  if (num_experts <= 0 || total_rows < 0 || n <= 0 || k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_grouped_gemm_w4a16: bad shape");
  if (k % 2 != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_grouped_gemm_w4a16: K must be even");
  const int gs = group_size > 0 ? group_size : static_cast<int>(k);
  if (k % gs != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_grouped_gemm_w4a16: group_size must divide K");
  if (dtype != KS_DTYPE_F16 && dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_grouped_gemm_w4a16: dtype must be f16 or bf16");
  if (num_experts > 65535 || k > 2147483647LL || n > (int64_t{1} << 36) ||
      (n + 63) / 64 * (num_experts + 7) > (int64_t{1} << 30))
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_grouped_gemm_w4a16: shape exceeds grid limits");
  if (total_rows == 0) return KS_SUCCESS;  // nothing routed
  auto st = ks::to_stream(stream);
  if (dtype == KS_DTYPE_BF16)
    ks::moe4::run<ks::bf16_t>(c, a, b_packed, scales, zeros, expert_offsets, num_experts,
                              total_rows, n, k, gs, st);
  else
    ks::moe4::run<ks::f16_t>(c, a, b_packed, scales, zeros, expert_offsets, num_experts,
                             total_rows, n, k, gs, st);
  KS_LAUNCH_STATUS("ks_moe_grouped_gemm_w4a16");
  return KS_SUCCESS;
}

}  // extern "C"
