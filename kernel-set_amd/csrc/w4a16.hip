// kernel-set (MI355X build) -- W4A16 group-wise int4 GEMV / GEMM.
//
// Semantics (kernels/src/gemm/gemm_w4a16.cu:1-17,74-129 of cklxx/kernel-set):
//   C[m,n] = sum_k A[m,k] * W[k,n] + bias[n],  W[k,n] = (q[k,n] - z[g,n]) * s[g,n]
//   g = k / group_size, q from the K-packed uint8 [K/2, N] stream (even k in the
//   low nibble), scales/zeros/A/C/bias all in the activation dtype, fp32 math,
//   output rounded to nearest even.
//
// Decode path (M <= 8): HBM-bound. Every byte of the 4-bit weight stream is
// read exactly once with 16-byte loads; a workgroup covers 128 columns (one
// 128-byte line per packed row) by 32*RPT packed rows, so the grid is
// (N/128) column tiles x S K-splits and fills all 256 CUs even at N = 4096.
// Each thread owns 16 columns x 2*RPT consecutive k of one quantization group,
// so the group's scale/zero are applied once per thread:
//   sum_k a_k (q_k - z) s = s * (sum_k a_k q_k - z * sum_k a_k).
// Partials are reduced with wave shuffles and LDS inside the workgroup, then
// across the S splits by the last workgroup to arrive at that column tile
// (fixed summation order, so results are deterministic). Split workgroups of
// one tile are mapped to the same XCD so the partials stay in one L2.
//
// Batched path (M > 8): MFMA, see w4a16_mfma.hpp. Workgroups own 64 columns x
// a range of quantization groups; K splits across workgroups are reduced by the
// last arrival exactly like the decode path.
#include <algorithm>

#include "kernel_set/gemm.h"
#include "ks_common.hpp"
#include "w4a16_mfma.hpp"
#include "workspace.hpp"

namespace ks {
namespace w4a16 {

constexpr int kThreads = 256;
constexpr int kLanesN = 8;                    // lanes across the column tile
constexpr int kTileN = kLanesN * 16;          // 128 columns per workgroup
constexpr int kRowsPar = kThreads / kLanesN;  // 32 packed rows in flight
constexpr int kMaxGemvM = 8;

template <typename T>
__device__ inline float h2f(uint16_t h) { return elem<T>::to_f32(h); }

// 16 consecutive 16-bit values as fp32.
template <typename T>
__device__ inline void load16h(const uint16_t* p, float v[16]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  const uint4 b = *reinterpret_cast<const uint4*>(p + 8);
  const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = h2f<T>(static_cast<uint16_t>(d[i] & 0xffffu));
    v[2 * i + 1] = h2f<T>(static_cast<uint16_t>(d[i] >> 16));
  }
}

// Workgroup id -> (column tile, k split). When the grid divides into the 8
// XCDs, consecutive logical ids land on one XCD (hardware dispatches ids
// round-robin over XCDs), so the S splits of a tile share an L2.
__device__ inline void map_tile(int bid, int nblocks, int splits, int* tile, int* split) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  *tile = logical / splits;
  *split = logical % splits;
}

template <typename T, int MT, int RPT>
__global__ void __launch_bounds__(kThreads)
gemv_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
            const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
            const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
            int m_rows, int n, int k, int gs, int splits, float* __restrict__ ws,
            unsigned* __restrict__ counters) {
  __shared__ float red[kThreads / kWave][MT][kTileN];
  __shared__ int last_flag;

  int tile, split;
  map_tile(blockIdx.x, gridDim.x, splits, &tile, &split);
  const int t = threadIdx.x;
  const int lane_n = t % kLanesN;
  const int rblk = t / kLanesN;
  const int col0 = tile * kTileN + lane_n * 16;
  const int kp0 = (split * kRowsPar + rblk) * RPT;  // first packed row of this thread
  const bool live = (col0 < n) && (kp0 < k / 2);

  float part[MT][16];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) part[m][j] = 0.f;

  if (live) {
    uint4 w[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      w[i] = load_stream16(b + static_cast<int64_t>(kp0 + i) * n + col0);

    float acc[MT][16];
    float asum[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      asum[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[m][j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float a_lo[MT], a_hi[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < m_rows) {
          const uint32_t pr = *reinterpret_cast<const uint32_t*>(
              a + static_cast<int64_t>(m) * k + 2 * (kp0 + i));
          a_lo[m] = h2f<T>(static_cast<uint16_t>(pr & 0xffffu));
          a_hi[m] = h2f<T>(static_cast<uint16_t>(pr >> 16));
        } else {
          a_lo[m] = 0.f;
          a_hi[m] = 0.f;
        }
        asum[m] += a_lo[m] + a_hi[m];
      }
      const uint32_t d[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = d[q] & 0x0f0f0f0fu;
        const uint32_t hi = (d[q] >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float ql = static_cast<float>((lo >> (8 * j)) & 0xffu);
          const float qh = static_cast<float>((hi >> (8 * j)) & 0xffu);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            acc[m][4 * q + j] = fmaf(a_lo[m], ql, acc[m][4 * q + j]);
            acc[m][4 * q + j] = fmaf(a_hi[m], qh, acc[m][4 * q + j]);
          }
        }
      }
    }
    // All 2*RPT k of this thread share one group (gs is a multiple of 2*RPT).
    const int64_t g = static_cast<int64_t>(2 * kp0 / gs) * n + col0;
    float s[16], z[16];
    load16h<T>(scales + g, s);
    if (zeros) {
      load16h<T>(zeros + g, z);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) z[j] = 0.f;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int j = 0; j < 16; ++j) part[m][j] = s[j] * fmaf(-z[j], asum[m], acc[m][j]);
  }

  // Reduce over the 8 row blocks inside a wave (lane bits 3..5) ...
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float v = part[m][j];
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      part[m][j] = v;
    }
  const int wave = t / kWave;
  if ((t % kWave) < kLanesN) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int j = 0; j < 16; ++j) red[wave][m][lane_n * 16 + j] = part[m][j];
  }
  __syncthreads();
  // ... then over the 4 waves, fixed order.
  for (int e = t; e < MT * kTileN; e += kThreads) {
    const int m = e / kTileN, cc = e % kTileN;
    const int col = tile * kTileN + cc;
    if (m >= m_rows || col >= n) continue;
    const float v = red[0][m][cc] + red[1][m][cc] + red[2][m][cc] + red[3][m][cc];
    if (splits == 1) {
      float o = v;
      if (bias) o += h2f<T>(bias[col]);
      c[static_cast<int64_t>(m) * n + col] = elem<T>::from_f32(o);
    } else {
      ws[(static_cast<int64_t>(split) * m_rows + m) * n + col] = v;
    }
  }
  if (splits == 1) return;

  // Publish this split; the last arrival reduces all splits in order.
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned prev = atomicAdd(&counters[tile], 1u);
    last_flag = (prev == static_cast<unsigned>(splits - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  for (int e = t; e < MT * kTileN; e += kThreads) {
    const int m = e / kTileN, cc = e % kTileN;
    const int col = tile * kTileN + cc;
    if (m >= m_rows || col >= n) continue;
    float o = 0.f;
    for (int sp = 0; sp < splits; ++sp)
      o += ws[(static_cast<int64_t>(sp) * m_rows + m) * n + col];
    if (bias) o += h2f<T>(bias[col]);
    c[static_cast<int64_t>(m) * n + col] = elem<T>::from_f32(o);
  }
  if (t == 0) counters[tile] = 0u;  // ready for the next call on this stream
}

// Any-shape fallback: one thread per output element, full K loop, the
// reference's per-element dequant order. Used only when the vector path's
// alignment/shape conditions do not hold.
template <typename T>
__global__ void __launch_bounds__(kThreads)
simple_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
              const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
              const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
              int64_t n, int64_t k, int gs) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t m = blockIdx.y;
  if (col >= n) return;
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; ++kk) {
    const uint8_t byte = b[(kk >> 1) * n + col];
    const int q = (kk & 1) ? (byte >> 4) : (byte & 0xf);
    const int64_t g = (kk / gs) * n + col;
    const float zp = zeros ? h2f<T>(zeros[g]) : 0.f;
    const float w = (static_cast<float>(q) - zp) * h2f<T>(scales[g]);
    acc = fmaf(h2f<T>(a[m * k + kk]), w, acc);
  }
  if (bias) acc += h2f<T>(bias[col]);
  c[m * n + col] = elem<T>::from_f32(acc);
}


// ---------------------------------------------------------------------------
// Batched MFMA path.
// ---------------------------------------------------------------------------
template <typename T, int MB>
__global__ void __launch_bounds__(w4mma::kThreads)
mfma_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
            const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
            const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
            int64_t row0, int64_t row1, int64_t n, int64_t k, int gs, int splits,
            int groups_per_split, float* __restrict__ ws, unsigned* __restrict__ counters) {
  constexpr int kRows = 16 * MB;
  constexpr int kPlane = kRows * w4mma::kTileN;
  __shared__ float red[4 * kPlane];
  __shared__ int last_flag;
  int tile, split;
  map_tile(blockIdx.x, gridDim.x, splits, &tile, &split);
  const int ng = static_cast<int>(k / gs);
  w4mma::TileArgs p;
  p.a = a; p.b = b; p.s = scales; p.z = zeros;
  p.row0 = row0; p.row1 = row1; p.n = n; p.k = k; p.gs = gs;
  p.n0 = static_cast<int64_t>(tile) * w4mma::kTileN;
  p.g_begin = split * groups_per_split;
  p.g_end = min(p.g_begin + groups_per_split, ng);
  w4mma::tile_partial<T, MB>(p, row0, red);
  const float* res = red + 3 * kPlane;
  const int t = threadIdx.x;
  const int64_t rows = row1 - row0;
  if (splits == 1) {
    for (int e = t; e < kPlane; e += w4mma::kThreads) {
      const int64_t r = e / w4mma::kTileN, col = p.n0 + e % w4mma::kTileN;
      if (r >= rows || col >= n) continue;
      float o = res[e];
      if (bias) o += h2f<T>(bias[col]);
      c[(row0 + r) * n + col] = elem<T>::from_f32(o);
    }
    return;
  }
  for (int e = t; e < kPlane; e += w4mma::kThreads) {
    const int64_t r = e / w4mma::kTileN, col = p.n0 + e % w4mma::kTileN;
    if (r >= rows || col >= n) continue;
    ws[(static_cast<int64_t>(split) * rows + r) * n + col] = res[e];
  }
  __threadfence();
  __syncthreads();
  if (t == 0) {
    const unsigned prev = atomicAdd(&counters[tile], 1u);
    last_flag = (prev == static_cast<unsigned>(splits - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  for (int e = t; e < kPlane; e += w4mma::kThreads) {
    const int64_t r = e / w4mma::kTileN, col = p.n0 + e % w4mma::kTileN;
    if (r >= rows || col >= n) continue;
    float o = 0.f;
    for (int sp = 0; sp < splits; ++sp) o += ws[(static_cast<int64_t>(sp) * rows + r) * n + col];
    if (bias) o += h2f<T>(bias[col]);
    c[(row0 + r) * n + col] = elem<T>::from_f32(o);
  }
  if (t == 0) counters[tile] = 0u;
}

template <typename T, int MB>
void launch_mfma(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                 const uint16_t* z, const uint16_t* bias, int64_t r0, int64_t r1, int64_t n,
                 int64_t k, int gs, int tiles, int splits, int gps, const Scratch& sc,
                 hipStream_t st) {
  hipLaunchKernelGGL((mfma_kernel<T, MB>), dim3(tiles * splits), dim3(w4mma::kThreads), 0, st,
                     c, a, b, s, z, bias, r0, r1, n, k, gs, splits, gps, sc.partial,
                     sc.counters);
}

template <typename T>
ks_status_t run_mfma(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                     const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n, int64_t k,
                     int gs, hipStream_t st) {
  const int tiles = static_cast<int>((n + w4mma::kTileN - 1) / w4mma::kTileN);
  const int ng = static_cast<int>(k / gs);
  // Aim for ~1024 workgroups but keep >= 4 groups (one per wave) per split.
  int splits = (1024 + tiles - 1) / tiles;
  splits = std::max(1, std::min(splits, ng / 4));
  const int gps = (ng + splits - 1) / splits;
  splits = (ng + gps - 1) / gps;
  const int mb_rows = m >= 64 ? 64 : (m > 16 ? 32 : 16);
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * mb_rows * n,
                                static_cast<size_t>(tiles), &sc, "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  for (int64_t r0 = 0; r0 < m; r0 += mb_rows) {
    const int64_t r1 = std::min(m, r0 + mb_rows);
    if (mb_rows == 64) launch_mfma<T, 4>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, gps, sc, st);
    else if (mb_rows == 32) launch_mfma<T, 2>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, gps, sc, st);
    else launch_mfma<T, 1>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, gps, sc, st);
  }
  return KS_SUCCESS;
}

inline bool aligned(const void* p, uintptr_t q) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % q) == 0;
}

template <typename T, int MT, int RPT>
void launch_gemv(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                 const uint16_t* z, const uint16_t* bias, int m, int n, int k, int gs,
                 int tiles, int splits, const Scratch& sc, hipStream_t st) {
  hipLaunchKernelGGL((gemv_kernel<T, MT, RPT>), dim3(tiles * splits), dim3(kThreads), 0, st, c,
                     a, b, s, z, bias, m, n, k, gs, splits, sc.partial, sc.counters);
}

template <typename T, int RPT>
void launch_gemv_m(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                   const uint16_t* z, const uint16_t* bias, int m, int n, int k, int gs,
                   int tiles, int splits, const Scratch& sc, hipStream_t st) {
  if (m <= 1) launch_gemv<T, 1, RPT>(c, a, b, s, z, bias, m, n, k, gs, tiles, splits, sc, st);
  else if (m <= 2) launch_gemv<T, 2, RPT>(c, a, b, s, z, bias, m, n, k, gs, tiles, splits, sc, st);
  else if (m <= 4) launch_gemv<T, 4, RPT>(c, a, b, s, z, bias, m, n, k, gs, tiles, splits, sc, st);
  else launch_gemv<T, 8, RPT>(c, a, b, s, z, bias, m, n, k, gs, tiles, splits, sc, st);
}

template <typename T>
ks_status_t run(void* c_, const void* a_, const void* b_, const void* s_, const void* z_,
                const void* bias_, int64_t m, int64_t n, int64_t k, int gs, hipStream_t st) {
  auto* c = static_cast<uint16_t*>(c_);
  const auto* a = static_cast<const uint16_t*>(a_);
  const auto* b = static_cast<const uint8_t*>(b_);
  const auto* s = static_cast<const uint16_t*>(s_);
  const auto* z = static_cast<const uint16_t*>(z_);
  const auto* bias = static_cast<const uint16_t*>(bias_);

  const bool mfma = m > kMaxGemvM && (gs % 32 == 0) && (n % 4 == 0) && aligned(a, 16) &&
                    aligned(s, 8) && aligned(z, 8) && aligned(b, 4);
  if (mfma) return run_mfma<T>(c, a, b, s, z, bias, m, n, k, gs, st);
  const bool vec = (n % 16 == 0) && (gs % 16 == 0) && n <= (int64_t{1} << 30) &&
                   k <= (int64_t{1} << 30) && aligned(b, 16) && aligned(s, 16) &&
                   aligned(z, 16) && aligned(a, 4);
  if (!vec) {
    hipLaunchKernelGGL((simple_kernel<T>), dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads),
                                                static_cast<unsigned>(m)),
                       dim3(kThreads), 0, st, c, a, b, s, z, bias, n, k, gs);
    return KS_SUCCESS;
  }
  const int tiles = static_cast<int>((n + kTileN - 1) / kTileN);
  const int64_t kp = k / 2;
  // Eight packed rows per thread unless that leaves fewer than 512 workgroups.
  int rpt = 8;
  int splits = static_cast<int>((kp + kRowsPar * rpt - 1) / (kRowsPar * rpt));
  if (static_cast<int64_t>(tiles) * splits < 512) {
    rpt = 4;
    splits = static_cast<int>((kp + kRowsPar * rpt - 1) / (kRowsPar * rpt));
  }
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * kMaxGemvM * n,
                                static_cast<size_t>(tiles), &sc, "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  for (int64_t m0 = 0; m0 < m; m0 += kMaxGemvM) {
    const int mm = static_cast<int>((m - m0) < kMaxGemvM ? (m - m0) : kMaxGemvM);
    uint16_t* cc = c + m0 * n;
    const uint16_t* aa = a + m0 * k;
    const int ki = static_cast<int>(k), ni = static_cast<int>(n);
    if (rpt == 8) launch_gemv_m<T, 8>(cc, aa, b, s, z, bias, mm, ni, ki, gs, tiles, splits, sc, st);
    else launch_gemv_m<T, 4>(cc, aa, b, s, z, bias, mm, ni, ki, gs, tiles, splits, sc, st);
  }
  return KS_SUCCESS;
}

}  // namespace w4a16
}  // namespace ks

extern "C" {

ks_status_t ks_gemm_w4a16(void* c, const void* a, const void* b_packed,
                          const void* scales, const void* zeros, const void* bias,
                          int64_t m, int64_t n, int64_t k, int group_size,
                          ks_dtype_t dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(c);
  KS_REQUIRE_PTR(a);
  KS_REQUIRE_PTR(b_packed);
  KS_REQUIRE_PTR(scales);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w4a16: bad shape");
  if (k % 2 != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w4a16: K must be even (two int4 per byte)");
  if (group_size > 0 && k % group_size != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w4a16: group_size must divide K");
  if (k > 2147483647LL) KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w4a16: K too large");
  if (dtype != KS_DTYPE_F16 && dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_w4a16: dtype must be f16 or bf16");
  if (m > 65535) KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w4a16: M exceeds grid limit");
  const int gs = group_size > 0 ? group_size : static_cast<int>(k);
  auto st = ks::to_stream(stream);
  ks_status_t r = (dtype == KS_DTYPE_BF16)
                      ? ks::w4a16::run<ks::bf16_t>(c, a, b_packed, scales, zeros, bias, m, n, k, gs, st)
                      : ks::w4a16::run<ks::f16_t>(c, a, b_packed, scales, zeros, bias, m, n, k, gs, st);
  if (r != KS_SUCCESS) return r;
  KS_LAUNCH_STATUS("ks_gemm_w4a16");
  return KS_SUCCESS;
}

}  // extern "C"
