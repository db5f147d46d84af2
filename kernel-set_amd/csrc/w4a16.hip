// kernel-set (MI355X build) -- W4A16 group-wise int4 GEMV / GEMM.
//
// Semantics (kernels/src/gemm/gemm_w4a16.cu:1-17,74-129 of cklxx/kernel-set):
//   C[m,n] = sum_k A[m,k] * W[k,n] + bias[n],  W[k,n] = (q[k,n] - z[g,n]) * s[g,n]
//   g = k / group_size, q from the K-packed uint8 [K/2, N] stream (even k in the
//   low nibble), scales/zeros/A/C/bias all in the activation dtype, fp32 math,
//   output rounded to nearest even.
//
// Decode path (M <= 8), HBM-bound: w4a16_dec.hpp (MFMA, no byte transpose)
// when gs % 32 == 0 and the operands are 16-byte aligned; the dot2 kernel
// below otherwise. Measured on MI355X: reading the weight stream reaches full
// bandwidth only when each workgroup reads whole 128-byte lines of consecutive
// packed rows (column strips narrower than a line read ~2x slower), so K is
// split over workgroups. A cross-workgroup reduction inside one kernel
// (last-arriver, through L2 or device-coherent memory, or fp32 atomics)
// measured slower than a second launch, so the split partials go to a scratch
// plane and a small reduce kernel sums them in a fixed order (deterministic)
// and adds the bias. The decode reduce runs each tile on the XCD that wrote
// its partials, which reads them from that XCD's L2.
//
// dot2 fallback: v_dot2_f32_bf16 (or _f16). The activation pair (a[2kp],
// a[2kp+1]) is used as loaded; each packed byte becomes the 16-bit float pair
// (base + q_even, base + q_odd) with two v_perm ops per 4 columns
// (bf16 0x4300|q = 128 + q; f16 0x5800|q = 128 + q/8, both exact), so
//   sum_k a_k * w_k = s * (u * (D - (128 + z/u) * sum_k a_k)),  u = 1 or 8,
// where D is the dot2 accumulator; each thread's 2*RPT k lie in one group.
//
// Batched path (M > 8): bf16/f16 MFMA, see w4a16_mfma.hpp, with the same
// split-plane + reduce scheme when K is split.
#include <algorithm>

#include "kernel_set/gemm.h"
#include "ks_common.hpp"
#include "w4a16_mfma.hpp"
#include "w4a16_pipe.hpp"
#include "w4a16_dq.hpp"
#include "w4a16_dqs.hpp"
#include "w4a16_dec.hpp"
#include "workspace.hpp"

#include <mutex>

namespace ks {
namespace w4a16 {

constexpr int kThreads = 256;
constexpr int kLanesN = 8;                    // lanes across the column tile
constexpr int kTileN = kLanesN * 16;          // 128 columns per workgroup
constexpr int kRowsPar = kThreads / kLanesN;  // 32 row lanes
constexpr int kMaxGemvM = 8;   // dot2 decode kernel
constexpr int kMaxDecM = 8;    // MFMA decode kernel (up to 2 blocks of 4 activation rows)
constexpr int kDqMinM = 64;  // above this M the dequantize-to-LDS MFMA GEMM runs (measured crossover)

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct dot;

template <>
struct dot<bf16_t> {
  static constexpr uint32_t base_byte = 0x43434343u;  // 0x43xx = bf16 128 + low 7 bits
  static constexpr uint32_t ones = 0x3f803f80u;
  static constexpr float unit = 1.0f;
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
};

template <>
struct dot<f16_t> {
  static constexpr uint32_t base_byte = 0x58585858u;  // 0x58xx = f16 128 + xx/8
  static constexpr uint32_t ones = 0x3c003c00u;
  static constexpr float unit = 0.125f;
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
};

template <typename T>
__device__ inline float h2f(uint16_t h) { return elem<T>::to_f32(h); }

// Workgroup id -> (column tile, k split); splits of one tile share an XCD
// when the grid divides into the 8 XCDs (ids are dispatched round-robin).
__device__ inline void map_tile(int bid, int nblocks, int splits, int* tile, int* split) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  *tile = logical / splits;
  *split = logical % splits;
}

// acc[m][c0..c0+3] += a_pair[m] . (base + q) for the 4 columns in packed dword d.
template <typename T, int MT>
__device__ inline void dword_dot(uint32_t d, const uint32_t (&ap)[MT], float (*acc)[16], int c0) {
  const uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
  const uint32_t x0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // lo0 hi0 lo1 hi1
  const uint32_t x1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo2 hi2 lo3 hi3
  constexpr uint32_t B = dot<T>::base_byte;
  const uint32_t w0 = __builtin_amdgcn_perm(B, x0, 0x04010400u);  // (base|lo0, base|hi0)
  const uint32_t w1 = __builtin_amdgcn_perm(B, x0, 0x04030402u);
  const uint32_t w2 = __builtin_amdgcn_perm(B, x1, 0x04010400u);
  const uint32_t w3 = __builtin_amdgcn_perm(B, x1, 0x04030402u);
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    acc[m][c0 + 0] = dot<T>::dot2(ap[m], w0, acc[m][c0 + 0]);
    acc[m][c0 + 1] = dot<T>::dot2(ap[m], w1, acc[m][c0 + 1]);
    acc[m][c0 + 2] = dot<T>::dot2(ap[m], w2, acc[m][c0 + 2]);
    acc[m][c0 + 3] = dot<T>::dot2(ap[m], w3, acc[m][c0 + 3]);
  }
}

// Partial GEMV over one (128-column, 32*RPT-packed-row) tile for MT <= 8 rows.
// splits == 1: writes C (+bias) directly; else writes ws[split][m][n].
template <typename T, int MT, int RPT>
__global__ void __launch_bounds__(kThreads)
gemv_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
            const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
            const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
            int m_rows, int n, int k, int gs, int splits, float* __restrict__ ws) {
  __shared__ float red[kRowsPar][kTileN + 4];

  int tile, split;
  map_tile(blockIdx.x, gridDim.x, splits, &tile, &split);
  const int t = threadIdx.x;
  const int lane_n = t % kLanesN;
  const int rblk = t / kLanesN;
  const int col0 = tile * kTileN + lane_n * 16;
  const int kp0 = (split * kRowsPar + rblk) * RPT;  // first packed row of this thread
  const bool live = (col0 < n) && (kp0 < k / 2);

  float part[MT][16];
  if (live) {
    // Issue every load of this thread before any math: weights (streamed),
    // activation pairs, then this group's scales and zeros.
    uint4 w[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) w[i] = load_stream16(b + static_cast<int64_t>(kp0 + i) * n + col0);
    uint32_t ap[RPT][MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint32_t* arow = reinterpret_cast<const uint32_t*>(a + static_cast<int64_t>(m) * k) + kp0;
#pragma unroll
      for (int i = 0; i < RPT; ++i) ap[i][m] = (m < m_rows) ? arow[i] : 0u;
    }
    const int64_t g = static_cast<int64_t>(2 * kp0 / gs) * n + col0;
    const uint4 s0 = *reinterpret_cast<const uint4*>(scales + g);
    const uint4 s1 = *reinterpret_cast<const uint4*>(scales + g + 8);
    uint4 z0 = make_uint4(0, 0, 0, 0), z1 = make_uint4(0, 0, 0, 0);
    if (zeros) {
      z0 = *reinterpret_cast<const uint4*>(zeros + g);
      z1 = *reinterpret_cast<const uint4*>(zeros + g + 8);
    }

    float acc[MT][16], asum[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      asum[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[m][j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int m = 0; m < MT; ++m) asum[m] = dot<T>::dot2(ap[i][m], dot<T>::ones, asum[m]);
      dword_dot<T, MT>(w[i].x, ap[i], acc, 0);
      dword_dot<T, MT>(w[i].y, ap[i], acc, 4);
      dword_dot<T, MT>(w[i].z, ap[i], acc, 8);
      dword_dot<T, MT>(w[i].w, ap[i], acc, 12);
    }
    const uint32_t sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t zv[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
    constexpr float u = dot<T>::unit;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float sj = h2f<T>(static_cast<uint16_t>(sv[j / 2] >> (16 * (j & 1))));
      const float zj = h2f<T>(static_cast<uint16_t>(zv[j / 2] >> (16 * (j & 1))));
      const float cj = 128.0f + zj * u;  // zero-point in the base+q*u encoding
      const float se = sj * (1.0f / u);
#pragma unroll
      for (int m = 0; m < MT; ++m) part[m][j] = se * fmaf(-cj, asum[m], acc[m][j]);
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int j = 0; j < 16; ++j) part[m][j] = 0.f;
  }

  // Row-lane reduction through LDS (fixed order), one activation row at a time.
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m > 0) __syncthreads();  // previous row's reads are done
#pragma unroll
    for (int j = 0; j < 16; j += 4)
      *reinterpret_cast<float4*>(&red[rblk][lane_n * 16 + j]) =
          make_float4(part[m][j], part[m][j + 1], part[m][j + 2], part[m][j + 3]);
    __syncthreads();
    if (t < kTileN && m < m_rows) {
      const int col = tile * kTileN + t;
      float v = 0.f;
#pragma unroll 8
      for (int r = 0; r < kRowsPar; ++r) v += red[r][t];
      if (col < n) {
        if (splits == 1) {
          if (bias) v += h2f<T>(bias[col]);
          c[static_cast<int64_t>(m) * n + col] = elem<T>::from_f32(v);
        } else {
          ws[(static_cast<int64_t>(split) * m_rows + m) * n + col] = v;
        }
      }
    }
  }
}

// Sum of the split planes ws[split][row][col] in split order, + bias, -> C.
template <typename T>
__global__ void __launch_bounds__(kThreads)
reduce_kernel(uint16_t* __restrict__ c, const float* __restrict__ ws,
              const uint16_t* __restrict__ bias, int64_t rows, int64_t n, int splits) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= rows * n) return;
  const int64_t plane = rows * n;
  // 8 independent loads in flight, added in split order; the tail batch is
  // clamped and guarded (a runtime-count tail loop would serialize its loads).
  float o = 0.f;
  int sp = 0;
  for (; sp + 8 <= splits; sp += 8) {
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = ws[(sp + i) * plane + idx];
#pragma unroll
    for (int i = 0; i < 8; ++i) o += p[i];
  }
  if (sp < splits) {
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = ws[min(sp + i, splits - 1) * plane + idx];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp + i < splits) o += p[i];
  }
  if (bias) o += h2f<T>(bias[idx % n]);
  c[idx] = elem<T>::from_f32(o);
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
            int groups_per_split, float* __restrict__ ws) {
  constexpr int kRows = 16 * MB;
  constexpr int kPlane = kRows * w4mma::kTileN;
  __shared__ float red[4 * kPlane];
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
  const int64_t rows = row1 - row0;
  for (int e = threadIdx.x; e < kPlane; e += w4mma::kThreads) {
    const int64_t r = e / w4mma::kTileN, col = p.n0 + e % w4mma::kTileN;
    if (r >= rows || col >= n) continue;
    if (splits == 1) {
      float o = res[e];
      if (bias) o += h2f<T>(bias[col]);
      c[(row0 + r) * n + col] = elem<T>::from_f32(o);
    } else {
      ws[(static_cast<int64_t>(split) * rows + r) * n + col] = res[e];
    }
  }
}

inline bool aligned(const void* p, uintptr_t q) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % q) == 0;
}

template <typename T>
void launch_reduce(uint16_t* c, const float* ws, const uint16_t* bias, int64_t rows, int64_t n,
                   int splits, hipStream_t st) {
  const int64_t total = rows * n;
  hipLaunchKernelGGL((reduce_kernel<T>), dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, st, c, ws, bias, rows, n, splits);
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
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * mb_rows * n, 0, &sc,
                                "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  for (int64_t r0 = 0; r0 < m; r0 += mb_rows) {
    const int64_t r1 = std::min(m, r0 + mb_rows);
    const dim3 grid(tiles * splits), block(w4mma::kThreads);
    if (mb_rows == 64)
      hipLaunchKernelGGL((mfma_kernel<T, 4>), grid, block, 0, st, c, a, b, s, z, bias, r0, r1, n, k, gs, splits, gps, sc.partial);
    else if (mb_rows == 32)
      hipLaunchKernelGGL((mfma_kernel<T, 2>), grid, block, 0, st, c, a, b, s, z, bias, r0, r1, n, k, gs, splits, gps, sc.partial);
    else
      hipLaunchKernelGGL((mfma_kernel<T, 1>), grid, block, 0, st, c, a, b, s, z, bias, r0, r1, n, k, gs, splits, gps, sc.partial);
    if (splits > 1) launch_reduce<T>(c + r0 * n, sc.partial, bias, r1 - r0, n, splits, st);
  }
  return KS_SUCCESS;
}

// Batched path on the LDS-ring tile: one launch covers rows [row0, row1)
// (<= 16*MB rows) for every 128-column tile and K split.
template <typename T, int MB, bool OG>
__global__ void __launch_bounds__(w4pipe::kThreads, 2)
pipe_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
            const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
            const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
            int64_t row0, int64_t row1, int64_t n, int64_t k, int gs, int splits,
            int stages_per_split, float* __restrict__ ws) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  int tile, split;
  map_tile(blockIdx.x, gridDim.x, splits, &tile, &split);
  w4pipe::PipeArgs p;
  p.a = a; p.b = b; p.s = scales; p.z = zeros;
  p.n = n; p.k = k; p.gs = gs;
  p.n0 = static_cast<int64_t>(tile) * w4pipe::kTileN;
  const int total = static_cast<int>(k / w4pipe::kStageK);
  const int st0 = split * stages_per_split;
  const int st1 = min(st0 + stages_per_split, total);
  w4mma::f32x4 O[MB][2];
  w4pipe::pipe_tile<T, MB, OG>(p, row0, row1, st0, st1, smem, O);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int li = lane % 16, q = lane / 16;
  const int64_t rows = row1 - row0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = p.n0 + 32 * wave + 16 * j + li;
    if (col >= n) continue;
    const float bv = (splits == 1 && bias) ? h2f<T>(bias[col]) : 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t lr = 16 * mb + 4 * q + r;
        if (lr >= rows) continue;
        if (splits == 1)
          c[(row0 + lr) * n + col] = elem<T>::from_f32(O[mb][j][r] + bv);
        else
          ws[(static_cast<int64_t>(split) * rows + lr) * n + col] = O[mb][j][r];
      }
  }
}

// Split sum for the ring tile: ws[split][rows][n] in split order, + bias, -> C.
// A workgroup takes 8 rows of one 128-column tile, a thread 4 adjacent
// columns (16-byte loads; the ring path has N % 16 == 0). With tiles % 8 == 0
// the pipe kernel ran every split of tile t on XCD t / (tiles / 8) (map_tile),
// so workgroup id b (dispatched to XCD b % 8) takes a tile of that XCD and
// reads the partials from the L2 they were written through.
template <typename T>
__global__ void __launch_bounds__(kThreads)
pipe_reduce_kernel(uint16_t* __restrict__ c, const float* __restrict__ ws,
                   const uint16_t* __restrict__ bias, int rows, int n, int splits, int tiles) {
  const int rbs = (rows + 7) / 8;  // 8-row blocks per tile
  int tile, rb;
  if ((tiles & 7) == 0) {
    const int i = blockIdx.x >> 3;
    tile = (blockIdx.x & 7) * (tiles >> 3) + i / rbs;
    rb = i % rbs;
  } else {
    tile = blockIdx.x / rbs;
    rb = blockIdx.x % rbs;
  }
  const int row = 8 * rb + threadIdx.x / 32;
  const int col = tile * w4pipe::kTileN + 4 * (threadIdx.x % 32);
  if (row >= rows || col >= n) return;
  const int64_t plane = static_cast<int64_t>(rows) * n;
  const float* p = ws + static_cast<int64_t>(row) * n + col;
  w4mma::f32x4 o = {0.f, 0.f, 0.f, 0.f};
  int sp = 0;
  for (; sp + 8 <= splits; sp += 8) {  // 8 loads in flight, added in order
    w4mma::f32x4 part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = *reinterpret_cast<const w4mma::f32x4*>(p + (sp + i) * plane);
#pragma unroll
    for (int i = 0; i < 8; ++i) o += part[i];
  }
  if (sp < splits) {  // tail: clamped, guarded, still one batch in flight
    w4mma::f32x4 part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      part[i] = *reinterpret_cast<const w4mma::f32x4*>(p + min(sp + i, splits - 1) * plane);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp + i < splits) o += part[i];
  }
  uint16_t v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = elem<T>::from_f32(bias ? o[e] + h2f<T>(bias[col + e]) : o[e]);
  uint2 w;
  w.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
  w.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
  *reinterpret_cast<uint2*>(c + static_cast<int64_t>(row) * n + col) = w;
}

template <typename T, int MB, bool OG>
void launch_pipe_og(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                    const uint16_t* z, const uint16_t* bias, int64_t r0, int64_t r1, int64_t n,
                    int64_t k, int gs, int tiles, int splits, int sps, float* ws, hipStream_t st) {
  constexpr int lds = w4pipe::Ring<MB>::kBytes;
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&pipe_kernel<T, MB, OG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)configured;
  hipLaunchKernelGGL((pipe_kernel<T, MB, OG>), dim3(static_cast<unsigned>(tiles * splits)),
                     dim3(w4pipe::kThreads), lds, st, c, a, b, s, z, bias, r0, r1, n, k, gs,
                     splits, sps, ws);
}

// gs == 128 (one quantization group per 128-k stage) takes the variant whose
// stage-opening MFMAs start from zero instead of clearing the accumulators.
template <typename T, int MB>
void launch_pipe(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                 const uint16_t* z, const uint16_t* bias, int64_t r0, int64_t r1, int64_t n,
                 int64_t k, int gs, int tiles, int splits, int sps, float* ws, hipStream_t st) {
  if (gs == w4pipe::kStageK)
    launch_pipe_og<T, MB, true>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, ws, st);
  else
    launch_pipe_og<T, MB, false>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, ws, st);
}

template <typename T>
ks_status_t run_pipe(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                     const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n, int64_t k,
                     int gs, hipStream_t st) {
  const int tiles = static_cast<int>((n + w4pipe::kTileN - 1) / w4pipe::kTileN);
  const int total = static_cast<int>(k / w4pipe::kStageK);
  const int spg = std::max(1, gs / w4pipe::kStageK);  // splits stay on group boundaries
  // ~448 workgroups, splits aligned to quantization groups and at least 4
  // stages long. Measured on MI355X (K=4096, M=16/64): N=4096 10.1/17.1 us
  // (13.0/20.0 us with an 8-stage minimum, which left 128 workgroups);
  // N=14336 18.6/30.7 us (896 workgroups were slower).
  int splits = std::max(1, (448 + tiles - 1) / tiles);
  int sps = (total + splits - 1) / splits;
  sps = std::max(sps, std::min(total, 4));
  sps = ((sps + spg - 1) / spg) * spg;
  splits = (total + sps - 1) / sps;
  const int64_t pass_rows = m > 48 ? 64 : (m > 32 ? 48 : (m > 16 ? 32 : 16));
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * pass_rows * n, 0, &sc,
                                "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  for (int64_t r0 = 0; r0 < m; r0 += pass_rows) {
    const int64_t r1 = std::min(m, r0 + pass_rows);
    if (pass_rows == 64)
      launch_pipe<T, 4>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, sc.partial, st);
    else if (pass_rows == 48)
      launch_pipe<T, 3>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, sc.partial, st);
    else if (pass_rows == 32)
      launch_pipe<T, 2>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, sc.partial, st);
    else
      launch_pipe<T, 1>(c, a, b, s, z, bias, r0, r1, n, k, gs, tiles, splits, sps, sc.partial, st);
    if (splits > 1 && !aligned(c, 8)) {
      launch_reduce<T>(c + r0 * n, sc.partial, bias, r1 - r0, n, splits, st);
    } else if (splits > 1) {  // 8-byte output stores (r0 * n is a multiple of 16)
      const int rows = static_cast<int>(r1 - r0);
      hipLaunchKernelGGL((pipe_reduce_kernel<T>), dim3(static_cast<unsigned>(tiles * ((rows + 7) / 8))),
                         dim3(kThreads), 0, st, c + r0 * n, sc.partial, bias, rows,
                         static_cast<int>(n), splits, tiles);
    }
  }
  return KS_SUCCESS;
}

// Larger M: weights dequantized once per workgroup into LDS, 32x32x16 MFMA.
template <typename T, int BM, int BN>
ks_status_t launch_dq(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
               const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n, int64_t k, int gs,
               hipStream_t st) {
  using C = w4dq::Cfg<BM == 256 ? 128 : BM, BN>;
  // 128 x 128 and 256 x 128 tiles run the role-split kernel (w4a16_dqs.hpp),
  // the others dq_kernel.
  constexpr bool kSplitRoles = BM >= 128 && BN == 128;
  constexpr int kLds = kSplitRoles ? w4dqs::Geo<BM>::kBytes : C::kBytes;
  constexpr unsigned kBlock = kSplitRoles ? w4dqs::kThreads : C::kThreads;
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    if constexpr (kSplitRoles)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&w4dqs::dqs_kernel<T, BM>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    else
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&w4dq::dq_kernel<T, BM, BN>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    return true;
  }();
  (void)configured;
  // Fewer than 192 workgroups: split K (whole quantization groups, at least two
  // groups per split) and sum the partial plane with the split reduce. The
  // kernel's stage loop is bound by the copy round trip of each stage, so a
  // small grid otherwise runs its whole K serially on few CUs.
  const int64_t wgs = (n / BN) * ((m + BM - 1) / BM);
  const int nst = static_cast<int>(k / w4dq::kStageK);
  const int spg = std::max(1, gs / w4dq::kStageK);
  int splits = 1, sps = nst;
  if (wgs < 192) {
    splits = static_cast<int>(std::min<int64_t>((224 + wgs - 1) / wgs, nst / (2 * spg)));
    // The role-split kernel holds one workgroup per CU: more than 256
    // workgroups would leave a second, mostly idle round (N = 4096 M = 384:
    // 96 tiles x 3 splits took 46 us, longer than M = 512's 2 x 128).
    if constexpr (kSplitRoles)
      while (splits > 1 && wgs * splits > 256) --splits;
    if (splits > 1) {
      sps = ((nst + splits - 1) / splits + spg - 1) / spg * spg;
      splits = (nst + sps - 1) / sps;
    } else {
      splits = 1;
      sps = nst;
    }
  }
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * m * n, 0, &sc, "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  const dim3 grid(static_cast<unsigned>(n / BN), static_cast<unsigned>((m + BM - 1) / BM),
                  static_cast<unsigned>(splits));
  if constexpr (kSplitRoles)
    hipLaunchKernelGGL((w4dqs::dqs_kernel<T, BM>), grid, dim3(kBlock), kLds, st, c, a, b, s, z, bias, m,
                       n, k, gs, sps, splits > 1 ? sc.partial : nullptr);
  else
    hipLaunchKernelGGL((w4dq::dq_kernel<T, BM, BN>), grid, dim3(kBlock), kLds, st, c, a, b, s, z,
                       bias, m, n, k, gs, sps, splits > 1 ? sc.partial : nullptr);
  if (splits > 1) launch_reduce<T>(c, sc.partial, bias, m, n, splits, st);
  return KS_SUCCESS;
}

template <typename T, int RPT>
void launch_gemv(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                 const uint16_t* z, const uint16_t* bias, int m, int n, int k, int gs,
                 int tiles, int splits, float* ws, hipStream_t st) {
  const dim3 grid(tiles * splits), block(kThreads);
  if (m <= 1) hipLaunchKernelGGL((gemv_kernel<T, 1, RPT>), grid, block, 0, st, c, a, b, s, z, bias, m, n, k, gs, splits, ws);
  else if (m <= 2) hipLaunchKernelGGL((gemv_kernel<T, 2, RPT>), grid, block, 0, st, c, a, b, s, z, bias, m, n, k, gs, splits, ws);
  else if (m <= 4) hipLaunchKernelGGL((gemv_kernel<T, 4, RPT>), grid, block, 0, st, c, a, b, s, z, bias, m, n, k, gs, splits, ws);
  else hipLaunchKernelGGL((gemv_kernel<T, 8, RPT>), grid, block, 0, st, c, a, b, s, z, bias, m, n, k, gs, splits, ws);
}

// Split-plane reduce for the decode kernel: one workgroup per 256-column tile
// and output row, placed on the XCD whose workgroups wrote that tile's
// partials (workgroup ids are dispatched to the 8 XCDs round-robin, and with
// tiles % 8 == 0 every grid row keeps that mapping), so the planes are read
// from that XCD's L2. Sums in split order, + bias. ROWS1: M = 1 with the plane
// size known at compile time (measured ~0.1 us faster per call than the
// general form at M = 1; at M = 8 a row per grid row beats one block doing
// every row: 7.4 against 8.4 us at N = 4096).
template <typename T, bool ROWS1>
__global__ void __launch_bounds__(w4dec::kTileN)
dec_reduce_kernel(uint16_t* __restrict__ c, const float* __restrict__ ws,
                  const uint16_t* __restrict__ bias, int rows, int n, int splits, int tiles) {
  int tile = blockIdx.x;
  if ((tiles & 7) == 0) tile = (blockIdx.x & 7) * (tiles >> 3) + (blockIdx.x >> 3);
  const int col = tile * w4dec::kTileN + threadIdx.x;
  if (col >= n) return;
  const int64_t plane = ROWS1 ? static_cast<int64_t>(n) : static_cast<int64_t>(rows) * n;
  const int m = ROWS1 ? 0 : static_cast<int>(blockIdx.y);
  const float bv = bias ? h2f<T>(bias[col]) : 0.f;
  const float* p = ws + static_cast<int64_t>(m) * n + col;
  float o = 0.f;
  int sp = 0;
  for (; sp + 8 <= splits; sp += 8) {  // 8 loads in flight, added in order
    float part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = p[(sp + i) * plane];
#pragma unroll
    for (int i = 0; i < 8; ++i) o += part[i];
  }
  if (sp < splits) {  // tail: clamped, guarded, still one batch in flight
    float part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = p[min(sp + i, splits - 1) * plane];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp + i < splits) o += part[i];
  }
  c[static_cast<int64_t>(m) * n + col] = elem<T>::from_f32(o + bv);
}

template <typename T>
void launch_dec_reduce(uint16_t* c, const float* ws, const uint16_t* bias, int m, int n,
                       int splits, int tiles, hipStream_t st) {
  if (m == 1)
    hipLaunchKernelGGL((dec_reduce_kernel<T, true>), dim3(tiles), dim3(w4dec::kTileN), 0, st, c,
                       ws, bias, m, n, splits, tiles);
  else
    hipLaunchKernelGGL((dec_reduce_kernel<T, false>), dim3(tiles, static_cast<unsigned>(m)),
                       dim3(w4dec::kTileN), 0, st, c, ws, bias, m, n, splits, tiles);
}

template <typename T, int MB, int WAVES, int RPT, int ITER>
void launch_dec(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                const uint16_t* z, const uint16_t* bias, int m, int n, int k, int gs, int tiles,
                int splits, float* ws, hipStream_t st) {
  hipLaunchKernelGGL((w4dec::dec_kernel<T, MB, WAVES, RPT, ITER>), dim3(tiles * splits),
                     dim3(64 * WAVES), 0, st, c, a, b, s, z, bias, m, n, k,
                     gs, splits, ws);
}

template <typename T, int MB, int WAVES, int RPT, int ITER>
ks_status_t dec_rows(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                     const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n, int64_t k,
                     int gs, hipStream_t st) {
  const int tiles = static_cast<int>((n + w4dec::kTileN - 1) / w4dec::kTileN);
  const int rows_wg = w4dec::Geo<WAVES, RPT, ITER>::kRowsWG;
  const int splits = static_cast<int>((k / 2 + rows_wg - 1) / rows_wg);
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * kMaxDecM * n, 0, &sc,
                                "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  const int ni = static_cast<int>(n), ki = static_cast<int>(k), mi = static_cast<int>(m);
  launch_dec<T, MB, WAVES, RPT, ITER>(c, a, b, s, z, bias, mi, ni, ki, gs, tiles, splits,
                                      sc.partial, st);
  if (splits > 1)
    launch_dec_reduce<T>(c, sc.partial, bias, mi, ni, splits, tiles, st);
  return KS_SUCCESS;
}

// Row blocks and K chunks per workgroup by shape. Measured on MI355X (K=4096,
// graph replay, cold): M <= 4 is fastest with one chunk (16 splits); M = 5..8
// with two chunks once one chunk would give >= 512 workgroups (N=14336 M=8:
// 14.7 us against 16.2 us), else one (N=4096 M=8: 9.8 us against 10.1 us).
template <typename T, int WAVES, int RPT>
ks_status_t dec_dispatch(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
                         const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n,
                         int64_t k, int gs, hipStream_t st) {
  if (m <= 4) return dec_rows<T, 1, WAVES, RPT, 1>(c, a, b, s, z, bias, m, n, k, gs, st);
  const int64_t tiles = (n + w4dec::kTileN - 1) / w4dec::kTileN;
  const int64_t rows1 = w4dec::Geo<WAVES, RPT, 1>::kRowsWG;
  const int64_t wgs1 = tiles * ((k / 2 + rows1 - 1) / rows1);
  if (wgs1 >= 512) return dec_rows<T, 2, WAVES, RPT, 2>(c, a, b, s, z, bias, m, n, k, gs, st);
  return dec_rows<T, 2, WAVES, RPT, 1>(c, a, b, s, z, bias, m, n, k, gs, st);
}

// Decode shapes (M <= 8) on MFMA; returns false when the shape or alignment
// does not fit the kernel's requirements.
template <typename T>
bool run_dec(uint16_t* c, const uint16_t* a, const uint8_t* b, const uint16_t* s,
             const uint16_t* z, const uint16_t* bias, int64_t m, int64_t n, int64_t k, int gs,
             hipStream_t st, ks_status_t* r) {
  if (n % 16 != 0 || k % 8 != 0 || n > (int64_t{1} << 26) || k > (int64_t{1} << 30) ||
      !aligned(a, 16) ||
      !aligned(b, 16) || !aligned(s, 16) || !aligned(z, 16))
    return false;
  // Measured on MI355X at M=1 K=N=4096: 4 waves x 8 rows per lane (256
  // workgroups, 16 splits) beats 8 waves x 4 rows, 4 waves x 4 rows and
  // 8 waves x 8 rows (fewer workgroups).
  if (gs % 64 == 0 && k % 64 == 0) {
    *r = dec_dispatch<T, 4, 8>(c, a, b, s, z, bias, m, n, k, gs, st);
    return true;
  }
  if (gs % 32 == 0 && k % 32 == 0) {
    *r = dec_dispatch<T, 4, 4>(c, a, b, s, z, bias, m, n, k, gs, st);
    return true;
  }
  return false;
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
  const bool pipe = m > kMaxGemvM && (gs % 64 == 0) && (k % w4pipe::kStageK == 0) && (n % 16 == 0) &&
                    aligned(a, 16) && aligned(b, 16) && aligned(s, 4) && aligned(z, 4) &&
                    k * n < (int64_t{1} << 40) && n < (int64_t{1} << 26) &&
                    m * k < (int64_t{1} << 31);  // the ring tile's 32-bit copy offsets
  // M <= 8: the MFMA decode kernel (measured on MI355X at K=4096, N=14336:
  // M=8 14.7 us against 33.3 us for the dot2 kernel; at M=16, four
  // block-diagonal row blocks measured 25 us against 18.8 us for the LDS-ring
  // tile).
  if (m <= kMaxDecM) {
    ks_status_t r;
    if (run_dec<T>(c, a, b, s, z, bias, m, n, k, gs, st, &r)) return r;
  }
  const bool dq = m > kDqMinM && (gs % 64 == 0) && (k % 64 == 0) && (n % 64 == 0) &&
                  aligned(a, 16) && aligned(b, 16) && aligned(s, 4) && aligned(z, 4) &&
                  (m + 127) / 128 < 65536;
  if (dq) {
    // Tile: the first of 128x128, 64x128, 128x64, 64x64 (wider N first: the
    // activation re-reads, the dominant copy stream, scale with N / BN) that
    // still gives >= 192 workgroups; the kernel is bound by each CU's copy
    // stream, so an under-filled grid costs more than a smaller tile (M=256
    // N=4096: 64 workgroups of 128x128 took 72.8 us).
    const bool wide = n % 128 == 0;
    auto wgs = [&](int bm, int bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); };
    // 128 x 128 tiles (the role-split kernel) from 32 tiles up, K-split below
    // 192 workgroups (against 64 x 128 / 64 x 64 tiles: N = 14336 M = 96/128
    // 51 -> 43 us; N = 8192 M = 128 40.8 -> 30.7 us; N = 4096 M = 256
    // 40.4 -> 29.1 us, M = 65 24.9 -> 21.2 us; at 16 tiles, N = 2048 M = 96,
    // 16.5 -> 18.4 us, so smaller grids keep the 64-row tiles).
    // 256 x 128 tiles (each weight dequantized once for 256 rows) when they
    // alone give >= 192 workgroups: N = 14336 M = 512 / 1024 106 / 201 ->
    // 95 / 180 us; with a K split instead (M = 256) they lost to 128 x 128.
    if (m >= 384 && wide && wgs(256, 128) >= 192) return launch_dq<T, 256, 128>(c, a, b, s, z, bias, m, n, k, gs, st);
    if (m > 64 && wide && wgs(128, 128) >= 32) return launch_dq<T, 128, 128>(c, a, b, s, z, bias, m, n, k, gs, st);
    if (wide && wgs(64, 128) >= 192) return launch_dq<T, 64, 128>(c, a, b, s, z, bias, m, n, k, gs, st);
    if (m > 64 && wgs(128, 64) >= 192) return launch_dq<T, 128, 64>(c, a, b, s, z, bias, m, n, k, gs, st);
    return launch_dq<T, 64, 64>(c, a, b, s, z, bias, m, n, k, gs, st);
  }
  if (pipe) return run_pipe<T>(c, a, b, s, z, bias, m, n, k, gs, st);
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
  // Eight packed rows per thread unless that leaves fewer than 256 workgroups.
  int rpt = 8;
  int splits = static_cast<int>((kp + kRowsPar * rpt - 1) / (kRowsPar * rpt));
  if (static_cast<int64_t>(tiles) * splits < 256) {
    rpt = 4;
    splits = static_cast<int>((kp + kRowsPar * rpt - 1) / (kRowsPar * rpt));
  }
  Scratch sc;
  if (splits > 1) {
    ks_status_t r = get_scratch(st, static_cast<size_t>(splits) * kMaxGemvM * n, 0, &sc,
                                "ks_gemm_w4a16");
    if (r != KS_SUCCESS) return r;
  }
  for (int64_t m0 = 0; m0 < m; m0 += kMaxGemvM) {
    const int mm = static_cast<int>((m - m0) < kMaxGemvM ? (m - m0) : kMaxGemvM);
    uint16_t* cc = c + m0 * n;
    const uint16_t* aa = a + m0 * k;
    const int ki = static_cast<int>(k), ni = static_cast<int>(n);
    if (rpt == 8) launch_gemv<T, 8>(cc, aa, b, s, z, bias, mm, ni, ki, gs, tiles, splits, sc.partial, st);
    else launch_gemv<T, 4>(cc, aa, b, s, z, bias, mm, ni, ki, gs, tiles, splits, sc.partial, st);
    if (splits > 1) launch_reduce<T>(cc, sc.partial, bias, mm, n, splits, st);
  }
  return KS_SUCCESS;
}

// ---- no-allocation variant: fixed per-device scratch --------------------
// The split partial planes of every ks_gemm_w4a16 path come from this array
// instead of library-allocated memory. Each device that the library runs on
// holds one copy until the process ends. Host code must never pass the
// symbol itself to a kernel (it names a host-side shadow): the device address
// comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoAllocScratchBytes = size_t{16} << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
float* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of this device's `scratch`, resolved on the first call on
// the device (with that device current).
ks_status_t noalloc_scratch(float** out) {
  int dev = 0;
  ks_status_t st = check_hip(hipGetDevice(&dev), "ks_gemm_w4a16_noalloc");
  if (st != KS_SUCCESS) return st;
  if (dev < 0 || dev >= kMaxDevices) {
    set_last_error("ks_gemm_w4a16_noalloc: device ordinal beyond the supported 64");
    return KS_ERROR_INVALID_ARGUMENT;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? static_cast<float*>(p) : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr)
    return check_hip(g_scratch_err[dev] != hipSuccess ? g_scratch_err[dev] : hipErrorInvalidSymbol,
                     "ks_gemm_w4a16_noalloc: hipGetSymbolAddress(scratch)");
  *out = g_scratch_ptr[dev];
  return KS_SUCCESS;
}

}  // namespace w4a16
}  // namespace ks

extern "C" {

static ks_status_t gemm_w4a16_body(void* c, const void* a, const void* b_packed,
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

ks_status_t ks_gemm_w4a16(void* c, const void* a, const void* b_packed,
                          const void* scales, const void* zeros, const void* bias,
                          int64_t m, int64_t n, int64_t k, int group_size,
                          ks_dtype_t dtype, ks_stream_t stream) {
  return gemm_w4a16_body(c, a, b_packed, scales, zeros, bias, m, n, k, group_size, dtype, stream);
}

// Same kernels and bits as ks_gemm_w4a16; split partials go to the fixed
// per-device `scratch` array, so the call never allocates. Calls that overlap
// on one device race on that array.
ks_status_t ks_gemm_w4a16_noalloc(void* c, const void* a, const void* b_packed,
                                  const void* scales, const void* zeros, const void* bias,
                                  int64_t m, int64_t n, int64_t k, int group_size,
                                  ks_dtype_t dtype, ks_stream_t stream) {
  float* ptr = nullptr;
  ks_status_t r = ks::w4a16::noalloc_scratch(&ptr);
  if (r != KS_SUCCESS) return r;
  ks::ScratchOverride use(ptr, ks::w4a16::kNoAllocScratchBytes / sizeof(float), nullptr, 0,
                          "16 MiB");
  return gemm_w4a16_body(c, a, b_packed, scales, zeros, bias, m, n, k, group_size, dtype, stream);
}

}  // extern "C"
