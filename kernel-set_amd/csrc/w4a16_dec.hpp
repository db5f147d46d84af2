// kernel-set (MI355X build) -- W4A16 decode GEMV/GEMM (M <= 8) on MFMA.
//
// Semantics are those of ks_gemm_w4a16 (kernels/src/gemm/gemm_w4a16.cu:74-129
// of cklxx/kernel-set): C[m,n] = sum_k A[m,k] * (q[k,n] - z[g,n]) * s[g,n].
//
// Weight stream: uint8 [K/2, N], byte (kp, n) = q(2kp, n) | q(2kp+1, n) << 4.
// Lane (li = lane % 16, g = lane / 16) of a wave loads 16 bytes = 16 columns of
// one packed row; the 16 lanes of a lane group cover 256 contiguous bytes (two
// whole 128-byte lines) of that row, and the four lane groups take four rows.
//
// No byte transpose. A packed dword d holds 4 columns x 2 k. One and-or per
// output dword turns it into a 16-bit float pair "base + q" (bf16 0x4300|q =
// 128 + q, f16 0x5800|q = 128 + q/8, both exact):
//   v0 = (d       & 0x000f000f) | base  -> (col 0, even k), (col 2, even k)
//   v1 = (d >>  8 & 0x000f000f) | base  -> (col 1, even k), (col 3, even k)
//   v2 = (d >>  4 & 0x000f000f) | base  -> (col 0, odd k),  (col 2, odd k)
//   v3 = (d >> 12 & 0x000f000f) | base  -> (col 1, odd k),  (col 3, odd k)
// {v0..v3} is the B fragment (8 k-slots) of one v_mfma_f32_16x16x32 for MFMA
// column li. The 8 slots belong to four different weight columns, so the A
// fragment is block-diagonal: MFMA row i = 4*mm + c (activation row mm, column
// c of the dword) carries a[mm, 2kp] in the slot of (c, even) and a[mm, 2kp+1]
// in the slot of (c, odd), zeros elsewhere. D[4*mm + c][li] is then the dot of
// activation row mm with weight column 16*li + 4*p + c (p = dword of the 16-byte
// load). One MFMA serves up to four activation rows at the same VALU cost, so
// M <= 4 costs what M = 1 costs; M <= 8 uses two A fragments.
//
// Zero-point: with an all-ones B the same A gives S = sum_k a, and per group
//   O += s * (P - (128 + z) * S)       (f16: s*8 * (P - (128 + z/8) * S))
// equals sum_k a * (q - z) * s. Each wave's K range lies inside one group.
//
// Workgroup = WAVES waves over one 256-column tile and WAVES*4*RPT packed rows;
// the waves are summed through LDS in a fixed order, and K splits go to a
// partial plane reduced by a second kernel in split order (deterministic).
#pragma once

#include "ks_common.hpp"
#include "w4a16_mfma.hpp"

namespace ks {
namespace w4dec {

using w4mma::f32x4;
using w4mma::u32x4v;

constexpr int kTileN = 256;

template <int WAVES, int RPT, int ITER>
struct Geo {
  static constexpr int kThreads = 64 * WAVES;
  static constexpr int kRowsChunk = WAVES * 4 * RPT;      // packed rows per chunk
  static constexpr int kRowsWG = kRowsChunk * ITER;       // packed rows per workgroup
};

// Workgroup id -> (column tile, k split); the splits of one tile share an XCD
// when the grid divides into the 8 XCDs (ids are dispatched round-robin).
__device__ inline void map_tile(int bid, int nblocks, int splits, int* tile, int* split) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  *tile = logical / splits;
  *split = logical % splits;
}

// (x & mask) | base. With the mask a wave-uniform SGPR value and the base a
// VGPR (VOP3 takes no literal on gfx9, one SGPR per instruction) this selects
// to a single v_and_or_b32.
__device__ inline uint32_t and_or(uint32_t x, uint32_t mask, uint32_t base) {
  return (x & mask) | base;
}

// Pins a value in a VGPR so the compiler does not rematerialize the constant.
__device__ inline uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Requirements (checked by the host): n % 16 == 0, k % (8*RPT) == 0,
// gs % (8*RPT) == 0, A 16-byte aligned with k % 8 == 0, b/s/z 16-byte aligned.
//
// A workgroup's K range is ITER chunks; in chunk `it` wave w owns packed rows
// split*kRowsWG + it*kRowsChunk + w*4*RPT .. +4*RPT (8*RPT k, inside one
// quantization group). Chunk it+1's loads are issued before chunk it's math,
// and every chunk is promoted with its own group's scales and zeros.
template <typename T, int MB, int WAVES, int RPT, int ITER>
__global__ void __launch_bounds__(64 * WAVES)
dec_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
           const uint8_t* __restrict__ b, const uint16_t* scales,
           const uint16_t* zeros, const uint16_t* __restrict__ bias,
           int m_rows, int n, int k, int gs, int splits, float* __restrict__ ws) {
  using G = Geo<WAVES, RPT, ITER>;
  constexpr int kRowsM = 4 * MB;
  __shared__ float red[WAVES][kRowsM][kTileN];

  int tile, split;
  map_tile(blockIdx.x, gridDim.x, splits, &tile, &split);
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int li = lane % 16, g = lane / 16;
  const int col0 = tile * kTileN + 16 * li;
  const int kph = k / 2;
  const int ng = k / gs;
  const bool col_ok = col0 < n;
  // Every load is unconditional (addresses clamped into the tensors) so the
  // loads stay branch-free and the math on row i waits only for load i. Rows
  // past K get zero activations (no contribution); columns past N are computed
  // on clamped data and never stored. A NULL zeros pointer reads the scales
  // and is replaced by 0.
  const int ccol0 = col_ok ? col0 : 0;
  const uint16_t* zsrc = zeros ? zeros : scales;

  struct Chunk {
    uint4 a[MB][RPT / 4];  // activation pairs of this lane's RPT rows, raw
    uint4 s[2], z[2];      // the chunk's group: 16 columns of scales / zeros
    uint4 w[RPT];          // the weight stream
    bool rows_ok;
  };
  auto issue = [&](int it, Chunk& ch) {
    const int wrow0 = split * G::kRowsWG + it * G::kRowsChunk + wave * 4 * RPT;
    const int row0 = wrow0 + g * RPT;
    ch.rows_ok = row0 < kph;  // k % (8*RPT) == 0: a lane's rows are all in or all out
    const int crow0 = ch.rows_ok ? row0 : 0;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int mm = 4 * mb + (li >> 2);
      const uint4* src = reinterpret_cast<const uint4*>(
                             a + static_cast<int64_t>(mm < m_rows ? mm : 0) * k) + crow0 / 4;
#pragma unroll
      for (int i = 0; i < RPT / 4; ++i) ch.a[mb][i] = src[i];
    }
    // Weight addresses: a wave-uniform row base (a wave's 4*RPT rows are all
    // in range or all out, since K/2 is a multiple of 4*RPT) plus a 32-bit
    // lane offset, one add per load instead of a 64-bit multiply-add.
    const uint8_t* bw = b + static_cast<int64_t>(wrow0 < kph ? wrow0 : 0) * n;
    const uint32_t loff = static_cast<uint32_t>(g * RPT * n + ccol0);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      ch.w[i] = load_stream16(bw + (loff + static_cast<uint32_t>(i * n)));
    // The group's scales / zeros are needed only by the promotion: issued last.
    const int grp = min((2 * wrow0) / gs, ng - 1);
    const int64_t gi = static_cast<int64_t>(grp) * n + ccol0;
    ch.s[0] = *reinterpret_cast<const uint4*>(scales + gi);
    ch.s[1] = *reinterpret_cast<const uint4*>(scales + gi + 8);
    ch.z[0] = *reinterpret_cast<const uint4*>(zsrc + gi);
    ch.z[1] = *reinterpret_cast<const uint4*>(zsrc + gi + 8);
  };

  // Per-lane perm selectors placing a_even / a_odd into the slots of column cdw.
  const int cdw = li & 3;
  constexpr uint32_t Z = 0x0c0c0c0cu, EL = 0x0c0c0100u, EH = 0x01000c0cu, OL = 0x0c0c0302u,
                     OH = 0x03020c0cu;
  const uint32_t sel0 = cdw == 0 ? EL : (cdw == 2 ? EH : Z);
  const uint32_t sel1 = cdw == 1 ? EL : (cdw == 3 ? EH : Z);
  const uint32_t sel2 = cdw == 0 ? OL : (cdw == 2 ? OH : Z);
  const uint32_t sel3 = cdw == 1 ? OL : (cdw == 3 ? OH : Z);
  const uint32_t base = opaque(w4mma::mfma_traits<T>::magic);
  const uint32_t mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
  const uint32_t one2 = opaque(w4mma::mfma_traits<T>::one2);
  const u32x4v ones = {one2, one2, one2, one2};
  constexpr float u = w4mma::code_scale<T>::unit;

  // Lane holds D[4*(lane/16) + r][li] -> activation row 4*mb + g, column
  // col0 + 4*p + r; O accumulates the promoted chunks.
  f32x4 O[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int p = 0; p < 4; ++p) O[mb][p] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The scale / zero loads must stay with the weight loads: the promotion
  // that consumes them is conditional on the lane holding a live activation
  // row, and as invariant loads (const __restrict__ pointers) they were sunk
  // into that branch, after the last MFMA, adding a memory round trip to
  // every workgroup's tail (M=1 K=N=4096: 6.04 -> 5.94 us per call with
  // them kept here). `scales` / `zeros` are therefore not __restrict__, and a
  // compiler barrier follows each issue.
  Chunk cur;
  issue(0, cur);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    Chunk nxt;
    if (it + 1 < ITER) issue(it + 1, nxt);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // next chunk's loads stay ahead of this math

    uint32_t ap[MB][RPT];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const bool ok = cur.rows_ok && (4 * mb + (li >> 2)) < m_rows;
#pragma unroll
      for (int i = 0; i < RPT; i += 4) {
        const uint4 v = cur.a[mb][i / 4];
        ap[mb][i] = ok ? v.x : 0u;
        ap[mb][i + 1] = ok ? v.y : 0u;
        ap[mb][i + 2] = ok ? v.z : 0u;
        ap[mb][i + 3] = ok ? v.w : 0u;
      }
    }
    f32x4 P[MB][4], S[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      S[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 4; ++p) P[mb][p] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      u32x4v af[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint32_t x = ap[mb][i];
        af[mb] = u32x4v{__builtin_amdgcn_perm(x, x, sel0), __builtin_amdgcn_perm(x, x, sel1),
                        __builtin_amdgcn_perm(x, x, sel2), __builtin_amdgcn_perm(x, x, sel3)};
      }
      const uint32_t dw[4] = {cur.w[i].x, cur.w[i].y, cur.w[i].z, cur.w[i].w};
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t d = dw[p];
        const u32x4v bf = {and_or(d, mask, base), and_or(d >> 8, mask, base),
                           and_or(d >> 4, mask, base), and_or(d >> 12, mask, base)};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) P[mb][p] = w4mma::mfma_traits<T>::mma(af[mb], bf, P[mb][p]);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) S[mb] = w4mma::mfma_traits<T>::mma(af[mb], ones, S[mb]);
    }
    // Promotion with the chunk's group: O += s * (P - (128 + z) * S).
    const uint32_t sv[8] = {cur.s[0].x, cur.s[0].y, cur.s[0].z, cur.s[0].w,
                            cur.s[1].x, cur.s[1].y, cur.s[1].z, cur.s[1].w};
    const uint32_t zv[8] = {cur.z[0].x, cur.z[0].y, cur.z[0].z, cur.z[0].w,
                            cur.z[1].x, cur.z[1].y, cur.z[1].z, cur.z[1].w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 4 * p + r;
        const float sj = elem<T>::to_f32(static_cast<uint16_t>(sv[j / 2] >> (16 * (j & 1))));
        const float zj = zeros ? elem<T>::to_f32(static_cast<uint16_t>(zv[j / 2] >> (16 * (j & 1))))
                               : 0.f;
        const float cz = 128.0f + zj * u;
        const float se = sj * (1.0f / u);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) O[mb][p][r] = fmaf(se, fmaf(-cz, S[mb][r], P[mb][p][r]), O[mb][p][r]);
      }
    }
    if (it + 1 < ITER) cur = nxt;
  }

  // Only the rows that hold activation rows (< m_rows) are written and summed:
  // at M = 1 that cuts the tail after the last weight row arrives from ~1400
  // to ~700 cycles (s_memtime stamps).
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    if (4 * mb + g < m_rows) {
#pragma unroll
      for (int p = 0; p < 4; ++p)
        *reinterpret_cast<f32x4*>(&red[wave][4 * mb + g][16 * li + 4 * p]) = O[mb][p];
    }
  __syncthreads();

  // Sum the waves in order; one thread per (row, column) entry.
  for (int e = threadIdx.x; e < m_rows * kTileN; e += G::kThreads) {
    const int mm = e / kTileN, cc = e % kTileN;
    const int col = tile * kTileN + cc;
    if (col >= n) continue;
    float v = red[0][mm][cc];
#pragma unroll
    for (int wv = 1; wv < WAVES; ++wv) v += red[wv][mm][cc];
    if (splits == 1) {
      if (bias) v += elem<T>::to_f32(bias[col]);
      c[static_cast<int64_t>(mm) * n + col] = elem<T>::from_f32(v);
    } else {
      ws[(static_cast<int64_t>(split) * m_rows + mm) * n + col] = v;
    }
  }
}

}  // namespace w4dec
}  // namespace ks
