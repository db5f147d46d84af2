// kernel-set (MI355X build) -- 8-bit MFMA GEMMs: fp8 blockwise-scaled and W8A8.
//
// Both take A [M,K] (K contiguous) and B [K,N] (N contiguous, the reference's
// quantized-linear layout, gemm.h:79-98 / gemm.h:39-49 of cklxx/kernel-set).
// MFMA wants both operands K-contiguous per lane, so each workgroup transposes
// its B tile once while staging it into LDS (register byte transpose with
// v_perm, then 32-bit LDS writes into a [n][k] layout); all four waves then read
// MFMA fragments with 128-bit LDS loads. A tiles are copied to LDS unchanged.
//
// Tiling: workgroup 128x128 output tile, 4 waves as 2x2 of 64x64, K step 128.
// Per K step each wave issues 4x4 MFMAs:
//   fp8 : v_mfma_scale_f32_16x16x128_f8f6f4 (unit scales)        -> fp32
//   int8: 2 x v_mfma_i32_16x16x64_i8                              -> int32
// The next K step's global loads are issued into registers before the current
// step's MFMAs (register double buffering) so HBM latency hides behind math.
//
// fp8 blockwise (gemm_fp8_blockwise.cu:107-161): inside one scale block of
// block_k (a multiple of 128) the MFMA accumulates the raw fp32 partial P; at
// the block end P is promoted: O = fma(P, a_s[m,kb] * b_s[kb,n/block_n], O).
// W8A8 (gemm_w8a8.cu:120-142): exact int32 accumulation over all of K, then
// v = (float(acc) * a_s) * b_s (+ bias), with no contraction of the multiplies.
#include "kernel_set/gemm.h"
#include "kernel_set/quant.h"
#include "kernel_set/testing.h"
#include "ks_common.hpp"
#include "gemm8_common.hpp"
#include "gemm8_skinny.hpp"
#include "workspace.hpp"

namespace ks {
namespace gemm8 {

// 4x4 byte transpose: in[r] holds bytes (r,0..3); out[c] holds bytes (0..3,c).
__device__ inline void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  // pair rows (0,1) and (2,3): interleave bytes
  const uint32_t t01lo = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // r0c0 r1c0 r0c1 r1c1
  const uint32_t t01hi = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // r0c2 r1c2 r0c3 r1c3
  const uint32_t t23lo = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t t23hi = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(t23lo, t01lo, 0x05040100u);  // c0: r0 r1 r2 r3
  out[1] = __builtin_amdgcn_perm(t23lo, t01lo, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t23hi, t01hi, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t23hi, t01hi, 0x07060302u);
}

template <typename Out>
__device__ inline void store_out(typename Out::storage* p, float v) {
  *p = elem<Out>::from_f32(v);
}


// Workgroup id -> (tile_m, tile_n). Tiles are walked column-major in groups so
// that concurrently running workgroups share B column panels in L2.
__device__ inline void tile_coords(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
  // Workgroup ids are dispatched round-robin over the 8 XCDs, each with its own
  // L2. Renumber so every XCD owns a contiguous range of tiles, then walk the
  // tiles in bands of kGroup tile rows: an XCD's range is then a compact
  // ~kGroup x (range/kGroup) block whose A and B panels stay in its L2 while
  // its workgroups move through K together (instead of every XCD streaming
  // the whole of B).
  constexpr int kGroup = 4;
  const int total = tiles_m * tiles_n;
  int l = bid;
  if ((total & 7) == 0) l = (bid & 7) * (total >> 3) + (bid >> 3);
  const int per_group = kGroup * tiles_n;
  const int g = l / per_group;
  const int first_m = g * kGroup;
  const int gm = min(tiles_m - first_m, kGroup);
  const int r = l % per_group;
  *tm = first_m + r % gm;
  *tn = r / gm;
}

template <int KIND, typename Out>
__global__ void __launch_bounds__(kThreads)
gemm8_kernel(Args p) {
  __shared__ __attribute__((aligned(16))) uint8_t sA[kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) uint8_t sB[kBN * kLdsStride];  // [n][k]
  __shared__ float sAs[kBM];
  __shared__ float sBs[kBN];

  const int tiles_m = static_cast<int>((p.m + kBM - 1) / kBM);
  const int tiles_n = static_cast<int>((p.n + kBN - 1) / kBN);
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int64_t m0 = static_cast<int64_t>(tm) * kBM;
  const int64_t n0 = static_cast<int64_t>(tn) * kBN;

  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int wm = (wave / 2) * 64;  // wave tile origin inside the workgroup tile
  const int wn = (wave % 2) * 64;

  // ---- global -> register staging assignments ----
  // A: 128 rows x 128 bytes = 1024 chunks of 16 B, 4 per thread.
  // B: thread covers 4 k rows x 16 columns (4 chunks of 16 B).
  const int b_cg = t % 8;   // 16-column group
  const int b_kg = t / 8;   // 4-row group (0..31)
  uint4 ra[4], rb[4];

  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + kThreads * i;
      const int row = c / 8, kc = c % 8;
      const int64_t gm = m0 + row, gk = k0 + 16 * kc;
      ra[i] = (gm < p.m && gk < p.k)
                  ? *reinterpret_cast<const uint4*>(p.a + gm * p.k + gk)
                  : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t gk = k0 + 4 * b_kg + r, gn = n0 + 16 * b_cg;
      rb[r] = (gk < p.k && gn < p.n)
                  ? *reinterpret_cast<const uint4*>(p.b + gk * p.n + gn)
                  : make_uint4(0, 0, 0, 0);
    }
  };

  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + kThreads * i;
      const int row = c / 8, kc = c % 8;
      *reinterpret_cast<uint4*>(sA + row * kLdsStride + 16 * kc) = ra[i];
    }
    const uint32_t d[4][4] = {{rb[0].x, rb[0].y, rb[0].z, rb[0].w},
                              {rb[1].x, rb[1].y, rb[1].z, rb[1].w},
                              {rb[2].x, rb[2].y, rb[2].z, rb[2].w},
                              {rb[3].x, rb[3].y, rb[3].z, rb[3].w}};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t in[4] = {d[0][q], d[1][q], d[2][q], d[3][q]};
      uint32_t o[4];
      transpose4x4(in, o);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int col = 16 * b_cg + 4 * q + c;
        *reinterpret_cast<uint32_t*>(sB + col * kLdsStride + 4 * b_kg) = o[c];
      }
    }
  };

  // Plain fp8 runs the blockwise path as one K block with unit scales (the
  // promotion is then fma(P, 1, 0) = P exactly) and the per-token /
  // per-channel epilogue of W8A8.
  constexpr bool kPlain = is_fp8_plain(KIND);
  constexpr bool kFp8 = is_fp8_block(KIND) || kPlain;
  // accumulators: 4x4 blocks of 16x16, 4 values per lane each
  f32x4 acc_o[4][4];   // fp8: promoted output; unused for int8
  f32x4 acc_p[4][4];   // fp8: raw partial of the current scale block
  i32x4 acc_i[4][4];   // int8: exact accumulator
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc_o[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc_p[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc_i[i][j] = i32x4{0, 0, 0, 0};
    }

  const int li = lane % 16;       // row (A) / column (B) inside a 16-block
  const int lk = lane / 16;       // k sub-slice
  const int steps = static_cast<int>((p.k + kBK - 1) / kBK);
  const int steps_per_block = kPlain ? steps : (kFp8 ? p.block_k / kBK : 1);

  load_tiles(0);
  for (int s = 0; s < steps; ++s) {
    const int64_t k0 = static_cast<int64_t>(s) * kBK;
    __syncthreads();  // previous step's LDS reads are done
    store_tiles();
    const bool promote = kFp8 && ((s + 1) % steps_per_block == 0 || s + 1 == steps);
    if (kFp8 && promote) {
      if (kPlain) {
        if (t < kBM) sAs[t] = 1.f; else sBs[t - kBM] = 1.f;
      } else {
        const int64_t kb = k0 / p.block_k;
        if (t < kBM) {
          const int64_t gm = m0 + t;
          sAs[t] = gm < p.m ? p.a_scale[gm * p.nkb + kb] : 0.f;
        } else {
          const int64_t gn = n0 + (t - kBM);
          sBs[t - kBM] = gn < p.n ? p.b_scale[kb * p.nnb + gn / p.block_n] : 0.f;
        }
      }
    }
    __syncthreads();
    if (s + 1 < steps) load_tiles(k0 + kBK);  // in flight during the MFMAs

    if constexpr (kFp8) {
      i32x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint8_t* pa = sA + (wm + 16 * i + li) * kLdsStride + 32 * lk;
        const uint4 x0 = *reinterpret_cast<const uint4*>(pa);
        const uint4 x1 = *reinterpret_cast<const uint4*>(pa + 16);
        fa[i] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                      (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        const uint8_t* pb = sB + (wn + 16 * i + li) * kLdsStride + 32 * lk;
        const uint4 y0 = *reinterpret_cast<const uint4*>(pb);
        const uint4 y1 = *reinterpret_cast<const uint4*>(pb + 16);
        fb[i] = i32x8{(int)y0.x, (int)y0.y, (int)y0.z, (int)y0.w,
                      (int)y1.x, (int)y1.y, (int)y1.z, (int)y1.w};
      }
      constexpr int fmt = fp8_fmt(KIND);  // 0 = fp8 e4m3, 1 = bf8 e5m2
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc_p[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              fa[i], fb[j], acc_p[i][j], fmt, fmt, 0, 127, 0, 127);
      if (promote) {
        // lane's output rows: wm + 16i + 4*lk + r ; column: wn + 16j + li
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float bs = sBs[wn + 16 * j + li];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float sc = sAs[wm + 16 * i + 4 * lk + r] * bs;
              acc_o[i][j][r] = fmaf(acc_p[i][j][r], sc, acc_o[i][j][r]);
            }
            acc_p[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        i32x4 fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 x = *reinterpret_cast<const uint4*>(
              sA + (wm + 16 * i + li) * kLdsStride + 64 * h + 16 * lk);
          fa[i] = i32x4{(int)x.x, (int)x.y, (int)x.z, (int)x.w};
          const uint4 y = *reinterpret_cast<const uint4*>(
              sB + (wn + 16 * i + li) * kLdsStride + 64 * h + 16 * lk);
          fb[i] = i32x4{(int)y.x, (int)y.y, (int)y.z, (int)y.w};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc_i[i][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue ----
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + wn + 16 * j + li;
      if (gn >= p.n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t gm = m0 + wm + 16 * i + 4 * lk + r;
        if (gm >= p.m) continue;
        if constexpr (kPlain) {
          const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
          const float bs = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn,
                         __fmul_rn(__fmul_rn(acc_o[i][j][r], as), bs));
        } else if constexpr (kFp8) {
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn,
                         acc_o[i][j][r]);
        } else if constexpr (KIND == INT8_RAW) {
          static_cast<int32_t*>(p.out)[gm * p.n + gn] = acc_i[i][j][r];
        } else {
          const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
          const float bs = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
          float v = __fmul_rn(__fmul_rn(static_cast<float>(acc_i[i][j][r]), as), bs);
          if (p.bias)
            v = __fadd_rn(v, elem<Out>::load(static_cast<const typename Out::storage*>(p.bias), gn));
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn, v);
        }
      }
    }
}


// ===========================================================================
// Fast path: 256x256 workgroup tile, 8 waves (2 x 4) of 128x64, K step 128,
// LDS double buffer, one barrier per K step, no VGPR staging:
//  * A [256 rows][128 B] and B [128 k][256 n] tiles are fetched with
//    global_load_lds_dwordx4 straight into LDS; every wave instruction fills a
//    contiguous 1 KB and each lane picks which 16-byte chunk lands in its slot,
//    which stores both tiles with their chunks XOR-swizzled (a_swz, b_swz).
//    The copies for step s+1 are issued as inline asm before step s's math,
//    so they overlap it (the compiler would otherwise hold every LDS read of
//    step s behind them with a vmcnt(0)).
//  * A fragments: two ds_read_b128 per 16x(32 k) lane slice. The 32 bytes of
//    lane group lk (lane / 16) are k = 16lk..16lk+15 and 64+16lk..64+16lk+15
//    of the 128-k step, and the B fragments read the same k-rows in the same
//    byte order (any k order shared by A and B gives the same dot products).
//    With k = 32lk..32lk+31 instead, every A read was a 2-way bank conflict
//    (SQ_LDS_BANK_CONFLICT a third of the LDS active cycles); this order is
//    the W8A8 path's and reads conflict-free.
//  * B fragments are read already transposed with ds_read_b64_tr_b8: in each
//    16-lane group, lanes (2j, 2j+1) address the two 8-byte halves of k-row j
//    of a 16-column block and lane i receives column i of those 8 rows, i.e.
//    8 consecutive k of one column, the MFMA operand order.
//  * fp8 (block_k == 128): each 16x16x128 MFMA is one whole scale block, so the
//    partial is promoted at once: O = fma(P, a_s * b_s, O). The two scale
//    vectors of a step are also fetched straight into LDS.
// ===========================================================================
constexpr int kFThreads = 512;
constexpr int kFBM = 256, kFBN = 256;
constexpr int kFARow = 128;  // bytes per A row in LDS
constexpr int kFBRow = 256;  // bytes per B k-row in LDS

typedef int i32x2 __attribute__((ext_vector_type(2)));

// LDS chunk swizzles (gfx950 LDS: 64 banks x 4 B, so 256 bytes per bank cycle).
// A rows are 128 B: rows r and r+2 share a bank range, so the 16 rows of a
// 16-lane fragment read (r = 0..15) get distinct chunks from (r >> 1) & 7.
// B k-rows are 256 B (every row starts at bank 0): the 8 rows of one transposed
// read get distinct chunks from r & 7, and bit 3 of the chunk flips between the
// two 16-lane groups that read in the same cycle (rows 32 apart for fp8, 16
// apart for int8).
__device__ inline int a_swz(int row) { return (row >> 1) & 7; }
__device__ inline int b_swz(int row) { return (row & 7) | ((((row >> 4) ^ (row >> 5)) & 1) << 3); }
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

// LDS buffers of the fast kernel per tile height (see gemm8_fast_kernel).
constexpr int fast_nb(int bm) { return bm <= 128 ? 3 : 2; }

// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// SPLIT: workgroup id = tile * p.splits + split; the split runs K steps
// [split * per, min(steps, (split + 1) * per)) and writes its raw accumulators
// (fp8 blockwise: the promoted O; plain fp8: the fp32 sum; int8: int32) to the
// partial plane p.ws, which skinny::skinny_reduce_kernel sums in split order
// before the epilogue.
template <int KIND, typename Out, bool UNIFORM_BS, bool SPLIT, int BM>
__global__ void __launch_bounds__(kFThreads)
gemm8_fast_kernel(Args p) {
  // BM = 256, 128 or 64 rows per tile: each wave owns BM/2 rows = kRB 16-row
  // blocks and issues kAL of the tile's 1 KB A copies per K step. NB LDS
  // buffers: tiles of <= 128 rows leave room for three, so two steps of copies are in
  // flight (their splits run few steps, each bound by the copy round trip).
  constexpr int kRB = BM / 32, kAL = BM / 64, NB = fast_nb(BM);
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* sA = smem;                                    // [NB][BM][128]
  uint8_t* sB = smem + NB * BM * kFARow;                 // [NB][128][256]
  float* sAs = reinterpret_cast<float*>(sB + NB * kBK * kFBRow);  // [NB][256]
  float* sBs = sAs + NB * kFBM;                                    // [NB][256]

  const int tiles_m = static_cast<int>((p.m + BM - 1) / BM);
  const int tiles_n = static_cast<int>(p.n / kFBN);
  int tm, tn;
  int bid = blockIdx.x, split = 0;
  if constexpr (SPLIT) {
    split = bid % p.splits;
    bid /= p.splits;
  }
  tile_coords(bid, tiles_m, tiles_n, &tm, &tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * kFBN;

  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int wm = (wave / 4) * (BM / 2);
  const int wn = (wave % 4) * 64;
  const int li = lane % 16, lk = lane / 16;
  constexpr bool kFp8 = is_fp8_block(KIND);
  constexpr bool kPlain = is_fp8_plain(KIND);
  constexpr int kL = kAL + 4 + (kFp8 ? 1 : 0);  // copies per wave per K step

  // ---- per-lane global offsets of the direct-to-LDS loads (32-bit, checked
  // on the host). A: wave instruction i fills rows 8*(kAL*wave+i)..+7 (rows
  // past M are clamped, never stored). B: wave instruction i fills k-rows
  // 4*(4*wave+i)..+3 from a wave-uniform base; the lane's chunk swizzle
  // depends on i only through its parity, so two per-lane offsets serve all
  // four.
  uint32_t a_off[kAL];
#pragma unroll
  for (int i = 0; i < kAL; ++i) {
    const int row = 8 * (kAL * wave + i) + lane / 8;
    const int64_t gm = min<int64_t>(m0 + row, p.m - 1);
    a_off[i] = static_cast<uint32_t>(gm * p.k + 16 * ((lane % 8) ^ a_swz(row)));
  }
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint8_t* b_sb = p.b + static_cast<int64_t>(16 * wave_u) * p.n + n0;
  uint32_t b_v[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int krow = 4 * (4 * wave + e) + lane / 16;
    b_v[e] = static_cast<uint32_t>((lane / 16) * p.n + 16 * ((lane % 16) ^ b_swz(krow)));
  }
  const uint32_t n32 = static_cast<uint32_t>(p.n);
  // scales: waves 0-3 fetch a_scale of rows 64*wave+lane, waves 4-7 b_scale
  const int s_idx = 64 * (wave % 4) + lane;
  const float* s_src = nullptr;
  int64_t s_step = 0;  // per K block
  if constexpr (kFp8) {
    s_src = (wave < 4) ? p.a_scale + min<int64_t>(m0 + s_idx, p.m - 1) * p.nkb
                       : p.b_scale + (n0 + s_idx) / p.block_n;
    s_step = (wave < 4) ? 1 : p.nnb;
  }

  // Copy q (0 <= q < kL) of K step `step` into LDS buffer `buf`: the kAL A
  // copies, then the four B copies, then (fp8 blockwise) the scale vector.
  auto issue_one = [&](int q, int step, int buf) {
    const uint32_t k0 = static_cast<uint32_t>(step * kBK);
    if (q < kAL) {
      uint8_t* a_dst = sA + buf * BM * kFARow + (kAL * wave_u) * 8 * kFARow;
      dma_to_lds_off<16>(p.a, a_off[q] + k0, a_dst + q * 8 * kFARow);
    } else if (q < kAL + 4) {
      const int i = q - kAL;
      uint8_t* b_dst = sB + buf * kBK * kFBRow + (4 * wave_u) * 4 * kFBRow;
      dma_to_lds_off<16>(b_sb + i * 4 * p.n, b_v[i & 1] + k0 * n32, b_dst + i * 4 * kFBRow);
    } else if constexpr (kFp8) {  // block_k == 128: K step `step` is scale block `step`
      float* s_dst = (wave_u < 4) ? sAs + buf * kFBM + 64 * wave_u : sBs + buf * kFBN + 64 * (wave_u - 4);
      dma_to_lds<4>(s_src + step * s_step, s_dst);
    }
  };
  auto issue_loads = [&](int step, int buf) {
#pragma unroll
    for (int q = 0; q < kL; ++q) issue_one(q, step, buf);
  };
  // In the main loop the copies of step s+NB-1 are issued kDmaPer at a time
  // at the head of the first row blocks, after the step's B-fragment reads:
  // issuing all of them at the step start stalled every wave on the copy
  // queue before its first MFMA (fp8 blockwise M=2048 N=K=7168: 141-146 ->
  // 124-127 us). The kinds without promotion spread them thinner (three per
  // row block: plain fp8 at that shape 105.5 -> 101.0 us, W8A8 4096^3
  // 69.2 -> 68.6 us; the blockwise kind is slower at three).
  constexpr int kDmaPer = kFp8 ? 5 : 3;
  static_assert(kDmaPer * kRB >= kL, "every copy gets a row block");

  f32x4 acc_o[kRB][4];
  i32x4 acc_i[kRB][4];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc_o[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc_i[i][j] = i32x4{0, 0, 0, 0};
    }

  // B transposed-read addressing: lane (2*jj + h) of its 16-lane group reads
  // k-row (kbase + jj), bytes 8h..8h+7 of the 16-column block.
  const int tr_jj = li >> 1, tr_h = li & 1;
  // Every transposed read of a step is at k-row 16*lk + c + tr_jj for a
  // constant c in {0, 8, 64, 72}, and b_swz gives the same chunk for all four
  // (row & 7 == tr_jj, and bit 3 depends only on lk), so the lane's byte
  // offset within a buffer is b_lane[j] + c * kFBRow: fixed per lane for the
  // whole K loop, with c folded into the reads' immediate offsets.
  uint32_t b_lane[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row0 = 16 * lk + tr_jj;
    b_lane[j] = static_cast<uint32_t>(row0 * kFBRow +
                                      ((((wn + 16 * j) >> 4) ^ b_swz(row0)) * 16) + 8 * tr_h);
  }

  // fp8: the last two partials of a step are promoted at the start of the next.
  f32x4 plast[2], sclast;
  float bslast[4];
  auto promote16 = [](f32x4& o, const f32x4& part, const f32x4& sc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = fmaf(part[r], sc[r], o[r]);
  };

  int s_begin = 0, steps = static_cast<int>(p.k / kBK);
  if constexpr (SPLIT) {
    const int per = (steps + p.splits - 1) / p.splits;
    s_begin = split * per;
    steps = min(steps, s_begin + per);
  }
  for (int j = 0; j < NB - 1 && s_begin + j < steps; ++j) issue_loads(s_begin + j, j);
  if (NB > 2 && s_begin + NB - 2 < steps) wait_vm<(NB - 2) * kL>();  // the first step landed
  else __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = s_begin; s < steps; ++s) {
    const int cur = (s - s_begin) % NB;
    const bool dma_now = s + NB - 1 < steps;
    const int dma_step = s + NB - 1, dma_buf = (cur + NB - 1) % NB;
    auto issue_group = [&](int i) {  // row block i's share of the step's copies
      if (dma_now) {
#pragma unroll
        for (int q = kDmaPer * i; q < kDmaPer * (i + 1); ++q)
          if (q < kL) issue_one(q, dma_step, dma_buf);
      }
    };
    const uint8_t* a_src = sA + cur * BM * kFARow;
    const uint8_t* b_src = sB + cur * kBK * kFBRow;

    // B fragment of n-block j: k rows 16*lk + c + (0..7) of columns wn+16j..+15
    auto b_tr8 = [&](int j, int c) -> i32x2 {
      const uint8_t* addr = b_src + b_lane[j] + c * kFBRow;
      return __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_i32x2*>(
          reinterpret_cast<uintptr_t>(addr)));
    };

    if constexpr (kFp8) {
      constexpr int fmt = fp8_fmt(KIND);
      // Explicit software pipeline over the step's 32 MFMAs t = 4*i + j (row
      // block i, column block j):
      //  * the A fragment and row scales of block i+1 are read before block
      //    i's MFMAs are issued;
      //  * partial t is promoted right after MFMA t+2 is issued, so the
      //    promotion never waits on an MFMA result and only three partials
      //    are live;
      //  * the step's last two partials are promoted at the start of the
      //    next step, under the latency of its B-fragment reads.
      // sched_barrier pins this order against the scheduler's reordering.
      // A fragment: the chunk swizzle of row wm + 16i + li is a_swz(li) for every i.
      const uint8_t* pa0 = a_src + (wm + li) * kFARow;
      const int ca0 = (lk ^ a_swz(li)) * 16, ca1 = ((4 + lk) ^ a_swz(li)) * 16;
      const float* sa0 = &sAs[cur * kFBM + wm + 4 * lk];
      uint4 xa[kRB][2];
      f32x4 scl[kRB];
      auto read_a = [&](int i) {
        xa[i][0] = *reinterpret_cast<const uint4*>(pa0 + i * 16 * kFARow + ca0);
        xa[i][1] = *reinterpret_cast<const uint4*>(pa0 + i * 16 * kFARow + ca1);
        scl[i] = *reinterpret_cast<const f32x4*>(sa0 + 16 * i);
      };
      read_a(0);
      i32x8 fb[4];
      float bs[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const i32x2 q0 = b_tr8(j, 0), q1 = b_tr8(j, 8);
        const i32x2 q2 = b_tr8(j, 64), q3 = b_tr8(j, 72);
        fb[j] = i32x8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
        bs[j] = sBs[cur * kFBN + wn + 16 * j + li];
      }
      if (s > s_begin) {
        promote16(acc_o[kRB - 1][2], plast[0], UNIFORM_BS ? sclast : sclast * bslast[2]);
        promote16(acc_o[kRB - 1][3], plast[1], UNIFORM_BS ? sclast : sclast * bslast[3]);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 part[4 * kRB];
      f32x4 sc[kRB];  // uniform b_scale: block scale; else the row scales
#pragma unroll
      for (int i = 0; i < kRB; ++i) {
        issue_group(i);
        if (i + 1 < kRB) read_a(i + 1);
        const i32x8 fa = i32x8{(int)xa[i][0].x, (int)xa[i][0].y, (int)xa[i][0].z, (int)xa[i][0].w,
                               (int)xa[i][1].x, (int)xa[i][1].y, (int)xa[i][1].z, (int)xa[i][1].w};
        sc[i] = UNIFORM_BS ? scl[i] * bs[0] : scl[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 4 * i + j;
          part[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              fa, fb[j], f32x4{0.f, 0.f, 0.f, 0.f}, fmt, fmt, 0, 127, 0, 127);
          __builtin_amdgcn_sched_barrier(0);
          if (t >= 2) {
            const int u = t - 2, ui = u / 4, uj = u % 4;
            promote16(acc_o[ui][uj], part[u], UNIFORM_BS ? sc[ui] : sc[ui] * bs[uj]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      plast[0] = part[4 * kRB - 2];
      plast[1] = part[4 * kRB - 1];
      sclast = sc[kRB - 1];
#pragma unroll
      for (int j = 0; j < 4; ++j) bslast[j] = bs[j];
    } else if constexpr (kPlain) {
      // Plain fp8: fp32 accumulation over all of K in the MFMA accumulator;
      // A fragments are read one row block ahead of their MFMAs.
      constexpr int fmt = fp8_fmt(KIND);
      const uint8_t* pa0 = a_src + (wm + li) * kFARow;
      const int ca0 = (lk ^ a_swz(li)) * 16, ca1 = ((4 + lk) ^ a_swz(li)) * 16;
      uint4 xa0 = *reinterpret_cast<const uint4*>(pa0 + ca0);
      uint4 xa1 = *reinterpret_cast<const uint4*>(pa0 + ca1);
      i32x8 fbp[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const i32x2 q0 = b_tr8(j, 0), q1 = b_tr8(j, 8);
        const i32x2 q2 = b_tr8(j, 64), q3 = b_tr8(j, 72);
        fbp[j] = i32x8{q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
      }
#pragma unroll
      for (int i = 0; i < kRB; ++i) {
        issue_group(i);
        const i32x8 fa = i32x8{(int)xa0.x, (int)xa0.y, (int)xa0.z, (int)xa0.w,
                               (int)xa1.x, (int)xa1.y, (int)xa1.z, (int)xa1.w};
        if (i + 1 < kRB) {
          xa0 = *reinterpret_cast<const uint4*>(pa0 + (i + 1) * 16 * kFARow + ca0);
          xa1 = *reinterpret_cast<const uint4*>(pa0 + (i + 1) * 16 * kFARow + ca1);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc_o[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              fa, fbp[j], acc_o[i][j], fmt, fmt, 0, 127, 0, 127);
      }
    } else {
      // A fragments are read one row block ahead of their MFMAs (the 16-row
      // fragment of row block i: row wm + 16i + li, swizzle a_swz(li)).
      auto read_a8 = [&](int h, int i) {
        const int row = wm + 16 * i + li;
        return *reinterpret_cast<const uint4*>(a_src + row * kFARow + ((4 * h + lk) ^ a_swz(li)) * 16);
      };
      uint4 xa = read_a8(0, 0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        i32x4 fb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const i32x2 q0 = b_tr8(j, 64 * h), q1 = b_tr8(j, 64 * h + 8);
          fb[j] = i32x4{q0[0], q0[1], q1[0], q1[1]};
        }
#pragma unroll
        for (int i = 0; i < kRB; ++i) {
          if (h == 0) issue_group(i);
          const i32x4 fa = i32x4{(int)xa.x, (int)xa.y, (int)xa.z, (int)xa.w};
          if (i + 1 < kRB) xa = read_a8(h, i + 1);
          else if (h == 0) xa = read_a8(1, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc_i[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa, fb[j], acc_i[i][j], 0, 0, 0);
        }
      }
    }
    // This wave's loads for step s+1 have landed (they were issued as inline
    // asm, so the compiler does not hold LDS reads of step s behind them).
    if (NB > 2 && s + NB - 1 < steps) wait_vm<(NB - 2) * kL>();
    else __builtin_amdgcn_s_waitcnt(0);
    barrier_no_wait();
  }

  if constexpr (kFp8) {
    promote16(acc_o[kRB - 1][2], plast[0], UNIFORM_BS ? sclast : sclast * bslast[2]);
    promote16(acc_o[kRB - 1][3], plast[1], UNIFORM_BS ? sclast : sclast * bslast[3]);
  }

  // ---- epilogue: lane holds rows wm+16i+4lk+r, column wn+16j+li ----
  if constexpr (SPLIT) {
    uint32_t* ws = static_cast<uint32_t*>(p.ws) + split * p.m * p.n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + wn + 16 * j + li;
#pragma unroll
      for (int i = 0; i < kRB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t gm = m0 + wm + 16 * i + 4 * lk + r;
          if (gm >= p.m) continue;
          if constexpr (KIND == INT8 || KIND == INT8_RAW)
            ws[gm * p.n + gn] = static_cast<uint32_t>(acc_i[i][j][r]);
          else
            ws[gm * p.n + gn] = __float_as_uint(acc_o[i][j][r]);
        }
    }
    return;
  }
  // 16-bit outputs: the tile is staged through LDS (the A/B buffers are free
  // after the last step's barrier) and written as whole 512-byte row segments
  // with 16-byte non-temporal stores, instead of 2-byte stores per lane
  // (fp8 blockwise config 3: ~4 us of a ~115 us call). Row stride 528 B: the
  // four rows one 2-byte LDS write touches land 16 banks apart.
  if constexpr (sizeof(typename Out::storage) == 2 && KIND != INT8_RAW) {
    constexpr int kRowB = 528;
    static_assert(BM * kRowB <= NB * (BM * kFARow + kBK * kFBRow + (kFBM + kFBN) * 4), "staging fits");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wn + 16 * j + li;
      const int64_t gn = n0 + col;
      float bsc = 0.f;
      if constexpr (KIND == INT8 || kPlain) bsc = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
#pragma unroll
      for (int i = 0; i < kRB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm + 16 * i + 4 * lk + r;
          const int64_t gm = min<int64_t>(m0 + row, p.m - 1);  // rows past M are never stored
          float v;
          if constexpr (kPlain) {
            const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
            v = __fmul_rn(__fmul_rn(acc_o[i][j][r], as), bsc);
          } else if constexpr (kFp8) {
            v = acc_o[i][j][r];
          } else {
            const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
            v = __fmul_rn(__fmul_rn(static_cast<float>(acc_i[i][j][r]), as), bsc);
            if (p.bias)
              v = __fadd_rn(v, elem<Out>::load(static_cast<const typename Out::storage*>(p.bias), gn));
          }
          *reinterpret_cast<uint16_t*>(smem + row * kRowB + 2 * col) = elem<Out>::from_f32(v);
        }
    }
    __syncthreads();
    uint16_t* outp = static_cast<uint16_t*>(p.out);
#pragma unroll 4
    for (int e = t; e < BM * 32; e += kFThreads) {
      const int row = e >> 5, ch = e & 31;
      const int64_t gm = m0 + row;
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + row * kRowB + 16 * ch);
      if (gm < p.m) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(outp + gm * p.n + n0 + 8 * ch));
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t gn = n0 + wn + 16 * j + li;
    float bsc = 0.f;
    if constexpr (KIND == INT8 || kPlain) bsc = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
#pragma unroll
    for (int i = 0; i < kRB; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t gm = m0 + wm + 16 * i + 4 * lk + r;
        if (gm >= p.m) continue;
        if constexpr (kPlain) {
          const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn,
                         __fmul_rn(__fmul_rn(acc_o[i][j][r], as), bsc));
        } else if constexpr (kFp8) {
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn, acc_o[i][j][r]);
        } else if constexpr (KIND == INT8_RAW) {
          static_cast<int32_t*>(p.out)[gm * p.n + gn] = acc_i[i][j][r];
        } else {
          const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
          float v = __fmul_rn(__fmul_rn(static_cast<float>(acc_i[i][j][r]), as), bsc);
          if (p.bias)
            v = __fadd_rn(v, elem<Out>::load(static_cast<const typename Out::storage*>(p.bias), gn));
          store_out<Out>(static_cast<typename Out::storage*>(p.out) + gm * p.n + gn, v);
        }
      }
  }
}

// LDS: A [NB][BM][128 B], B [NB][128][256 B], a_scale and b_scale [NB][256] fp32.
constexpr size_t fast_lds(int bm) {
  return fast_nb(bm) * (static_cast<size_t>(bm) * kFARow + kBK * kFBRow + (kFBM + kFBN) * sizeof(float));
}

// Any-shape fp8 blockwise fallback (one thread per output, reference order).
template <typename Dec, typename Out>
__global__ void __launch_bounds__(kThreads)
fp8_blockwise_simple_kernel(Args p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= p.m * p.n) return;
  const int64_t gm = idx / p.n, gn = idx % p.n;
  float out = 0.f;
  for (int64_t kb = 0; kb < p.nkb; ++kb) {
    const int64_t k0 = kb * p.block_k;
    const int64_t k1 = (k0 + p.block_k < p.k) ? k0 + p.block_k : p.k;
    float part = 0.f;
    for (int64_t kk = k0; kk < k1; ++kk)
      part = fmaf(Dec::dec(p.a[gm * p.k + kk]), Dec::dec(p.b[kk * p.n + gn]), part);
    out = fmaf(part, p.a_scale[gm * p.nkb + kb] * p.b_scale[kb * p.nnb + gn / p.block_n], out);
  }
  store_out<Out>(static_cast<typename Out::storage*>(p.out) + idx, out);
}

// Any-shape plain fp8 fallback: k-ascending fp32 fma, then (acc * a_s) * b_s
// (gemm_fp8.cu:120-157 order).
template <typename Dec, typename Out>
__global__ void __launch_bounds__(kThreads)
fp8_plain_simple_kernel(Args p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= p.m * p.n) return;
  const int64_t gm = idx / p.n, gn = idx % p.n;
  float acc = 0.f;
  for (int64_t kk = 0; kk < p.k; ++kk)
    acc = fmaf(Dec::dec(p.a[gm * p.k + kk]), Dec::dec(p.b[kk * p.n + gn]), acc);
  const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
  const float bs = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
  store_out<Out>(static_cast<typename Out::storage*>(p.out) + idx, __fmul_rn(__fmul_rn(acc, as), bs));
}

// Any-shape W8A8 fallback.
template <int KIND, typename Out>
__global__ void __launch_bounds__(kThreads)
w8a8_simple_kernel(Args p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= p.m * p.n) return;
  const int64_t gm = idx / p.n, gn = idx % p.n;
  const int8_t* a = reinterpret_cast<const int8_t*>(p.a);
  const int8_t* b = reinterpret_cast<const int8_t*>(p.b);
  int32_t acc = 0;
  for (int64_t kk = 0; kk < p.k; ++kk) acc += static_cast<int32_t>(a[gm * p.k + kk]) * b[kk * p.n + gn];
  if constexpr (KIND == INT8_RAW) {
    static_cast<int32_t*>(p.out)[idx] = acc;
  } else {
    const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
    const float bs = p.b_per_channel ? p.b_scale[gn] : p.b_scale[0];
    float v = __fmul_rn(__fmul_rn(static_cast<float>(acc), as), bs);
    if (p.bias) v = __fadd_rn(v, elem<Out>::load(static_cast<const typename Out::storage*>(p.bias), gn));
    store_out<Out>(static_cast<typename Out::storage*>(p.out) + idx, v);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline bool tiled_ok(const Args& p) {
  return p.k % 16 == 0 && p.n % 16 == 0 && aligned16(p.a) && aligned16(p.b) &&
         p.m < (int64_t{1} << 31) && p.n < (int64_t{1} << 31);
}

template <int KIND, typename Out>
void launch_tiled(const Args& p, hipStream_t s) {
  const int64_t tiles = ((p.m + kBM - 1) / kBM) * ((p.n + kBN - 1) / kBN);
  hipLaunchKernelGGL((gemm8_kernel<KIND, Out>), dim3(static_cast<unsigned>(tiles)),
                     dim3(kThreads), 0, s, p);
}

// The fast kernel covers shapes without K/N tails whose operands fit 32-bit
// byte offsets; everything else takes the general tiled kernel.
inline bool fast_ok(const Args& p) {
  return p.k % kBK == 0 && p.n % kFBN == 0 && p.m * p.k < (int64_t{1} << 31) &&
         p.k * p.n < (int64_t{1} << 31) && (reinterpret_cast<uintptr_t>(p.a) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(p.b) & 15u) == 0;
}

template <int KIND, typename Out, bool UBS, bool SPLIT, int BM>
void launch_fast_kernel(const Args& p, int64_t wgs, hipStream_t s) {
  constexpr size_t kLds = fast_lds(BM);
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm8_fast_kernel<KIND, Out, UBS, SPLIT, BM>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLds));
    return true;
  }();
  (void)configured;
  hipLaunchKernelGGL((gemm8_fast_kernel<KIND, Out, UBS, SPLIT, BM>), dim3(static_cast<unsigned>(wgs)),
                     dim3(kFThreads), kLds, s, p);
}

// Fewer tiles than CUs (M <= 512 at N = 7168): split K so tiles * splits
// fills the 256 CUs (one 130 KB-LDS workgroup each), at least two K steps
// per split; the splits' raw accumulators are summed in split order by
// skinny_reduce_kernel, which also applies the epilogue.
inline int fast_splits(const Args& p, int bm) {
  const int64_t tiles = ((p.m + bm - 1) / bm) * ((p.n + kFBN - 1) / kFBN);
  const int64_t steps = p.k / kBK;
  int64_t sp = std::min<int64_t>(256 / std::max<int64_t>(tiles, 1), steps / 2);
  if (sp <= 1 || (sp * p.m * p.n) >= (int64_t{1} << 31)) return 1;
  const int64_t per = (steps + sp - 1) / sp;
  return static_cast<int>((steps + per - 1) / per);  // every split gets >= 1 step
}

template <int KIND, typename Out, bool UBS, int BM>
ks_status_t launch_fast_impl(Args p, hipStream_t s) {
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + kFBN - 1) / kFBN);
  p.splits = fast_splits(p, BM);
  if (p.splits == 1) {
    launch_fast_kernel<KIND, Out, UBS, false, BM>(p, tiles, s);
    return KS_SUCCESS;
  }
  Scratch sc;
  ks_status_t st = get_scratch(s, static_cast<size_t>(p.splits) * p.m * p.n, 0, &sc, "gemm8 split-K");
  if (st != KS_SUCCESS) return st;
  p.ws = sc.partial;
  launch_fast_kernel<KIND, Out, UBS, true, BM>(p, tiles * p.splits, s);
  skinny::launch_reduce<KIND, Out>(p, s);
  return KS_SUCCESS;
}

// A wave's 64 columns share one b_scale entry when block_n is a multiple of 64
// (n0 and the wave offsets are multiples of 64).
// M <= 64 takes 64-row tiles and M <= 384 128-row tiles: a 256-row tile would
// spend up to three quarters of its MFMAs and A copies on clamped rows past M,
// and the smaller tiles' 3-deep ring suits the few K steps of their splits
// (fp8 blockwise N = K = 7168, M = 160/192/256: 36/37/41 -> 33.7/33.5/35.3 us;
// M = 384 56.9 -> 54.1 us; at M = 512, 57.8 against 60.1 us, and at M = 2048
// the 256-row tile is faster).
template <int KIND, typename Out>
ks_status_t launch_fast(const Args& p, hipStream_t s) {
  const bool ubs = (KIND == FP8_E4M3 || KIND == FP8_E5M2) && p.block_n % 64 == 0;
  if (p.m <= 64)
    return ubs ? launch_fast_impl<KIND, Out, true, 64>(p, s) : launch_fast_impl<KIND, Out, false, 64>(p, s);
  if (p.m <= 384)
    return ubs ? launch_fast_impl<KIND, Out, true, 128>(p, s) : launch_fast_impl<KIND, Out, false, 128>(p, s);
  return ubs ? launch_fast_impl<KIND, Out, true, 256>(p, s) : launch_fast_impl<KIND, Out, false, 256>(p, s);
}

inline unsigned simple_grid(const Args& p) {
  return static_cast<unsigned>((p.m * p.n + kThreads - 1) / kThreads);
}

// Decode shapes (M <= 8) take the skinny kernel: B streamed once, K split
// over enough workgroups to fill the chip, partials reduced in split order.
// From M = 9 the split-K 256x256 kernel is as fast: four row fragments need
// ~168 VGPRs, so a CU holds one 8-wave workgroup (half the bytes in flight of
// M <= 8) and the grid runs in 1.5 rounds (N = K = 7168: M = 9..16 21.6-23.6
// us skinny against 23.0 us split-K at M = 17).
inline bool skinny_ok(const Args& p) {
  return p.m <= skinny::kMaxM && p.n % 16 == 0 && p.k % skinny::kChunk == 0 &&
         p.m * p.k < (int64_t{1} << 31) && p.k * p.n < (int64_t{1} << 31) &&
         (p.k / skinny::kChunk) * p.m * p.n < (int64_t{1} << 31) &&
         (reinterpret_cast<uintptr_t>(p.a) & 15u) == 0 && (reinterpret_cast<uintptr_t>(p.b) & 15u) == 0;
}

template <int KIND, typename Out, int MB, int CH, typename In = void>
ks_status_t launch_skinny(Args p, hipStream_t s, const char* who) {
  constexpr bool kBlock = is_fp8_block(KIND);
  const int64_t tiles = (p.n + skinny::kTileN - 1) / skinny::kTileN;
  const int64_t kwg = static_cast<int64_t>(skinny::kWaves) * CH * skinny::kChunk;
  p.splits = static_cast<int>((p.k + kwg - 1) / kwg);
  Scratch sc;
  ks_status_t st = get_scratch(s, static_cast<size_t>(p.splits) * p.m * p.n, 0, &sc, who);
  if (st != KS_SUCCESS) return st;
  p.ws = sc.partial;
  const unsigned grid = static_cast<unsigned>(tiles * p.splits);
  if (kBlock && p.block_k % (CH * skinny::kChunk) == 0)
    hipLaunchKernelGGL((skinny::skinny_kernel<KIND, MB, CH, In, kBlock>), dim3(grid),
                       dim3(skinny::kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((skinny::skinny_kernel<KIND, MB, CH, In, false>), dim3(grid),
                       dim3(skinny::kThreads), 0, s, p);
  skinny::launch_reduce<KIND, Out>(p, s);
  return KS_SUCCESS;
}

// Chunks per wave: the most (4, 2, 1) that still gives >= 192 workgroups.
// Measured on MI355X (graph replay, N = K = 7168, fp8 blockwise): M = 1/4/8
// 13.7/13.6/15.1 us with 4 chunks against 13.9/14.2/18.0 with 2; at
// N = K = 4096 only one chunk per wave fills the chip.
template <int KIND, typename Out, int MB, typename In = void>
ks_status_t skinny_chunks(const Args& p, hipStream_t s, const char* who) {
  const int64_t tiles = (p.n + skinny::kTileN - 1) / skinny::kTileN;
  auto wgs = [&](int ch) {
    const int64_t kwg = int64_t{ch} * skinny::kWaves * skinny::kChunk;
    return tiles * ((p.k + kwg - 1) / kwg);
  };
  if (wgs(4) >= 192) return launch_skinny<KIND, Out, MB, 4, In>(p, s, who);
  if (wgs(2) >= 192) return launch_skinny<KIND, Out, MB, 2, In>(p, s, who);
  return launch_skinny<KIND, Out, MB, 1, In>(p, s, who);
}

template <int KIND, typename Out, typename In = void>
ks_status_t run_skinny(const Args& p, hipStream_t s, const char* who) {
  if (p.m <= 4) return skinny_chunks<KIND, Out, 1, In>(p, s, who);
  return skinny_chunks<KIND, Out, 2, In>(p, s, who);
}

// Fused quantize + blockwise GEMM at decode shapes: by output and input type.
template <int KIND, typename In>
ks_status_t run_fused_in(const Args& p, ks_dtype_t out_dtype, hipStream_t s, const char* who) {
  switch (out_dtype) {
    case KS_DTYPE_F32: return run_skinny<KIND, f32_t, In>(p, s, who);
    case KS_DTYPE_F16: return run_skinny<KIND, f16_t, In>(p, s, who);
    default: return run_skinny<KIND, bf16_t, In>(p, s, who);
  }
}

template <int KIND>
ks_status_t run_fused(const Args& p, ks_dtype_t a_dtype, ks_dtype_t out_dtype, hipStream_t s,
                      const char* who) {
  switch (a_dtype) {
    case KS_DTYPE_F32: return run_fused_in<KIND, f32_t>(p, out_dtype, s, who);
    case KS_DTYPE_F16: return run_fused_in<KIND, f16_t>(p, out_dtype, s, who);
    default: return run_fused_in<KIND, bf16_t>(p, out_dtype, s, who);
  }
}

template <int KIND>
ks_status_t run_skinny_out(const Args& p, ks_dtype_t out_dtype, hipStream_t s, const char* who) {
  switch (out_dtype) {
    case KS_DTYPE_F32: return run_skinny<KIND, f32_t>(p, s, who);
    case KS_DTYPE_F16: return run_skinny<KIND, f16_t>(p, s, who);
    default: return run_skinny<KIND, bf16_t>(p, s, who);
  }
}

template <typename Out>
ks_status_t run_fp8(const Args& p, ks_dtype_t fp8, hipStream_t s) {
  const bool tiled = tiled_ok(p) && p.block_k % kBK == 0;
  const bool fast = tiled && p.block_k == kBK && fast_ok(p);
  if (fp8 == KS_DTYPE_F8E4M3) {
    if (fast) return launch_fast<FP8_E4M3, Out>(p, s);
    else if (tiled) launch_tiled<FP8_E4M3, Out>(p, s);
    else hipLaunchKernelGGL((fp8_blockwise_simple_kernel<e4m3_t, Out>), dim3(simple_grid(p)), dim3(kThreads), 0, s, p);
  } else {
    if (fast) return launch_fast<FP8_E5M2, Out>(p, s);
    else if (tiled) launch_tiled<FP8_E5M2, Out>(p, s);
    else hipLaunchKernelGGL((fp8_blockwise_simple_kernel<e5m2_t, Out>), dim3(simple_grid(p)), dim3(kThreads), 0, s, p);
  }
  return KS_SUCCESS;
}

template <typename Out>
ks_status_t run_fp8_plain(const Args& p, ks_dtype_t fp8, hipStream_t s) {
  const bool tiled = tiled_ok(p);
  const bool fast = tiled && fast_ok(p);
  if (fp8 == KS_DTYPE_F8E4M3) {
    if (fast) return launch_fast<FP8P_E4M3, Out>(p, s);
    else if (tiled) launch_tiled<FP8P_E4M3, Out>(p, s);
    else hipLaunchKernelGGL((fp8_plain_simple_kernel<e4m3_t, Out>), dim3(simple_grid(p)), dim3(kThreads), 0, s, p);
  } else {
    if (fast) return launch_fast<FP8P_E5M2, Out>(p, s);
    else if (tiled) launch_tiled<FP8P_E5M2, Out>(p, s);
    else hipLaunchKernelGGL((fp8_plain_simple_kernel<e5m2_t, Out>), dim3(simple_grid(p)), dim3(kThreads), 0, s, p);
  }
  return KS_SUCCESS;
}

template <int KIND, typename Out>
ks_status_t run_w8a8(const Args& p, hipStream_t s) {
  if (tiled_ok(p) && fast_ok(p)) return launch_fast<KIND, Out>(p, s);
  if (tiled_ok(p)) launch_tiled<KIND, Out>(p, s);
  else hipLaunchKernelGGL((w8a8_simple_kernel<KIND, Out>), dim3(simple_grid(p)), dim3(kThreads), 0, s, p);
  return KS_SUCCESS;
}

}  // namespace gemm8
}  // namespace ks

using namespace ks;
using namespace ks::gemm8;

namespace {
constexpr int64_t kI64Max = 9223372036854775807LL;
bool mul_overflows(int64_t a, int64_t b) { return a > kI64Max / b; }
constexpr int64_t kMaxTiles = 2147483647LL;
}  // namespace

extern "C" {

ks_status_t ks_gemm_fp8_blockwise(void* out, const void* a_fp8, const void* b_fp8,
                                  const float* a_scale, const float* b_scale, int64_t m,
                                  int64_t n, int64_t k, int block_n, int block_k,
                                  ks_dtype_t fp8_dtype, ks_dtype_t out_dtype,
                                  ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(a_fp8);
  KS_REQUIRE_PTR(b_fp8);
  KS_REQUIRE_PTR(a_scale);
  KS_REQUIRE_PTR(b_scale);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8_blockwise: bad shape");
  if (block_n <= 0 || block_k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8_blockwise: block_n/block_k must be > 0");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n))
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_fp8_blockwise: M*K / K*N / M*N exceeds int64 range");
  if (fp8_dtype != KS_DTYPE_F8E4M3 && fp8_dtype != KS_DTYPE_F8E5M2)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8_blockwise: fp8_dtype must be e4m3 or e5m2");
  if (out_dtype != KS_DTYPE_F32 && out_dtype != KS_DTYPE_F16 && out_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8_blockwise: out_dtype must be f32/f16/bf16");
  if (((m + kBM - 1) / kBM) > kMaxTiles / ((n + kBN - 1) / kBN) || m * n / kThreads >= kMaxTiles)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_fp8_blockwise: tile grid exceeds grid limits");
  Args p{};
  p.out = out;
  p.a = static_cast<const uint8_t*>(a_fp8);
  p.b = static_cast<const uint8_t*>(b_fp8);
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.m = m; p.n = n; p.k = k;
  p.block_n = block_n; p.block_k = block_k;
  p.nkb = (k + block_k - 1) / block_k;
  p.nnb = (n + block_n - 1) / block_n;
  auto s = to_stream(stream);
  if (skinny_ok(p) && block_k % skinny::kChunk == 0 && block_n % 16 == 0) {
    const ks_status_t st = fp8_dtype == KS_DTYPE_F8E4M3
        ? run_skinny_out<FP8_E4M3>(p, out_dtype, s, "ks_gemm_fp8_blockwise")
        : run_skinny_out<FP8_E5M2>(p, out_dtype, s, "ks_gemm_fp8_blockwise");
    if (st != KS_SUCCESS) return st;
    KS_LAUNCH_STATUS("ks_gemm_fp8_blockwise");
    return KS_SUCCESS;
  }
  ks_status_t st = KS_SUCCESS;
  switch (out_dtype) {
    case KS_DTYPE_F32: st = run_fp8<f32_t>(p, fp8_dtype, s); break;
    case KS_DTYPE_F16: st = run_fp8<f16_t>(p, fp8_dtype, s); break;
    default: st = run_fp8<bf16_t>(p, fp8_dtype, s); break;
  }
  if (st != KS_SUCCESS) return st;
  KS_LAUNCH_STATUS("ks_gemm_fp8_blockwise");
  return KS_SUCCESS;
}

ks_status_t ks_gemm_fp8_blockwise_fused_quant(void* out, const void* a, const void* b_fp8,
                                              const float* b_scale, int64_t m, int64_t n,
                                              int64_t k, int block_n, int block_k,
                                              ks_dtype_t a_dtype, ks_dtype_t fp8_dtype,
                                              ks_dtype_t out_dtype, ks_stream_t stream) {
  static const char* who = "ks_gemm_fp8_blockwise_fused_quant";
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(a);
  KS_REQUIRE_PTR(b_fp8);
  KS_REQUIRE_PTR(b_scale);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8_blockwise_fused_quant: bad shape");
  if (block_n <= 0 || block_k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8_blockwise_fused_quant: block_n/block_k must be > 0");
  if (a_dtype != KS_DTYPE_F32 && a_dtype != KS_DTYPE_F16 && a_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8_blockwise_fused_quant: a_dtype must be f32/f16/bf16");
  if (fp8_dtype != KS_DTYPE_F8E4M3 && fp8_dtype != KS_DTYPE_F8E5M2)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8_blockwise_fused_quant: fp8_dtype must be e4m3 or e5m2");
  if (out_dtype != KS_DTYPE_F32 && out_dtype != KS_DTYPE_F16 && out_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8_blockwise_fused_quant: out_dtype must be f32/f16/bf16");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n))
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_fp8_blockwise_fused_quant: M*K / K*N / M*N exceeds int64 range");
  Args p{};
  p.out = out;
  p.a_in = a;
  p.b = static_cast<const uint8_t*>(b_fp8);
  p.b_scale = b_scale;
  p.m = m; p.n = n; p.k = k;
  p.block_n = block_n; p.block_k = block_k;
  p.nkb = (k + block_k - 1) / block_k;
  p.nnb = (n + block_n - 1) / block_n;
  auto s = to_stream(stream);
  // One pass at decode shapes: the skinny kernel quantizes its own slice.
  // Its checks see the activation pointer as operand A (16-byte aligned rows).
  Args q = p;
  q.a = static_cast<const uint8_t*>(a);
  const bool gs_ok = block_k == 32 || block_k == 64 || block_k == 128 || block_k == 256;
  if (skinny_ok(q) && gs_ok && block_n % 16 == 0 && (reinterpret_cast<uintptr_t>(a) & 15u) == 0) {
    const ks_status_t st = fp8_dtype == KS_DTYPE_F8E4M3
        ? run_fused<FP8_E4M3>(p, a_dtype, out_dtype, s, who)
        : run_fused<FP8_E5M2>(p, a_dtype, out_dtype, s, who);
    if (st != KS_SUCCESS) return st;
    KS_LAUNCH_STATUS("ks_gemm_fp8_blockwise_fused_quant");
    return KS_SUCCESS;
  }
  // Otherwise the per-token-group quantizer writes codes and scales to library
  // staging and the blockwise GEMM reads them (same stream, so ordered).
  const size_t codes = static_cast<size_t>((m * k + 255) / 256 * 256);
  Scratch sc;
  ks_status_t st = get_scratch(s, 0, codes + static_cast<size_t>(m * p.nkb) * sizeof(float), &sc, who);
  if (st != KS_SUCCESS) return st;
  uint8_t* a8 = static_cast<uint8_t*>(sc.staging);
  float* a_s = reinterpret_cast<float*>(a8 + codes);
  st = ks_quantize_fp8_group(a8, a_s, a, m, k, block_k, a_dtype, fp8_dtype, stream);
  if (st != KS_SUCCESS) return st;
  return ks_gemm_fp8_blockwise(out, a8, b_fp8, a_s, b_scale, m, n, k, block_n, block_k, fp8_dtype,
                               out_dtype, stream);
}

ks_status_t ks_gemm_fp8(void* out, const void* a_fp8, const void* b_fp8, const float* a_scale,
                        const float* b_scale, int64_t m, int64_t n, int64_t k,
                        ks_quant_mode_t a_mode, ks_quant_mode_t b_mode, ks_dtype_t fp8_dtype,
                        ks_dtype_t out_dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(a_fp8);
  KS_REQUIRE_PTR(b_fp8);
  KS_REQUIRE_PTR(a_scale);
  KS_REQUIRE_PTR(b_scale);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8: bad shape");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n))
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_fp8: M*K / K*N / M*N exceeds int64 range");
  if (m * n / kThreads >= kMaxTiles)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_fp8: tile grid exceeds grid limits");
  if (a_mode != KS_QUANT_PER_TENSOR && a_mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8: a_mode must be per-tensor or per-token");
  if (b_mode != KS_QUANT_PER_TENSOR && b_mode != KS_QUANT_PER_CHANNEL)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_fp8: b_mode must be per-tensor or per-channel");
  if (fp8_dtype != KS_DTYPE_F8E4M3 && fp8_dtype != KS_DTYPE_F8E5M2)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8: fp8_dtype must be e4m3 or e5m2");
  if (out_dtype != KS_DTYPE_F32 && out_dtype != KS_DTYPE_F16 && out_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_fp8: out_dtype must be f32/f16/bf16");
  Args p{};
  p.out = out;
  p.a = static_cast<const uint8_t*>(a_fp8);
  p.b = static_cast<const uint8_t*>(b_fp8);
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.m = m; p.n = n; p.k = k;
  p.a_per_token = a_mode == KS_QUANT_PER_TOKEN;
  p.b_per_channel = b_mode == KS_QUANT_PER_CHANNEL;
  auto s = to_stream(stream);
  if (skinny_ok(p)) {
    const ks_status_t st = fp8_dtype == KS_DTYPE_F8E4M3
        ? run_skinny_out<FP8P_E4M3>(p, out_dtype, s, "ks_gemm_fp8")
        : run_skinny_out<FP8P_E5M2>(p, out_dtype, s, "ks_gemm_fp8");
    if (st != KS_SUCCESS) return st;
    KS_LAUNCH_STATUS("ks_gemm_fp8");
    return KS_SUCCESS;
  }
  ks_status_t st = KS_SUCCESS;
  switch (out_dtype) {
    case KS_DTYPE_F32: st = run_fp8_plain<f32_t>(p, fp8_dtype, s); break;
    case KS_DTYPE_F16: st = run_fp8_plain<f16_t>(p, fp8_dtype, s); break;
    default: st = run_fp8_plain<bf16_t>(p, fp8_dtype, s); break;
  }
  if (st != KS_SUCCESS) return st;
  KS_LAUNCH_STATUS("ks_gemm_fp8");
  return KS_SUCCESS;
}

ks_status_t ks_gemm_w8a8(void* c, const void* a_i8, const void* b_i8, const float* a_scale,
                         const float* b_scale, const void* bias, int64_t m, int64_t n,
                         int64_t k, ks_quant_mode_t a_mode, ks_quant_mode_t b_mode,
                         ks_dtype_t out_dtype, ks_stream_t stream) {
  KS_REQUIRE_PTR(c);
  KS_REQUIRE_PTR(a_i8);
  KS_REQUIRE_PTR(b_i8);
  KS_REQUIRE_PTR(a_scale);
  KS_REQUIRE_PTR(b_scale);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8: bad shape");
  if (a_mode != KS_QUANT_PER_TENSOR && a_mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8: a_mode must be per-tensor or per-token");
  if (b_mode != KS_QUANT_PER_TENSOR && b_mode != KS_QUANT_PER_CHANNEL)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8: b_mode must be per-tensor or per-channel");
  if (out_dtype != KS_DTYPE_F32 && out_dtype != KS_DTYPE_F16 && out_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_w8a8: out_dtype must be f32/f16/bf16");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n) || m * n / kThreads >= kMaxTiles)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w8a8: shape exceeds grid limits");
  if (k > 260000)  // 127*127*k must stay below 2^31 for exact int32 accumulation
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w8a8: K too large for exact int32 accumulation");
  Args p{};
  p.out = c;
  p.a = static_cast<const uint8_t*>(a_i8);
  p.b = static_cast<const uint8_t*>(b_i8);
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.bias = bias;
  p.m = m; p.n = n; p.k = k;
  p.a_per_token = a_mode == KS_QUANT_PER_TOKEN;
  p.b_per_channel = b_mode == KS_QUANT_PER_CHANNEL;
  auto s = to_stream(stream);
  if (skinny_ok(p)) {
    const ks_status_t st = run_skinny_out<INT8>(p, out_dtype, s, "ks_gemm_w8a8");
    if (st != KS_SUCCESS) return st;
    KS_LAUNCH_STATUS("ks_gemm_w8a8");
    return KS_SUCCESS;
  }
  ks_status_t st = KS_SUCCESS;
  switch (out_dtype) {
    case KS_DTYPE_F32: st = run_w8a8<INT8, f32_t>(p, s); break;
    case KS_DTYPE_F16: st = run_w8a8<INT8, f16_t>(p, s); break;
    default: st = run_w8a8<INT8, bf16_t>(p, s); break;
  }
  if (st != KS_SUCCESS) return st;
  KS_LAUNCH_STATUS("ks_gemm_w8a8");
  return KS_SUCCESS;
}

ks_status_t ks_gemm_w8a8_fused_quant(void* c, const void* a, const void* b_i8,
                                     const float* b_scale, const void* bias, int64_t m, int64_t n,
                                     int64_t k, ks_quant_mode_t a_mode, ks_quant_mode_t b_mode,
                                     ks_dtype_t a_dtype, ks_dtype_t out_dtype,
                                     ks_stream_t stream) {
  static const char* who = "ks_gemm_w8a8_fused_quant";
  KS_REQUIRE_PTR(c);
  KS_REQUIRE_PTR(a);
  KS_REQUIRE_PTR(b_i8);
  KS_REQUIRE_PTR(b_scale);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8_fused_quant: bad shape");
  if (a_mode != KS_QUANT_PER_TENSOR && a_mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8_fused_quant: a_mode must be per-tensor or per-token");
  if (b_mode != KS_QUANT_PER_TENSOR && b_mode != KS_QUANT_PER_CHANNEL)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_gemm_w8a8_fused_quant: b_mode must be per-tensor or per-channel");
  if (a_dtype != KS_DTYPE_F32 && a_dtype != KS_DTYPE_F16 && a_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_w8a8_fused_quant: a_dtype must be f32/f16/bf16");
  if (out_dtype != KS_DTYPE_F32 && out_dtype != KS_DTYPE_F16 && out_dtype != KS_DTYPE_BF16)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_gemm_w8a8_fused_quant: out_dtype must be f32/f16/bf16");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n) || m * n / kThreads >= kMaxTiles)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w8a8_fused_quant: shape exceeds grid limits");
  if (k > 260000)  // 127*127*k must stay below 2^31 for exact int32 accumulation
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_gemm_w8a8_fused_quant: K too large for exact int32 accumulation");
  auto s = to_stream(stream);
  const bool per_token = a_mode == KS_QUANT_PER_TOKEN;
  const size_t nscale = per_token ? static_cast<size_t>(m) : 1;
  Args p{};
  p.out = c;
  p.a = static_cast<const uint8_t*>(a);  // the skinny checks see the activations as operand A
  p.a_in = a;
  p.b = static_cast<const uint8_t*>(b_i8);
  p.b_scale = b_scale;
  p.bias = bias;
  p.m = m; p.n = n; p.k = k;
  p.a_per_token = per_token;
  p.b_per_channel = b_mode == KS_QUANT_PER_CHANNEL;
  // One pass for M <= 4: every workgroup reduces the row maxima itself and
  // quantizes its own K slice; workgroup 0 leaves the scales in library
  // staging for the split reduce's epilogue. Measured on MI355X (graph replay,
  // bf16 in/out, one pass vs quantize + GEMM): N = K = 4096 M = 1/4/8
  // 9.9/10.9/13.6 us vs 10.8/11.8/13.1 us; N = K = 7168 15.8/16.4/21.5 us vs
  // 16.5/17.6/19.5 us. Above M = 4 every workgroup's full-row pass costs more
  // than the separate quantizer, so those shapes stage.
  if (skinny_ok(p) && m <= 4) {
    Scratch sc;
    ks_status_t st = get_scratch(s, 0, nscale * sizeof(float), &sc, who);
    if (st != KS_SUCCESS) return st;
    p.a_scale_out = static_cast<float*>(sc.staging);
    p.a_scale = p.a_scale_out;
    st = run_fused<INT8>(p, a_dtype, out_dtype, s, who);
    if (st != KS_SUCCESS) return st;
    KS_LAUNCH_STATUS("ks_gemm_w8a8_fused_quant");
    return KS_SUCCESS;
  }
  // Otherwise the int8 quantizer writes codes and scales to library staging
  // and the W8A8 GEMM reads them (same stream, so ordered).
  const size_t codes = static_cast<size_t>((m * k + 255) / 256 * 256);
  Scratch sc;
  ks_status_t st = get_scratch(s, 0, codes + nscale * sizeof(float), &sc, who);
  if (st != KS_SUCCESS) return st;
  uint8_t* a8 = static_cast<uint8_t*>(sc.staging);
  float* a_s = reinterpret_cast<float*>(a8 + codes);
  st = ks_quantize_int8(a8, a_s, a, m, k, a_dtype, a_mode, stream);
  if (st != KS_SUCCESS) return st;
  return ks_gemm_w8a8(c, a8, b_i8, a_s, b_scale, bias, m, n, k, a_mode, b_mode, out_dtype, stream);
}

ks_status_t ks_testing_gemm_w8a8_i32(int32_t* acc, const void* a_i8, const void* b_i8,
                                     int64_t m, int64_t n, int64_t k, ks_stream_t stream) {
  KS_REQUIRE_PTR(acc);
  KS_REQUIRE_PTR(a_i8);
  KS_REQUIRE_PTR(b_i8);
  if (m <= 0 || n <= 0 || k <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_testing_gemm_w8a8_i32: bad shape");
  if (mul_overflows(m, k) || mul_overflows(k, n) || mul_overflows(m, n) || m * n / kThreads >= kMaxTiles)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_testing_gemm_w8a8_i32: shape exceeds grid limits");
  Args p{};
  p.out = acc;
  p.a = static_cast<const uint8_t*>(a_i8);
  p.b = static_cast<const uint8_t*>(b_i8);
  p.m = m; p.n = n; p.k = k;
  if (skinny_ok(p)) {
    const ks_status_t st = run_skinny<INT8_RAW, f32_t>(p, to_stream(stream), "ks_testing_gemm_w8a8_i32");
    if (st != KS_SUCCESS) return st;
  } else {
    const ks_status_t st = run_w8a8<INT8_RAW, f32_t>(p, to_stream(stream));
    if (st != KS_SUCCESS) return st;
  }
  KS_LAUNCH_STATUS("ks_testing_gemm_w8a8_i32");
  return KS_SUCCESS;
}

}  // extern "C"
