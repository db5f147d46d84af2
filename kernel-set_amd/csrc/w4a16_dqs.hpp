// kernel-set (MI355X build) -- W4A16 GEMM for larger M, 128x128 or 256x128
// tiles, with the waves split by role (warp specialization):
//
//  * waves 4-7 (producers, one per SIMD) copy the operands global -> LDS
//    through a kDepth-stage ring (direct copies, no VGPRs) and dequantize
//    the next stage's weights into the bf16/f16 tile Wd [128 n][64 k];
//  * waves 0-3 (consumers, one per SIMD) run the 32x32x16 MFMAs of a 64x64
//    (128-row tile) or 128x64 (256-row tile) output tile each on the current
//    stage's A and Wd.
//
// The two roles run separate loops that pass the same per-stage barriers, so
// the consumers' accumulators are not live across the producers' code (one
// shared loop held 174 VGPRs for the 128-row tile and spilled for the 256-row
// one; now 112 / 208, and the 128-row tile measured 5-10 % faster, e.g. M =
// 256 N = 14336 K = 4096 62 -> 56 us). The 256-row tile dequantizes each
// weight once for twice the rows; it serves M >= 384 when it alone fills 192
// workgroups (N = 14336 M = 512 / 1024: 106 / 201 -> 95 / 180 us); with a
// K split (M = 256) it was slower than the 128-row tile (63 against 56 us).
//
// Both roles work on different stages between the same per-stage barrier, so
// a stage costs max(copy + dequantize, MFMA) instead of their sum. Every
// producer copies the 8 packed rows it dequantizes and its own copy of the
// stage's scales and zeros, so it dequantizes after waiting for its own copies
// only (no barrier between copy and use); the A copies, spread over the four
// producers, are published to the consumers by the stage barrier.
//
// What bounds it (s_memtime stamps of one workgroup, M = 256, N = 14336,
// K = 4096: ~2140 cycles per 64-k stage): the producer chain -- issuing its 7
// copies ~670 cycles (the CU moves ~50 B/clk global -> LDS, and a stage is
// 22 KB), waiting ~160, dequantizing ~950 -- while the consumers' 16 MFMAs
// and fragment reads take ~1340 and they then wait ~700 at the barrier.
// Moving the A copies to the consumers (before or after their MFMAs) made the
// stage slower (2490 cycles): a copy issue waits on the CU's DMA rate
// whichever wave makes it. Fewer copied bytes per MFMA (a wider tile) is the
// remaining lever.
//
// Arithmetic is that of dq_kernel (w4a16_dq.hpp): w = fma(q, s, -z*s) rounded
// once to the activation dtype, fp32 MFMA accumulation over k in stage order,
// the same MFMA sequence per output element. Bit identity of the two kernels
// on one shape is not tested (the dispatch picks one per shape); each is
// checked against the oracle within the W4A16 tolerance. LDS swizzles: A rows by (row & 7), raw W rows by (row & 7), Wd columns
// by (n & 7) (16-byte chunks).
#pragma once

#include "w4a16_dq.hpp"

namespace ks {
namespace w4dqs {

using w4dq::kStageK;
using w4dq::dq_traits;
using w4dq::f32x16;
using w4dq::i32x2;
using w4dq::lds_i32x2;
using w4dq::wait_lgkm0;
using w4dq::wait_vmcnt;

constexpr int kBN = 128;
constexpr int kThreads = 512;
constexpr int kWBytes = (kStageK / 2) * kBN;    // raw packed rows of a stage: 4 KB
constexpr int kSzBytes = 2 * kBN * 2;           // one producer's scales + zeros
constexpr int kWdBytes = kBN * kStageK * 2;     // Wd [128 n][64 k]: 16 KB

// Tile height BM = 128 or 256 rows (256: each consumer wave owns 128 x 64 and
// the tile copies half the activation bytes per MFMA of the 128-row tile).
template <int BM>
struct Geo {
  static constexpr int kABytes = BM * kStageK * 2;     // A [BM rows][64 k]: 16 / 32 KB
  static constexpr int kSlot = kABytes + kWBytes + 4 * kSzBytes;
  static constexpr int kDepth = BM == 128 ? 4 : 3;  // 4 x 21.5 / 3 x 37.5 KB + Wd
  static constexpr int kBytes = kSlot * kDepth + 2 * kWdBytes;
  static constexpr int kACopies = BM / 32;             // A copies per producer per stage
  static constexpr int kLoads = kACopies + 1 + 2;      // copies per producer per stage
  static constexpr int kRB = BM / 64;                  // 32-row MFMA blocks per consumer
  static_assert(kBytes <= 160 * 1024, "LDS");
};

// Rows [m0, m0+BM) (clamped reads at row_end-1, outputs past row_end dropped)
// x columns [n0, n0+128), K stages [st0, st0 + sps) of grid z. Requires
// K % 64 == 0, gs % 64 == 0, N % 128 == 0, 16-byte aligned a and b, 4-byte
// aligned scales and zeros; sps a multiple of gs / 64.
template <typename T, int BM>
__global__ void __launch_bounds__(kThreads)
dqs_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
           const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
           const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
           int64_t row_end, int64_t n, int64_t k, int gs, int sps, float* __restrict__ ws) {
  using G = Geo<BM>;
  constexpr int D = G::kDepth, kSlot = G::kSlot, kABytes = G::kABytes, kLoads = G::kLoads;
  constexpr int kAC = G::kACopies, kRB = G::kRB;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* ring = smem;
  uint8_t* wd = smem + kSlot * D;  // [2][128 n][128 B]

  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kBN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const bool producer = wave >= 4;
  const int st0 = static_cast<int>(blockIdx.z) * sps;
  const int nst = min(static_cast<int>(k / kStageK) - st0, sps);
  const int spg = gs / kStageK;  // stages per quantization group

  // ---- producer state (wave p = wave - 4) ----
  const int p = wave & 3;
  const uint16_t* a_cur[kAC];
#pragma unroll
  for (int i = 0; i < kAC; ++i) {  // A copy kAC*p + i: rows 8(kAC*p+i) .. +7, one 128-B row per 8 lanes
    const int row = 8 * (kAC * p + i) + lane / 8;
    const int cc = (lane % 8) ^ (row & 7);
    const int64_t gr = min<int64_t>(m0 + row, row_end - 1);
    a_cur[i] = a + gr * k + static_cast<int64_t>(st0) * kStageK + 8 * cc;
  }
  const int w_row = 8 * p + lane / 8;  // this producer's packed rows 8p .. 8p+7
  const int w_c = (lane % 8) ^ (w_row & 7);
  const uint8_t* w_cur = b + (static_cast<int64_t>(st0) * (kStageK / 2) + w_row) * n + n0 + 16 * w_c;
  const int64_t g0 = st0 / spg;
  const uint16_t* s_cur = scales + g0 * n + n0 + 2 * lane;
  const uint16_t* z_cur = (zeros ? zeros : scales) + g0 * n + n0 + 2 * lane;
  int sz_left = spg;
  int is_slot = 0;
  auto issue = [&]() {
    uint8_t* slot = ring + is_slot * kSlot;
#pragma unroll
    for (int i = 0; i < kAC; ++i) {
      dma_to_lds<16>(a_cur[i], slot + 1024 * (kAC * p + i));
      a_cur[i] += kStageK;
    }
    dma_to_lds<16>(w_cur, slot + kABytes + 1024 * p);
    w_cur += (kStageK / 2) * n;
    uint8_t* szd = slot + kABytes + kWBytes + kSzBytes * p;
    dma_to_lds<4>(s_cur, szd);
    dma_to_lds<4>(z_cur, szd + 2 * kBN);
    if (--sz_left == 0) {
      sz_left = spg;
      s_cur += n;
      z_cur += n;
    }
    is_slot = (is_slot + 1 == D) ? 0 : is_slot + 1;
  };
  // Dequantize packed rows 8p .. 8p+7 (k 16p .. 16p+15) of columns lane and
  // 64 + lane: ds_read_b64_tr_b8 gives lane i of each 16-lane group column i
  // of the 8 rows (lanes 2j, 2j+1 address the two halves of row j).
  const bool has_z = zeros != nullptr;
  const int tr_row = 8 * p + ((lane % 16) >> 1);
  auto dequant = [&](const uint8_t* slot, uint8_t* wd_buf) {
    const uint16_t* szl = reinterpret_cast<const uint16_t*>(slot + kABytes + kWBytes + kSzBytes * p);
    i32x2 d[2];
    uint16_t sr[2], zr[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int dn = 64 * h + lane;
      const int src = tr_row * kBN + (((dn / 16) ^ (tr_row & 7)) * 16) + 8 * (lane & 1);
      d[h] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(slot + kABytes + src)));
      sr[h] = szl[dn];
      zr[h] = szl[kBN + dn];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int dn = 64 * h + lane;
      const float s = elem<T>::to_f32(sr[h]);
      const float z = has_z ? elem<T>::to_f32(zr[h]) : 0.f;
      const float zs = s * z;  // exact: at most 2 x 11 significant bits
      uint32_t o[8];
      w4dq::dequant_dword<T>(static_cast<uint32_t>(d[h][0]), s, -zs, o);
      w4dq::dequant_dword<T>(static_cast<uint32_t>(d[h][1]), s, -zs, o + 4);
      uint8_t* dst = wd_buf + dn * 128;
      *reinterpret_cast<uint4*>(dst + ((2 * p) ^ (dn & 7)) * 16) = make_uint4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<uint4*>(dst + ((2 * p + 1) ^ (dn & 7)) * 16) = make_uint4(o[4], o[5], o[6], o[7]);
    }
  };

  if (producer) {
    // The producers' loop is separate from the consumers', so the
    // accumulators are not live across the dequantization (both loops pass
    // the same barriers, one per stage).
#pragma unroll 1
    for (int i = 0; i < D - 1 && i < nst; ++i) issue();
    if (nst >= D - 1) wait_vmcnt<(D - 2) * kLoads>();
    else wait_vmcnt<0>();
    dequant(ring, wd);
    wait_lgkm0();
    barrier_no_wait();  // stage 0: A landed, Wd[0] written
#pragma unroll 1
    for (int st = 0; st < nst; ++st) {
      // Slot (st + D - 1) % D held stage st - 1, which the consumers finished
      // before the last barrier; Wd[(st + 1) & 1] likewise.
      const bool more = st + D - 1 < nst;
      if (more) issue();
      if (st + 1 < nst) {
        if (more) wait_vmcnt<(D - 2) * kLoads>();  // stage st + 1 landed (own copies)
        else wait_vmcnt<0>();
        const int nx = (st + 1) % D;
        dequant(ring + nx * kSlot, wd + ((st + 1) & 1) * kWdBytes);
        wait_lgkm0();
      }
      barrier_no_wait();  // stage st consumed; stage st + 1's A and Wd published
    }
    return;
  }

  // ---- consumer state: wave (wr, wc) -> rows BM/2 wr .., columns 64 wc .. ----
  const int cm = (wave >> 1) * (BM / 2), cn = (wave & 1) * 64;
  const int l32 = lane % 32, lh = lane / 32;
  f32x16 acc[kRB][2];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  barrier_no_wait();  // stage 0 published

#pragma unroll 1
  for (int st = 0; st < nst; ++st) {
    const uint8_t* as = ring + (st % D) * kSlot;
    const uint8_t* bs = wd + (st & 1) * kWdBytes;
#pragma unroll
    for (int ks = 0; ks < kStageK / 16; ++ks) {
      const int chunk = 2 * ks + lh;  // 8 k per lane: k = 16ks + 8lh .. +7
      uint4 af[kRB], bf[2];
#pragma unroll
      for (int i = 0; i < kRB; ++i) {
        const int am = cm + 32 * i + l32;
        af[i] = *reinterpret_cast<const uint4*>(as + am * 128 + ((chunk ^ (am & 7)) * 16));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int bn = cn + 32 * i + l32;
        bf[i] = *reinterpret_cast<const uint4*>(bs + bn * 128 + ((chunk ^ (bn & 7)) * 16));
      }
#pragma unroll
      for (int i = 0; i < kRB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = dq_traits<T>::mma(af[i], bf[j], acc[i][j]);
    }
    barrier_no_wait();  // stage st consumed; stage st + 1's A and Wd published
  }

  // ---- epilogue: acc[i][j][r] -> row 8*(r/4) + 4*lh + r%4 of 32x32 tile (i, j) ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + cn + 32 * j + l32;
    const float bv = (bias && !ws) ? elem<T>::to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < kRB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + cm + 32 * i + 8 * (r / 4) + 4 * lh + (r % 4);
        if (row >= row_end) continue;
        if (ws)  // split partial, summed (with the bias) by the reduce kernel
          ws[(static_cast<int64_t>(blockIdx.z) * row_end + row) * n + col] = acc[i][j][r];
        else
          c[row * n + col] = elem<T>::from_f32(acc[i][j][r] + bv);
      }
  }
}

}  // namespace w4dqs
}  // namespace ks
