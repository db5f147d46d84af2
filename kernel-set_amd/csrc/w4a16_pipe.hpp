// kernel-set (MI355X build) -- W4A16 batched tile with an LDS load ring, shared
// by the dense GEMM (ks_gemm_w4a16, M > 8) and the MoE grouped GEMM.
//
// Why a ring: at these sizes the kernel is HBM-bound (M <= 64) and a workgroup
// has only a few MFMAs per 64-k step, so a one-step prefetch leaves the HBM
// latency (~2 us under load) exposed every step. Here every operand moves
// global -> LDS directly (global_load_lds, no VGPRs held), D stages deep, so
// ~(D-1) x 5-13 KB per workgroup and two workgroups per CU are in flight.
//
// Tile: 16*MB rows x 128 columns, 4 waves side by side over N (32 columns,
// two 16-column MFMA blocks each); one stage = 64 k = 32 packed rows.
// Per stage and ring slot (all 16-byte chunks XOR-swizzled by row & 7):
//   W  [32 packed rows][128 B]     raw int4 pairs, one 128-byte line per row
//   A  [16*MB rows][64 bf16/f16]   activations
//   SZ [4][64 x 4 B]               scales (wave 0 slot), zeros (wave 1 slot)
// B fragments are read already transposed with ds_read_b64_tr_b8: lane li of
// 16-lane group q receives column li's bytes of packed rows 8q..8q+7, i.e.
// codes k = 16q..16q+15. Each dword (8 codes) becomes an MFMA B fragment with
// one and-or per pair: 0x4300|q is bf16 128+q (f16 0x5800|q = 128+q/8), pairs
// ordered (0,4),(1,5),(2,6),(3,7); the activation fragment uses that order.
// Per quantization group the MFMAs accumulate P = A*(128+q) and S = A*1, then
//   O += s * (P - (128 + z) * S)   (f16: the code axis is scaled by 1/8),
// which is sum_k a*(q - z)*s over the group in fp32.
#pragma once

#include "ks_common.hpp"
#include "w4a16_mfma.hpp"

namespace ks {
namespace w4pipe {

using w4mma::f32x4;
using w4mma::u32x4v;

constexpr int kThreads = 256;
constexpr int kTileN = 128;
constexpr int kStageK = 64;          // k per stage
constexpr int kStageRows = 32;       // packed rows per stage
constexpr int kWBytes = kStageRows * 128;
constexpr int kSZBytes = 4 * 256;

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

template <int MB>
struct Ring {
  static constexpr int kABytes = 16 * MB * 128;
  static constexpr int kSlot = kWBytes + kABytes + kSZBytes;
  static constexpr int kDepth = MB >= 4 ? 6 : 8;
  static constexpr int kBytes = kSlot * kDepth;
  // global_load_lds instructions per thread per stage (identical in every wave)
  static constexpr int kLoads = 1 + (MB == 1 ? 2 : MB / 2) + 1;
};

// s_waitcnt vmcnt(N) only (expcnt / lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

struct PipeArgs {
  const uint16_t* a;   // activations, row-major [*, K]
  const uint8_t* b;    // packed weights [K/2, N]
  const uint16_t* s;   // scales [K/gs, N]
  const uint16_t* z;   // zeros [K/gs, N] or null
  int64_t n, k;
  int gs;
  int64_t n0;          // first column of the tile (n0 % 128 == 0)
};

// Computes O[mb][j][r] = sum over stages [st0, st1) for rows r0 + 16*mb + 4*q + r
// (rows >= r_end read row r_end - 1 and must not be stored) and columns
// n0 + 32*wave + 16*j + li. Requires K % 64 == 0, gs % 64 == 0, N % 16 == 0 and
// 16-byte aligned a / b. All threads of the workgroup must call it.
template <typename T, int MB>
__device__ inline void pipe_tile(const PipeArgs& p, int64_t r0, int64_t r_end, int st0, int st1,
                                 uint8_t* smem, f32x4 (&O)[MB][2]) {
  using R = Ring<MB>;
  constexpr int D = R::kDepth;
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int li = lane % 16, q = lane / 16;
  const int64_t n = p.n, k = p.k;
  const int64_t last_chunk = n / 16 - 1;  // last valid 16-column chunk

#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j) O[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nst = st1 - st0;
  if (nst <= 0) return;

  // ---- per-lane global sources of the ring loads (stage-invariant parts) ----
  // W: wave instruction fills rows 8*wave..8*wave+7; lane -> (row, physical chunk).
  const int w_row = 8 * wave + lane / 8;
  const int w_c = (lane % 8) ^ (w_row & 7);
  const int64_t w_col = min<int64_t>(p.n0 / 16 + w_c, last_chunk) * 16;
  const uint8_t* w_src = p.b + static_cast<int64_t>(w_row) * n + w_col;
  // A: MB == 1 uses two 4-byte loads per lane (2 rows per instruction),
  // otherwise MB/2 16-byte loads (8 rows per instruction).
  constexpr int kALd = MB == 1 ? 2 : MB / 2;
  const uint16_t* a_src[kALd];
#pragma unroll
  for (int i = 0; i < kALd; ++i) {
    int row, c, word;
    if (MB == 1) {
      row = 2 * (2 * wave + i) + lane / 32;
      c = ((lane % 32) / 4) ^ (row & 7);
      word = lane % 4;
    } else {
      row = 8 * (wave * kALd + i) + lane / 8;
      c = (lane % 8) ^ (row & 7);
      word = 0;
    }
    const int64_t gr = min<int64_t>(r0 + row, r_end - 1);
    a_src[i] = p.a + gr * k + 8 * c + 2 * word;
  }
  // SZ: wave 0 scales, wave 1 zeros (scales again when zeros are absent),
  // waves 2-3 scales into unused slots so every wave issues the same loads.
  const uint16_t* sz_base = (wave == 1 && p.z) ? p.z : p.s;
  const int64_t sz_col = min<int64_t>(p.n0 + 2 * lane, n - 2);

  auto issue = [&](int st) {
    uint8_t* slot = smem + (st % D) * R::kSlot;
    const int64_t kk = static_cast<int64_t>(st) * kStageK;
    dma_to_lds<16>(w_src + (kk / 2) * n, slot + 1024 * wave);
    uint8_t* a_dst = slot + kWBytes;
#pragma unroll
    for (int i = 0; i < kALd; ++i) {
      if (MB == 1)
        dma_to_lds<4>(a_src[i] + kk, a_dst + 256 * (2 * wave + i));
      else
        dma_to_lds<16>(a_src[i] + kk, a_dst + 1024 * (wave * kALd + i));
    }
    const int64_t g = kk / p.gs;
    dma_to_lds<4>(sz_base + g * n + sz_col, slot + kWBytes + R::kABytes + 256 * wave);
  };

  const u32x4v ones = {w4mma::mfma_traits<T>::one2, w4mma::mfma_traits<T>::one2,
                       w4mma::mfma_traits<T>::one2, w4mma::mfma_traits<T>::one2};
  constexpr float unit = w4mma::code_scale<T>::unit;
  constexpr float inv_unit = 1.0f / unit;
  const int stages_per_group = p.gs / kStageK;
  const bool has_z = p.z != nullptr;

  // tr8 source: lane (2*jj + h) of group q addresses half h of packed row 8q+jj.
  const int tr_row = 8 * q + (li >> 1);
  const int tr_half = 8 * (li & 1);

#pragma unroll 1
  for (int i = 0; i < D - 1 && i < nst; ++i) issue(st0 + i);

  f32x4 P[MB][2], S[MB];
#pragma unroll 1
  for (int i = 0; i < nst; ++i) {
    const int st = st0 + i;
    if (i + D - 2 < nst) wait_vmcnt<(D - 2) * R::kLoads>();
    else wait_vmcnt<0>();
    barrier_no_wait();  // stage st visible to all; slot (st-1) % D free
    if (i + D - 1 < nst) issue(st + D - 1);

    const uint8_t* slot = smem + (st % D) * R::kSlot;
    const uint8_t* wl = slot;
    const uint8_t* al = slot + kWBytes;
    const uint8_t* szl = slot + kWBytes + R::kABytes;
    const int in_group = st % stages_per_group;
    if (in_group == 0 || i == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        S[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 2; ++j) P[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    u32x4v bfr[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cblk = 2 * wave + j;
      const int pc = cblk ^ (tr_row & 7);
      const uint8_t* addr = wl + tr_row * 128 + pc * 16 + tr_half;
      const i32x2 d = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(addr)));
      bfr[j][0] = w4mma::codes_to_frag<T>(static_cast<uint32_t>(d[0]));
      bfr[j][1] = w4mma::codes_to_frag<T>(static_cast<uint32_t>(d[1]));
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int row = 16 * mb + li;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int pc = (2 * q + sub) ^ (row & 7);
        const uint4 v = *reinterpret_cast<const uint4*>(al + row * 128 + pc * 16);
        const u32x4v af = w4mma::act_frag(v);
#pragma unroll
        for (int j = 0; j < 2; ++j) P[mb][j] = w4mma::mfma_traits<T>::mma(af, bfr[j][sub], P[mb][j]);
        S[mb] = w4mma::mfma_traits<T>::mma(af, ones, S[mb]);
      }
    }
    if (in_group == stages_per_group - 1 || i == nst - 1) {
      // Promote with this group's scale/zero of columns 32*wave + 16*j + li.
      const uint16_t* sl = reinterpret_cast<const uint16_t*>(szl);
      const uint16_t* zl = reinterpret_cast<const uint16_t*>(szl + 256);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int cc = 32 * wave + 16 * j + li;
        const float sc = elem<T>::to_f32(sl[cc]);
        const float zz = has_z ? elem<T>::to_f32(zl[cc]) : 0.f;
        const float cz = 128.0f + zz * unit;
        const float se = sc * inv_unit;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            O[mb][j][r] = fmaf(se, fmaf(-cz, S[mb][r], P[mb][j][r]), O[mb][j][r]);
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();  // the ring may be reused by the caller's next pass
}

}  // namespace w4pipe
}  // namespace ks
