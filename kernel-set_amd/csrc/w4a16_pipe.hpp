// kernel-set (MI355X build) -- W4A16 batched tile with an LDS load ring, shared
// by the dense GEMM (ks_gemm_w4a16, M > 8) and the MoE grouped GEMM.
//
// Every operand moves global -> LDS directly (global_load_lds, no VGPRs
// held) through a ring of D stages. Measured on MI355X (graph replay, cold,
// K = 4096, N = 14336), two stages beat deeper rings at every pass height
// (1024 cold calls: M = 16 / 64 16.5 / 25.8 -> 14.8 / 25.0 us against 6 / 3
// stages; MoE config 5 gate_up 43.3 -> 40.1 us): a small ring lets more
// workgroups share a CU (48-row MoE passes: three instead of two, so the
// 768 (tile, expert) workgroups run in one round), and the other workgroups
// on the CU hide the copy latency that one stage of prefetch leaves exposed.
// Measured on MI355X the tile is instruction-issue bound before it is HBM
// bound, so a stage is 128 k deep and all per-stage bookkeeping is
// incremental (no division, no 64-bit multiply in the loop).
//
// Tile: 16*MB rows x 128 columns, 4 waves side by side over N (32 columns,
// two 16-column MFMA blocks each); one stage = 128 k = 64 packed rows.
// Per stage and ring slot:
//   W  [64 packed rows][128 B]     raw int4 pairs, 16-byte chunks swizzled by row & 7
//   A  [16*MB rows][128 bf16/f16]  activations, chunks swizzled by row & 15
//   SZ [4][256 B]                  scales / zeros of the stage's first 64 k
//                                  (slots 0, 1) and last 64 k (slots 2, 3)
// B fragments are read already transposed with ds_read_b64_tr_b8: lane li of
// 16-lane group q receives column li's bytes of packed rows 32h+8q..+7, i.e.
// codes k = 64h+16q..+15. Each dword (8 codes) becomes an MFMA B fragment in
// natural k order with one v_perm and one v_and_or per pair: 0x4300|q is bf16
// 128+q (f16 0x5800|q = 128+q/8). The activation fragment is then the 16 bytes
// read from LDS as they are, shared unchanged by the four waves.
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
constexpr int kStageK = 128;         // k per stage
constexpr int kStageRows = 64;       // packed rows per stage
constexpr int kWBytes = kStageRows * 128;
constexpr int kSZBytes = 4 * 256;

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

template <int MB>
struct Ring {
  static constexpr int kABytes = 16 * MB * 256;
  static constexpr int kSlot = kWBytes + kABytes + kSZBytes;
  static constexpr int kDepth = 2;  // 26 / 34 / 42 / 50 KB for MB = 1..4
  static constexpr int kBytes = kSlot * kDepth;
  static constexpr int kALoads = MB;  // 16-byte A loads per thread per stage
  // global_load_lds instructions per thread per stage (identical in every wave)
  static constexpr int kLoads = 2 + kALoads + 1;
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
// n0 + 32*wave + 16*j + li. Requires K % 128 == 0, gs % 64 == 0, N % 16 == 0,
// 16-byte aligned a / b, 4-byte aligned scales / zeros, and st0 on a
// quantization-group boundary, and 32-bit byte offsets: 64 * N and
// rows(A) * K * 2 below 2^32 (checked on the host). All threads of the
// workgroup must call it.
// OG (one group per stage, gs == 128): each stage's first MFMAs start from a
// zero accumulator, so the promotion clears no P / S registers.
template <typename T, int MB, bool OG = false>
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

  // ---- ring producer: wave-uniform bases (advanced one stage per issue(),
  // scalar adds) plus fixed 32-bit per-lane byte offsets ----
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // W: wave instruction i fills packed rows 8*(2*wave+i)..+7 (1 KB).
  const uint8_t* w_base = p.b + static_cast<int64_t>(st0) * kStageRows * n;
  uint32_t w_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * (2 * wave + i) + lane / 8;
    const int c = (lane % 8) ^ (row & 7);
    const int64_t col = min<int64_t>(p.n0 / 16 + c, last_chunk) * 16;
    w_off[i] = static_cast<uint32_t>(row * n + col);
  }
  // A: wave instruction i fills rows 4*(wave*MB+i)..+3 (256 B per row).
  const uint8_t* a_base = reinterpret_cast<const uint8_t*>(p.a) + static_cast<int64_t>(st0) * kStageK * 2;
  uint32_t a_off[R::kALoads];
#pragma unroll
  for (int i = 0; i < R::kALoads; ++i) {
    const int row = 4 * (wave * MB + i) + lane / 16;
    const int c = (lane % 16) ^ (row & 15);
    const int64_t gr = min<int64_t>(r0 + row, r_end - 1);
    a_off[i] = static_cast<uint32_t>((gr * k + 8 * c) * 2);
  }
  // SZ: waves 0/1 take scales/zeros of the stage's first 64 k, waves 2/3 of
  // its last 64 k (the same group unless gs == 64); scales stand in for
  // absent zeros so every wave issues the same loads.
  const uint16_t* sz_src = ((wave_u & 1) && p.z) ? p.z : p.s;
  const uint32_t sz_off = static_cast<uint32_t>(min<int64_t>(p.n0 + 2 * lane, n - 2) * 2);
  const int64_t k_first = static_cast<int64_t>(st0) * kStageK + (wave_u >= 2 ? 64 : 0);
  const uint16_t* sz_base = sz_src + (k_first / p.gs) * n;
  const int spg64 = p.gs / 64;  // 64-k halves per group
  // halves left before this wave's group index changes
  int sz_left = spg64 - static_cast<int>((k_first / 64) % spg64);
  uint32_t is_slot = 0;
  const int64_t w_step = kStageRows * n;

  auto issue = [&]() {
    uint8_t* slot = smem + is_slot * R::kSlot;
#pragma unroll
    for (int i = 0; i < 2; ++i) dma_to_lds_off<16>(w_base, w_off[i], slot + 1024 * (2 * wave_u + i));
    w_base += w_step;
#pragma unroll
    for (int i = 0; i < R::kALoads; ++i)
      dma_to_lds_off<16>(a_base, a_off[i], slot + kWBytes + 1024 * (wave_u * MB + i));
    a_base += kStageK * 2;
    dma_to_lds_off<4>(sz_base, sz_off, slot + kWBytes + R::kABytes + 256 * wave_u);
    sz_left -= 2;  // a stage is two 64-k halves
    if (sz_left <= 0) {
      sz_left += spg64;
      sz_base += n;
      if (sz_left <= 0) {  // gs == 64: both halves moved on
        sz_left += spg64;
        sz_base += n;
      }
    }
    is_slot = (is_slot + 1 == D) ? 0 : is_slot + 1;
  };

  const u32x4v ones = {w4mma::mfma_traits<T>::one2, w4mma::mfma_traits<T>::one2,
                       w4mma::mfma_traits<T>::one2, w4mma::mfma_traits<T>::one2};
  uint32_t code_base = w4mma::mfma_traits<T>::magic;
  asm volatile("" : "+v"(code_base));  // kept in a VGPR (see codes_to_frag_nat)
  const uint32_t code_mask = __builtin_amdgcn_readfirstlane(0x000f000fu);
  constexpr float unit = w4mma::code_scale<T>::unit;
  constexpr float inv_unit = 1.0f / unit;
  const bool has_z = p.z != nullptr;
  const bool half_groups = p.gs == 64;  // promote after each 64-k half
  const int sps = p.gs / kStageK;       // stages per group when gs >= 128

  // tr8 source: lane (2*jj + hh) of group q addresses half hh of packed row 8q+jj.
  const int tr_row = 8 * q + (li >> 1);
  const int tr_half = 8 * (li & 1);
  const int tr_pc0 = ((2 * wave) ^ (tr_row & 7)) * 16 + tr_half;
  const int tr_pc1 = ((2 * wave + 1) ^ (tr_row & 7)) * 16 + tr_half;

#pragma unroll 1
  for (int i = 0; i < D - 1 && i < nst; ++i) issue();

  f32x4 P[MB][2], S[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    S[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) P[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Promotion with the scale/zero slot pair `half` (0: first 64 k, 1: last);
  // leaves P and S cleared for the next group (OG: the next stage's first
  // MFMAs overwrite them instead).
  // The promotion's per-column factors of scale/zero slot pair `half`: read
  // at the stage start (their LDS latency then hides under the MFMAs), both
  // values read unconditionally (the zero slot holds scales when there are
  // no zeros) and selected, so no branch splits the stage.
  struct Fac { float se[2], cz[2]; };
  auto factors = [&](const uint8_t* szl, int half) {
    const uint16_t* sl = reinterpret_cast<const uint16_t*>(szl + 512 * half);
    const uint16_t* zl = reinterpret_cast<const uint16_t*>(szl + 512 * half + 256);
    Fac f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cc = 32 * wave + 16 * j + li;
      const float sc = elem<T>::to_f32(sl[cc]);
      const float zr = elem<T>::to_f32(zl[cc]);
      const float zz = has_z ? zr : 0.f;
      f.cz[j] = 128.0f + zz * unit;
      f.se[j] = sc * inv_unit;
    }
    return f;
  };
  auto promote = [&](const Fac& f) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float cz = f.cz[j];
      const float se = f.se[j];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          O[mb][j][r] = fmaf(se, fmaf(-cz, S[mb][r], P[mb][j][r]), O[mb][j][r]);
          if constexpr (!OG) P[mb][j][r] = 0.f;
        }
    }
    if constexpr (!OG) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) S[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  int grp_pos = 0;  // stage index within its group (gs >= 128); st0 is group-aligned
  uint32_t slot_i = 0;
#pragma unroll 1
  for (int i = 0; i < nst; ++i) {
    if (i + D - 2 < nst) wait_vmcnt<(D - 2) * R::kLoads>();
    else wait_vmcnt<0>();
    barrier_no_wait();  // this stage is visible to all; the previous slot is free
    if (i + D - 1 < nst) issue();

    const uint8_t* slot = smem + slot_i * R::kSlot;
    slot_i = (slot_i + 1 == D) ? 0 : slot_i + 1;
    const uint8_t* al = slot + kWBytes;
    const uint8_t* szl = slot + kWBytes + R::kABytes;
    const Fac f0 = factors(szl, 0);
    Fac f1 = f0;
    if (half_groups) f1 = factors(szl, 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint8_t* wl = slot + (32 * h + tr_row) * 128;
      const i32x2 d0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(wl + tr_pc0)));
      const i32x2 d1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(wl + tr_pc1)));
      u32x4v bfr[2][2];
      bfr[0][0] = w4mma::codes_to_frag_nat<T>(static_cast<uint32_t>(d0[0]), code_mask, code_base);
      bfr[0][1] = w4mma::codes_to_frag_nat<T>(static_cast<uint32_t>(d0[1]), code_mask, code_base);
      bfr[1][0] = w4mma::codes_to_frag_nat<T>(static_cast<uint32_t>(d1[0]), code_mask, code_base);
      bfr[1][1] = w4mma::codes_to_frag_nat<T>(static_cast<uint32_t>(d1[1]), code_mask, code_base);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int row = 16 * mb + li;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          const int pc = (8 * h + 2 * q + sub) ^ li;  // row & 15 == li
          const uint4 v = *reinterpret_cast<const uint4*>(al + row * 256 + pc * 16);
          const u32x4v af = {v.x, v.y, v.z, v.w};
          const bool fresh = OG && h == 0 && sub == 0;  // compile-time
          P[mb][0] = w4mma::mfma_traits<T>::mma(af, bfr[0][sub], fresh ? zero4 : P[mb][0]);
          P[mb][1] = w4mma::mfma_traits<T>::mma(af, bfr[1][sub], fresh ? zero4 : P[mb][1]);
          S[mb] = w4mma::mfma_traits<T>::mma(af, ones, fresh ? zero4 : S[mb]);
        }
      }
      if (!OG && half_groups) promote(h == 0 ? f0 : f1);
    }
    if constexpr (OG) {
      promote(f0);
    } else if (!half_groups) {
      if (++grp_pos == sps || i == nst - 1) {
        grp_pos = 0;
        promote(f0);
      }
    }
  }
  wait_vmcnt<0>();
  __syncthreads();  // the ring may be reused by the caller's next pass
}

}  // namespace w4pipe
}  // namespace ks
