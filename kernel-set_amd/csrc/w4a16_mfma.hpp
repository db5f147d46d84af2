// kernel-set (MI355X build) -- W4A16 on bf16/f16 MFMA, shared by the dense
// batched GEMM (ks_gemm_w4a16, M > 8) and the MoE grouped GEMM.
//
// Roles: activations are the MFMA A operand (rows = tokens m), int4 weights the
// B operand (columns = n), v_mfma_f32_16x16x32_{bf16,f16}.
//
// Weight fragments without LDS: lane (li = lane%16, q = lane/16) loads one
// dword (4 columns) from each of the 4 packed rows kp0+4q+{0..3}; a 4x4 byte
// transpose gives, per column, the 8 codes k0+8q+{0..7}. Each code becomes the
// 16-bit float "base + q" with one and-or: 0x4300|q is bf16 128+q and
// 0x5800|q is f16 128+q (both exact). The lane pairs codes (0,4),(1,5),(2,6),
// (3,7); the activation fragment is permuted the same way, so the dot product
// over the 8 k is unchanged. MFMA j of a step uses column n0 + 4*li + j.
//
// Per quantization group (gs % 32 == 0) the MFMAs accumulate
//   P[m,n] = sum_k a[m,k] * (128 + q[k,n])        and, with an all-ones B,
//   S[m]   = sum_k a[m,k],
// then promote  O[m,n] += s[g,n] * (P - (128 + z[g,n]) * S)
// which equals sum_k a[m,k] * (q - z) * s over the group.
//
// A workgroup (4 waves) owns 64 columns; the waves split the K range of the
// workgroup (intra-workgroup split-K) and are summed through LDS in a fixed
// order, so each weight byte is fetched and converted exactly once.
#pragma once

#include "ks_common.hpp"

namespace ks {
namespace w4mma {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTileN = 64;  // columns per workgroup (16 lane slots x 4)

template <typename T>
struct mfma_traits;

template <>
struct mfma_traits<bf16_t> {
  static constexpr uint32_t magic = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr uint32_t one2 = 0x3f803f80u;   // bf16 1.0 pair
  __device__ static inline f32x4 mma(u32x4v a, u32x4v b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct mfma_traits<f16_t> {
  static constexpr uint32_t magic = 0x58005800u;  // f16 128.0 (ulp 0.125 -> 0x5800|q = 128+q/8)
  static constexpr uint32_t one2 = 0x3c003c00u;
  __device__ static inline f32x4 mma(u32x4v a, u32x4v b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// f16 has 10 mantissa bits: 0x5800 is 128.0 with ulp 1/8, so OR-ing q into the
// low bits gives 128 + q/8. The code scale is folded into the promotion.
template <typename T>
struct code_scale;
template <>
struct code_scale<bf16_t> {
  static constexpr float unit = 1.0f;  // one code step in the base+q encoding
};
template <>
struct code_scale<f16_t> {
  static constexpr float unit = 0.125f;
};

__device__ inline void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  const uint32_t t01lo = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);
  const uint32_t t01hi = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);
  const uint32_t t23lo = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t t23hi = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(t23lo, t01lo, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(t23lo, t01lo, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(t23hi, t01hi, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(t23hi, t01hi, 0x07060302u);
}

// One column's 8 codes (packed rows in the 4 bytes of t) -> B fragment.
template <typename T>
__device__ inline u32x4v codes_to_frag(uint32_t t) {
  constexpr uint32_t mg = mfma_traits<T>::magic;
  const uint32_t m = 0x000f000fu;
  return u32x4v{(t & m) | mg, ((t >> 4) & m) | mg, ((t >> 8) & m) | mg, ((t >> 12) & m) | mg};
}

// One column's 8 codes (packed rows in the 4 bytes of t) -> B fragment in
// natural k order: dword r = codes (2r, 2r+1), the low and high nibble of byte
// r, so the A fragment is 8 consecutive activations as loaded. v_perm puts
// byte r of t in byte 0 and byte r of t >> 4 in byte 2 (zeros elsewhere), one
// v_and_or_b32 keeps the two nibbles and adds the 128 base. `mask` must be the
// wave-uniform 0x000f000f and `base` the magic in a VGPR (VOP3 takes no
// literal on gfx9, and one SGPR per instruction), or the and-or splits in two.
template <typename T>
__device__ inline u32x4v codes_to_frag_nat(uint32_t t, uint32_t mask, uint32_t base) {
  const uint32_t t4 = t >> 4;
  return u32x4v{(__builtin_amdgcn_perm(t4, t, 0x0c040c00u) & mask) | base,
                (__builtin_amdgcn_perm(t4, t, 0x0c050c01u) & mask) | base,
                (__builtin_amdgcn_perm(t4, t, 0x0c060c02u) & mask) | base,
                (__builtin_amdgcn_perm(t4, t, 0x0c070c03u) & mask) | base};
}

// 8 consecutive activations (16 B) -> A fragment in the (0,4),(1,5),(2,6),(3,7) order.
__device__ inline u32x4v act_frag(uint4 d) {
  return u32x4v{__builtin_amdgcn_perm(d.z, d.x, 0x05040100u),
                __builtin_amdgcn_perm(d.z, d.x, 0x07060302u),
                __builtin_amdgcn_perm(d.w, d.y, 0x05040100u),
                __builtin_amdgcn_perm(d.w, d.y, 0x07060302u)};
}

struct TileArgs {
  const uint16_t* a;      // activations [rows, K] (row pointer base)
  const uint8_t* b;       // packed weights [K/2, N]
  const uint16_t* s;      // scales [K/gs, N]
  const uint16_t* z;      // zeros [K/gs, N] or null
  int64_t row0, row1;     // token rows [row0, row1) of `a`
  int64_t n, k;
  int gs;
  int64_t n0;             // first column of the tile
  int g_begin, g_end;     // quantization groups of this workgroup
};

// Computes the workgroup's partial sums O[m][n0..n0+63] for rows [r0, r0+16*MB)
// over groups [g_begin, g_end). Result lands in `red` (LDS, [16*MB][64] floats,
// wave 0's final sum) after the call; all threads must call it.
template <typename T, int MB>
__device__ inline void tile_partial(const TileArgs& p, int64_t r0, float* red /* [3][16*MB][64] + out */) {
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int li = lane % 16, q = lane / 16;
  const int64_t col = p.n0 + 4 * li;
  const bool col_ok = col < p.n;
  const int steps_per_group = p.gs / 32;
  const int ng = p.g_end - p.g_begin;
  const int gw = (ng + 3) / 4;  // groups per wave
  const int gw0 = p.g_begin + wave * gw;
  const int gw1 = min(gw0 + gw, p.g_end);

  f32x4 O[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) O[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const u32x4v ones = {mfma_traits<T>::one2, mfma_traits<T>::one2, mfma_traits<T>::one2,
                       mfma_traits<T>::one2};
  const int total_steps = (gw1 > gw0) ? (gw1 - gw0) * steps_per_group : 0;
  const int64_t kp_first = static_cast<int64_t>(gw0) * p.gs / 2;

  uint32_t wcur[4], wnext[4];
  auto load_w = [&](int st, uint32_t* w) {
    const int64_t kp = kp_first + static_cast<int64_t>(st) * 16 + 4 * q;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      w[r] = col_ok ? __builtin_nontemporal_load(
                          reinterpret_cast<const uint32_t*>(p.b + (kp + r) * p.n + col))
                    : 0u;
  };
  // Activation fragments are prefetched one step ahead like the weights, so
  // neither operand's load latency sits on the MFMA chain.
  uint4 acur[MB], anext[MB];
  auto load_a = [&](int st, uint4* av) {
    const int64_t k0 = 2 * (kp_first + static_cast<int64_t>(st) * 16) + 8 * q;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t row = r0 + 16 * mb + li;
      av[mb] = (row < p.row1) ? *reinterpret_cast<const uint4*>(p.a + row * p.k + k0)
                              : make_uint4(0, 0, 0, 0);
    }
  };
  if (total_steps > 0) {
    load_w(0, wcur);
    load_a(0, acur);
  }

  f32x4 P[MB][4], S[MB];
  for (int st = 0; st < total_steps; ++st) {
    const int in_group = st % steps_per_group;
    if (in_group == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        S[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) P[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if (st + 1 < total_steps) {
      load_w(st + 1, wnext);
      load_a(st + 1, anext);
    }

    uint32_t tr[4];
    transpose4x4(wcur, tr);
    u32x4v bf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = codes_to_frag<T>(tr[j]);

#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const u32x4v af = act_frag(acur[mb]);
#pragma unroll
      for (int j = 0; j < 4; ++j) P[mb][j] = mfma_traits<T>::mma(af, bf[j], P[mb][j]);
      S[mb] = mfma_traits<T>::mma(af, ones, S[mb]);
    }

    if (in_group == steps_per_group - 1) {
      // promote: O += s * (unit*P - (128 + z) * S) ... for f16 the code axis
      // is scaled by 1/8: P = sum a*(128 + q/8) -> sum a*q = 8*(P - 128*S).
      const int64_t g = gw0 + st / steps_per_group;
      float sc[4], cz[4];
      if (col_ok) {
        const uint2 sv = *reinterpret_cast<const uint2*>(p.s + g * p.n + col);
        const uint32_t s2[2] = {sv.x, sv.y};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sc[j] = elem<T>::to_f32(static_cast<uint16_t>(s2[j / 2] >> (16 * (j % 2))));
        if (p.z) {
          const uint2 zv = *reinterpret_cast<const uint2*>(p.z + g * p.n + col);
          const uint32_t z2[2] = {zv.x, zv.y};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            cz[j] = elem<T>::to_f32(static_cast<uint16_t>(z2[j / 2] >> (16 * (j % 2))));
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) cz[j] = 0.f;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = cz[j] = 0.f;
      }
      constexpr float inv_unit = 1.0f / code_scale<T>::unit;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // value = s * inv_unit * (P - (128 + z*unit) * S)
        const float c = 128.0f + cz[j] * code_scale<T>::unit;
        const float se = sc[j] * inv_unit;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            O[mb][j][r] = fmaf(se, fmaf(-c, S[mb][r], P[mb][j][r]), O[mb][j][r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) wcur[r] = wnext[r];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acur[mb] = anext[mb];
  }

  // ---- cross-wave reduction in a fixed order: waves 1..3 stage, wave 0 sums.
  // red layout: [3][16*MB rows][64 cols] then result [16*MB][64].
  constexpr int kPlane = 16 * MB * kTileN;
  if (wave > 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[(wave - 1) * kPlane + (16 * mb + 4 * q + r) * kTileN + 4 * li + j] = O[mb][j][r];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = (16 * mb + 4 * q + r) * kTileN + 4 * li + j;
          red[3 * kPlane + e] = ((O[mb][j][r] + red[e]) + red[kPlane + e]) + red[2 * kPlane + e];
        }
  }
  __syncthreads();
}

}  // namespace w4mma
}  // namespace ks
