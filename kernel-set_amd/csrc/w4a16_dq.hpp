// kernel-set (MI355X build) -- W4A16 GEMM for larger M: weights dequantized
// once per workgroup into an LDS bf16/f16 tile, then a plain 32x32x16 MFMA
// GEMM (no per-group promotion in the inner loop).
//
// Each workgroup (2 x BN/32 waves) owns BM rows x BN columns and walks K in
// 64-deep stages. Activations A [BM][64] and the raw int4 tile W [32 packed rows][BN]
// arrive global -> LDS through a D-stage ring (direct copies, no VGPRs), with
// the stage's scales and zeros. One
// stage ahead of the MFMAs the waves turn W into Wd [BN n][64 k] of the
// activation dtype: a wave reads 8 packed rows of 64 columns with
// ds_read_b64_tr_b8 (lane = column), computes w = fma(q, s, -z*s) -- equal to (q - z) * s in
// fp32 because z*s is exact -- and rounds once to bf16/f16, exactly the
// dequantized weight the reference's "dequantize, then matmul" forms. The MFMA
// B operand is then 8 consecutive k of one column, one ds_read_b128.
//
// LDS chunks (16 B) are XOR-swizzled against bank conflicts: A rows by
// (row & 7), W rows by (row & 7) (BN = 128) or ((row >> 2) & 3) (BN = 64),
// Wd columns by (n & 7). A larger BN divides the activation re-reads (one per
// column tile) -- the dominant traffic at M = 256.
#pragma once

#include "ks_common.hpp"

namespace ks {
namespace w4dq {

constexpr int kStageK = 64;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

template <int BM, int BN>
struct Cfg {
  static constexpr int kWavesN = BN / 32;
  static constexpr int kWaves = 2 * kWavesN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kABytes = BM * 128;
  static constexpr int kWBytes = 32 * BN;               // raw packed rows of one stage
  static constexpr int kWdBytes = BN * kStageK * 2;
  // A, W (+ a spare W copy filled by the second half of the waves) and one
  // 256 B scale/zero copy per wave: every wave issues the same copies, so the
  // per-wave vmcnt bookkeeping is uniform.
  static constexpr int kSlot = kABytes + 2 * kWBytes + 256 * kWaves;
  static constexpr int kDepth = BN == 64 ? 6 : 4;
  static constexpr int kALoads = BM / (8 * kWaves);     // 1 KB A copies per wave per stage
  static constexpr int kLoads = kALoads + 2;
  static constexpr int kBytes = kSlot * kDepth + 2 * kWdBytes;
  static_assert(kALoads >= 1, "tile");
};

template <typename T>
struct dq_traits;

template <>
struct dq_traits<bf16_t> {
  __device__ static inline uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(lo), static_cast<__bf16>(hi)});
  }
  __device__ static inline f32x16 mma(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct dq_traits<f16_t> {
  __device__ static inline uint32_t pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(lo), static_cast<_Float16>(hi)});
  }
  __device__ static inline f32x16 mma(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Dequantizes the 8 codes of one packed dword (byte r = rows r: low nibble k
// even, high nibble k odd) into 4 packed pairs o[r] = (w(k even), w(k odd)),
// w = fma(q, s, -zs). The two nibble planes are split with one mask each and
// every byte then converts with one v_cvt_f32_ubyteN (no per-code extract).
template <typename T>
__device__ inline void dequant_dword(uint32_t d, float s, float mzs, uint32_t* o) {
  uint32_t lo = d & 0x0f0f0f0fu, hi = (d >> 4) & 0x0f0f0f0fu;
  // opaque to the compiler, which would otherwise fold each byte back into a
  // per-code bit-field extract
  asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
  for (int r = 0; r < 4; ++r)
    o[r] = dq_traits<T>::pack(fmaf(static_cast<float>((lo >> (8 * r)) & 0xffu), s, mzs),
                              fmaf(static_cast<float>((hi >> (8 * r)) & 0xffu), s, mzs));
}

template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS writes of this wave complete (the caller's barrier then publishes them).
__device__ inline void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));
}

// Rows [m0, m0+BM) (clamped reads at row_end-1, outputs past row_end dropped)
// x columns [n0, n0+BN) over all of K. Requires K % 64 == 0, gs % 64 == 0,
// N % BN == 0, 16-byte aligned a and b, 4-byte aligned scales and zeros.
template <typename T, int BM, int BN>
__global__ void __launch_bounds__((Cfg<BM, BN>::kThreads))
dq_kernel(uint16_t* __restrict__ c, const uint16_t* __restrict__ a,
          const uint8_t* __restrict__ b, const uint16_t* __restrict__ scales,
          const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ bias,
          int64_t row_end, int64_t n, int64_t k, int gs, int sps, float* __restrict__ ws) {
  using R = Cfg<BM, BN>;
  constexpr int D = R::kDepth;
  constexpr int TM = BM / 64;  // 32x32 tiles per wave along M (wave tile BM/2 x 32)
  constexpr int kWChunks = BN / 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* ring = smem;
  uint8_t* wd = smem + R::kSlot * D;  // [2][BN n][128 B]

  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  // K split (grid z): stages [st0, st0 + nst); sps is a multiple of the
  // stages per quantization group, so every split starts on a group.
  const int st0 = static_cast<int>(blockIdx.z) * sps;
  const int nst = min(static_cast<int>(k / kStageK) - st0, sps);
  auto wswz = [](int row) { return BN == 64 ? ((row >> 2) & 3) : (row & 7); };

  // ---- producer (direct global -> LDS), advanced one stage per issue() ----
  const uint16_t* a_cur[R::kALoads];
#pragma unroll
  for (int i = 0; i < R::kALoads; ++i) {
    const int row = 8 * (wave * R::kALoads + i) + lane / 8;
    const int cc = (lane % 8) ^ (row & 7);
    const int64_t gr = min<int64_t>(m0 + row, row_end - 1);
    a_cur[i] = a + gr * k + static_cast<int64_t>(st0) * kStageK + 8 * cc;
  }
  // W: the first half of the waves fill W, the second half a spare copy;
  // a 1 KB copy covers 1024 / BN packed rows.
  constexpr int kRowsPerCopy = 1024 / BN;
  const int wv = wave % (R::kWaves / 2);
  const int w_row = wv * kRowsPerCopy + lane / kWChunks;
  const int w_c = (lane % kWChunks) ^ wswz(w_row);
  const uint8_t* w_cur = b + (static_cast<int64_t>(st0) * (kStageK / 2) + w_row) * n + n0 + 16 * w_c;
  const int w_dst = (wave / (R::kWaves / 2)) * R::kWBytes + wv * 1024;
  // Scales / zeros of the stage's group, 2 columns per lane: BN = 64 -> lanes
  // 0-31 scales, 32-63 zeros of wave 0's copy; BN = 128 -> wave 0 scales,
  // wave 1 zeros. Scales stand in for absent zeros.
  const bool sz_zero_lane = BN == 64 ? lane >= 32 : (wave & 1) != 0;
  const int sz_c = BN == 64 ? 2 * (lane % 32) : 2 * lane;
  const int spg = gs / kStageK;  // stages per quantization group
  const uint16_t* sz_col = ((sz_zero_lane && zeros) ? zeros : scales) +
                           static_cast<int64_t>(st0 / spg) * n + n0 + sz_c;
  int sz_left = spg;
  int is_slot = 0;
  auto issue = [&]() {
    uint8_t* slot = ring + is_slot * R::kSlot;
#pragma unroll
    for (int i = 0; i < R::kALoads; ++i) {
      dma_to_lds<16>(a_cur[i], slot + 1024 * (wave * R::kALoads + i));
      a_cur[i] += kStageK;
    }
    dma_to_lds<16>(w_cur, slot + R::kABytes + w_dst);
    w_cur += 32 * n;
    dma_to_lds<4>(sz_col, slot + R::kABytes + 2 * R::kWBytes + 256 * wave);
    if (--sz_left == 0) {
      sz_left = spg;
      sz_col += n;
    }
    is_slot = (is_slot + 1 == D) ? 0 : is_slot + 1;
  };

  // ---- dequant role: wave -> packed rows 8*(wave%4).. (k 16*(wave%4)..+15),
  // lane -> column 64*(wave/4) + lane ----
  const int dq_rg = wave % 4;
  const int dq_n = 64 * (wave / 4) + lane;
  const int dq_row = 8 * dq_rg + ((lane % 16) >> 1);
  const int dq_cb = dq_n / 16;
  const int dq_src = dq_row * BN + ((dq_cb ^ wswz(dq_row)) * 16) + 8 * (lane & 1);
  const bool has_z = zeros != nullptr;
  auto dequant = [&](const uint8_t* wslot, uint8_t* wd_buf) {
    const uint16_t* szl = reinterpret_cast<const uint16_t*>(wslot + 2 * R::kWBytes);
    const float s = elem<T>::to_f32(szl[dq_n]);
    const float z = has_z ? elem<T>::to_f32(BN == 64 ? szl[64 + dq_n] : szl[128 + dq_n]) : 0.f;
    const float zs = s * z;  // exact: at most 2 x 11 significant bits
    const i32x2 d = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(wslot + dq_src)));
    uint32_t o[8];
    dequant_dword<T>(static_cast<uint32_t>(d[0]), s, -zs, o);
    dequant_dword<T>(static_cast<uint32_t>(d[1]), s, -zs, o + 4);
    uint8_t* dst = wd_buf + dq_n * 128;
    *reinterpret_cast<uint4*>(dst + ((2 * dq_rg) ^ (dq_n & 7)) * 16) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(dst + ((2 * dq_rg + 1) ^ (dq_n & 7)) * 16) = make_uint4(o[4], o[5], o[6], o[7]);
  };

  // ---- MFMA role: wave (wr, wc) -> rows wr*BM/2 .., columns wc*32 .. ----
  const int wr = wave / R::kWavesN, wc = wave % R::kWavesN;
  const int l32 = lane % 32, lh = lane / 32;
  f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) acc[i] = f32x16{};

#pragma unroll 1
  for (int i = 0; i < D - 1 && i < nst; ++i) issue();
  // stage 0 must be dequantized before the loop
  if (nst >= D - 1) wait_vmcnt<(D - 2) * R::kLoads>();
  else wait_vmcnt<0>();
  barrier_no_wait();
  dequant(ring + R::kABytes, wd);

  int slot_i = 0;
#pragma unroll 1
  for (int st = 0; st < nst; ++st) {
    // stage st+1 has landed (its loads were issued >= D-2 stages ago)
    if (st + D - 2 < nst) wait_vmcnt<(D - 3) * R::kLoads>();
    else wait_vmcnt<0>();
    wait_lgkm0();       // this wave's Wd writes of the previous iteration
    barrier_no_wait();  // Wd[st] visible, Wd[st+1] and ring slot st-1 free
    if (st + D - 1 < nst) issue();
    const int nx_slot = (slot_i + 1 == D) ? 0 : slot_i + 1;
    const uint8_t* as = ring + slot_i * R::kSlot;
    const uint8_t* bs = wd + (st & 1) * R::kWdBytes;
#pragma unroll
    for (int ks = 0; ks < kStageK / 16; ++ks) {
      const int chunk = 2 * ks + lh;  // 8 k per lane: k = 16ks + 8lh .. +7
      const int bn = wc * 32 + l32;
      const uint4 bf = *reinterpret_cast<const uint4*>(bs + bn * 128 + ((chunk ^ (bn & 7)) * 16));
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int am = wr * (BM / 2) + i * 32 + l32;
        const uint4 af = *reinterpret_cast<const uint4*>(as + am * 128 + ((chunk ^ (am & 7)) * 16));
        acc[i] = dq_traits<T>::mma(af, bf, acc[i]);
      }
    }
    // The next stage's dequantization after this stage's MFMAs are issued:
    // its VALU and LDS work then runs while the MFMAs execute.
    if (st + 1 < nst) dequant(ring + nx_slot * R::kSlot + R::kABytes, wd + ((st + 1) & 1) * R::kWdBytes);
    slot_i = nx_slot;
  }
  wait_vmcnt<0>();

  // ---- epilogue: acc[i][r] -> row 8*(r/4) + 4*lh + r%4 of the 32x32 tile ----
  const int64_t col = n0 + wc * 32 + l32;
  const float bv = (bias && !ws) ? elem<T>::to_f32(bias[col]) : 0.f;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = m0 + wr * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * lh + (r % 4);
      if (row >= row_end) continue;
      if (ws)  // split partial, summed (with the bias) by the reduce kernel
        ws[(static_cast<int64_t>(blockIdx.z) * row_end + row) * n + col] = acc[i][r];
      else
        c[row * n + col] = elem<T>::from_f32(acc[i][r] + bv);
    }
}

}  // namespace w4dq
}  // namespace ks
