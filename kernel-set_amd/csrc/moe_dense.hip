// kernel-set (MI355X build) -- dense grouped GEMM for Mixture-of-Experts:
// ks_moe_grouped_gemm (moe.h:57-65, kernels/src/moe/moe_grouped_gemm.cu:136-198
// of cklxx/kernel-set). For each expert e, rows [off_e, off_{e+1}) of
// A [total_rows, K] times that expert's weights b[e] = [K, N] (N contiguous)
// give the same rows of C [total_rows, N]; all three share one dtype
// (f32, f16, bf16, fp8 e4m3fn, fp8 e5m2), products are accumulated in fp32 and
// the result is rounded once to the storage type (moe_grouped_gemm.cu:68-127).
//
// Differences from the reference's form, not its results:
//  * no tile-schedule buffer, no allocation and no stream synchronization: the
//    grid is (128-column tiles) x (experts), and every workgroup reads its
//    expert's row range from expert_offsets on the device and walks it in
//    16*MB-row passes (the call is asynchronous like every other entry point,
//    and can be captured in a HIP graph);
//  * MFMA instead of SIMT: v_mfma_f32_16x16x32_{bf16,f16}, the scaled
//    16x16x128 fp8 MFMA at unit scales, v_mfma_f32_16x16x4_f32 for f32; the
//    fp32 sum is taken in the MFMA's order rather than k-ascending.
//
// Tile: 16*MB rows x 128 columns, 4 waves side by side over N (32 columns, two
// 16-column MFMA blocks each). One stage holds SK = 128 / sizeof(T) k: the B
// stage is always 16 KB ([SK k-rows][128 columns]) and the A stage 128 bytes
// per row, both copied global -> LDS directly (global_load_lds_dwordx4) into a
// 3-deep ring with 16-byte chunks XOR-swizzled per row. B fragments are read
// already transposed (ds_read_b64_tr_b16 / _tr_b8), so each lane receives the
// consecutive k of one column that the MFMA operand wants.
#include <algorithm>
#include <type_traits>

#include "kernel_set/moe.h"
#include "ks_common.hpp"

namespace ks {
namespace moed {

constexpr int kThreads = 256;
constexpr int kTileN = 128;
constexpr int kBStage = 16384;  // B bytes per stage
constexpr int kARow = 128;      // A bytes per row per stage
constexpr int kDepth = 3;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

// Storage and conversions per dtype tag (rounding: bf16/f16 RNE, fp8 RNE with
// saturation to the finite maximum and NaN kept, as ks_common.hpp states).
template <typename T>
struct Dt;
template <>
struct Dt<f32_t> {
  using st = float;
  static constexpr int es = 4;
  __device__ static float dec(float v) { return v; }
  __device__ static float enc(float v) { return v; }
};
template <>
struct Dt<f16_t> {
  using st = uint16_t;
  static constexpr int es = 2;
  __device__ static float dec(uint16_t v) { return f16_bits_to_f32(v); }
  __device__ static uint16_t enc(float v) { return f32_to_f16_bits(v); }
};
template <>
struct Dt<bf16_t> {
  using st = uint16_t;
  static constexpr int es = 2;
  __device__ static float dec(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ static uint16_t enc(float v) { return f32_to_bf16_bits(v); }
};
template <>
struct Dt<e4m3_t> {
  using st = uint8_t;
  static constexpr int es = 1;
  static constexpr int fmt = 0;  // MFMA operand format: fp8 e4m3
  __device__ static float dec(uint8_t v) { return e4m3_to_f32(v); }
  __device__ static uint8_t enc(float v) { return f32_to_e4m3(v); }
};
template <>
struct Dt<e5m2_t> {
  using st = uint8_t;
  static constexpr int es = 1;
  static constexpr int fmt = 1;  // bf8 (e5m2)
  __device__ static float dec(uint8_t v) { return e5m2_to_f32(v); }
  __device__ static uint8_t enc(float v) { return f32_to_e5m2(v); }
};

// Chunk swizzles (LDS: 64 banks x 4 B). A rows are 128 B, so rows r and r+1
// share a 256-byte bank line in opposite halves and rows 2 apart collide
// unless their chunks differ: (r >> 1) & 7 spreads a 16-row fragment read over
// all 64 banks.
__device__ inline int a_swz(int r) { return (r >> 1) & 7; }
// B k-rows are 128 * es bytes. es = 2: a transposed read touches rows j = 0..3
// (and the 16-lane group 8 rows on), 32 bytes each at the same column, so the
// chunk pair is moved by 2 * (r & 3) and the next group's by 8. es = 1: the 8
// rows of a transposed read get chunks r & 7. es = 4: the four rows q = 0..3
// of one f32 fragment read get 64-byte groups 4 * (r & 3).
template <int ES>
__device__ inline int b_swz(int r) {
  if constexpr (ES == 2) return (2 * (r & 3)) | (((r >> 3) & 1) << 3);
  else if constexpr (ES == 1) return r & 7;
  else return 4 * (r & 3);
}

// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int MB>
struct Ring {
  static constexpr int kABytes = 16 * MB * kARow;
  static constexpr int kSlot = kBStage + kABytes;
  static constexpr int kBytes = kDepth * kSlot;
  static constexpr int kAInstr = 2 * MB;                  // 1 KB A copies per stage
  static constexpr int kAL = MB >= 2 ? MB / 2 : 1;        // per wave (MB = 1: waves 2, 3 repeat 0, 1)
  static constexpr int kLoads = 4 + kAL;                  // copies per wave per stage
};

// Rows [r0, min(r0 + 16 MB, r_end)) x columns [n0, n0 + 128) of one expert,
// over all of K. Requires K % SK == 0, (N * es) % 16 == 0 and 16-byte aligned
// a / b (checked on the host). All threads of the workgroup call it.
template <typename T, int MB>
__device__ inline void dense_pass(typename Dt<T>::st* __restrict__ c,
                                  const typename Dt<T>::st* __restrict__ a,
                                  const typename Dt<T>::st* __restrict__ be, int64_t r0,
                                  int64_t r_end, int64_t n0, int64_t n, int64_t k,
                                  uint8_t* smem) {
  using R = Ring<MB>;
  constexpr int ES = Dt<T>::es;
  constexpr int SK = 128 / ES;          // k per stage
  constexpr int RB = 128 * ES;          // bytes per B k-row
  constexpr int CPR = RB / 16;          // chunks per B k-row
  constexpr int RPI = 1024 / RB;        // B k-rows per 1 KB copy
  const int t = threadIdx.x;
  const int lane = t % kWave;
  const int wave = t / kWave;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int li = lane % 16, q = lane / 16;
  const int nst = static_cast<int>(k / SK);

  // ---- producer: per-lane sources, advanced one stage per issue() ----
  const uint8_t* b_cur[4];
  const int64_t last_chunk = n * ES / 16 - 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = RPI * (4 * wave + i) + lane / CPR;
    const int pc = lane % CPR;
    const int64_t chunk = min<int64_t>(n0 * ES / 16 + (pc ^ b_swz<ES>(row)), last_chunk);
    b_cur[i] = reinterpret_cast<const uint8_t*>(be) + row * n * ES + 16 * chunk;
  }
  const uint8_t* a_cur[R::kAL];
#pragma unroll
  for (int i = 0; i < R::kAL; ++i) {
    const int idx = (wave * R::kAL + i) % R::kAInstr;
    const int row = 8 * idx + lane / 8;
    const int64_t gr = min<int64_t>(r0 + row, r_end - 1);  // rows past the expert: never stored
    a_cur[i] = reinterpret_cast<const uint8_t*>(a) + gr * k * ES + 16 * ((lane % 8) ^ a_swz(row));
  }
  const int64_t b_step = static_cast<int64_t>(SK) * n * ES;
  uint32_t is_slot = 0;
  auto issue = [&]() {
    uint8_t* slot = smem + is_slot * R::kSlot;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma_to_lds<16>(b_cur[i], slot + 1024 * (4 * wave_u + i));
      b_cur[i] += b_step;
    }
#pragma unroll
    for (int i = 0; i < R::kAL; ++i) {
      const int idx = (wave_u * R::kAL + i) % R::kAInstr;
      dma_to_lds<16>(a_cur[i], slot + kBStage + 1024 * idx);
      a_cur[i] += kARow;
    }
    is_slot = (is_slot + 1 == kDepth) ? 0 : is_slot + 1;
  };

  f32x4 O[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j) O[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
  for (int i = 0; i < kDepth - 1 && i < nst; ++i) issue();

  uint32_t slot_i = 0;
#pragma unroll 1
  for (int s = 0; s < nst; ++s) {
    if (s + kDepth - 2 < nst) wait_vm<(kDepth - 2) * R::kLoads>();
    else wait_vm<0>();
    barrier_no_wait();  // stage s is visible to all; the slot issued next is free
    if (s + kDepth - 1 < nst) issue();
    const uint8_t* sb = smem + slot_i * R::kSlot;
    const uint8_t* sa = sb + kBStage;
    slot_i = (slot_i + 1 == kDepth) ? 0 : slot_i + 1;

    if constexpr (ES == 2) {
      // 2 substeps of 32 k: lane (li, q) holds k = 8q..8q+7 of its row / column.
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        i16x4 bf[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            // lane 4*jj + cc of the group addresses k-row 32h + 8q + 4e + jj,
            // bytes 8*cc..+7 of the 16-column block
            const int row = 32 * h + 8 * q + 4 * e + (li >> 2);
            const int lc = 4 * wave + 2 * j + ((li & 3) >> 1);
            const uint8_t* p = sb + row * RB + 16 * (lc ^ b_swz<ES>(row)) + 8 * (li & 1);
            bf[j][e] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<lds_i16x4*>(reinterpret_cast<uintptr_t>(p)));
          }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = 16 * mb + li;
          const uint4 av = *reinterpret_cast<const uint4*>(sa + row * kARow +
                                                          16 * ((4 * h + q) ^ a_swz(row)));
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const i16x4 b0 = bf[j][0], b1 = bf[j][1];
            const uint4 bv = make_uint4(
                (uint32_t)(uint16_t)b0[0] | ((uint32_t)(uint16_t)b0[1] << 16),
                (uint32_t)(uint16_t)b0[2] | ((uint32_t)(uint16_t)b0[3] << 16),
                (uint32_t)(uint16_t)b1[0] | ((uint32_t)(uint16_t)b1[1] << 16),
                (uint32_t)(uint16_t)b1[2] | ((uint32_t)(uint16_t)b1[3] << 16));
            if constexpr (std::is_same<T, bf16_t>::value)
              O[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), O[mb][j], 0, 0, 0);
            else
              O[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  __builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), O[mb][j], 0, 0, 0);
          }
        }
      }
    } else if constexpr (ES == 1) {
      // one 128-k MFMA: lane (li, q) holds k = 32q..32q+31.
      i32x8 bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        i32x2 d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // lane 2*jj + hh addresses k-row 32q + 8u + jj, half hh of the chunk
          const int row = 32 * q + 8 * u + (li >> 1);
          const int lc = 2 * wave + j;
          const uint8_t* p = sb + row * RB + 16 * (lc ^ b_swz<ES>(row)) + 8 * (li & 1);
          d[u] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              reinterpret_cast<lds_i32x2*>(reinterpret_cast<uintptr_t>(p)));
        }
        bf[j] = i32x8{d[0][0], d[0][1], d[1][0], d[1][1], d[2][0], d[2][1], d[3][0], d[3][1]};
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int row = 16 * mb + li;
        const uint4 x0 = *reinterpret_cast<const uint4*>(sa + row * kARow + 16 * ((2 * q) ^ a_swz(row)));
        const uint4 x1 = *reinterpret_cast<const uint4*>(sa + row * kARow + 16 * ((2 * q + 1) ^ a_swz(row)));
        const i32x8 af = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                               (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
#pragma unroll
        for (int j = 0; j < 2; ++j)
          O[mb][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              af, bf[j], O[mb][j], Dt<T>::fmt, Dt<T>::fmt, 0, 127, 0, 127);
      }
    } else {
      // f32: 8 substeps of 4 k; lane (li, q) holds A[li][4u + q] and B[4u + q][col].
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        float bv[2];
        const int brow = 4 * u + q;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = 32 * wave + 16 * j + li;
          bv[j] = *reinterpret_cast<const float*>(sb + brow * RB +
                                                  16 * ((col >> 2) ^ b_swz<ES>(brow)) + 4 * (col & 3));
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const int row = 16 * mb + li;
          const float av = *reinterpret_cast<const float*>(sa + row * kARow + 16 * (u ^ a_swz(row)) + 4 * q);
#pragma unroll
          for (int j = 0; j < 2; ++j)
            O[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[j], O[mb][j], 0, 0, 0);
        }
      }
    }
  }
  wait_vm<0>();
  __syncthreads();  // the ring is refilled by the next pass

  // lane holds rows 16 mb + 4 q + r, column 32 wave + 16 j + li
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + 32 * wave + 16 * j + li;
    if (col >= n) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = r0 + 16 * mb + 4 * q + r;
        if (row < r_end) c[row * n + col] = Dt<T>::enc(O[mb][j][r]);
      }
  }
}

// One workgroup per (128-column tile, expert). Workgroup ids are dispatched to
// the 8 XCDs round-robin; id L serves expert (L % 8) + 8 * (L / 8 / tiles_n),
// so every column tile of an expert runs on one XCD and the expert's rows of A
// come from HBM into that XCD's L2 once, not into all eight.
template <typename T, int MB>
__global__ void __launch_bounds__(kThreads, 2)
dense_kernel(typename Dt<T>::st* __restrict__ c, const typename Dt<T>::st* __restrict__ a,
             const typename Dt<T>::st* __restrict__ b, const int32_t* __restrict__ offsets,
             int num_experts, int tiles_n, int64_t total_rows, int64_t n, int64_t k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int L = blockIdx.x;
  const int e = (L & 7) + 8 * ((L >> 3) / tiles_n);
  if (e >= num_experts) return;
  // Row range clamped to [0, total_rows]: malformed offsets cannot make the
  // kernel touch memory outside A and C.
  const int64_t r_begin = min<int64_t>(max<int64_t>(offsets[e], 0), total_rows);
  const int64_t r_end = min<int64_t>(max<int64_t>(offsets[e + 1], r_begin), total_rows);
  if (r_end <= r_begin) return;  // uniform across the workgroup
  const typename Dt<T>::st* be = b + static_cast<int64_t>(e) * k * n;
  const int64_t n0 = static_cast<int64_t>((L >> 3) % tiles_n) * kTileN;
  for (int64_t r0 = r_begin; r0 < r_end; r0 += 16 * MB)
    dense_pass<T, MB>(c, a, be, r0, r_end, n0, n, k, smem);
}

// Any shape / alignment: one thread per output, k-ascending fp32 fma (the
// reference kernel's order, moe_grouped_gemm.cu:99-124). Rows outside every
// expert's range are left untouched.
template <typename T>
__global__ void __launch_bounds__(kThreads)
dense_simple_kernel(typename Dt<T>::st* __restrict__ c, const typename Dt<T>::st* __restrict__ a,
                    const typename Dt<T>::st* __restrict__ b, const int32_t* __restrict__ offsets,
                    int num_experts, int64_t total_rows, int64_t n, int64_t k) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total_rows * n) return;
  const int64_t row = idx / n, col = idx % n;
  int lo = 0, hi = num_experts;  // last e with offsets[e] <= row
  while (hi - lo > 1) {
    const int mid = (lo + hi) / 2;
    if (offsets[mid] <= row) lo = mid; else hi = mid;
  }
  if (row < offsets[lo] || row >= offsets[lo + 1]) return;  // row not routed
  const typename Dt<T>::st* be = b + static_cast<int64_t>(lo) * k * n;
  float acc = 0.f;
  for (int64_t kk = 0; kk < k; ++kk)
    acc = fmaf(Dt<T>::dec(a[row * k + kk]), Dt<T>::dec(be[kk * n + col]), acc);
  c[row * n + col] = Dt<T>::enc(acc);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

template <typename T, int MB>
void launch_tile(void* c, const void* a, const void* b, const int32_t* offs, int E, int64_t rows,
                 int64_t n, int64_t k, hipStream_t st) {
  constexpr int lds = Ring<MB>::kBytes;
  // opt in to the LDS size once per process (thread-safe static initialization)
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&dense_kernel<T, MB>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return true;
  }();
  (void)configured;
  using S = typename Dt<T>::st;
  const int tiles_n = static_cast<int>((n + kTileN - 1) / kTileN);
  const unsigned grid = static_cast<unsigned>(tiles_n * ((E + 7) / 8) * 8);
  hipLaunchKernelGGL((dense_kernel<T, MB>), dim3(grid), dim3(kThreads), lds, st, static_cast<S*>(c),
                     static_cast<const S*>(a), static_cast<const S*>(b), offs, E, tiles_n, rows, n, k);
}

template <typename T>
void run(void* c, const void* a, const void* b, const int32_t* offs, int E, int64_t rows,
         int64_t n, int64_t k, hipStream_t st) {
  constexpr int ES = Dt<T>::es;
  const bool tile = (k % (128 / ES) == 0) && ((n * ES) % 16 == 0) && aligned16(a) && aligned16(b);
  if (!tile) {
    using S = typename Dt<T>::st;
    hipLaunchKernelGGL((dense_simple_kernel<T>),
                       dim3(static_cast<unsigned>((rows * n + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, st, static_cast<S*>(c), static_cast<const S*>(a),
                       static_cast<const S*>(b), offs, E, rows, n, k);
    return;
  }
  // Pass height from the average rows per expert: an expert taller than a
  // pass streams its weights once more per pass, a pass taller than the
  // expert spends MFMAs on rows that are not stored.
  const int64_t avg = (rows + E - 1) / E;
  if (avg <= 16) launch_tile<T, 1>(c, a, b, offs, E, rows, n, k, st);
  else if (avg <= 32) launch_tile<T, 2>(c, a, b, offs, E, rows, n, k, st);
  else launch_tile<T, 4>(c, a, b, offs, E, rows, n, k, st);
}

}  // namespace moed
}  // namespace ks

extern "C" {

// moe_grouped_gemm.cu:136-198: same arguments, checks and statuses.
ks_status_t ks_moe_grouped_gemm(void* c, const void* a, const void* b,
                                const int32_t* expert_offsets, int num_experts,
                                int64_t total_rows, int64_t n, int64_t k, ks_dtype_t dtype,
                                ks_stream_t stream) {
  KS_REQUIRE_PTR(c);
  KS_REQUIRE_PTR(a);
  KS_REQUIRE_PTR(b);
  KS_REQUIRE_PTR(expert_offsets);
  if (num_experts <= 0 || total_rows < 0 || n <= 0 || k <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_moe_grouped_gemm: bad shape");
  if (dtype != KS_DTYPE_F32 && dtype != KS_DTYPE_F16 && dtype != KS_DTYPE_BF16 &&
      dtype != KS_DTYPE_F8E4M3 && dtype != KS_DTYPE_F8E5M2)
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_moe_grouped_gemm: unsupported dtype");
  if (total_rows == 0) return KS_SUCCESS;  // nothing routed
  if (num_experts > 65535 ||
      (n + ks::moed::kTileN - 1) / ks::moed::kTileN * (num_experts + 7) > (int64_t{1} << 30) ||
      total_rows * n / ks::moed::kThreads > 2147483647LL)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_moe_grouped_gemm: shape exceeds grid limits");
  auto st = ks::to_stream(stream);
  switch (dtype) {
    case KS_DTYPE_F32:
      ks::moed::run<ks::f32_t>(c, a, b, expert_offsets, num_experts, total_rows, n, k, st);
      break;
    case KS_DTYPE_F16:
      ks::moed::run<ks::f16_t>(c, a, b, expert_offsets, num_experts, total_rows, n, k, st);
      break;
    case KS_DTYPE_BF16:
      ks::moed::run<ks::bf16_t>(c, a, b, expert_offsets, num_experts, total_rows, n, k, st);
      break;
    case KS_DTYPE_F8E4M3:
      ks::moed::run<ks::e4m3_t>(c, a, b, expert_offsets, num_experts, total_rows, n, k, st);
      break;
    default:
      ks::moed::run<ks::e5m2_t>(c, a, b, expert_offsets, num_experts, total_rows, n, k, st);
      break;
  }
  KS_LAUNCH_STATUS("ks_moe_grouped_gemm");
  return KS_SUCCESS;
}

}  // extern "C"
