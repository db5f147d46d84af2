// kernel-set (MI355X build) -- dynamic activation quantizers, their dequant
// partners, and the int4 weight-format helpers.
//
// Arithmetic contract (shared with the CPU oracle, bit for bit):
//   amax  = max |float(x)|                         (fmaxf: NaN inputs ignored)
//   scale = fmaxf(amax / qmax, 1e-12f)             (IEEE-correct fp32 divide)
//   inv   = 1.0f / scale                           (IEEE-correct fp32 divide)
//   fp8   : code = enc_rne_satfinite(float(x) * inv)
//   int8  : code = rint(clamp(float(x) * inv, -127, 127))
// as in kernels/src/quant/quant_fp8_group.cu:94-106, quant_fp8.cu:51-65 and
// quant_int8.cu:32-45 of cklxx/kernel-set.
//
// MI355X layout: these passes are HBM-bound byte streams. Every fast path
// moves 16 B per lane per load (8 x 16-bit or 2 x 4 x f32), keeps the data it
// must revisit in registers (one HBM read per element), and reduces amax with
// wave64 xor-shuffles; scales are written by one lane per group/row.
#include <type_traits>

#include "kernel_set/quant.h"
#include "kernel_set/testing.h"
#include "ks_common.hpp"

namespace ks {
namespace quant {

constexpr int kThreads = 256;  // 4 waves per workgroup

// ---- 8-element vector loads into fp32 ------------------------------------
template <typename T>
__device__ inline void load8(const typename T::storage* p, float v[8]);

template <>
__device__ inline void load8<bf16_t>(const uint16_t* p, float v[8]) {
  const uint4 w = load_stream16(p);
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(d[i] << 16);
    v[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
  }
}

template <>
__device__ inline void load8<f16_t>(const uint16_t* p, float v[8]) {
  const uint4 w = load_stream16(p);
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = f16_bits_to_f32(static_cast<uint16_t>(d[i] & 0xffffu));
    v[2 * i + 1] = f16_bits_to_f32(static_cast<uint16_t>(d[i] >> 16));
  }
}

template <>
__device__ inline void load8<f32_t>(const float* p, float v[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ---- encoders: scaled fp32 value -> one code byte -------------------------
// i8_t (the int8 encoder) and its enc8 live in ks_common.hpp.


template <typename Enc>
__device__ inline void store8(uint8_t* dst, const float v[8], float inv) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo |= static_cast<uint32_t>(Enc::enc(v[i] * inv)) << (8 * i);
    hi |= static_cast<uint32_t>(Enc::enc(v[i + 4] * inv)) << (8 * i);
  }
  *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
}

// ===========================================================================
// Per-(row, group) quantization, vector path.
// A "slot" of L = group_size/8 lanes (power of two, <= 64) owns one group; each
// lane holds 8 consecutive elements in registers, so the amax reduction and the
// encode pass share one HBM read. Slots are packed densely over the grid, so a
// wave covers 64/L consecutive groups of one row (or the tail of one row and
// the head of the next): 16 B per lane, contiguous across the wave.
// fp8 codes come from the hardware converters (v_cvt_pk_fp8_f32 /
// v_cvt_pk_bf8_f32, round to nearest even): every value they see is x * (1/s)
// with s >= amax/qmax, so |x/s| <= qmax(1 + 2^-23) and both the saturating
// and the non-saturating conversion give the same code. Index math is 32-bit
// when the tensor allows it (Idx = uint32_t), with L a compile-time power of 2.
// ===========================================================================
// enc8<e4m3_t> / enc8<e5m2_t> (hardware converters) live in ks_common.hpp.
}  // namespace quant



namespace quant {

constexpr int kGroupUnroll = 1;  // slots per thread (2 and 4 measured slower)
constexpr unsigned kLoopBlocks = 2048;  // persistent grid of the per-block quantizer

template <typename In, typename Enc, int LOG_L, typename Idx>
__global__ void __launch_bounds__(kThreads)
group_quant_vec_kernel(uint8_t* __restrict__ out, float* __restrict__ scale,
                       const typename In::storage* __restrict__ in,
                       Idx rows, Idx cols, Idx group_size, Idx ngroups) {
  constexpr int L = 1 << LOG_L;
  constexpr int U = kGroupUnroll;
  const Idx base = static_cast<Idx>(blockIdx.x) * (kThreads * U) + threadIdx.x;
  const int sub = static_cast<int>(threadIdx.x & (L - 1));
  const Idx nslots = rows * ngroups;
  float v[U][8];
  float amax[U];
  Idx off[U], sidx[U];
  bool live[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {  // issue every load before any math
    const Idx slot = (base + static_cast<Idx>(u) * kThreads) >> LOG_L;
    const bool live_slot = slot < nslots;
    const Idx row = live_slot ? slot / ngroups : 0;
    const Idx grp = live_slot ? slot - row * ngroups : 0;
    const Idx col = grp * group_size + static_cast<Idx>(sub) * 8;
    live[u] = live_slot && col < cols;
    off[u] = live[u] ? row * cols + col : 0;  // unconditional load (branch-free)
    sidx[u] = row * ngroups + grp;
    amax[u] = 0.f;
    load8<In>(in + off[u], v[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) amax[u] = fmaxf(amax[u], live[u] ? fabsf(v[u][i]) : 0.f);
    amax[u] = group_max(amax[u], L);
    const float sc = scale_from_amax<Enc>(amax[u]);
    const float inv = 1.0f / sc;
    if (live[u]) {
      const uint2 code = enc8<Enc>::run(v[u], inv);
      __builtin_nontemporal_store(code.x, reinterpret_cast<uint32_t*>(out + off[u]));
      __builtin_nontemporal_store(code.y, reinterpret_cast<uint32_t*>(out + off[u]) + 1);
      if (sub == 0) scale[sidx[u]] = sc;
    }
  }
}

// Persistent variant: a fixed grid walks the slots with stride gridDim *
// kThreads, loading slot i+1 before it quantizes slot i.
template <typename In, typename Enc, int LOG_L, typename Idx>
__global__ void __launch_bounds__(kThreads)
group_quant_loop_kernel(uint8_t* __restrict__ out, float* __restrict__ scale,
                        const typename In::storage* __restrict__ in,
                        Idx rows, Idx cols, Idx group_size, Idx ngroups) {
  constexpr int L = 1 << LOG_L;
  const int sub = static_cast<int>(threadIdx.x & (L - 1));
  const Idx nthreads = rows * ngroups * L;
  const Idx stride = static_cast<Idx>(gridDim.x) * kThreads;
  Idx tid = static_cast<Idx>(blockIdx.x) * kThreads + threadIdx.x;
  auto locate = [&](Idx t, Idx* off, Idx* sidx, bool* live) {
    const Idx slot = t >> LOG_L;
    const bool ls = t < nthreads;
    const Idx row = ls ? slot / ngroups : 0;
    const Idx grp = ls ? slot - row * ngroups : 0;
    const Idx col = grp * group_size + static_cast<Idx>(sub) * 8;
    *live = ls && col < cols;
    *off = *live ? row * cols + col : 0;
    *sidx = row * ngroups + grp;
  };
  Idx off, sidx;
  bool live;
  locate(tid, &off, &sidx, &live);
  float v[8];
  load8<In>(in + off, v);
  // every lane of a wave runs the same number of rounds (uniform trip count)
  const Idx wave0 = tid - (threadIdx.x & (kWave - 1));
  for (Idx t0 = wave0; t0 < nthreads; t0 += stride) {
    Idx noff, nsidx;
    bool nlive;
    locate(tid + stride, &noff, &nsidx, &nlive);
    float nv[8];
    load8<In>(in + noff, nv);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, live ? fabsf(v[i]) : 0.f);
    amax = group_max(amax, L);
    const float sc = scale_from_amax<Enc>(amax);
    const float inv = 1.0f / sc;
    if (live) {
      const uint2 code = enc8<Enc>::run(v, inv);
      __builtin_nontemporal_store(code.x, reinterpret_cast<uint32_t*>(out + off));
      __builtin_nontemporal_store(code.y, reinterpret_cast<uint32_t*>(out + off) + 1);
      if (sub == 0) scale[sidx] = sc;
    }
    tid += stride;
    off = noff; sidx = nsidx; live = nlive;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = nv[i];
  }
}

// Generic per-(row, group): one wave per group, element-wise, two passes over
// the group (the second pass re-reads from cache). Serves any group size and
// any alignment.
template <typename In, typename Enc>
__global__ void __launch_bounds__(kThreads)
group_quant_scalar_kernel(uint8_t* __restrict__ out, float* __restrict__ scale,
                          const typename In::storage* __restrict__ in,
                          int64_t rows, int64_t cols, int group_size,
                          int64_t ngroups) {
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  if (wave >= rows * ngroups) return;  // whole wave exits together
  const int64_t row = wave / ngroups, grp = wave % ngroups;
  const int64_t c0 = grp * group_size;
  const int64_t c1 = (c0 + group_size < cols) ? c0 + group_size : cols;
  const typename In::storage* x = in + row * cols;
  float amax = 0.f;
  for (int64_t c = c0 + lane; c < c1; c += kWave) amax = fmaxf(amax, fabsf(elem<In>::load(x, c)));
  amax = wave_max(amax);
  const float sc = scale_from_amax<Enc>(amax);
  const float inv = 1.0f / sc;
  if (lane == 0) scale[row * ngroups + grp] = sc;
  for (int64_t c = c0 + lane; c < c1; c += kWave)
    out[row * cols + c] = Enc::enc(elem<In>::load(x, c) * inv);
}

// ===========================================================================
// Per-row (per-token) quantization: one 256-thread workgroup per row.
// Vector path keeps up to kRowCache x 8 elements per lane in registers
// (rows up to 256*8*kRowCache elements are read once); longer rows re-read.
// ===========================================================================
constexpr int kRowCache = 8;

__device__ inline float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x % kWave) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / kWave; ++i) r = fmaxf(r, red[i]);
  return r;
}

template <typename In, typename Enc>
__global__ void __launch_bounds__(kThreads)
row_quant_vec_kernel(uint8_t* __restrict__ out, float* __restrict__ scale,
                     const typename In::storage* __restrict__ in, int64_t cols) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const typename In::storage* x = in + row * cols;
  uint8_t* y = out + row * cols;
  const int64_t nvec = cols / 8;
  const bool cached = nvec <= static_cast<int64_t>(kThreads) * kRowCache;

  float v[kRowCache][8];
  float amax = 0.f;
  if (cached) {
#pragma unroll
    for (int r = 0; r < kRowCache; ++r) {
      const int64_t vi = static_cast<int64_t>(r) * kThreads + threadIdx.x;
      if (vi < nvec) {
        load8<In>(x + vi * 8, v[r]);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[r][i]));
      }
    }
  } else {
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kThreads) {
      float t[8];
      load8<In>(x + vi * 8, t);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(t[i]));
    }
  }
  amax = block_max(amax, red);
  const float sc = scale_from_amax<Enc>(amax);
  const float inv = 1.0f / sc;
  if (threadIdx.x == 0) scale[row] = sc;
  if (cached) {
#pragma unroll
    for (int r = 0; r < kRowCache; ++r) {
      const int64_t vi = static_cast<int64_t>(r) * kThreads + threadIdx.x;
      if (vi < nvec) store8<Enc>(y + vi * 8, v[r], inv);
    }
  } else {
    for (int64_t vi = threadIdx.x; vi < nvec; vi += kThreads) {
      float t[8];
      load8<In>(x + vi * 8, t);
      store8<Enc>(y + vi * 8, t, inv);
    }
  }
}

template <typename In, typename Enc>
__global__ void __launch_bounds__(kThreads)
row_quant_scalar_kernel(uint8_t* __restrict__ out, float* __restrict__ scale,
                        const typename In::storage* __restrict__ in, int64_t cols) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const typename In::storage* x = in + row * cols;
  float amax = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads)
    amax = fmaxf(amax, fabsf(elem<In>::load(x, c)));
  amax = block_max(amax, red);
  const float sc = scale_from_amax<Enc>(amax);
  const float inv = 1.0f / sc;
  if (threadIdx.x == 0) scale[row] = sc;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads)
    out[row * cols + c] = Enc::enc(elem<In>::load(x, c) * inv);
}

// ===========================================================================
// Per-tensor quantization: zero -> amax (atomicMax on the bit pattern of a
// non-negative float, which orders like the value) -> encode -> finalize.
// scale[0] holds amax until the finalize kernel turns it into the scale. The
// zeroing is a kernel, not a memset, so the sequence can be graph-captured.
// ===========================================================================
__global__ void zero_f32_kernel(float* p) { *p = 0.f; }

template <typename In>
__global__ void __launch_bounds__(kThreads)
tensor_amax_kernel(float* __restrict__ amax_out, const typename In::storage* __restrict__ in,
                   int64_t numel) {
  __shared__ float red[kThreads / kWave];
  float amax = 0.f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride)
    amax = fmaxf(amax, fabsf(elem<In>::load(in, i)));
  amax = block_max(amax, red);
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<int*>(amax_out), __float_as_int(amax));
}

template <typename In, typename Enc>
__global__ void __launch_bounds__(kThreads)
tensor_encode_kernel(uint8_t* __restrict__ out, const float* __restrict__ amax_in,
                     const typename In::storage* __restrict__ in, int64_t numel) {
  const float inv = 1.0f / scale_from_amax<Enc>(*amax_in);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride)
    out[i] = Enc::enc(elem<In>::load(in, i) * inv);
}

template <typename Enc>
__global__ void tensor_finalize_kernel(float* scale) {
  *scale = scale_from_amax<Enc>(*scale);
}

// ===========================================================================
// Dequantization: out = float(code) * scale (per-token or per-tensor).
// ===========================================================================
struct i8_dec {
  __device__ static inline float dec(uint8_t c) {
    return static_cast<float>(static_cast<int8_t>(c));
  }
};

template <typename Out, typename Dec>
__global__ void __launch_bounds__(kThreads)
dequant_kernel(typename Out::storage* __restrict__ out, const uint8_t* __restrict__ in,
               const float* __restrict__ scale, int64_t rows, int64_t cols,
               bool per_token) {
  const int64_t numel = rows * cols;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride) {
    const float sc = per_token ? scale[i / cols] : scale[0];
    out[i] = elem<Out>::from_f32(Dec::dec(in[i]) * sc);
  }
}

// ===========================================================================
// int4 weight helpers.
// repack: int32 [K/8, N] -> uint8 [K/2, N]. Packed byte kp of column n holds
// codes k=2kp (bits 0-3) and 2kp+1 (bits 4-7); both live in byte (kp % 4) of
// input word (kp/4, n), so without a permutation the repack is a byte gather.
// With an act-order permutation, output code k is input code perm[k].
// ===========================================================================
__global__ void __launch_bounds__(kThreads)
repack_int4_kernel(uint8_t* __restrict__ out, const uint32_t* __restrict__ in,
                   int64_t k, int64_t n) {
  const int64_t numel = (k / 2) * n;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride) {
    const int64_t kp = i / n, col = i % n;
    const uint32_t word = in[(kp >> 2) * n + col];
    out[i] = static_cast<uint8_t>(word >> (8 * (kp & 3)));
  }
}

__device__ inline uint32_t int4_code(const uint32_t* in, int64_t krow, int64_t n, int64_t col) {
  return (in[(krow >> 3) * n + col] >> (4 * (krow & 7))) & 0xfu;
}

__global__ void __launch_bounds__(kThreads)
repack_int4_perm_kernel(uint8_t* __restrict__ out, const uint32_t* __restrict__ in,
                        const int32_t* __restrict__ perm, int64_t k, int64_t n) {
  const int64_t numel = (k / 2) * n;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride) {
    const int64_t kp = i / n, col = i % n;
    const uint32_t lo = int4_code(in, perm[2 * kp], n, col);
    const uint32_t hi = int4_code(in, perm[2 * kp + 1], n, col);
    out[i] = static_cast<uint8_t>(lo | (hi << 4));
  }
}

// dequant_int4 (kernels/src/quant/dequant_int4.cu:35-60 of the reference):
// out[k,n] = (float(code) - float(zero[g,n])) * float(scale[g,n]), g = k/gs.
template <typename Out>
__global__ void __launch_bounds__(kThreads)
dequant_int4_kernel(typename Out::storage* __restrict__ out, const uint32_t* __restrict__ in,
                    const typename Out::storage* __restrict__ scales,
                    const typename Out::storage* __restrict__ zeros, int64_t k,
                    int64_t n, int group_size) {
  const int64_t numel = k * n;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < numel; i += stride) {
    const int64_t kk = i / n, col = i % n;
    const float q = static_cast<float>(int4_code(in, kk, n, col));
    const int64_t g = (kk / group_size) * n + col;
    out[i] = elem<Out>::from_f32((q - elem<Out>::load(zeros, g)) * elem<Out>::load(scales, g));
  }
}

inline unsigned stride_grid(int64_t numel) {
  int64_t g = (numel + kThreads - 1) / kThreads;
  if (g < 1) g = 1;
  if (g > 8192) g = 8192;  // 32 workgroups per CU on 256 CUs; loops cover the rest
  return static_cast<unsigned>(g);
}

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

template <typename T>
struct type_tag {
  using type = T;
};

// ---- host launchers (templated on input element and encoder) --------------
template <typename In, typename Enc>
void launch_group(uint8_t* out, float* scale, const void* input, int64_t rows,
                  int64_t cols, int gs, hipStream_t s) {
  const int64_t ngroups = (cols + gs - 1) / gs;
  using S = typename In::storage;
  const int lanes = gs / 8;
  const bool vec = (gs % 8 == 0) && (cols % 8 == 0) && lanes <= kWave &&
                   (lanes & (lanes - 1)) == 0 && aligned(input, 16) && aligned(out, 8);
  if (vec) {
    const int64_t threads = rows * ngroups * lanes;
    const int64_t per_block = static_cast<int64_t>(kThreads) * kGroupUnroll;
    const int64_t blocks = (threads + per_block - 1) / per_block;
    const bool small = blocks * per_block < (int64_t{1} << 31) && rows * cols < (int64_t{1} << 31);
    int log_l = 0;
    while ((1 << log_l) < lanes) ++log_l;
    auto go = [&](auto log_tag, auto idx_tag) {
      constexpr int LL = decltype(log_tag)::value;
      using I = typename decltype(idx_tag)::type;
      // Large inputs: a persistent grid of kLoopBlocks workgroups (measured on
      // MI355X at 2048x7168: 10.1 us against 10.6 us for one slot per thread;
      // 512 or 1024 workgroups were slower).
      if (blocks > kLoopBlocks)
        hipLaunchKernelGGL((group_quant_loop_kernel<In, Enc, LL, I>), dim3(kLoopBlocks),
                           dim3(kThreads), 0, s, out, scale, static_cast<const S*>(input),
                           static_cast<I>(rows), static_cast<I>(cols), static_cast<I>(gs),
                           static_cast<I>(ngroups));
      else
        hipLaunchKernelGGL((group_quant_vec_kernel<In, Enc, LL, I>),
                           dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, out,
                           scale, static_cast<const S*>(input), static_cast<I>(rows),
                           static_cast<I>(cols), static_cast<I>(gs), static_cast<I>(ngroups));
    };
    auto by_idx = [&](auto log_tag) {
      if (small) go(log_tag, type_tag<uint32_t>{});
      else go(log_tag, type_tag<int64_t>{});
    };
    switch (log_l) {
      case 0: by_idx(std::integral_constant<int, 0>{}); break;
      case 1: by_idx(std::integral_constant<int, 1>{}); break;
      case 2: by_idx(std::integral_constant<int, 2>{}); break;
      case 3: by_idx(std::integral_constant<int, 3>{}); break;
      case 4: by_idx(std::integral_constant<int, 4>{}); break;
      case 5: by_idx(std::integral_constant<int, 5>{}); break;
      default: by_idx(std::integral_constant<int, 6>{}); break;
    }
  } else {
    const int64_t waves = rows * ngroups;
    const int64_t blocks = (waves * kWave + kThreads - 1) / kThreads;
    hipLaunchKernelGGL((group_quant_scalar_kernel<In, Enc>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kThreads), 0, s, out, scale, static_cast<const S*>(input), rows,
                       cols, gs, ngroups);
  }
}

template <typename In, typename Enc>
void launch_row(uint8_t* out, float* scale, const void* input, int64_t rows,
                int64_t cols, hipStream_t s) {
  using S = typename In::storage;
  const bool vec = (cols % 8 == 0) && aligned(input, 16) && aligned(out, 8);
  if (vec)
    hipLaunchKernelGGL((row_quant_vec_kernel<In, Enc>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, s, out, scale, static_cast<const S*>(input), cols);
  else
    hipLaunchKernelGGL((row_quant_scalar_kernel<In, Enc>), dim3(static_cast<unsigned>(rows)),
                       dim3(kThreads), 0, s, out, scale, static_cast<const S*>(input), cols);
}

template <typename In, typename Enc>
void launch_tensor(uint8_t* out, float* scale, const void* input, int64_t numel,
                   hipStream_t s) {
  using S = typename In::storage;
  const unsigned g = stride_grid(numel);
  hipLaunchKernelGGL(zero_f32_kernel, dim3(1), dim3(1), 0, s, scale);
  hipLaunchKernelGGL((tensor_amax_kernel<In>), dim3(g), dim3(kThreads), 0, s, scale,
                     static_cast<const S*>(input), numel);
  hipLaunchKernelGGL((tensor_encode_kernel<In, Enc>), dim3(g), dim3(kThreads), 0, s, out,
                     scale, static_cast<const S*>(input), numel);
  hipLaunchKernelGGL((tensor_finalize_kernel<Enc>), dim3(1), dim3(1), 0, s, scale);
}

// Runtime dtype -> template dispatch for f32/f16/bf16 element tags.
template <template <typename> class F, typename... Args>
bool dispatch_float(ks_dtype_t dt, Args&&... args) {
  switch (dt) {
    case KS_DTYPE_F32: F<f32_t>::run(args...); return true;
    case KS_DTYPE_F16: F<f16_t>::run(args...); return true;
    case KS_DTYPE_BF16: F<bf16_t>::run(args...); return true;
    default: return false;
  }
}

template <typename Enc>
struct GroupOp {
  template <typename In>
  struct With {
    template <typename... A>
    static void run(A... a) { launch_group<In, Enc>(a...); }
  };
};
template <typename Enc>
struct RowOp {
  template <typename In>
  struct With {
    template <typename... A>
    static void run(A... a) { launch_row<In, Enc>(a...); }
  };
};
template <typename Enc>
struct TensorOp {
  template <typename In>
  struct With {
    template <typename... A>
    static void run(A... a) { launch_tensor<In, Enc>(a...); }
  };
};
template <typename Dec>
struct DequantOp {
  template <typename Out>
  struct With {
    static void run(void* out, const uint8_t* in, const float* scale, int64_t rows,
                    int64_t cols, bool per_token, hipStream_t s) {
      hipLaunchKernelGGL((dequant_kernel<Out, Dec>), dim3(stride_grid(rows * cols)),
                         dim3(kThreads), 0, s, static_cast<typename Out::storage*>(out), in,
                         scale, rows, cols, per_token);
    }
  };
};
template <typename Out>
struct DequantInt4Op {
  static void run(void* out, const uint32_t* in, const void* scales, const void* zeros,
                  int64_t k, int64_t n, int gs, hipStream_t s) {
    using S = typename Out::storage;
    hipLaunchKernelGGL((dequant_int4_kernel<Out>), dim3(stride_grid(k * n)), dim3(kThreads), 0,
                       s, static_cast<S*>(out), in, static_cast<const S*>(scales),
                       static_cast<const S*>(zeros), k, n, gs);
  }
};

// out[i] = the 16-bit output rounding every kernel applies (elem<Out>::from_f32)
// to the fp32 bit pattern start + i (test hook: no input buffer needed).
template <typename Out>
__global__ void __launch_bounds__(kThreads)
round_bits_kernel(uint16_t* __restrict__ out, uint32_t start, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    out[i] = elem<Out>::from_f32(__uint_as_float(start + static_cast<uint32_t>(i)));
}

}  // namespace quant
}  // namespace ks

using namespace ks;
using namespace ks::quant;

namespace {
bool is_fp8(ks_dtype_t d) { return d == KS_DTYPE_F8E4M3 || d == KS_DTYPE_F8E5M2; }
}  // namespace

extern "C" {

ks_status_t ks_quantize_fp8_group(void* out, float* scale, const void* input,
                                  int64_t rows, int64_t cols, int group_size,
                                  ks_dtype_t in_dtype, ks_dtype_t fp8_dtype,
                                  ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(scale);
  KS_REQUIRE_PTR(input);
  if (rows <= 0 || cols <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_fp8_group: bad shape");
  if (group_size <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_fp8_group: group_size must be > 0");
  if (!is_fp8(fp8_dtype))
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_quantize_fp8_group: fp8_dtype must be e4m3 or e5m2");
  const int64_t ngroups = (cols + group_size - 1) / group_size;
  // Each group occupies at least one lane; bound the flattened launch.
  if (rows > (int64_t{1} << 40) / ngroups)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_quantize_fp8_group: too many groups");
  auto s = to_stream(stream);
  auto* o = static_cast<uint8_t*>(out);
  bool ok = (fp8_dtype == KS_DTYPE_F8E4M3)
                ? dispatch_float<GroupOp<e4m3_t>::With>(in_dtype, o, scale, input, rows, cols, group_size, s)
                : dispatch_float<GroupOp<e5m2_t>::With>(in_dtype, o, scale, input, rows, cols, group_size, s);
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_quantize_fp8_group: unsupported dtype");
  KS_LAUNCH_STATUS("ks_quantize_fp8_group");
  return KS_SUCCESS;
}

ks_status_t ks_quantize_fp8(void* out, float* scale, const void* input,
                            int64_t rows, int64_t cols, ks_dtype_t in_dtype,
                            ks_dtype_t fp8_dtype, ks_quant_mode_t mode,
                            ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(scale);
  KS_REQUIRE_PTR(input);
  if (rows <= 0 || cols <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_fp8: bad shape");
  if (mode != KS_QUANT_PER_TENSOR && mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_fp8: mode must be per-tensor or per-token");
  if (!is_fp8(fp8_dtype))
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_quantize_fp8: fp8_dtype must be e4m3 or e5m2");
  if (mode == KS_QUANT_PER_TOKEN && rows > 2147483647LL)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_quantize_fp8: rows exceeds grid limit");
  auto s = to_stream(stream);
  auto* o = static_cast<uint8_t*>(out);
  const bool e4 = fp8_dtype == KS_DTYPE_F8E4M3;
  bool ok;
  if (mode == KS_QUANT_PER_TOKEN) {
    ok = e4 ? dispatch_float<RowOp<e4m3_t>::With>(in_dtype, o, scale, input, rows, cols, s)
            : dispatch_float<RowOp<e5m2_t>::With>(in_dtype, o, scale, input, rows, cols, s);
  } else {
    ok = e4 ? dispatch_float<TensorOp<e4m3_t>::With>(in_dtype, o, scale, input, rows * cols, s)
            : dispatch_float<TensorOp<e5m2_t>::With>(in_dtype, o, scale, input, rows * cols, s);
  }
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_quantize_fp8: unsupported dtype");
  KS_LAUNCH_STATUS("ks_quantize_fp8");
  return KS_SUCCESS;
}

ks_status_t ks_quantize_int8(void* out, float* scale, const void* input,
                             int64_t rows, int64_t cols, ks_dtype_t in_dtype,
                             ks_quant_mode_t mode, ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(scale);
  KS_REQUIRE_PTR(input);
  if (rows <= 0 || cols <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_int8: bad shape");
  if (mode != KS_QUANT_PER_TENSOR && mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_quantize_int8: mode must be per-tensor or per-token");
  if (mode == KS_QUANT_PER_TOKEN && rows > 2147483647LL)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_quantize_int8: rows exceeds grid limit");
  auto s = to_stream(stream);
  auto* o = static_cast<uint8_t*>(out);
  const bool ok = (mode == KS_QUANT_PER_TOKEN)
                      ? dispatch_float<RowOp<i8_t>::With>(in_dtype, o, scale, input, rows, cols, s)
                      : dispatch_float<TensorOp<i8_t>::With>(in_dtype, o, scale, input, rows * cols, s);
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_quantize_int8: unsupported dtype");
  KS_LAUNCH_STATUS("ks_quantize_int8");
  return KS_SUCCESS;
}

ks_status_t ks_dequantize_fp8(void* out, const void* input, const float* scale,
                              int64_t rows, int64_t cols, ks_dtype_t out_dtype,
                              ks_dtype_t fp8_dtype, ks_quant_mode_t mode,
                              ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(input);
  KS_REQUIRE_PTR(scale);
  if (rows <= 0 || cols <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_fp8: bad shape");
  if (mode != KS_QUANT_PER_TENSOR && mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_fp8: mode must be per-tensor or per-token");
  if (!is_fp8(fp8_dtype))
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_dequantize_fp8: fp8_dtype must be e4m3 or e5m2");
  auto s = to_stream(stream);
  const auto* in = static_cast<const uint8_t*>(input);
  const bool pt = mode == KS_QUANT_PER_TOKEN;
  const bool ok = (fp8_dtype == KS_DTYPE_F8E4M3)
                      ? dispatch_float<DequantOp<e4m3_t>::With>(out_dtype, out, in, scale, rows, cols, pt, s)
                      : dispatch_float<DequantOp<e5m2_t>::With>(out_dtype, out, in, scale, rows, cols, pt, s);
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_dequantize_fp8: unsupported dtype");
  KS_LAUNCH_STATUS("ks_dequantize_fp8");
  return KS_SUCCESS;
}

ks_status_t ks_dequantize_int8(void* out, const void* input, const float* scale,
                               int64_t rows, int64_t cols, ks_dtype_t out_dtype,
                               ks_quant_mode_t mode, ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(input);
  KS_REQUIRE_PTR(scale);
  if (rows <= 0 || cols <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_int8: bad shape");
  if (mode != KS_QUANT_PER_TENSOR && mode != KS_QUANT_PER_TOKEN)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_int8: mode must be per-tensor or per-token");
  auto s = to_stream(stream);
  const bool ok = dispatch_float<DequantOp<i8_dec>::With>(
      out_dtype, out, static_cast<const uint8_t*>(input), scale, rows, cols,
      mode == KS_QUANT_PER_TOKEN, s);
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_dequantize_int8: unsupported dtype");
  KS_LAUNCH_STATUS("ks_dequantize_int8");
  return KS_SUCCESS;
}

ks_status_t ks_dequantize_int4(void* out, const void* qweight_packed,
                               const void* scales, const void* zeros, int64_t k,
                               int64_t n, int group_size, ks_dtype_t out_dtype,
                               ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  KS_REQUIRE_PTR(qweight_packed);
  KS_REQUIRE_PTR(scales);
  KS_REQUIRE_PTR(zeros);
  if (k <= 0 || n <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_int4: bad shape");
  if (group_size <= 0)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_dequantize_int4: group_size must be > 0");
  if (k % 8 != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_dequantize_int4: K must be a multiple of 8 (8 codes/word)");
  if (k % group_size != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_dequantize_int4: K must be a multiple of group_size");
  auto s = to_stream(stream);
  const auto* in = static_cast<const uint32_t*>(qweight_packed);
  bool ok = true;
  switch (out_dtype) {
    case KS_DTYPE_F32: DequantInt4Op<f32_t>::run(out, in, scales, zeros, k, n, group_size, s); break;
    case KS_DTYPE_F16: DequantInt4Op<f16_t>::run(out, in, scales, zeros, k, n, group_size, s); break;
    case KS_DTYPE_BF16: DequantInt4Op<bf16_t>::run(out, in, scales, zeros, k, n, group_size, s); break;
    default: ok = false;
  }
  if (!ok) KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_dequantize_int4: unsupported dtype");
  KS_LAUNCH_STATUS("ks_dequantize_int4");
  return KS_SUCCESS;
}

ks_status_t ks_repack_int4(void* out_packed, const void* qweight, const void* perm,
                           int64_t size_k, int64_t size_n, int num_bits,
                           ks_stream_t stream) {
  KS_REQUIRE_PTR(out_packed);
  KS_REQUIRE_PTR(qweight);
  if (size_k <= 0 || size_n <= 0) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_repack_int4: bad shape");
  if (num_bits != 4) KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_repack_int4: only 4-bit supported");
  if (size_k % 8 != 0)
    KS_FAIL(KS_ERROR_UNSUPPORTED_SHAPE, "ks_repack_int4: K must be a multiple of 8 (8 codes/word)");
  auto s = to_stream(stream);
  const unsigned g = stride_grid((size_k / 2) * size_n);
  if (perm == nullptr)
    hipLaunchKernelGGL(repack_int4_kernel, dim3(g), dim3(kThreads), 0, s,
                       static_cast<uint8_t*>(out_packed), static_cast<const uint32_t*>(qweight),
                       size_k, size_n);
  else
    hipLaunchKernelGGL(repack_int4_perm_kernel, dim3(g), dim3(kThreads), 0, s,
                       static_cast<uint8_t*>(out_packed), static_cast<const uint32_t*>(qweight),
                       static_cast<const int32_t*>(perm), size_k, size_n);
  KS_LAUNCH_STATUS("ks_repack_int4");
  return KS_SUCCESS;
}

ks_status_t ks_testing_round_bits(void* out, uint32_t start, int64_t n, ks_dtype_t out_dtype,
                                  ks_stream_t stream) {
  KS_REQUIRE_PTR(out);
  if (n <= 0 || n > (int64_t{1} << 32) - start)
    KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "ks_testing_round_bits: bad range");
  auto s = to_stream(stream);
  const unsigned g = stride_grid(n);
  if (out_dtype == KS_DTYPE_BF16)
    hipLaunchKernelGGL((round_bits_kernel<bf16_t>), dim3(g), dim3(kThreads), 0, s,
                       static_cast<uint16_t*>(out), start, n);
  else if (out_dtype == KS_DTYPE_F16)
    hipLaunchKernelGGL((round_bits_kernel<f16_t>), dim3(g), dim3(kThreads), 0, s,
                       static_cast<uint16_t*>(out), start, n);
  else
    KS_FAIL(KS_ERROR_UNSUPPORTED_DTYPE, "ks_testing_round_bits: out_dtype must be bf16 or f16");
  KS_LAUNCH_STATUS("ks_testing_round_bits");
  return KS_SUCCESS;
}

}  // extern "C"
