// kernel-set (MI355X build) -- shared host/device helpers for every HIP source.
//
// Contents:
//   * status/error plumbing behind ks_last_error_string (same message
//     conventions as the reference: "null arg: <name>", "<func>: <hip msg>",
//     kernels/src/common/dispatch.cuh:23-50 of cklxx/kernel-set);
//   * element load/store for f32 / f16 / bf16 with round-to-nearest-even;
//   * OCP fp8 (e4m3fn, e5m2) encode with saturation to the finite maximum and
//     decode, written from the OCP 8-bit floating point specification;
//   * wave64 reductions.
// Everything here is gfx950-only: wave size 64 is assumed, not queried.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "kernel_set/types.h"

namespace ks {

// ---------------------------------------------------------------------------
// Error plumbing (host)
// ---------------------------------------------------------------------------
void set_last_error(const std::string& msg);

inline ks_status_t check_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return KS_SUCCESS;
  set_last_error(std::string(where) + ": " + hipGetErrorString(e));
  return KS_ERROR_CUDA;
}

inline hipStream_t to_stream(ks_stream_t s) {
  return reinterpret_cast<hipStream_t>(s);
}

}  // namespace ks

#define KS_FAIL(status, msg)       \
  do {                             \
    ::ks::set_last_error(msg);     \
    return (status);               \
  } while (0)

#define KS_REQUIRE_PTR(p)                                          \
  do {                                                             \
    if ((p) == nullptr)                                            \
      KS_FAIL(KS_ERROR_INVALID_ARGUMENT, "null arg: " #p);         \
  } while (0)

// After a launch: report a launch error as KS_ERROR_CUDA "<func>: <msg>".
#define KS_LAUNCH_STATUS(func)                                              \
  do {                                                                      \
    ks_status_t _st = ::ks::check_hip(hipGetLastError(), func);             \
    if (_st != KS_SUCCESS) return _st;                                      \
  } while (0)

namespace ks {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load: marked non-temporal so single-use weight bytes do not
// evict data that is reused (activations, scales, partials).
__device__ inline uint4 load_stream16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---------------------------------------------------------------------------
// 16-bit float storage. Values are carried as raw uint16_t bits so one kernel
// template serves f16 and bf16; the tag types below pick the conversion.
// ---------------------------------------------------------------------------
struct f32_t {
  using storage = float;
};
struct f16_t {
  using storage = uint16_t;
};
struct bf16_t {
  using storage = uint16_t;
};

__device__ inline float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN (its top 16 bits
// with the quiet bit set). gfx950 converts in hardware (v_cvt_pk_bf16_f32);
// checked on MI355X against the integer form
//   NaN: (u >> 16) | 0x40, else (u + 0x7fff + ((u >> 16) & 1)) >> 16
// for all 2^32 inputs, with no difference.
__device__ inline uint16_t f32_to_bf16_bits(float f) {
  const __bf16 b = static_cast<__bf16>(f);
  uint16_t u;
  __builtin_memcpy(&u, &b, 2);
  return u;
}

__device__ inline float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return static_cast<float>(v);
}

__device__ inline uint16_t f32_to_f16_bits(float f) {
  _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32: round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

template <typename T>
struct elem;

template <>
struct elem<f32_t> {
  static constexpr int bytes = 4;
  __device__ static inline float load(const float* p, int64_t i) { return p[i]; }
  __device__ static inline float to_f32(float v) { return v; }
  __device__ static inline float from_f32(float v) { return v; }
};

template <>
struct elem<f16_t> {
  static constexpr int bytes = 2;
  __device__ static inline float load(const uint16_t* p, int64_t i) {
    return f16_bits_to_f32(p[i]);
  }
  __device__ static inline float to_f32(uint16_t v) { return f16_bits_to_f32(v); }
  __device__ static inline uint16_t from_f32(float v) { return f32_to_f16_bits(v); }
};

template <>
struct elem<bf16_t> {
  static constexpr int bytes = 2;
  __device__ static inline float load(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
  }
  __device__ static inline float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ static inline uint16_t from_f32(float v) { return f32_to_bf16_bits(v); }
};

// ---------------------------------------------------------------------------
// OCP fp8 encoders (round to nearest even, saturate to the finite max, NaN ->
// 0x7f). Derivation, e4m3fn (bias 7, max 1.75*2^8 = 448, min normal 2^-6,
// subnormal step 2^-9):
//   |x| >= 2^-6 : the fp32 exponent/mantissa fields shifted right by 20 keep 3
//                 mantissa bits; adding 0x7ffff + lsb before the shift rounds
//                 to nearest even, and subtracting (127-7)<<3 rebiases. A carry
//                 out of the mantissa bumps the exponent, which is the correct
//                 encoding of the rounded value.
//   |x| <  2^-6 : the code equals rint(|x| * 2^9) (0..8); 8 is the encoding of
//                 2^-6, so rounding up into the normal range is also right.
// e5m2 is the same with bias 15, 2 mantissa bits, max 1.75*2^15 = 57344,
// min normal 2^-14, subnormal step 2^-16.
// ---------------------------------------------------------------------------
__device__ inline uint8_t f32_to_e4m3(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7f;             // NaN
  if (a > 0x43e00000u) return sign | 0x7eu;     // > 448 (incl. inf): saturate
  uint32_t code;
  if (a >= 0x3c800000u) {                       // >= 2^-6: normal
    code = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
  } else {
    code = static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 512.0f));
  }
  return static_cast<uint8_t>(sign | code);
}

__device__ inline uint8_t f32_to_e5m2(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7f;             // NaN
  if (a > 0x47600000u) return sign | 0x7bu;     // > 57344 (incl. inf): saturate
  uint32_t code;
  if (a >= 0x38800000u) {                       // >= 2^-14: normal
    code = ((a + 0xfffffu + ((a >> 21) & 1u)) >> 21) - (112u << 2);
  } else {
    code = static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 65536.0f));
  }
  return static_cast<uint8_t>(sign | code);
}

// Decoders (exact). e4m3fn: exponent field 15 with mantissa 7 is NaN.
__device__ inline float e4m3_to_f32(uint8_t c) {
  const uint32_t sign = static_cast<uint32_t>(c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  if (e == 15u && m == 7u) return __uint_as_float(0x7fc00000u | sign);
  float mag;
  if (e == 0u) {
    mag = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  } else {
    mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}

__device__ inline float e5m2_to_f32(uint8_t c) {
  const uint32_t sign = static_cast<uint32_t>(c & 0x80u) << 24;
  const uint32_t e = (c >> 2) & 0x1fu, m = c & 3u;
  if (e == 31u) return __uint_as_float((m ? 0x7fc00000u : 0x7f800000u) | sign);
  float mag;
  if (e == 0u) {
    mag = static_cast<float>(m) * 1.52587890625e-05f;  // m * 2^-16
  } else {
    mag = __uint_as_float(((e + 112u) << 23) | (m << 21));
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}

struct e4m3_t {
  static constexpr float qmax = 448.0f;
  __device__ static inline uint8_t enc(float x) { return f32_to_e4m3(x); }
  __device__ static inline float dec(uint8_t c) { return e4m3_to_f32(c); }
};
struct e5m2_t {
  static constexpr float qmax = 57344.0f;
  __device__ static inline uint8_t enc(float x) { return f32_to_e5m2(x); }
  __device__ static inline float dec(uint8_t c) { return e5m2_to_f32(c); }
};

constexpr float kEpsScale = 1e-12f;  // floor of every dynamic scale
constexpr float kInt8Max = 127.0f;

// Dynamic quantization scale of a group/row/tensor with max |x| = amax
// (quant_fp8_group.cu:94-106 of cklxx/kernel-set): IEEE-correct fp32 divide,
// floored at kEpsScale. Codes are then enc(x * (1.0f / scale)).
template <typename Enc>
__device__ inline float scale_from_amax(float amax) {
  return fmaxf(amax / Enc::qmax, kEpsScale);
}

// Eight scaled values -> eight fp8 codes (two dwords, element i in byte i % 4
// of dword i / 4). fp8 codes come from the hardware converters
// (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32, round to nearest even): every value
// they see is x * (1/s) with s >= amax/qmax, so |x/s| <= qmax(1 + 2^-23) and
// the saturating and non-saturating conversions give the same code.
template <typename Enc>
struct enc8;  // specialized per code type

// NaN codes are canonicalized to 0x7F (the code the reference's
// __nv_fp8_e4m3 / __nv_fp8_e5m2 conversions give for the canonical NaN, and
// the software encoders' code). The hardware converters keep a NaN's sign, and
// the NaN this hardware produces for an invalid operation (an infinite group
// amax gives inf * (1/inf) = inf * 0) has its sign bit set. Per byte b (SWAR):
// e4m3 NaN iff (b & 0x7f) == 0x7f; e5m2 NaN iff (b & 0x7f) > 0x7c (no infinity
// code can arise here: every other input is finite and |x * inv| <= qmax).
__device__ inline uint32_t canon_nan_e4m3(uint32_t c) {
  const uint32_t nan_sign = ((c & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
  return c & ~nan_sign;  // 0xff -> 0x7f
}
__device__ inline uint32_t canon_nan_e5m2(uint32_t c) {
  const uint32_t nan_hi = ((c & 0x7f7f7f7fu) + 0x03030303u) & 0x80808080u;
  const uint32_t m = (nan_hi >> 7) * 0xffu;  // 0xff in each NaN byte
  return (c & ~m) | (0x7f7f7f7fu & m);
}

template <>
struct enc8<e4m3_t> {
  __device__ static inline uint2 run(const float v[8], float inv) {
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] * inv, v[1] * inv, 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] * inv, v[3] * inv, lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4] * inv, v[5] * inv, 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6] * inv, v[7] * inv, hi, true);
    return make_uint2(canon_nan_e4m3(static_cast<uint32_t>(lo)),
                      canon_nan_e4m3(static_cast<uint32_t>(hi)));
  }
};

template <>
struct enc8<e5m2_t> {
  __device__ static inline uint2 run(const float v[8], float inv) {
    int lo = __builtin_amdgcn_cvt_pk_bf8_f32(v[0] * inv, v[1] * inv, 0, false);
    lo = __builtin_amdgcn_cvt_pk_bf8_f32(v[2] * inv, v[3] * inv, lo, true);
    int hi = __builtin_amdgcn_cvt_pk_bf8_f32(v[4] * inv, v[5] * inv, 0, false);
    hi = __builtin_amdgcn_cvt_pk_bf8_f32(v[6] * inv, v[7] * inv, hi, true);
    return make_uint2(canon_nan_e5m2(static_cast<uint32_t>(lo)),
                      canon_nan_e5m2(static_cast<uint32_t>(hi)));
  }
};


// int8 code: round-half-even of the scaled value clamped to [-127, 127]
// (quant_int8.cu:44 and :80 of cklxx/kernel-set).
struct i8_t {
  static constexpr float qmax = kInt8Max;
  __device__ static inline uint8_t enc(float v) {
    // Same comparison order as a clamp written v<lo?lo:(v>hi?hi:v).
    const float c = v < -kInt8Max ? -kInt8Max : (v > kInt8Max ? kInt8Max : v);
    return static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(__builtin_rintf(c))));
  }
};

template <>
struct enc8<i8_t> {
  __device__ static inline uint2 run(const float v[8], float inv) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= static_cast<uint32_t>(i8_t::enc(v[i] * inv)) << (8 * i);
      hi |= static_cast<uint32_t>(i8_t::enc(v[i + 4] * inv)) << (8 * i);
    }
    return make_uint2(lo, hi);
  }
};

// ---------------------------------------------------------------------------
// wave64 reductions (xor butterflies over all 64 lanes)
// ---------------------------------------------------------------------------
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Max over aligned groups of `width` lanes (width a power of two <= 64).
// Direct global -> LDS copy: lane i's `Bytes` (4 or 16) land at lds + i*Bytes
// (lds must be the same for the whole wave). Issued as inline asm so the
// compiler does not treat later LDS reads as depending on it (it would insert
// a full vmcnt(0) wait before every LDS read, serializing a load ring); the
// caller orders it explicitly with s_waitcnt vmcnt + s_barrier. M0 is saved
// and restored around the instruction.
template <int Bytes>
__device__ inline void dma_to_lds(const void* gptr, const void* lds) {
  static_assert(Bytes == 4 || Bytes == 16, "dword or dwordx4");
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  uint32_t saved;
  if constexpr (Bytes == 16)
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved) : "v"(gptr), "s"(l) : "memory");
  else
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
        "global_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved) : "v"(gptr), "s"(l) : "memory");
}

// Same copy addressed as a wave-uniform base plus a 32-bit per-lane byte
// offset (saddr form): one VGPR per lane instead of a 64-bit address pair.
template <int Bytes>
__device__ inline void dma_to_lds_off(const void* sbase, uint32_t voff, const void* lds) {
  static_assert(Bytes == 4 || Bytes == 16, "dword or dwordx4");
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  uint32_t saved;
  if constexpr (Bytes == 16)
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(l) : "memory");
  else
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved) : "v"(voff), "s"(sbase), "s"(l) : "memory");
}

// Workgroup barrier that emits no memory-counter waits of its own (the
// caller has already waited for what it needs); also a compiler barrier.
__device__ inline void barrier_no_wait() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ inline float group_max(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace ks
