// kernel-set (MI355X build) -- shared definitions of the 8-bit MFMA GEMMs
// (gemm8.hip and gemm8_skinny.hpp): operand kinds, vector types and the kernel
// argument block.
#pragma once

#include <cstdint>

#include "ks_common.hpp"

namespace ks {
namespace gemm8 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kLdsStride = kBK + 16;  // bytes per LDS row (16 B pad vs bank conflicts)

// FP8_*: blockwise-scaled (ks_gemm_fp8_blockwise); FP8P_*: plain fp32
// accumulation over all of K with per-token/per-channel scales (ks_gemm_fp8).
enum Kind { FP8_E4M3 = 0, FP8_E5M2 = 1, INT8 = 2, INT8_RAW = 3, FP8P_E4M3 = 4, FP8P_E5M2 = 5 };

constexpr bool is_fp8_block(int kind) { return kind == FP8_E4M3 || kind == FP8_E5M2; }
constexpr bool is_fp8_plain(int kind) { return kind == FP8P_E4M3 || kind == FP8P_E5M2; }
constexpr int fp8_fmt(int kind) { return (kind == FP8_E5M2 || kind == FP8P_E5M2) ? 1 : 0; }

struct Args {
  void* out;
  const uint8_t* a;
  const uint8_t* b;
  const float* a_scale;
  const float* b_scale;
  const void* bias;
  int64_t m, n, k;
  int block_n, block_k;    // fp8 blockwise
  int64_t nkb, nnb;        // scale grid dims
  int a_per_token, b_per_channel;  // w8a8
  int splits;                      // skinny path: K splits
  void* ws;                        // skinny path: split partial plane
  const void* a_in;                // fused quantize + GEMM: unquantized activations [M, K]
  float* a_scale_out;              // fused int8: workgroup 0 publishes the activation scales
};

}  // namespace gemm8
}  // namespace ks
