// kernel-set (MI355X build) -- 8-bit GEMMs for decode shapes (M <= 8):
// ks_gemm_fp8_blockwise, ks_gemm_fp8 and ks_gemm_w8a8 when A has few rows.
//
// At these shapes the call streams B ([K, N], N contiguous) once from HBM and
// the MFMA work is small, so the kernel feeds B's bytes to the MFMA exactly as
// they are loaded, with no transpose and no LDS staging:
//
//  * Lane (li = lane % 16, g = lane / 16) loads 16 bytes = 16 columns of one
//    k-row; the 16 lanes of a lane group cover 256 contiguous bytes of that
//    row, and lane group g takes k-rows 8g..8g+7 of a 32-row chunk.
//  * Dword p of the 16-byte load holds columns 16*li + 4p + c (c = 0..3) of
//    its row. The lane's dword p from its 8 rows is an MFMA B operand of 32
//    byte slots, slot 4r + c = B[row r, column 16*li + 4p + c].
//  * The A operand is block-diagonal: MFMA row i = 4*q + c (q = activation row
//    within the fragment, c = column within the dword) carries A[q, row r] in
//    slot 4r + c and zeros elsewhere. Then D[4q + c][li] is the dot product of
//    activation row q with column 16*li + 4p + c over the chunk's 32 rows.
//    Slot order is the same for A and B, so it does not matter how the MFMA
//    orders its k slots. One v_perm per dword builds the A operand.
//  * fp8: one v_mfma_scale_f32_16x16x128_f8f6f4 per (row fragment, p);
//    int8: two v_mfma_i32_16x16x64_i8 (rows 0-3 and 4-7 of the lane group).
//    One fragment serves 4 activation rows, so M <= 4 costs what M = 1 costs
//    and M <= 8 uses two fragments.
//
// Output lane (li, g) of fragment f holds D rows 4g..4g+3 = activation row
// 4f + g, columns 16*li + 4p + r. A workgroup's 8 waves take consecutive K
// ranges of one 256-column tile; they are summed through LDS in a fixed order,
// and each K split writes a partial plane that skinny_reduce_kernel sums in
// split order before the epilogue. W8A8 partials are int32 and add exactly,
// so its results are identical to a single pass.
//
// fp8 blockwise (gemm_fp8_blockwise.cu:107-161 of cklxx/kernel-set): each
// 32-row chunk lies inside one scale block (block_k % 32 == 0); its fp32 chunk
// partial is promoted as O = fma(P, a_s * b_s, O). The reference promotes per
// whole block; per-chunk promotion changes only fp32 rounding.
#pragma once

#include <type_traits>

#include "gemm8_common.hpp"

namespace ks {
namespace gemm8 {
namespace skinny {

constexpr int kTileN = 256;   // columns per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;    // k-rows per chunk (8 per lane group)
constexpr int kMaxM = 8;

// Workgroup id -> (column tile, k split); the splits of one tile share an XCD
// when the grid divides into the 8 XCDs (ids are dispatched round-robin).
__device__ inline void map_tile(int bid, int nblocks, int splits, int* tile, int* split) {
  int logical = bid;
  if ((nblocks & 7) == 0) logical = (bid & 7) * (nblocks >> 3) + (bid >> 3);
  *tile = logical / splits;
  *split = logical % splits;
}

// Unquantized activations of the fused path: 8 consecutive elements as raw
// words (plain loads: every column tile's workgroups re-read these rows), and
// their conversion to fp32, kept apart so the conversion does not make the
// compiler wait on the load before the B stream is issued.
template <typename In>
__device__ inline void load8_act_raw(const typename In::storage* p, uint4 w[2]) {
  w[0] = *reinterpret_cast<const uint4*>(p);
  if constexpr (std::is_same<In, f32_t>::value) w[1] = *reinterpret_cast<const uint4*>(p + 4);
}

template <typename In>
__device__ inline void act_to_f32(const uint4 w[2], float v[8]) {
  if constexpr (std::is_same<In, f32_t>::value) {
    const uint32_t d[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(d[i]);
  } else {
    const uint32_t d[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = elem<In>::to_f32(static_cast<uint16_t>(d[i] & 0xffffu));
      v[2 * i + 1] = elem<In>::to_f32(static_cast<uint16_t>(d[i] >> 16));
    }
  }
}

// Requirements (checked by the host): m <= 4*MB, n % 16 == 0, k % 32 == 0,
// a and b 16-byte aligned, M*K, K*N and splits*M*N below 2^31;
// blockwise: block_k % 32 == 0, block_n % 16 == 0.
//
// In != void: fused activation quantization. The workgroup quantizes its own
// slice A_in[0:M, kwg0 : kwg0 + 256*CH] into LDS with the standalone
// quantizer's arithmetic (scale_from_amax, enc8), then reads A codes (and
// scales) from LDS. Its slice loads are issued before the B stream, so B stays
// in flight while it quantizes.
//  * fp8 blockwise kinds: 1 x block_k groups (block_k in {32, 64, 128, 256},
//    so the slice holds whole groups).
//  * INT8: per-token (a_per_token) or per-tensor scales, which need the amax
//    of whole rows. A prologue, run before any other load while the registers
//    are free, reads all M x K activations (they stay in L2: every workgroup
//    reads the same M <= 8 rows) and reduces the row maxima (fmaxf, so the
//    order does not change the value). Every workgroup derives the same
//    scales; workgroup 0 also writes them to a_scale_out, from which the split
//    reduce takes the epilogue's a_s.
//
// WB (blockwise only): block_k is a multiple of a wave's CH * 32 rows, so all
// of a wave's chunks lie in one scale block; the MFMA then accumulates the
// wave's whole K range and the partial is promoted once, O = P * (a_s * b_s)
// (the same value as fma(P, a_s * b_s, 0)), which keeps the per-chunk O
// registers out of the loop.
template <int KIND, int MB, int CH, typename In = void, bool WB = false>
__global__ void __launch_bounds__(kThreads)
skinny_kernel(Args p) {
  constexpr bool kInt = KIND == INT8 || KIND == INT8_RAW;
  constexpr bool kBlock = is_fp8_block(KIND);
  static_assert(!WB || kBlock, "one-block promotion serves the blockwise kinds");
  constexpr bool kChunkPromote = kBlock && !WB;
  constexpr bool kFused = !std::is_void<In>::value;
  static_assert(!kFused || kBlock || KIND == INT8, "fused quantization: fp8 blockwise or INT8");
  constexpr bool kFusedI8 = kFused && KIND == INT8;
  constexpr int kRows = 4 * MB;
  constexpr int kSliceK = kWaves * CH * kChunk;  // k-rows per workgroup
  __shared__ uint32_t red[kWaves / 2][kRows][kTileN];
  // The workgroup's activation slice (codes, or the fused path's quantized
  // values) and its a_scale entries, staged through LDS: a few 16-byte loads
  // per thread issued before the B stream, rather than per-fragment 8-byte
  // loads that the compiler may serialize under register pressure.
  constexpr int kSB = kSliceK / kChunk + 1;  // scale blocks a slice can touch
  __shared__ __attribute__((aligned(16))) uint8_t sa[kRows][kSliceK];
  __shared__ float ss[kRows][kSB];

  int tile, split;
  map_tile(blockIdx.x, gridDim.x, p.splits, &tile, &split);
  const int lane = threadIdx.x % 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int li = lane % 16, g = lane / 16;
  const int m = static_cast<int>(p.m), n = static_cast<int>(p.n), k = static_cast<int>(p.k);
  const int col = tile * kTileN + 16 * li;
  const int colc = col < n ? col : n - 16;  // lanes past N load a valid line, store nothing
  const int kwg0 = split * kSliceK;
  const int kw = kwg0 + wave * CH * kChunk;
  const int kb0 = kBlock ? kwg0 / p.block_k : 0;  // first scale block of the slice

  __shared__ float srow[kRows];
  // ---- fused int8: per-row (or per-tensor) scales from a full-row prologue.
  // (Issuing its loads behind the B stream instead measured no faster: the
  // first MFMA then waits for the whole stream.)
  if constexpr (kFusedI8) {
    using S = typename In::storage;
    const S* x = static_cast<const S*>(p.a_in);
    const int ppr = k / 8;  // 8-element pieces per row (K % 32 == 0)
    const int np = m * ppr;
    float ra[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) ra[r] = 0.f;
    for (int base = 0; base < np; base += 8 * kThreads) {
      uint4 w[8][2];  // 8 pieces in flight; rows are contiguous, so piece i is x + 8i
#pragma unroll
      for (int i = 0; i < 8; ++i)
        load8_act_raw<In>(x + 8 * static_cast<int64_t>(min(base + i * kThreads + static_cast<int>(threadIdx.x), np - 1)), w[i]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int pc = base + i * kThreads + static_cast<int>(threadIdx.x);
        float v[8];
        act_to_f32<In>(w[i], v);
        float am = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(v[e]));
        const int row = pc < np ? pc / ppr : kRows;  // kRows: dropped
#pragma unroll
        for (int r = 0; r < kRows; ++r) ra[r] = row == r ? fmaxf(ra[r], am) : ra[r];
      }
    }
    __shared__ float rmax[kWaves][kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float v = wave_max(ra[r]);
      if (lane == 0) rmax[wave][r] = v;
    }
    __syncthreads();
    if (threadIdx.x < kRows) {
      float am = 0.f;
      if (p.a_per_token) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) am = fmaxf(am, rmax[w][threadIdx.x]);
      } else {
        for (int r = 0; r < m; ++r)
#pragma unroll
          for (int w = 0; w < kWaves; ++w) am = fmaxf(am, rmax[w][r]);
      }
      const float sc = scale_from_amax<i8_t>(am);
      srow[threadIdx.x] = sc;
      if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < (p.a_per_token ? m : 1))
        p.a_scale_out[threadIdx.x] = sc;
    }
  }

  // ---- loads, in issue order: activation slice, scales, then B ----
  // Fused: unquantized activations, 8 elements per slot.
  constexpr int kPieces = kSliceK / 8;            // 8-element pieces per row
  constexpr int kSlots = kRows * kPieces;
  constexpr int kU = kFused ? (kSlots + kThreads - 1) / kThreads : 1;
  uint4 xr[kU][2];
  bool xlive[kU];
  // Pre-quantized: codes, 16 bytes per slot (rows and columns clamped; rows
  // past M and chunks past K are masked out of the math).
  constexpr int kAPieces = kRows * kSliceK / 16;
  constexpr int kUA = kFused ? 1 : (kAPieces + kThreads - 1) / kThreads;
  uint4 araw[kUA];
  constexpr int kUS = (kRows * kSB + kThreads - 1) / kThreads;
  float sraw[kUS];
  if constexpr (kFused) {
    using S = typename In::storage;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int slot = threadIdx.x + u * kThreads;
      const int row = slot / kPieces, kc = kwg0 + 8 * (slot % kPieces);
      xlive[u] = slot < kSlots && row < m && kc < k;
      const int64_t off = xlive[u] ? static_cast<int64_t>(row) * k + kc : 0;
      load8_act_raw<In>(static_cast<const S*>(p.a_in) + off, xr[u]);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kUA; ++u) {
      const int piece = threadIdx.x + u * kThreads;
      const int row = min(piece / (kSliceK / 16), m - 1);
      const int kc = min(kwg0 + 16 * (piece % (kSliceK / 16)), k - 16);
      araw[u] = *reinterpret_cast<const uint4*>(p.a + static_cast<int64_t>(row) * k + kc);
    }
    if constexpr (kBlock) {
#pragma unroll
      for (int u = 0; u < kUS; ++u) {
        const int e = threadIdx.x + u * kThreads;
        const int row = min(e / kSB, m - 1);
        const int kb = min(kb0 + e % kSB, static_cast<int>(p.nkb) - 1);
        sraw[u] = p.a_scale[static_cast<int64_t>(row) * p.nkb + kb];
      }
    }
  }
  uint2 av[CH][MB];
  float bsc[CH], asc[CH][MB];
  // b_scale of each chunk's block, per lane column group.
  if constexpr (kBlock) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int kb = min(kw + kChunk * c, k - kChunk) / p.block_k;
      bsc[c] = p.b_scale[static_cast<int64_t>(kb) * p.nnb + colc / p.block_n];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // All of the wave's B bytes (CH * 8 x 16 B per lane), non-temporal.
  uint4 bv[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int row = min(kw + kChunk * c + 8 * g + r, k - 1);
      bv[c][r] = load_stream16(p.b + static_cast<int64_t>(row) * n + colc);
    }
  // Keep every load above the math: the scheduler would otherwise sink later
  // chunks' loads below earlier chunks' MFMAs and serialize their latency.
  __builtin_amdgcn_sched_barrier(0);
  // ---- activation slice -> LDS (waits only for the loads issued before B) ----
  if constexpr (kFusedI8) {
    __syncthreads();  // srow complete
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int slot = threadIdx.x + u * kThreads;
      const int row = slot / kPieces, pc = slot % kPieces;
      float xv[8];
      act_to_f32<In>(xr[u], xv);
      // Rows past M and pieces past K hold clamped loads; the math masks them.
      const float inv = 1.0f / srow[row < kRows ? row : 0];
      const uint2 code = enc8<i8_t>::run(xv, inv);
      if (slot < kSlots) *reinterpret_cast<uint2*>(&sa[row][8 * pc]) = code;
    }
  } else if constexpr (kFused) {
    // 1 x block_k groups of G = block_k / 8 consecutive lanes (G divides 64
    // and the slice width, so a group never straddles a wave or a row; the
    // slice starts on a group boundary, so its group j is block kb0 + j).
    using Enc = typename std::conditional<fp8_fmt(KIND) == 1, e5m2_t, e4m3_t>::type;
    const int gl = p.block_k / 8;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int slot = threadIdx.x + u * kThreads;
      const int row = slot / kPieces, pc = slot % kPieces;
      float xv[8];
      act_to_f32<In>(xr[u], xv);
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, xlive[u] ? fabsf(xv[i]) : 0.f);
      amax = group_max(amax, gl);
      const float sc = scale_from_amax<Enc>(amax);
      const uint2 code = enc8<Enc>::run(xv, 1.0f / sc);
      if (slot < kSlots) {
        *reinterpret_cast<uint2*>(&sa[row][8 * pc]) = code;
        if (pc % gl == 0) ss[row][pc / gl] = sc;
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < kUA; ++u) {
      const int piece = threadIdx.x + u * kThreads;
      if (piece < kAPieces)
        *reinterpret_cast<uint4*>(&sa[piece / (kSliceK / 16)][16 * (piece % (kSliceK / 16))]) = araw[u];
    }
    if constexpr (kBlock) {
#pragma unroll
      for (int u = 0; u < kUS; ++u) {
        const int e = threadIdx.x + u * kThreads;
        if (e < kRows * kSB) ss[e / kSB][e % kSB] = sraw[u];
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int k0 = min(kw + kChunk * c, k - kChunk);  // chunk start (clamped past K)
#pragma unroll
    for (int f = 0; f < MB; ++f) {
      av[c][f] = *reinterpret_cast<const uint2*>(&sa[4 * f + li / 4][k0 - kwg0 + 8 * g]);
      if constexpr (kBlock) asc[c][f] = ss[4 * f + g][k0 / p.block_k - kb0];
    }
  }

  // A operand selectors: byte r of the lane's 8 activation bytes goes to byte
  // li % 4 of dword r, the other bytes are zero (v_perm selector 0x0c).
  const int c4 = li % 4;
  uint32_t sel[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) sel[r] = 0x0c0c0c0cu ^ ((0x0cu ^ r) << (8 * c4));

  typedef typename std::conditional<kInt, i32x4, f32x4>::type acc_t;
  acc_t acc[MB][4];
  f32x4 o[MB][4];
#pragma unroll
  for (int f = 0; f < MB; ++f)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[f][q] = acc_t{0, 0, 0, 0};
      o[f][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

#pragma unroll
  for (int c = 0; c < CH; ++c) {
    // A chunk past K (wave-uniform) loaded clamped rows; its A operand is
    // zeroed so it adds nothing, which keeps every load ahead of the math.
    const bool chunk_ok = kw + kChunk * c < k;
    // One fragment at a time: its A operand (8 perms) and, for blockwise, its
    // chunk partials live only while its MFMAs run.
#pragma unroll
    for (int f = 0; f < MB; ++f) {
      const bool am_ok = chunk_ok && 4 * f + li / 4 < m;
      const uint32_t lo = am_ok ? av[c][f].x : 0u, hi = am_ok ? av[c][f].y : 0u;
      uint32_t fa[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) fa[r] = __builtin_amdgcn_perm(hi, lo, sel[r]);
      acc_t part[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t bq[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint4 v = bv[c][r];
          bq[r] = q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
        }
        const acc_t cin = kChunkPromote ? acc_t{0, 0, 0, 0} : acc[f][q];
        if constexpr (kInt) {
          part[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              i32x4{(int)fa[0], (int)fa[1], (int)fa[2], (int)fa[3]},
              i32x4{(int)bq[0], (int)bq[1], (int)bq[2], (int)bq[3]}, cin, 0, 0, 0);
          part[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              i32x4{(int)fa[4], (int)fa[5], (int)fa[6], (int)fa[7]},
              i32x4{(int)bq[4], (int)bq[5], (int)bq[6], (int)bq[7]}, part[q], 0, 0, 0);
        } else {
          constexpr int fmt = fp8_fmt(KIND);
          part[q] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              i32x8{(int)fa[0], (int)fa[1], (int)fa[2], (int)fa[3],
                    (int)fa[4], (int)fa[5], (int)fa[6], (int)fa[7]},
              i32x8{(int)bq[0], (int)bq[1], (int)bq[2], (int)bq[3],
                    (int)bq[4], (int)bq[5], (int)bq[6], (int)bq[7]},
              cin, fmt, fmt, 0, 127, 0, 127);
        }
      }
      if constexpr (kChunkPromote) {
        const float sc = asc[c][f] * bsc[c];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[f][q][r] = fmaf(part[q][r], sc, o[f][q][r]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[f][q] = part[q];
      }
    }
  }
  if constexpr (WB) {
    // Every chunk of the wave is in chunk 0's scale block (chunks past K
    // added zeros).
#pragma unroll
    for (int f = 0; f < MB; ++f) {
      const float sc = asc[0][f] * bsc[0];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[f][q][r] = fmaf(acc[f][q][r], sc, 0.f);
    }
  }

  // Sum the 8 waves in a fixed order: (w, w + 4) pairs, then the four pairs.
  auto val = [&](int f, int q, int r) -> uint32_t {
    if constexpr (kInt) return static_cast<uint32_t>(acc[f][q][r]);
    else if constexpr (kBlock) return __float_as_uint(o[f][q][r]);
    else return __float_as_uint(acc[f][q][r]);
  };
  auto add = [](uint32_t x, uint32_t y) -> uint32_t {
    if constexpr (kInt) return x + y;  // two's-complement int32 add
    else return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
  };
  if (wave >= kWaves / 2) {
#pragma unroll
    for (int f = 0; f < MB; ++f)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - kWaves / 2][4 * f + g][16 * li + 4 * q + r] = val(f, q, r);
  }
  __syncthreads();
  if (wave < kWaves / 2) {
#pragma unroll
    for (int f = 0; f < MB; ++f)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          uint32_t& e = red[wave][4 * f + g][16 * li + 4 * q + r];
          e = add(val(f, q, r), e);
        }
  }
  __syncthreads();
  uint32_t* ws = static_cast<uint32_t*>(p.ws);
  for (int e = threadIdx.x; e < kRows * kTileN; e += kThreads) {
    const int row = e / kTileN, cc = e % kTileN;
    const int gc = tile * kTileN + cc;
    if (row >= m || gc >= n) continue;
    uint32_t v = red[0][row][cc];
#pragma unroll
    for (int w = 1; w < kWaves / 2; ++w) v = add(v, red[w][row][cc]);
    ws[(static_cast<int64_t>(split) * m + row) * n + gc] = v;
  }
}

// Sums the split partials in split order, then applies the entry point's
// epilogue (the same operation order as the tiled kernels). A thread takes
// V adjacent outputs of one row (V = 4: 16-byte partial loads; the host uses
// it when N % 4 == 0 and the output is aligned to V elements).
template <int KIND, typename Out, int V>
__global__ void __launch_bounds__(256)
skinny_reduce_kernel(Args p) {
  const int64_t idx = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * V;
  const int64_t plane = p.m * p.n;
  if (idx >= plane) return;
  const int64_t gm = idx / p.n, gn = idx % p.n;
  constexpr bool kInt = KIND == INT8 || KIND == INT8_RAW;
  typedef uint32_t vec __attribute__((ext_vector_type(V)));
  const uint32_t* ws = static_cast<const uint32_t*>(p.ws) + idx;
  auto load = [&](int sp) { return *reinterpret_cast<const vec*>(ws + sp * plane); };
  uint32_t si[V];
  float sf[V];
#pragma unroll
  for (int e = 0; e < V; ++e) { si[e] = 0; sf[e] = 0.f; }
  auto add = [&](const vec& v) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
      if constexpr (kInt) si[e] += v[e];
      else sf[e] += __uint_as_float(v[e]);
    }
  };
  int sp = 0;
  for (; sp + 8 <= p.splits; sp += 8) {  // 8 loads in flight, added in order
    vec part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = load(sp + i);
#pragma unroll
    for (int i = 0; i < 8; ++i) add(part[i]);
  }
  if (sp < p.splits) {  // tail: clamped, guarded, still one batch in flight
    vec part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = load(min(sp + i, p.splits - 1));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (sp + i < p.splits) add(part[i]);
  }
  const float as = p.a_per_token ? p.a_scale[gm] : p.a_scale[0];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if constexpr (KIND == INT8_RAW) {
      static_cast<int32_t*>(p.out)[idx + e] = static_cast<int32_t>(si[e]);
    } else if constexpr (kInt) {
      const float bsc = p.b_per_channel ? p.b_scale[gn + e] : p.b_scale[0];
      float v = __fmul_rn(__fmul_rn(static_cast<float>(static_cast<int32_t>(si[e])), as), bsc);
      if (p.bias)
        v = __fadd_rn(v, elem<Out>::load(static_cast<const typename Out::storage*>(p.bias), gn + e));
      static_cast<typename Out::storage*>(p.out)[idx + e] = elem<Out>::from_f32(v);
    } else {
      float v = sf[e];
      if constexpr (is_fp8_plain(KIND)) {
        const float bsc = p.b_per_channel ? p.b_scale[gn + e] : p.b_scale[0];
        v = __fmul_rn(__fmul_rn(v, as), bsc);
      }
      static_cast<typename Out::storage*>(p.out)[idx + e] = elem<Out>::from_f32(v);
    }
  }
}

template <int KIND, typename Out>
inline void launch_reduce(const Args& p, hipStream_t s) {
  constexpr uintptr_t kOutBytes = KIND == INT8_RAW ? 4 : sizeof(typename Out::storage);
  const int64_t plane = p.m * p.n;
  // V = 4 only for large planes: at decode sizes fewer, wider threads were
  // slower (N = K = 7168 fp8 blockwise, A/B: M = 1 13.0 -> 13.2 us; M = 128 /
  // 256 26.3 / 35.1 -> 25.9 / 34.7 us).
  if (plane >= (int64_t{1} << 19) && p.n % 4 == 0 &&
      reinterpret_cast<uintptr_t>(p.out) % (4 * kOutBytes) == 0)
    hipLaunchKernelGGL((skinny_reduce_kernel<KIND, Out, 4>),
                       dim3(static_cast<unsigned>((plane / 4 + 255) / 256)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((skinny_reduce_kernel<KIND, Out, 1>),
                       dim3(static_cast<unsigned>((plane + 255) / 256)), dim3(256), 0, s, p);
}

}  // namespace skinny
}  // namespace gemm8
}  // namespace ks
