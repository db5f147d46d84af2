/*
 * kernel-set CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference's arithmetic for the quantized
 * inference path (cklxx/kernel-set, kernels/src/quant and kernels/src/gemm).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker: it is never the product path.
 *
 * Build: see oracle/build.py (gcc -O2 -ffp-contract=off, no fast-math, so
 * every fp32 operation is one IEEE-754 operation as written).
 *
 * fp8 encoding here is written independently of the HIP encoder: it finds the
 * binade with frexpf, rounds |x| / quantum with nearbyintf (round half to even
 * in the default rounding mode) and rebuilds the code from (exponent, mantissa).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EPS_SCALE 1e-12f

/* ---- OCP fp8 ----------------------------------------------------------- */
/* fmt 0 = e4m3fn (bias 7, 3 mantissa bits, max 448, NaN = 0x7f, no inf)
 * fmt 1 = e5m2   (bias 15, 2 mantissa bits, max 57344, inf = 0x7c)
 * Saturating conversion as used by the reference quantizers
 * (quant_fp8.cu:62-64, quant_fp8_group.cu:65-66: "the FP8 cast saturates to
 * the finite max"). */
static uint8_t fp8_encode(float x, int fmt) {
  const int mbits = fmt == 0 ? 3 : 2;
  const int bias = fmt == 0 ? 7 : 15;
  const float fmax = fmt == 0 ? 448.0f : 57344.0f;
  const uint8_t maxcode = fmt == 0 ? 0x7e : 0x7b;
  if (isnan(x)) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0x00;
  float a = fabsf(x);
  if (a > fmax) return sign | maxcode;
  if (a == 0.0f) return sign;
  int e2;
  (void)frexpf(a, &e2);      /* a = f * 2^e2, f in [0.5, 1) -> binade exponent e2-1 */
  int e = e2 - 1;
  const int emin = 1 - bias; /* smallest normal exponent */
  if (e < emin) e = emin;    /* subnormals share the quantum of the lowest binade */
  const float quantum = ldexpf(1.0f, e - mbits);
  float q = nearbyintf(a / quantum); /* exact division by a power of two */
  /* q in [0, 2^(mbits+1)]; q == 2^(mbits+1) means a carry into the next binade */
  if (q >= (float)(1 << (mbits + 1))) {
    q = q / 2.0f;
    e += 1;
  }
  int code;
  if (q < (float)(1 << mbits)) {
    code = (int)q; /* subnormal (only possible when e == emin) */
  } else {
    code = ((e + bias) << mbits) | ((int)q - (1 << mbits));
  }
  return sign | (uint8_t)code;
}

static float fp8_decode(uint8_t c, int fmt) {
  const int mbits = fmt == 0 ? 3 : 2;
  const int bias = fmt == 0 ? 7 : 15;
  const int ebits = fmt == 0 ? 4 : 5;
  const float s = (c & 0x80) ? -1.0f : 1.0f;
  const int e = (c >> mbits) & ((1 << ebits) - 1);
  const int m = c & ((1 << mbits) - 1);
  if (fmt == 0 && e == 15 && m == 7) return NAN;
  if (fmt == 1 && e == 31) return m ? NAN : s * INFINITY;
  if (e == 0) return s * ldexpf((float)m, 1 - bias - mbits);
  return s * ldexpf((float)((1 << mbits) | m), e - bias - mbits);
}

void oracle_fp8_encode(const float* x, uint8_t* out, int64_t n, int fmt) {
  for (int64_t i = 0; i < n; ++i) out[i] = fp8_encode(x[i], fmt);
}

void oracle_fp8_decode(const uint8_t* c, float* out, int64_t n, int fmt) {
  for (int64_t i = 0; i < n; ++i) out[i] = fp8_decode(c[i], fmt);
}

/* ---- int8 -------------------------------------------------------------- */
/* quant_int8.cu:44 + quant_common.cuh:35-44: rne(clamp(x*inv, -127, 127)). */
static int8_t int8_encode(float v) {
  const float c = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
  return (int8_t)(int)nearbyintf(c);
}

/* Dynamic scale: fmaxf(amax/qmax, 1e-12f) (quant_fp8_group.cu:100,
 * quant_fp8.cu:58, quant_int8.cu:39). fmaxf ignores a NaN amax operand the
 * same way the reference's block reductions do. */
static float dyn_scale(float amax, float qmax) { return fmaxf(amax / qmax, EPS_SCALE); }

static float qmax_of(int target) { /* 0 e4m3, 1 e5m2, 2 int8 */
  return target == 0 ? 448.0f : (target == 1 ? 57344.0f : 127.0f);
}

static uint8_t encode_target(float v, int target) {
  if (target == 2) return (uint8_t)int8_encode(v);
  return fp8_encode(v, target);
}

/* quant_fp8_group.cu:74-107 (cached) and :38-70 (generic): per (row, group). */
void oracle_quant_group(const float* x, uint8_t* out, float* scale, int64_t rows,
                        int64_t cols, int64_t gs, int target) {
  const int64_t ng = (cols + gs - 1) / gs;
  const float qmax = qmax_of(target);
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < ng; ++g) {
      const int64_t c0 = g * gs, c1 = (c0 + gs < cols) ? c0 + gs : cols;
      float amax = 0.0f;
      for (int64_t c = c0; c < c1; ++c) amax = fmaxf(amax, fabsf(x[r * cols + c]));
      const float sc = dyn_scale(amax, qmax);
      scale[r * ng + g] = sc;
      const float inv = 1.0f / sc;
      for (int64_t c = c0; c < c1; ++c)
        out[r * cols + c] = encode_target(x[r * cols + c] * inv, target);
    }
  }
}

/* Per-token (quant_fp8.cu:42-66, quant_int8.cu:23-47) is the group case with
 * one group spanning the row. */
void oracle_quant_row(const float* x, uint8_t* out, float* scale, int64_t rows,
                      int64_t cols, int target) {
  oracle_quant_group(x, out, scale, rows, cols, cols, target);
}

/* Per-tensor (quant_fp8.cu:69-100, quant_int8.cu:50-83). */
void oracle_quant_tensor(const float* x, uint8_t* out, float* scale, int64_t numel,
                         int target) {
  float amax = 0.0f;
  for (int64_t i = 0; i < numel; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const float sc = dyn_scale(amax, qmax_of(target));
  *scale = sc;
  const float inv = 1.0f / sc;
  for (int64_t i = 0; i < numel; ++i) out[i] = encode_target(x[i] * inv, target);
}

/* ---- int4 weight formats ------------------------------------------------ */
/* repack_int4.cu:10-34: int32 [K/8,N] -> uint8 [K/2,N], even k low nibble.
 * perm (may be NULL): output row k takes input row perm[k]. */
void oracle_repack_int4(const uint32_t* in, const int32_t* perm, uint8_t* out,
                        int64_t k, int64_t n) {
  for (int64_t kp = 0; kp < k / 2; ++kp) {
    for (int64_t c = 0; c < n; ++c) {
      const int64_t ke = perm ? perm[2 * kp] : 2 * kp;
      const int64_t ko = perm ? perm[2 * kp + 1] : 2 * kp + 1;
      const uint32_t qe = (in[(ke / 8) * n + c] >> (4 * (ke % 8))) & 0xf;
      const uint32_t qo = (in[(ko / 8) * n + c] >> (4 * (ko % 8))) & 0xf;
      out[kp * n + c] = (uint8_t)(qe | (qo << 4));
    }
  }
}

/* dequant_int4.cu:47-58 in fp32 (before rounding to the output dtype). */
void oracle_dequant_int4(const uint32_t* in, const float* scales, const float* zeros,
                         float* out, int64_t k, int64_t n, int64_t gs) {
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t c = 0; c < n; ++c) {
      const float q = (float)((in[(kk / 8) * n + c] >> (4 * (kk % 8))) & 0xf);
      const int64_t g = (kk / gs) * n + c;
      out[kk * n + c] = (q - zeros[g]) * scales[g];
    }
}

/* ---- GEMMs (fp32 scalar, reference kernel order) ------------------------ */
/* gemm_w4a16.cu:74-129: w = (q - z) * s in fp32, acc = fma(a, w, acc) over
 * increasing k, + bias. a/scales/zeros/bias already widened to fp32.
 * zeros == NULL means 0, bias == NULL means none. Output fp32 (caller rounds). */
void oracle_w4a16(const float* a, const uint8_t* b, const float* scales,
                  const float* zeros, const float* bias, float* c, int64_t m,
                  int64_t n, int64_t k, int64_t gs) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (int64_t kk = 0; kk < k; ++kk) {
        const uint8_t byte = b[(kk / 2) * n + j];
        const int q = (kk & 1) ? (byte >> 4) & 0xf : byte & 0xf;
        const int64_t g = (kk / gs) * n + j;
        const float zp = zeros ? zeros[g] : 0.0f;
        const float w = ((float)q - zp) * scales[g];
        acc = fmaf(a[i * k + kk], w, acc);
      }
      if (bias) acc += bias[j];
      c[i * n + j] = acc;
    }
}

/* gemm_fp8_blockwise.cu:107-161: per K-block fp32 partial, promoted as
 * out += part * (a_s * b_s). Operands are fp8 codes of format fmt. */
void oracle_fp8_blockwise(const uint8_t* a, const uint8_t* b, const float* as,
                          const float* bs, float* c, int64_t m, int64_t n, int64_t k,
                          int64_t bn, int64_t bk, int fmt) {
  const int64_t nkb = (k + bk - 1) / bk, nnb = (n + bn - 1) / bn;
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float out = 0.0f;
      for (int64_t kb = 0; kb < nkb; ++kb) {
        float part = 0.0f;
        const int64_t k0 = kb * bk, k1 = (k0 + bk < k) ? k0 + bk : k;
        for (int64_t kk = k0; kk < k1; ++kk)
          part = fmaf(fp8_decode(a[i * k + kk], fmt), fp8_decode(b[kk * n + j], fmt), part);
        out = fmaf(part, as[i * nkb + kb] * bs[kb * nnb + j / bn], out);
      }
      c[i * n + j] = out;
    }
}

/* gemm_fp8.cu:98-157: fp32 accumulation over all of K in ascending k (the
 * reference's acc += a*b, contracted to an fma), then (acc * a_s) * b_s. */
void oracle_fp8_gemm(const uint8_t* a, const uint8_t* b, const float* as,
                     const float* bs, float* c, int64_t m, int64_t n, int64_t k,
                     int a_per_token, int b_per_channel, int fmt) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (int64_t kk = 0; kk < k; ++kk)
        acc = fmaf(fp8_decode(a[i * k + kk], fmt), fp8_decode(b[kk * n + j], fmt), acc);
      float v = acc * (a_per_token ? as[i] : as[0]);
      v = v * (b_per_channel ? bs[j] : bs[0]);
      c[i * n + j] = v;
    }
}

/* gemm_w8a8.cu:120-142: exact int32 accumulation. */
void oracle_w8a8_acc(const int8_t* a, const int8_t* b, int32_t* acc, int64_t m,
                     int64_t n, int64_t k) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      int64_t s = 0;
      for (int64_t kk = 0; kk < k; ++kk) s += (int64_t)a[i * k + kk] * b[kk * n + j];
      acc[i * n + j] = (int32_t)s;
    }
}

/* gemm_w8a8.cu:134-141: v = (float(acc) * a_s) * b_s (+ bias), left to right. */
void oracle_w8a8_epilogue(const int32_t* acc, const float* as, const float* bs,
                          const float* bias, float* c, int64_t m, int64_t n,
                          int a_per_token, int b_per_channel) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float v = (float)acc[i * n + j] * (a_per_token ? as[i] : as[0]);
      v = v * (b_per_channel ? bs[j] : bs[0]);
      if (bias) v += bias[j];
      c[i * n + j] = v;
    }
}

/* moe_grouped_gemm.cu:68-127: for each expert e, rows [offs[e], offs[e+1]) of
 * A times B_e = b + e*k*n ([k, n]), acc = fma(a, b, acc) over increasing k in
 * fp32 (the reference's acc += as*bs, contracted to an fma). Rows outside
 * every expert's range are not written; ranges are clamped to [0, rows].
 * Operands already decoded to fp32; output fp32 (the caller rounds). */
void oracle_grouped_gemm(const float* a, const float* b, const int32_t* offs, int ne,
                         float* c, int64_t rows, int64_t n, int64_t k) {
  for (int e = 0; e < ne; ++e) {
    int64_t r0 = offs[e] < 0 ? 0 : offs[e];
    int64_t r1 = offs[e + 1];
    if (r0 > rows) r0 = rows;
    if (r1 > rows) r1 = rows;
    const float* be = b + (int64_t)e * k * n;
    for (int64_t i = r0; i < r1; ++i)
      for (int64_t j = 0; j < n; ++j) {
        float acc = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) acc = fmaf(a[i * k + kk], be[kk * n + j], acc);
        c[i * n + j] = acc;
      }
  }
}
