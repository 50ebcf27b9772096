/*
 * CPU oracle for the w8g64 quantized linear and the int8 GEMM tier.
 *
 * TEST INFRASTRUCTURE ONLY: the checker, never the thing measured or
 * shipped. See oracle.h for what pins each function.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include "oracle.h"

#include <stdlib.h>

#include <math.h>
#include <string.h>

/* bf16 <-> f32, round to nearest even on the upper 16 bits.
 * Follows src/ltx25-metal-ops.cc:23-31 and tests/ltx25-qlinear-test.cc:67-74
 * (add 0x7fff plus the LSB of the kept half, then truncate). NaN inputs are
 * returned as a quiet NaN rather than run through the adder, which would
 * carry a NaN payload into the exponent. */
uint16_t orc_bf16_rne(float f)
{
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    return (uint16_t)((u >> 16) | 0x0040u);
  }
  const uint32_t r = ((u >> 16) & 1u) + 0x7fffu;
  return (uint16_t)((u + r) >> 16);
}

/* src/ltx25-metal-ops.cc:33-39 */
float orc_bf16_to_f32(uint16_t h)
{
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n)
{
  for (size_t i = 0; i < n; ++i) { out[i] = orc_bf16_rne(in[i]); }
}

void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n)
{
  for (size_t i = 0; i < n; ++i) { out[i] = orc_bf16_to_f32(in[i]); }
}

/* IEEE binary16 -> binary32, exact (every half is a float). */
static float f16_decode(uint16_t h)
{
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0x1fu) {
    u = sign | 0x7f800000u | (man << 13);
  } else if (exp != 0) {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    u = sign;
  } else {
    /* subnormal half: man * 2^-24, renormalised */
    int e = -1;
    uint32_t m = man;
    do { m <<= 1; ++e; } while ((m & 0x400u) == 0);
    u = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3ffu) << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* The loader's F16 -> BF16 conversion of scales and biases:
 * src/ltx25-dit-weights.cc:250-259 (decode the half, then RNE to bf16). */
void orc_f16_to_bf16_n(const uint16_t* in_f16, uint16_t* out_bf16, size_t n)
{
  for (size_t i = 0; i < n; ++i) {
    out_bf16[i] = orc_bf16_rne(f16_decode(in_f16[i]));
  }
}

static int bits_ok(int bits) { return bits == 4 || bits == 8; }

/* Group-affine quantize one [N][K] row-major weight, MLX layout.
 * Follows tests/ltx25-qlinear-test.cc:93-141 step for step:
 *   lo, hi = fmin/fmax over the group                       (:110-116)
 *   sc = (hi - lo) / (2^bits - 1)                           (:117)
 *   scale and bias rounded to bf16 BEFORE coding            (:121-125)
 *   q = scr > 0 ? lround((w - lor) / scr) : 0, clamped      (:129-132)
 *   deq = scr * q + lor                                     (:133)
 *   codes LOW bits first, 32/bits per u32 word              (:134-137)
 * `deq` may be NULL. Returns 0, or -1 on a shape the layout cannot hold. */
int orc_quantize_affine(const float* w, int N, int K, int bits, int group,
                        uint32_t* codes, uint16_t* scales, uint16_t* biases,
                        float* deq)
{
  if (!bits_ok(bits) || group <= 0 || N < 0 || K <= 0 || K % group != 0 ||
      (K * bits) % 32 != 0) {
    return -1;
  }
  const int per_word = 32 / bits;
  const int gcols = K / group;
  const int wcols = K / per_word;
  const float qmax = (float)((1 << bits) - 1);

  memset(codes, 0, (size_t)N * wcols * sizeof(uint32_t));
  for (int n = 0; n < N; ++n) {
    for (int g = 0; g < gcols; ++g) {
      const int k0 = g * group;
      const float* wr = w + (size_t)n * K + k0;
      float lo = wr[0], hi = lo;
      for (int j = 1; j < group; ++j) {
        lo = fminf(lo, wr[j]);
        hi = fmaxf(hi, wr[j]);
      }
      const float sc = (hi - lo) / qmax;
      const uint16_t sc_b = orc_bf16_rne(sc);
      const uint16_t lo_b = orc_bf16_rne(lo);
      const float scr = orc_bf16_to_f32(sc_b);
      const float lor = orc_bf16_to_f32(lo_b);
      scales[(size_t)n * gcols + g] = sc_b;
      biases[(size_t)n * gcols + g] = lo_b;
      for (int j = 0; j < group; ++j) {
        const int k = k0 + j;
        long q = scr > 0.0f ? lroundf((wr[j] - lor) / scr) : 0;
        if (q < 0) { q = 0; }
        if (q > (long)qmax) { q = (long)qmax; }
        if (deq != NULL) {
          const float p = scr * (float)q;
          deq[(size_t)n * K + k] = p + lor;
        }
        codes[(size_t)n * wcols + k / per_word] |=
            ((uint32_t)q) << (bits * (k % per_word));
      }
    }
  }
  return 0;
}

/* Codes -> u32 words, LOW bits first (tests/ltx25-qlinear-test.cc:134-137).
 * For bits == 8 this is exactly the little-endian byte layout of u8 [N][K]. */
int orc_pack_codes(const uint8_t* q, int N, int K, int bits, uint32_t* codes)
{
  if (!bits_ok(bits) || (K * bits) % 32 != 0) { return -1; }
  const int per_word = 32 / bits;
  const int wcols = K / per_word;
  const uint32_t mask = (1u << bits) - 1u;
  for (int n = 0; n < N; ++n) {
    for (int wd = 0; wd < wcols; ++wd) {
      uint32_t v = 0;
      for (int s = 0; s < per_word; ++s) {
        v |= ((uint32_t)q[(size_t)n * K + wd * per_word + s] & mask)
             << (bits * s);
      }
      codes[(size_t)n * wcols + wd] = v;
    }
  }
  return 0;
}

/* Inverse of orc_pack_codes. */
int orc_unpack_codes(const uint32_t* codes, int N, int K, int bits,
                     uint8_t* q)
{
  if (!bits_ok(bits) || (K * bits) % 32 != 0) { return -1; }
  const int per_word = 32 / bits;
  const int wcols = K / per_word;
  const uint32_t mask = (1u << bits) - 1u;
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) {
      const uint32_t v = codes[(size_t)n * wcols + k / per_word];
      q[(size_t)n * K + k] = (uint8_t)((v >> (bits * (k % per_word))) & mask);
    }
  }
  return 0;
}

/* The dequant-once expansion (libvpipe affine_dequant, dispatched at
 * src/ltx25-metal-ops.cc:488-498): w = bf16(scale * q + bias) into [N][K].
 * The product-sum is ONE fused multiply-add, fmaf(scale, q, bias), which
 * is the rounding the HIP kernels implement in front of the MFMA. Either
 * output may be NULL. */
int orc_dequant(const uint32_t* codes, const uint16_t* scales,
                const uint16_t* biases, int N, int K, int bits, int group,
                float* w_f32, uint16_t* w_bf16)
{
  if (!bits_ok(bits) || group <= 0 || K % group != 0 ||
      (K * bits) % 32 != 0) {
    return -1;
  }
  const int per_word = 32 / bits;
  const int wcols = K / per_word;
  const int gcols = K / group;
  const uint32_t mask = (1u << bits) - 1u;
  for (int n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) {
      const uint32_t v = codes[(size_t)n * wcols + k / per_word];
      const float q = (float)((v >> (bits * (k % per_word))) & mask);
      const float s = orc_bf16_to_f32(scales[(size_t)n * gcols + k / group]);
      const float b = orc_bf16_to_f32(biases[(size_t)n * gcols + k / group]);
      const float d = fmaf(s, q, b);
      if (w_f32 != NULL) { w_f32[(size_t)n * K + k] = d; }
      if (w_bf16 != NULL) { w_bf16[(size_t)n * K + k] = orc_bf16_rne(d); }
    }
  }
  return 0;
}

/* out[r][o] = sum_i x[r][i] * w[o][i] + b[o], accumulated in double in
 * index order with the bias as the initial value.
 * Restates src/ltx25-block-ref.cc:11-28 (linear_). `bias` may be NULL. */
void orc_linear_f64(const float* x, const float* w, const float* bias, int M,
                    int K, int N, float* out)
{
  for (int r = 0; r < M; ++r) {
    const float* xr = x + (size_t)r * K;
    for (int c = 0; c < N; ++c) {
      const float* wr = w + (size_t)c * K;
      double acc = bias == NULL ? 0.0 : (double)bias[c];
      for (int i = 0; i < K; ++i) { acc += (double)xr[i] * wr[i]; }
      out[(size_t)r * N + c] = (float)acc;
    }
  }
}

/* The same sum, kept in double (the tolerance reference for bf16 outputs). */
void orc_linear_f64_d(const float* x, const float* w, const float* bias,
                      int M, int K, int N, double* out)
{
  for (int r = 0; r < M; ++r) {
    const float* xr = x + (size_t)r * K;
    for (int c = 0; c < N; ++c) {
      const float* wr = w + (size_t)c * K;
      double acc = bias == NULL ? 0.0 : (double)bias[c];
      for (int i = 0; i < K; ++i) { acc += (double)xr[i] * wr[i]; }
      out[(size_t)r * N + c] = acc;
    }
  }
}

/* The multithreaded f32 CPU path (OpenMP over output rows and columns),
 * used only as a timing baseline. Same operation as orc_linear_f64 with an
 * f32 accumulator, so its results differ from it by f32 rounding. */
void orc_linear_f32_omp(const float* x, const float* w, const float* bias,
                        int M, int K, int N, float* out, int threads)
{
  if (threads <= 0) { threads = 1; }
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
  for (int r = 0; r < M; ++r) {
    for (int c = 0; c < N; ++c) {
      const float* xr = x + (size_t)r * K;
      const float* wr = w + (size_t)c * K;
      float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
      for (int i = 0; i < K; ++i) { acc += xr[i] * wr[i]; }
      out[(size_t)r * N + c] = acc + (bias == NULL ? 0.0f : bias[c]);
    }
  }
}

/* GELU, tanh approximation, evaluated in double and rounded once to float.
 * Restates src/ltx25-block-ref.cc:265-272. */
void orc_gelu_tanh(const float* in, float* out, size_t n)
{
  for (size_t i = 0; i < n; ++i) {
    const double x = in[i];
    const double t = 0.7978845608028654 * (x + 0.044715 * x * x * x);
    out[i] = (float)(0.5 * x * (1.0 + tanh(t)));
  }
}

/* y[i] = bf16(float(y[i]) + float(bias[i % N])), in place.
 * Restates src/ltx25-kernels.metal:1431-1441 (ltx_bias_add). */
void orc_bias_add_bf16(uint16_t* y, const uint16_t* bias, int M, int N)
{
  const size_t total = (size_t)M * N;
  for (size_t i = 0; i < total; ++i) {
    const float v = orc_bf16_to_f32(y[i]) + orc_bf16_to_f32(bias[i % N]);
    y[i] = orc_bf16_rne(v);
  }
}

/* Per-head gating of an attention output, in place on bf16 y [tokens]
 * [heads * head_dim]: gate = 2 / (1 + exp(-logit)) in float, from the bf16
 * logit of (token, head); y = bf16(float(y) * gate). Restates
 * src/ltx25-kernels.metal:85-103 (ltx_gate_heads; storage rounding of y)
 * with the gate expression of src/ltx25-block-ref.cc:123. */
void orc_gate_heads(uint16_t* y, const uint16_t* logits, int heads, int tokens, int head_dim)
{
  for (int t = 0; t < tokens; ++t) {
    for (int h = 0; h < heads; ++h) {
      const float lg = orc_bf16_to_f32(logits[(size_t)t * heads + h]);
      const float gate = 2.0f / (1.0f + expf(-lg));
      uint16_t* row = y + ((size_t)t * heads + h) * head_dim;
      for (int d = 0; d < head_dim; ++d) {
        row[d] = orc_bf16_rne(orc_bf16_to_f32(row[d]) * gate);
      }
    }
  }
}

/* The low-rank adapter delta y += (x . a^T) . b^T, in place on bf16 y,
 * following MetalOps::lora_add (src/ltx25-metal-ops.cc:989-1004) in its
 * matrix-core form (:940-987): r = x . a^T is written to a bf16 scratch
 * (rounded once), and the second product accumulates onto y, seeded from y,
 * with one rounding to bf16 at the store. a is [rank][K] and b is [N][rank]
 * (src/ltx25-metal-ops.h:107-117); accumulation here is double. */
void orc_lora_add(const uint16_t* x, const uint16_t* a, const uint16_t* b,
                  uint16_t* y, int M, int K, int N, int rank)
{
  if (M <= 0 || K <= 0 || N <= 0 || rank <= 0) { return; }
  float* r = (float*)malloc(sizeof(float) * (size_t)rank);
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x + (size_t)m * K;
    for (int j = 0; j < rank; ++j) {
      const uint16_t* ar = a + (size_t)j * K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        acc += (double)orc_bf16_to_f32(xr[k]) * (double)orc_bf16_to_f32(ar[k]);
      }
      r[j] = orc_bf16_to_f32(orc_bf16_rne((float)acc));
    }
    uint16_t* yr = y + (size_t)m * N;
    for (int n = 0; n < N; ++n) {
      const uint16_t* br = b + (size_t)n * rank;
      double acc = (double)orc_bf16_to_f32(yr[n]);
      for (int j = 0; j < rank; ++j) { acc += (double)r[j] * (double)orc_bf16_to_f32(br[j]); }
      yr[n] = orc_bf16_rne((float)acc);
    }
  }
  free(r);
}

/* Per-row symmetric int8: scale = absmax / 127 (f32 division),
 * q = clamp(rint(x / scale), -127, 127), and q = 0, scale = 0 for an
 * all-zero row. Used for activations per token and for weights per output
 * channel (a weight's rows are its output channels).
 *
 * The reference's int8 tier lives in libvpipe's I8GemmContext, which is not
 * in the reference tree; its stated contract is per-(row, group) symmetric
 * quantization with ~1e-2 rel-L2 per GEMM (src/ltx25-metal-ops.h:810-817).
 * The per-token / per-channel form here, and round-half-to-even, are this
 * build's definition and are pinned by the fixtures under tests/golden. */
void orc_i8_quantize_rows(const uint16_t* x_bf16, int M, int K, int8_t* q,
                          float* scale)
{
  for (int m = 0; m < M; ++m) {
    const uint16_t* xr = x_bf16 + (size_t)m * K;
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) {
      amax = fmaxf(amax, fabsf(orc_bf16_to_f32(xr[k])));
    }
    const float s = amax / 127.0f;
    scale[m] = s;
    for (int k = 0; k < K; ++k) {
      float v = 0.0f;
      if (s > 0.0f) {
        v = rintf(orc_bf16_to_f32(xr[k]) / s);
        if (v > 127.0f) { v = 127.0f; }
        if (v < -127.0f) { v = -127.0f; }
      }
      q[(size_t)m * K + k] = (int8_t)v;
    }
  }
}

/* acc[m][n] = sum_k xq[m][k] * wq[n][k], exact in int32. */
void orc_i8_gemm_i32(const int8_t* xq, const int8_t* wq, int M, int K, int N,
                     int32_t* acc)
{
  for (int m = 0; m < M; ++m) {
    const int8_t* xr = xq + (size_t)m * K;
    for (int n = 0; n < N; ++n) {
      const int8_t* wr = wq + (size_t)n * K;
      int32_t a = 0;
      for (int k = 0; k < K; ++k) { a += (int32_t)xr[k] * (int32_t)wr[k]; }
      acc[(size_t)m * N + n] = a;
    }
  }
}

/* The fused dequant epilogue of the int8 GEMM, in a fixed f32 order:
 *   y = bf16(fmaf(float(acc), sx[m] * sw[n], b)),  b = bias[n] or +0.0f
 * bias_dtype: 0 none, 1 bf16, 2 f32. */
void orc_i8_epilogue(const int32_t* acc, const float* sx, const float* sw,
                     const void* bias, int bias_dtype, int M, int N,
                     uint16_t* y)
{
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      float b = 0.0f;
      if (bias != NULL && bias_dtype == 1) {
        b = orc_bf16_to_f32(((const uint16_t*)bias)[n]);
      } else if (bias != NULL && bias_dtype == 2) {
        b = ((const float*)bias)[n];
      }
      const float sc = sx[m] * sw[n];
      const float v = fmaf((float)acc[(size_t)m * N + n], sc, b);
      y[(size_t)m * N + n] = orc_bf16_rne(v);
    }
  }
}

/* orc_i8_epilogue followed by the feed-forward's GELU-tanh (epilogue 1)
 * before the one rounding: y = bf16(gelu(fma(float(acc), sx[m] * sw[n],
 * bias[n]))), gelu as orc_gelu_tanh. epilogue 0 is orc_i8_epilogue. The
 * composition the int8 tier computes under ff_in (src/ltx25-block-metal.cc:
 * 639-645 runs linear then gelu; the tier sits under that linear,
 * src/ltx25-metal-ops.cc:376-391). */
void orc_i8_epilogue_ex(const int32_t* acc, const float* sx, const float* sw,
                        const void* bias, int bias_dtype, int epilogue, int M, int N,
                        uint16_t* y)
{
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      float b = 0.0f;
      if (bias != NULL && bias_dtype == 1) {
        b = orc_bf16_to_f32(((const uint16_t*)bias)[n]);
      } else if (bias != NULL && bias_dtype == 2) {
        b = ((const float*)bias)[n];
      }
      const float sc = sx[m] * sw[n];
      float v = fmaf((float)acc[(size_t)m * N + n], sc, b);
      if (epilogue == 1) { orc_gelu_tanh(&v, &v, 1); }
      y[(size_t)m * N + n] = orc_bf16_rne(v);
    }
  }
}

/* splitmix64 stream + Box-Muller in double: a seeded N(mean, stddev)
 * generator whose output does not depend on the C library. */
static uint64_t splitmix64(uint64_t* s)
{
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean,
                     float stddev)
{
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    /* 53-bit uniforms in (0, 1] and [0, 1) */
    const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(splitmix64(&s) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1));
    out[i] = (float)(mean + stddev * r * cos(two_pi * u2));
    if (i + 1 < n) {
      out[i + 1] = (float)(mean + stddev * r * sin(two_pi * u2));
    }
  }
}
