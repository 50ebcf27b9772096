// Bandwidth-bound kernels around the quantized linear: the standalone bias
// pass, GELU-tanh, the dequant-once expansion, the packed-weight format
// (pack / unpack / quantize) and the loader's F16 -> bf16 conversion.
// All are HBM-bound byte work: 16-byte vector loads and stores, no LDS.
#include "common.h"

namespace ltx25 {
namespace {

constexpr int kBlock = 256;

unsigned blocks_for(size_t work_items)
{
  return (unsigned)((work_items + kBlock - 1) / kBlock);
}

// y = bf16(f32(y) + f32(bias[i % N])), 8 elements per thread.
// Semantics of ltx_bias_add (src/ltx25-kernels.metal:1431-1441).
__global__ void __launch_bounds__(kBlock)
bias_add_kernel(uint16_t* y, const void* bias, int bias_type, int N,
                size_t total)
{
  const size_t i0 = ((size_t)blockIdx.x * kBlock + threadIdx.x) * 8;
  if (i0 >= total) { return; }
  auto bias_at = [&](size_t i) -> float {
    const int n = (int)(i % (size_t)N);
    return bias_type == kBiasF32 ? ((const float*)bias)[n]
                                 : bf16_to_f32(((const uint16_t*)bias)[n]);
  };
  if (i0 + 8 <= total && (N & 7) == 0) {
    uint4 v = *(const uint4*)(y + i0);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16_to_f32((uint16_t)(w[j] & 0xffffu)) + bias_at(i0 + 2 * j);
      const float b = bf16_to_f32((uint16_t)(w[j] >> 16)) + bias_at(i0 + 2 * j + 1);
      w[j] = pack_bf16x2(a, b);
    }
    *(uint4*)(y + i0) = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  for (size_t i = i0; i < i0 + 8 && i < total; ++i) {
    y[i] = f32_to_bf16(bf16_to_f32(y[i]) + bias_at(i));
  }
}

__global__ void __launch_bounds__(kBlock)
gelu_kernel(const uint16_t* x, uint16_t* y, size_t n)
{
  const size_t i0 = ((size_t)blockIdx.x * kBlock + threadIdx.x) * 8;
  if (i0 >= n) { return; }
  if (i0 + 8 <= n) {
    const uint4 v = *(const uint4*)(x + i0);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(gelu_tanh(bf16_to_f32((uint16_t)(w[j] & 0xffffu))),
                         gelu_tanh(bf16_to_f32((uint16_t)(w[j] >> 16))));
    }
    *(uint4*)(y + i0) = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  for (size_t i = i0; i < n; ++i) {
    y[i] = f32_to_bf16(gelu_tanh(bf16_to_f32(x[i])));
  }
}

// Per-head gate on the attention output, y[t][h][d] *= 2 sigmoid(logit[t][h]),
// rounded once to bf16 (the reference rounds y to its storage type there
// too). Eight d per thread: one 16-byte load and store when the head width
// allows it, else element by element.
__global__ void __launch_bounds__(kBlock)
gate_heads_kernel(uint16_t* y, const uint16_t* logits, int heads, int head_dim,
                  size_t chunks_per_row, size_t total_chunks, bool vec)
{
  const size_t c = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= total_chunks) { return; }
  const size_t row = c / chunks_per_row;          // token t * heads + h
  const int d0 = (int)(c % chunks_per_row) * 8;
  const float lg = bf16_to_f32(logits[row]);
  const float g = 2.0f / (1.0f + expf(-lg));
  uint16_t* p = y + row * (size_t)head_dim + d0;
  if (vec) {
    const uint4 v = *(const uint4*)p;
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(bf16_to_f32((uint16_t)(w[j] & 0xffffu)) * g,
                         bf16_to_f32((uint16_t)(w[j] >> 16)) * g);
    }
    *(uint4*)p = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  for (int d = d0; d < d0 + 8 && d < head_dim; ++d) {
    p[d - d0] = f32_to_bf16(bf16_to_f32(p[d - d0]) * g);
  }
}

// Dequant-once: one thread per run of 8 codes (8 bytes of w8, 4 of w4) ->
// 8 bf16 (16 bytes), w = bf16(fma(scale, q, qbias)). Block (row n, part p)
// covers kBlock * kDeqRuns consecutive runs of row n and consecutive lanes
// take consecutive runs, so each load and each store instruction is one
// contiguous span of the row; each thread has kDeqRuns runs in flight.
constexpr int kDeqRuns = 2;

template <int BITS>
__global__ void __launch_bounds__(kBlock)
dequant_kernel(const uint8_t* codes, const uint16_t* scales,
               const uint16_t* qbias, int gshift, int gcols, uint16_t* out,
               int N, int K, int ldo, const uint16_t* tail, int tail_cols, int tail_ld)
{
  const int n = blockIdx.x;
  const int runs = K >> 3;
  const int r0 = blockIdx.y * kBlock * kDeqRuns + threadIdx.x;
  const uint8_t* crow = codes + (size_t)n * K * BITS / 8;
  const uint16_t* srow = scales + (size_t)n * gcols;
  const uint16_t* qrow = qbias + (size_t)n * gcols;
  uint16_t* orow = out + (size_t)n * ldo;
  uint32_t v[kDeqRuns][2];
  float s[kDeqRuns], b[kDeqRuns];
#pragma unroll
  for (int j = 0; j < kDeqRuns; ++j) {
    const int r = r0 + j * kBlock;
    v[j][0] = v[j][1] = 0u;
    s[j] = b[j] = 0.0f;
    if (r < runs) {
      if constexpr (BITS == 8) {
        const uint2 c = *(const uint2*)(crow + (size_t)r * 8);
        v[j][0] = c.x;
        v[j][1] = c.y;
      } else {
        v[j][0] = *(const uint32_t*)(crow + (size_t)r * 4);
      }
      const int g = (r << 3) >> gshift;
      s[j] = bf16_to_f32(srow[g]);
      b[j] = bf16_to_f32(qrow[g]);
    }
  }
  // Columns [K, ldo) of the row: tail row n (tail_cols of it, zeros past
  // them), 8 columns per thread, strided by the block so any width is
  // covered. Loaded after the codes, so that both loads are in flight
  // together; one 16-byte load where the 8 columns are whole and aligned.
  for (int c = (int)threadIdx.x * 8; tail != nullptr && blockIdx.y == 0 && c < ldo - K;
       c += kBlock * 8) {
    const uint16_t* trow = tail + (size_t)n * tail_ld;
    uint32_t w[4];
    if (c + 8 <= tail_cols && ((uintptr_t)(trow + c) & 15u) == 0) {
      const uint4 t4 = *(const uint4*)(trow + c);
      w[0] = t4.x;
      w[1] = t4.y;
      w[2] = t4.z;
      w[3] = t4.w;
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t lo = c + 2 * t < tail_cols ? trow[c + 2 * t] : 0u;
        const uint32_t hi = c + 2 * t + 1 < tail_cols ? trow[c + 2 * t + 1] : 0u;
        w[t] = lo | (hi << 16);
      }
    }
    *(uint4*)(orow + K + c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
#pragma unroll
  for (int j = 0; j < kDeqRuns; ++j) {
    const int r = r0 + j * kBlock;
    if (r >= runs) { return; }
    uint32_t o[4];
    if constexpr (BITS == 8) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t w = v[j][h];
        o[2 * h] = pack_bf16x2(fmaf(s[j], (float)(w & 0xffu), b[j]),
                               fmaf(s[j], (float)((w >> 8) & 0xffu), b[j]));
        o[2 * h + 1] = pack_bf16x2(fmaf(s[j], (float)((w >> 16) & 0xffu), b[j]),
                                   fmaf(s[j], (float)(w >> 24), b[j]));
      }
    } else {
      // code c at bits 4c of the word
      const uint32_t w = v[j][0];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        o[t] = pack_bf16x2(fmaf(s[j], (float)((w >> (8 * t)) & 0xfu), b[j]),
                           fmaf(s[j], (float)((w >> (8 * t + 4)) & 0xfu), b[j]));
      }
    }
    *(uint4*)(orow + (size_t)r * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Group-affine quantize, one thread per (row, group). Step for step the
// quantizer of tests/ltx25-qlinear-test.cc:108-139: fmin/fmax over the
// group, scale and min rounded to bf16 first, codes by round-half-away of
// (w - bias) / scale with IEEE division, clamped; LOW bits first.
__global__ void __launch_bounds__(kBlock)
quantize_affine_kernel(const float* w, uint32_t* codes, uint16_t* scales,
                       uint16_t* qbias, int N, int K, int bits, int group)
{
  const int gcols = K / group;
  const size_t gid = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (gid >= (size_t)N * gcols) { return; }
  const int n = (int)(gid / gcols);
  const int g = (int)(gid % gcols);
  const float* wr = w + (size_t)n * K + (size_t)g * group;
  float lo = wr[0], hi = wr[0];
  for (int j = 1; j < group; ++j) {
    lo = fminf(lo, wr[j]);
    hi = fmaxf(hi, wr[j]);
  }
  const float qmax = (float)((1 << bits) - 1);
  const uint16_t sc_b = f32_to_bf16((hi - lo) / qmax);
  const uint16_t lo_b = f32_to_bf16(lo);
  scales[gid] = sc_b;
  qbias[gid] = lo_b;
  const float scr = bf16_to_f32(sc_b);
  const float lor = bf16_to_f32(lo_b);
  const int per_word = 32 / bits;
  uint32_t* dst = codes + ((size_t)n * K + (size_t)g * group) / per_word;
  for (int wd = 0; wd < group / per_word; ++wd) {
    uint32_t word = 0;
    for (int s = 0; s < per_word; ++s) {
      const float v = wr[wd * per_word + s];
      float q = scr > 0.0f ? roundf((v - lor) / scr) : 0.0f;
      q = fminf(fmaxf(q, 0.0f), qmax);
      word |= (uint32_t)q << (bits * s);
    }
    dst[wd] = word;
  }
}

// u8 codes [N][K] <-> u32 words, LOW bits first; one word per thread.
__global__ void __launch_bounds__(kBlock)
pack_kernel(const uint8_t* q, uint32_t* codes, size_t words, int bits)
{
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= words) { return; }
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t v = 0;
  for (int s = 0; s < per_word; ++s) {
    v |= ((uint32_t)q[i * per_word + s] & mask) << (bits * s);
  }
  codes[i] = v;
}

__global__ void __launch_bounds__(kBlock)
unpack_kernel(const uint32_t* codes, uint8_t* q, size_t words, int bits)
{
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= words) { return; }
  const int per_word = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const uint32_t v = codes[i];
  for (int s = 0; s < per_word; ++s) {
    q[i * per_word + s] = (uint8_t)((v >> (bits * s)) & mask);
  }
}

// F16 -> f32 (exact) -> bf16 (RNE), 8 per thread; in place allowed.
__global__ void __launch_bounds__(kBlock)
f16_to_bf16_kernel(const uint16_t* in, uint16_t* out, size_t n)
{
  const size_t i0 = ((size_t)blockIdx.x * kBlock + threadIdx.x) * 8;
  if (i0 >= n) { return; }
  auto cvt = [](uint16_t h) -> float {
    return (float)__builtin_bit_cast(_Float16, h);
  };
  if (i0 + 8 <= n) {
    const uint4 v = *(const uint4*)(in + i0);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[j] = pack_bf16x2(cvt((uint16_t)(w[j] & 0xffffu)), cvt((uint16_t)(w[j] >> 16)));
    }
    *(uint4*)(out + i0) = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  for (size_t i = i0; i < n; ++i) { out[i] = f32_to_bf16(cvt(in[i])); }
}

int ilog2(int v)
{
  int s = 0;
  while ((1 << s) < v) { ++s; }
  return s;
}

}  // namespace

hipError_t launch_bias_add(uint16_t* y, const void* bias, int bias_type,
                           int M, int N, hipStream_t stream)
{
  const size_t total = (size_t)M * N;
  hipLaunchKernelGGL(bias_add_kernel, dim3(blocks_for((total + 7) / 8)),
                     dim3(kBlock), 0, stream, y, bias, bias_type, N, total);
  return hipGetLastError();
}

hipError_t launch_gelu(const uint16_t* x, uint16_t* y, size_t n,
                       hipStream_t stream)
{
  hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for((n + 7) / 8)), dim3(kBlock),
                     0, stream, x, y, n);
  return hipGetLastError();
}

hipError_t launch_gate_heads(uint16_t* y, const uint16_t* logits, int heads, int tokens,
                             int head_dim, hipStream_t stream)
{
  const size_t chunks_per_row = ((size_t)head_dim + 7) / 8;
  const size_t total = (size_t)tokens * heads * chunks_per_row;
  if (total == 0) { return hipSuccess; }
  const bool vec = head_dim % 8 == 0 && ((uintptr_t)y & 15u) == 0;
  hipLaunchKernelGGL(gate_heads_kernel, dim3(blocks_for(total)), dim3(kBlock), 0, stream, y,
                     logits, heads, head_dim, chunks_per_row, total, vec);
  return hipGetLastError();
}

hipError_t launch_dequant(const void* codes, const uint16_t* scales,
                          const uint16_t* qbias, int bits, int group,
                          uint16_t* out, int N, int K, hipStream_t stream, int ldo,
                          const uint16_t* tail, int tail_cols, int tail_ld)
{
  if (ldo == 0) { ldo = K; }
  if (ldo < K || ldo % 8 != 0 ||
      (tail != nullptr && (tail_cols > ldo - K || tail_ld < tail_cols))) {
    return hipErrorInvalidValue;
  }
  const int gshift = ilog2(group);
  const int gcols = K / group;
  const int parts = (K / 8 + kBlock * kDeqRuns - 1) / (kBlock * kDeqRuns);
  const dim3 grid((unsigned)N, (unsigned)parts, 1);
  if (bits == 8) {
    hipLaunchKernelGGL(dequant_kernel<8>, grid, dim3(kBlock), 0, stream,
                       (const uint8_t*)codes, scales, qbias, gshift, gcols, out, N, K, ldo,
                       tail, tail_cols, tail_ld);
  } else {
    hipLaunchKernelGGL(dequant_kernel<4>, grid, dim3(kBlock), 0, stream,
                       (const uint8_t*)codes, scales, qbias, gshift, gcols, out, N, K, ldo,
                       tail, tail_cols, tail_ld);
  }
  return hipGetLastError();
}

hipError_t launch_quantize_affine(const float* w, uint32_t* codes,
                                  uint16_t* scales, uint16_t* qbias, int N,
                                  int K, int bits, int group,
                                  hipStream_t stream)
{
  const size_t groups = (size_t)N * (K / group);
  hipLaunchKernelGGL(quantize_affine_kernel, dim3(blocks_for(groups)),
                     dim3(kBlock), 0, stream, w, codes, scales, qbias, N, K,
                     bits, group);
  return hipGetLastError();
}

hipError_t launch_pack(const uint8_t* q, uint32_t* codes, int N, int K,
                       int bits, hipStream_t stream)
{
  const size_t words = (size_t)N * K * bits / 32;
  hipLaunchKernelGGL(pack_kernel, dim3(blocks_for(words)), dim3(kBlock), 0,
                     stream, q, codes, words, bits);
  return hipGetLastError();
}

hipError_t launch_unpack(const uint32_t* codes, uint8_t* q, int N, int K,
                         int bits, hipStream_t stream)
{
  const size_t words = (size_t)N * K * bits / 32;
  hipLaunchKernelGGL(unpack_kernel, dim3(blocks_for(words)), dim3(kBlock), 0,
                     stream, codes, q, words, bits);
  return hipGetLastError();
}

hipError_t launch_f16_to_bf16(const uint16_t* in, uint16_t* out, size_t n,
                              hipStream_t stream)
{
  hipLaunchKernelGGL(f16_to_bf16_kernel, dim3(blocks_for((n + 7) / 8)),
                     dim3(kBlock), 0, stream, in, out, n);
  return hipGetLastError();
}

}  // namespace ltx25
