// The int8 tier on gfx950: per-row symmetric int8 quantization of
// activations and of (dequantized) weights. The int8 x int8 -> int32 GEMM
// itself runs on the bf16 GEMM's tile machinery (qgemm.hip, operand mode
// kI8Ops: v_mfma_i32_32x32x32_i8, 128 int8 of K per step in the same
// 128-byte LDS rows) with the dequant epilogue fused:
//   y = bf16(fma(float(acc), sx[m] * sw[n], bias[n] or +0)).
// Integer accumulation is exact, so the int32 results are bit-identical to
// any other order of the same sum; the epilogue is a fixed f32 sequence.
//
// Reference: the int8 tier under MetalOps::dense_mma_ (I8GemmContext::gemm,
// src/ltx25-metal-ops.cc:386-391; contract at src/ltx25-metal-ops.h:810-817).
#include "common.h"

namespace ltx25 {
namespace {

constexpr int kThreads = 256;

// Rows longer than kCacheChunks 16-byte chunks per thread are re-read for
// the second pass; up to that they stay in registers between the passes.
constexpr int kCacheChunks = 8;

__device__ __forceinline__ uint32_t q8(float v, float s)
{
  float r = 0.0f;
  if (s > 0.0f) {
    r = rintf(v / s);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
  }
  return (uint32_t)(int)r & 0xffu;
}

__device__ __forceinline__ float block_absmax(float amax, float* red)
{
  for (int off = 32; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  }
  if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = amax; }
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One workgroup per row: absmax, then q = clamp(rint(x / s), -127, 127),
// s = absmax / 127. Works on bf16 activations (values exact in f32); the
// row is read once, 16 bytes (8 values) per load.
__global__ void __launch_bounds__(kThreads)
i8_quantize_rows_kernel(const uint16_t* x, int8_t* q, float* scale, int K)
{
  __shared__ float red[kThreads / 64];
  const int m = blockIdx.x;
  const uint16_t* xr = x + (size_t)m * K;
  int8_t* qr = q + (size_t)m * K;
  const int chunks = K / 8;
  uint4 cache[kCacheChunks];
  float amax = 0.0f;
  auto absmax8 = [&](const uint4& v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(bf16_to_f32((uint16_t)(w[j] & 0xffffu))));
      amax = fmaxf(amax, fabsf(bf16_to_f32((uint16_t)(w[j] >> 16))));
    }
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = (int)threadIdx.x + c * kThreads;
    if (i < chunks) {
      cache[c] = *(const uint4*)(xr + (size_t)i * 8);
      absmax8(cache[c]);
    }
  }
  for (int i = (int)threadIdx.x + kCacheChunks * kThreads; i < chunks; i += kThreads) {
    absmax8(*(const uint4*)(xr + (size_t)i * 8));
  }
  amax = block_absmax(amax, red);
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) { scale[m] = s; }
  auto quant8 = [&](const uint4& v, int i) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
      packed[j >> 2] |= q8(bf16_to_f32(h), s) << (8 * (j & 3));
    }
    *(uint2*)(qr + (size_t)i * 8) = make_uint2(packed[0], packed[1]);
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = (int)threadIdx.x + c * kThreads;
    if (i < chunks) { quant8(cache[c], i); }
  }
  for (int i = (int)threadIdx.x + kCacheChunks * kThreads; i < chunks; i += kThreads) {
    quant8(*(const uint4*)(xr + (size_t)i * 8), i);
  }
}

// The same for the dequantized values of a group-affine weight row,
// w = bf16(fma(scale, q, qbias)): one 16-byte load of codes (16 w8 or 32 w4
// codes, all in one group) per chunk, kept in registers between the absmax
// and the quantize pass; 16-byte int8 stores.
template <int BITS>
__global__ void __launch_bounds__(kThreads)
i8_quantize_qweight_kernel(const uint8_t* codes, const uint16_t* scales,
                           const uint16_t* qbias, int gshift, int gcols,
                           int8_t* q, float* scale, int K)
{
  __shared__ float red[kThreads / 64];
  constexpr int CPC = 128 / BITS;                 // codes per 16-byte chunk
  const int n = blockIdx.x;
  const uint8_t* cr = codes + (size_t)n * ((size_t)K * BITS / 8);
  const uint16_t* srow = scales + (size_t)n * gcols;
  const uint16_t* brow = qbias + (size_t)n * gcols;
  int8_t* qr = q + (size_t)n * K;
  const int chunks = K / CPC;
  uint4 cache[kCacheChunks];
  float amax = 0.0f;
  // the CPC dequantized values of chunk i, in order, into v
  auto dequant = [&](const uint4& c, int i, float* v) {
    const int g = (i * CPC) >> gshift;
    const float s = bf16_to_f32(srow[g]);
    const float b = bf16_to_f32(brow[g]);
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < CPC; ++j) {
      uint32_t code;
      if constexpr (BITS == 8) {
        code = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
      } else {
        code = (w[j >> 3] >> (4 * (j & 7))) & 0xfu;
      }
      v[j] = bf16_to_f32(f32_to_bf16(fmaf(s, (float)code, b)));
    }
  };
  auto absmax_chunk = [&](const uint4& c, int i) {
    float v[CPC];
    dequant(c, i, v);
#pragma unroll
    for (int j = 0; j < CPC; ++j) { amax = fmaxf(amax, fabsf(v[j])); }
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = (int)threadIdx.x + c * kThreads;
    if (i < chunks) {
      cache[c] = *(const uint4*)(cr + (size_t)i * 16);
      absmax_chunk(cache[c], i);
    }
  }
  for (int i = (int)threadIdx.x + kCacheChunks * kThreads; i < chunks; i += kThreads) {
    absmax_chunk(*(const uint4*)(cr + (size_t)i * 16), i);
  }
  amax = block_absmax(amax, red);
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) { scale[n] = s; }
  auto quant_chunk = [&](const uint4& c, int i) {
    float v[CPC];
    dequant(c, i, v);
    uint32_t packed[CPC / 4];
#pragma unroll
    for (int t = 0; t < CPC / 4; ++t) {
      packed[t] = q8(v[4 * t], s) | (q8(v[4 * t + 1], s) << 8) | (q8(v[4 * t + 2], s) << 16) |
                  (q8(v[4 * t + 3], s) << 24);
    }
#pragma unroll
    for (int t = 0; t < CPC / 16; ++t) {
      *(uint4*)(qr + (size_t)i * CPC + 16 * t) =
          make_uint4(packed[4 * t], packed[4 * t + 1], packed[4 * t + 2], packed[4 * t + 3]);
    }
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = (int)threadIdx.x + c * kThreads;
    if (i < chunks) { quant_chunk(cache[c], i); }
  }
  for (int i = (int)threadIdx.x + kCacheChunks * kThreads; i < chunks; i += kThreads) {
    quant_chunk(*(const uint4*)(cr + (size_t)i * 16), i);
  }
}

int ilog2(int v)
{
  int s = 0;
  while ((1 << s) < v) { ++s; }
  return s;
}

}  // namespace

hipError_t launch_i8_quantize_rows(const uint16_t* x, int8_t* q, float* s,
                                   int M, int K, hipStream_t stream)
{
  hipLaunchKernelGGL(i8_quantize_rows_kernel, dim3(M), dim3(kThreads), 0,
                     stream, x, q, s, K);
  return hipGetLastError();
}

hipError_t launch_i8_quantize_qweight(const void* codes,
                                      const uint16_t* scales,
                                      const uint16_t* qbias, int bits,
                                      int group, int8_t* q, float* s, int N,
                                      int K, hipStream_t stream)
{
  const int gshift = ilog2(group);
  const int gcols = K / group;
  if (bits == 8) {
    hipLaunchKernelGGL(i8_quantize_qweight_kernel<8>, dim3(N), dim3(kThreads),
                       0, stream, (const uint8_t*)codes, scales, qbias, gshift,
                       gcols, q, s, K);
  } else {
    hipLaunchKernelGGL(i8_quantize_qweight_kernel<4>, dim3(N), dim3(kThreads),
                       0, stream, (const uint8_t*)codes, scales, qbias, gshift,
                       gcols, q, s, K);
  }
  return hipGetLastError();
}


}  // namespace ltx25
