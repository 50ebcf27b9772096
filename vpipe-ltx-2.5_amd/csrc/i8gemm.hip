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
constexpr int kRowsPerBlock = kThreads / 64;   // one wave per row

// 16-byte chunks a lane keeps in registers between the absmax pass and the
// quantize pass (K up to 8192 bf16 or 16384 w8 codes); chunks past them are
// read again for the second pass.
constexpr int kCacheChunks = 16;

// q = clamp(rint(v / s), -127, 127) with v / s correctly rounded, given
// rs = 1 / s rounded, for four values packed low byte first. t = v * rs is
// within 2^-24 |v / s| (1 + 2^-24) of the quotient, i.e. within 2^-15 for
// |t| < 256; so rint(t) = rint(v / s) unless t lies within 2^-13 of a
// half-integer. Those values, and any t that is not a finite number below
// 256 (s tiny, v or s not finite), take the division itself. The test for
// that fallback is made once for the four values (a test per value was a
// branch per value around the rarely taken division); s <= 0 gives 0.
__device__ __forceinline__ uint32_t q8x4(const float* v, float s, float rs)
{
  if (!(s > 0.0f)) { return 0u; }
  float r[4];
  int slow = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float t = v[j] * rs;
    r[j] = rintf(t);
    slow |= (int)!(fabsf(t) < 256.0f) | (int)(fabsf(t - r[j]) > 0.5f - 0x1p-13f);
  }
  if (slow) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = v[j] * rs;
      if (!(fabsf(t) < 256.0f) || fabsf(t - r[j]) > 0.5f - 0x1p-13f) { r[j] = rintf(v[j] / s); }
    }
  }
  uint32_t out = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out |= ((uint32_t)(int)fminf(fmaxf(r[j], -127.0f), 127.0f) & 0xffu) << (8 * j);
  }
  return out;
}

__device__ __forceinline__ float wave_absmax(float amax)
{
  for (int off = 32; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  }
  return amax;
}

// One wave per row: absmax, then q = clamp(rint(x / s), -127, 127),
// s = absmax / 127. Works on bf16 activations (values exact in f32). Lane l
// takes 16-byte chunks l, l + 64, ...: every load instruction of the wave
// covers 1 KB of the row, up to 16 of them in flight per lane, and the
// row's maximum is a shuffle reduction (no LDS, no barrier).
__global__ void __launch_bounds__(kThreads)
i8_quantize_rows_kernel(const uint16_t* x, int8_t* q, float* scale, int M, int K)
{
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (m >= M) { return; }
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
    const int i = lane + c * 64;
    if (i < chunks) { cache[c] = *(const uint4*)(xr + (size_t)i * 8); }
  }
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    if (lane + c * 64 < chunks) { absmax8(cache[c]); }
  }
  for (int i = lane + kCacheChunks * 64; i < chunks; i += 64) {
    absmax8(*(const uint4*)(xr + (size_t)i * 8));
  }
  amax = wave_absmax(amax);
  const float s = amax / 127.0f;
  const float rs = 1.0f / s;
  if (lane == 0) { scale[m] = s; }
  auto quant8 = [&](const uint4& v, int i) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) { f[j] = bf16_to_f32((uint16_t)(w[j >> 1] >> (16 * (j & 1)))); }
    *(uint2*)(qr + (size_t)i * 8) = make_uint2(q8x4(f, s, rs), q8x4(f + 4, s, rs));
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = lane + c * 64;
    if (i < chunks) { quant8(cache[c], i); }
  }
  for (int i = lane + kCacheChunks * 64; i < chunks; i += 64) {
    quant8(*(const uint4*)(xr + (size_t)i * 8), i);
  }
}

// The same for the dequantized values of a group-affine weight row,
// w = bf16(fma(scale, q, qbias)): one wave per row, one 16-byte load of
// codes (16 w8 or 32 w4 codes, all in one group) per chunk, kept in
// registers between the absmax and the quantize pass; 16-byte int8 stores.
template <int BITS>
__global__ void __launch_bounds__(kThreads)
i8_quantize_qweight_kernel(const uint8_t* codes, const uint16_t* scales,
                           const uint16_t* qbias, int gshift, int gcols,
                           int8_t* q, float* scale, int N, int K)
{
  constexpr int CPC = 128 / BITS;                 // codes per 16-byte chunk
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (n >= N) { return; }
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
    const int i = lane + c * 64;
    if (i < chunks) { cache[c] = *(const uint4*)(cr + (size_t)i * 16); }
  }
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = lane + c * 64;
    if (i < chunks) { absmax_chunk(cache[c], i); }
  }
  for (int i = lane + kCacheChunks * 64; i < chunks; i += 64) {
    absmax_chunk(*(const uint4*)(cr + (size_t)i * 16), i);
  }
  amax = wave_absmax(amax);
  const float s = amax / 127.0f;
  const float rs = 1.0f / s;
  if (lane == 0) { scale[n] = s; }
  auto quant_chunk = [&](const uint4& c, int i) {
    float v[CPC];
    dequant(c, i, v);
    uint32_t packed[CPC / 4];
#pragma unroll
    for (int t = 0; t < CPC / 4; ++t) { packed[t] = q8x4(v + 4 * t, s, rs); }
#pragma unroll
    for (int t = 0; t < CPC / 16; ++t) {
      *(uint4*)(qr + (size_t)i * CPC + 16 * t) =
          make_uint4(packed[4 * t], packed[4 * t + 1], packed[4 * t + 2], packed[4 * t + 3]);
    }
  };
#pragma unroll
  for (int c = 0; c < kCacheChunks; ++c) {
    const int i = lane + c * 64;
    if (i < chunks) { quant_chunk(cache[c], i); }
  }
  for (int i = lane + kCacheChunks * 64; i < chunks; i += 64) {
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
  const dim3 grid((unsigned)((M + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL(i8_quantize_rows_kernel, grid, dim3(kThreads), 0, stream, x, q, s, M, K);
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
  const dim3 grid((unsigned)((N + kRowsPerBlock - 1) / kRowsPerBlock));
  if (bits == 8) {
    hipLaunchKernelGGL(i8_quantize_qweight_kernel<8>, grid, dim3(kThreads), 0, stream,
                       (const uint8_t*)codes, scales, qbias, gshift, gcols, q, s, N, K);
  } else {
    hipLaunchKernelGGL(i8_quantize_qweight_kernel<4>, grid, dim3(kThreads), 0, stream,
                       (const uint8_t*)codes, scales, qbias, gshift, gcols, q, s, N, K);
  }
  return hipGetLastError();
}


}  // namespace ltx25
