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

// One workgroup per row: absmax, then q = clamp(rint(x / s), -127, 127).
// Works on bf16 activations (values exact in f32).
__global__ void __launch_bounds__(kThreads)
i8_quantize_rows_kernel(const uint16_t* x, int8_t* q, float* scale, int K)
{
  __shared__ float red[kThreads / 64];
  const int m = blockIdx.x;
  const uint16_t* xr = x + (size_t)m * K;
  int8_t* qr = q + (size_t)m * K;
  float amax = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += kThreads * 8) {
    const uint4 v = *(const uint4*)(xr + k);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(bf16_to_f32((uint16_t)(w[j] & 0xffffu))));
      amax = fmaxf(amax, fabsf(bf16_to_f32((uint16_t)(w[j] >> 16))));
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  }
  if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = amax; }
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) { scale[m] = s; }
  for (int k = threadIdx.x * 8; k < K; k += kThreads * 8) {
    const uint4 v = *(const uint4*)(xr + k);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
      float r = 0.0f;
      if (s > 0.0f) {
        r = rintf(bf16_to_f32(h) / s);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
      }
      packed[j >> 2] |= ((uint32_t)(int)r & 0xffu) << (8 * (j & 3));
    }
    *(uint2*)(qr + k) = make_uint2(packed[0], packed[1]);
  }
}

// The same for the dequantized values of a group-affine weight row:
// w = bf16(fma(scale, q, qbias)), read from the codes twice (absmax pass,
// then the quantize pass) rather than materialised.
template <int BITS>
__global__ void __launch_bounds__(kThreads)
i8_quantize_qweight_kernel(const uint8_t* codes, const uint16_t* scales,
                           const uint16_t* qbias, int gshift, int gcols,
                           int8_t* q, float* scale, int K)
{
  __shared__ float red[kThreads / 64];
  const int n = blockIdx.x;
  const size_t row_bytes = (size_t)K * BITS / 8;
  const uint8_t* cr = codes + (size_t)n * row_bytes;
  auto value = [&](int k) -> float {
    uint32_t c;
    if constexpr (BITS == 8) {
      c = cr[k];
    } else {
      c = (cr[k >> 1] >> (4 * (k & 1))) & 0xfu;
    }
    const size_t gi = (size_t)n * gcols + (k >> gshift);
    const float d = fmaf(bf16_to_f32(scales[gi]), (float)c, bf16_to_f32(qbias[gi]));
    return bf16_to_f32(f32_to_bf16(d));
  };
  float amax = 0.0f;
  for (int k = threadIdx.x; k < K; k += kThreads) {
    amax = fmaxf(amax, fabsf(value(k)));
  }
  for (int off = 32; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  }
  if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = amax; }
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax / 127.0f;
  if (threadIdx.x == 0) { scale[n] = s; }
  int8_t* qr = q + (size_t)n * K;
  for (int k = threadIdx.x; k < K; k += kThreads) {
    float r = 0.0f;
    if (s > 0.0f) {
      r = rintf(value(k) / s);
      r = fminf(fmaxf(r, -127.0f), 127.0f);
    }
    qr[k] = (int8_t)(int)r;
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
