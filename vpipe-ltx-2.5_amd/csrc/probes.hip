// Measurement probes: the two ceilings the GEMM kernels are judged against.
// Neither computes anything the linear needs; bench.py's --ceilings leg
// times them.
//   - stream read: `bytes` of device memory read once with 16-byte loads,
//     four in flight per lane, every workgroup on its own contiguous span
//     (the HBM ceiling of a kernel that moves a C1 audio GEMM's bytes);
//   - MFMA stream: independent v_mfma_f32_16x16x32_bf16 on operands held in
//     registers, zero or random bf16, one or two waves per SIMD (the rate
//     the matrix cores hold on such data at the clock that power allows).
#include "common.h"

namespace ltx25 {
namespace {

constexpr int kReadThreads = 256;

__global__ void __launch_bounds__(kReadThreads)
stream_read_kernel(const i32x4* __restrict__ src, size_t n16, size_t per_block, uint32_t* sink)
{
  const size_t b0 = (size_t)blockIdx.x * per_block;
  const size_t b1 = min(n16, b0 + per_block);
  uint32_t x = 0;
  for (size_t i = b0 + threadIdx.x; i < b1; i += 4 * kReadThreads) {
    i32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t j = i + (size_t)u * kReadThreads;
      v[u] = j < b1 ? __builtin_nontemporal_load(src + j) : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) { x ^= (uint32_t)(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]); }
  }
  // one word per workgroup keeps the loads live
  __shared__ uint32_t red[kReadThreads];
  red[threadIdx.x] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int t = 0; t < kReadThreads; ++t) { r ^= red[t]; }
    sink[blockIdx.x] = r;
  }
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <bool RANDOM>
__global__ void __launch_bounds__(512)
mfma_stream_kernel(int iters, float* out)
{
  uint32_t h = (blockIdx.x * 512u + threadIdx.x) * 2654435761u;
  uint32_t ra[4][4], rb[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (RANDOM) {
        // bf16 pairs of magnitude ~1 with random mantissas and signs
        h ^= h << 13;
        h ^= h >> 17;
        h ^= h << 5;
        ra[k][e] = (h & 0x807f807fu) | 0x3f003f00u;
        h ^= h << 13;
        h ^= h >> 17;
        h ^= h << 5;
        rb[k][e] = (h & 0x807f807fu) | 0x3f003f00u;
      } else {
        // 0, from a kernel argument so that the compiler cannot fold it
        ra[k][e] = (uint32_t)iters >> 31;
        rb[k][e] = (uint32_t)iters >> 31;
      }
    }
  }
  bf16x8 a[4], b[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = __builtin_bit_cast(bf16x8, make_uint4(ra[k][0], ra[k][1], ra[k][2], ra[k][3]));
    b[k] = __builtin_bit_cast(bf16x8, make_uint4(rb[k][0], rb[k][1], rb[k][2], rb[k][3]));
  }
  f32x4v acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) { acc[k] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f}; }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[k & 3], b[(k >> 1) & 3], acc[k], 0, 0, 0);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) { s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3]; }
  if (s == 1.2345f) { out[blockIdx.x] = s; }   // practically never: keeps the MFMAs live
}

}  // namespace

hipError_t launch_probe_read(const void* src, size_t bytes, uint32_t* sink, int blocks,
                             hipStream_t stream)
{
  const size_t n16 = bytes / 16;
  const size_t per_block = (n16 + (size_t)blocks - 1) / (size_t)blocks;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(kReadThreads), 0, stream,
                     (const i32x4*)src, n16, per_block, sink);
  return hipGetLastError();
}

hipError_t launch_probe_mfma(int iters, int random, int waves_per_simd, float* out,
                             hipStream_t stream)
{
  const dim3 block((unsigned)(256 * waves_per_simd));
  if (random) {
    hipLaunchKernelGGL(mfma_stream_kernel<true>, dim3(256), block, 0, stream, iters, out);
  } else {
    hipLaunchKernelGGL(mfma_stream_kernel<false>, dim3(256), block, 0, stream, iters, out);
  }
  return hipGetLastError();
}

}  // namespace ltx25
