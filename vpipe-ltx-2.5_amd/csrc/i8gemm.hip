// The int8 tier on gfx950: per-row symmetric int8 quantization and an
// int8 x int8 -> int32 GEMM on v_mfma_i32_32x32x32_i8 with the dequant
// epilogue fused:
//   y = bf16(fma(float(acc), sx[m] * sw[n], bias[n] or +0)).
// Integer accumulation is exact, so the int32 results are bit-identical to
// any other order of the same sum; the epilogue is a fixed f32 sequence.
//
// Tile geometry mirrors the bf16 GEMM: 128 int8 of K per step occupy the
// same 128-byte LDS row (144 B pitch) that 64 bf16 do there.
//
// Reference: the int8 tier under MetalOps::dense_mma_ (I8GemmContext::gemm,
// src/ltx25-metal-ops.cc:386-391; contract at src/ltx25-metal-ops.h:810-817).
#include "common.h"

namespace ltx25 {
namespace {

constexpr int kThreads = 256;
constexpr int kBKB = 128;            // K bytes (= int8 elements) per step
constexpr int kLdsRowB = kBKB + 16;  // 144 B pitch

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

struct I8Params {
  const int8_t* xq;
  const float* sx;
  const int8_t* wq;
  const float* sw;
  const void* bias;
  int bias_type;
  uint16_t* y;
  int32_t* acc_out;
  int M, N, K;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ void map_tile_i8(int bid, int tiles_m, int tiles_n,
                                            int& tm, int& tn)
{
  const int total = tiles_m * tiles_n;
  const int total8 = total & ~7;
  int pid = bid;
  if (bid < total8) { pid = (bid & 7) * (total8 >> 3) + (bid >> 3); }
  constexpr int kGroupM = 8;
  const int per_group = kGroupM * tiles_n;
  const int gid = pid / per_group;
  const int first_m = gid * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int r = pid - gid * per_group;
  tm = first_m + r % gsz;
  tn = r / gsz;
}

template <int BM, int BN>
__global__ void __launch_bounds__(kThreads)
i8_gemm_kernel(I8Params p)
{
  constexpr int WTM = BM / 2;
  constexpr int WTN = BN / 2;
  constexpr int FM = WTM / 32;
  constexpr int FN = WTN / 32;
  constexpr int A_LD = BM * 8 / kThreads;   // 16-byte chunks per thread
  constexpr int B_LD = BN * 8 / kThreads;

  __shared__ __attribute__((aligned(16))) int8_t lds_a[2][BM * kLdsRowB];
  __shared__ __attribute__((aligned(16))) int8_t lds_b[2][BN * kLdsRowB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;

  int tm, tn;
  map_tile_i8(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int nsteps = p.K / kBKB;

  const int c = tid & 7;
  const int r0 = tid >> 3;
  uint4 areg[A_LD];
  uint4 breg[B_LD];

  auto load_tiles = [&](int k) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int m = m0 + r0 + 32 * i;
      areg[i] = make_uint4(0u, 0u, 0u, 0u);
      if (m < p.M) { areg[i] = *(const uint4*)(p.xq + (size_t)m * p.K + k + c * 16); }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int n = n0 + r0 + 32 * i;
      breg[i] = make_uint4(0u, 0u, 0u, 0u);
      if (n < p.N) { breg[i] = *(const uint4*)(p.wq + (size_t)n * p.K + k + c * 16); }
    }
  };
  auto store_tiles = [&](int st) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      *(uint4*)&lds_a[st][(r0 + 32 * i) * kLdsRowB + c * 16] = areg[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      *(uint4*)&lds_b[st][(r0 + 32 * i) * kLdsRowB + c * 16] = breg[i];
    }
  };

  i32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { acc[i][j][r] = 0; }
    }
  }

  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int st = s & 1;
    const bool more = s + 1 < nsteps;
    if (more) { load_tiles((s + 1) * kBKB); }
    const int8_t* la = lds_a[st] + (wm * WTM + (lane & 31)) * kLdsRowB + (lane >> 5) * 16;
    const int8_t* lb = lds_b[st] + (wn * WTN + (lane & 31)) * kLdsRowB + (lane >> 5) * 16;
#pragma unroll
    for (int kk = 0; kk < kBKB / 32; ++kk) {
      i32x4 af[FM];
      i32x4 bfv[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) { af[i] = *(const i32x4*)(la + i * 32 * kLdsRowB + kk * 32); }
#pragma unroll
      for (int j = 0; j < FN; ++j) { bfv[j] = *(const i32x4*)(lb + j * 32 * kLdsRowB + kk * 32); }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bfv[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (more) { store_tiles(st ^ 1); }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * WTN + j * 32 + (lane & 31);
    float bv = 0.0f;
    float swn = 0.0f;
    if (n < p.N) {
      swn = p.sw[n];
      if (p.bias_type == kBiasBf16) { bv = bf16_to_f32(((const uint16_t*)p.bias)[n]); }
      else if (p.bias_type == kBiasF32) { bv = ((const float*)p.bias)[n]; }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int mb = m0 + wm * WTM + i * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + (r >> 2) * 8 + (r & 3);
        if (m < p.M && n < p.N) {
          const int a = acc[i][j][r];
          if (p.acc_out != nullptr) { p.acc_out[(size_t)m * p.N + n] = a; }
          const float sc = p.sx[m] * swn;
          p.y[(size_t)m * p.N + n] = f32_to_bf16(fmaf((float)a, sc, bv));
        }
      }
    }
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

hipError_t launch_i8_gemm(const int8_t* xq, const float* sx,
                          const int8_t* wq, const float* sw, const void* bias,
                          int bias_type, uint16_t* y, int32_t* acc, int M,
                          int K, int N, hipStream_t stream)
{
  I8Params p;
  p.xq = xq;
  p.sx = sx;
  p.wq = wq;
  p.sw = sw;
  p.bias = bias;
  p.bias_type = bias != nullptr ? bias_type : kBiasNone;
  p.y = y;
  p.acc_out = acc;
  p.M = M;
  p.N = N;
  p.K = K;
  int dev = 0;
  int cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    cus = 256;
  }
  const long tall = (long)((M + 255) / 256) * ((N + 255) / 256);
  if (tall >= cus) {
    p.tiles_m = (M + 255) / 256;
    p.tiles_n = (N + 255) / 256;
    hipLaunchKernelGGL((i8_gemm_kernel<256, 256>), dim3(p.tiles_m * p.tiles_n),
                       dim3(kThreads), 0, stream, p);
  } else {
    p.tiles_m = (M + 127) / 128;
    p.tiles_n = (N + 127) / 128;
    hipLaunchKernelGGL((i8_gemm_kernel<128, 128>), dim3(p.tiles_m * p.tiles_n),
                       dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace ltx25
