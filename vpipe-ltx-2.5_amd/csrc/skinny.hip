// The skinny quantized linear on gfx950, for M <= 128 rows (the audio
// stream's ~126 tokens): y = x . dequant(W)^T (+ bias) (+ GELU).
//
// These GEMMs sit near the bf16 ridge (about 256 FLOP per weight byte
// against a ridge of about 300), so the weight stream from HBM and the
// MFMA work both have to run near their peaks at once. The layout:
//
//   - Each wave owns 32 output columns for ALL rows (up to 128 = four
//     32-row v_mfma_f32_32x32x16_bf16 tiles). Every weight element is
//     therefore dequantized exactly once, in registers, straight from its
//     16-byte global load: weights never touch LDS.
//   - The workgroup's NW waves cover BN = 32*NW adjacent columns and share
//     the activation tile, staged through LDS one 64-deep K step at a time.
//   - Lane l of a wave loads the 32 consecutive codes [32h, 32h+32) of a
//     step for column l%32 (h = l/32). MFMA slice j uses codes
//     [32h+8j, 32h+8j+8): the K order inside a step is permuted the same
//     way for the activation fragments, which the dot product allows.
//   - Weight loads run kDepth steps ahead in a register ring, so each
//     wave keeps about kDepth * 2 KB of the weight stream in flight.
//   - K is split over `splits` workgroups per column tile. Each writes an
//     f32 partial tile; the last to arrive (an atomic counter per tile)
//     sums the partials in split order, adds the bias, applies GELU and
//     rounds once to bf16 -- deterministic, and the linear is one launch.
//     The counter is reset by that last workgroup, so the counters are
//     zero again when the launch ends.
//
// Reference semantics: MetalOps::linear(QWeight) (src/ltx25-metal-ops.cc:
// 531-569) over the affine_dequant weight, then ltx_bias_add.
#include "common.h"

#include <algorithm>

namespace ltx25 {
namespace {

constexpr int kSkBK = 64;                 // K per step
constexpr int kSkRows = 128;              // rows per workgroup
constexpr int kSkLdsRow = kSkBK + 8;      // bf16 pitch of an activation row (144 B)
constexpr int kSkDepth = 4;               // weight steps in flight per wave

struct SkParams {
  const uint16_t* x;
  const void* w;
  const uint16_t* scales;
  const uint16_t* qbias;
  const void* bias;
  uint16_t* y;
  float* partial;        // [splits][M][N] f32
  int* counters;         // [tiles_n], zero between launches
  int M, N, K;
  int gshift, gcols;
  int k_chunk, splits;
  int bias_type, epilogue;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, size_t bytes)
{
  // Raw buffer: loads past `bytes` return zeros (rows past M, columns past N).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)(uint32_t)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 sk_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff)
{
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

__device__ __forceinline__ float sk_bias(const void* bias, int type, int n)
{
  if (type == kBiasBf16) { return bf16_to_f32(((const uint16_t*)bias)[n]); }
  if (type == kBiasF32) { return ((const float*)bias)[n]; }
  return 0.0f;
}

// 8 codes (two u32 words of u8, or one u32 of u4) -> one bf16x8 fragment,
// w = bf16(fma(scale, q, qbias)).
template <int BITS>
__device__ __forceinline__ bf16x8 dequant8(const uint32_t* words, float s, float b)
{
  uint32_t o[4];
  if constexpr (BITS == 8) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t v = words[t];
      o[2 * t] = pack_bf16x2(fmaf(s, (float)(v & 0xffu), b), fmaf(s, (float)((v >> 8) & 0xffu), b));
      o[2 * t + 1] = pack_bf16x2(fmaf(s, (float)((v >> 16) & 0xffu), b), fmaf(s, (float)(v >> 24), b));
    }
  } else {
    // u4: code 2c sits in the low nibble of byte c, code 2c+1 in the high.
    const uint32_t v = words[0];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t byte = (v >> (8 * t)) & 0xffu;
      o[t] = pack_bf16x2(fmaf(s, (float)(byte & 0xfu), b), fmaf(s, (float)(byte >> 4), b));
    }
  }
  return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

template <int NW, int BITS>
__global__ void __launch_bounds__(NW * 64)
skinny_kernel(SkParams p)
{
  constexpr bool QUANT = BITS != 16;
  constexpr int WB = QUANT ? 32 * BITS / 8 : 64;        // weight bytes per lane per step
  constexpr int WL = WB / 16;                            // 16 B loads per lane per step
  constexpr int WLOADS = WL + (QUANT ? 2 : 0);           // + scale and zero point
  constexpr int NT = NW * 64;
  constexpr int XL = kSkRows * kSkBK * 2 / 16 / NT;      // activation 16 B loads per thread per step
  static_assert(XL >= 1, "too many threads for one activation tile");

  // The activation tile of a step, 128 rows x 64 bf16, in two LDS stages
  // with a 144 B row pitch: the 16 B fragment reads of 16 rows at one
  // column then hit 16 distinct bank groups.
  __shared__ __attribute__((aligned(16))) uint16_t lds_x[2][kSkRows * kSkLdsRow];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int tn = blockIdx.x;
  const int split = blockIdx.y;
  const int col = tn * 32 * NW + wave * 32 + (lane & 31);
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nsteps = (kend - kbeg) / kSkBK;

  const size_t row_bytes = (size_t)p.K * (QUANT ? BITS : 16) / 8;
  const __amdgpu_buffer_rsrc_t xr = sk_rsrc(p.x, (size_t)p.M * p.K * 2);
  const __amdgpu_buffer_rsrc_t wr = sk_rsrc(p.w, (size_t)p.N * row_bytes);
  const __amdgpu_buffer_rsrc_t sr = sk_rsrc(p.scales, QUANT ? (size_t)p.N * p.gcols * 2 : 0);
  const __amdgpu_buffer_rsrc_t qr = sk_rsrc(p.qbias, QUANT ? (size_t)p.N * p.gcols * 2 : 0);

  // Steps at or past nsteps load with a per-lane offset (voffset) past
  // every buffer's end: the buffer unit's range check returns zeros
  // without touching memory, and the zero codes (scale and zero point 0)
  // dequantize to 0 and add nothing. The range check covers the per-lane
  // offset, so every offset that can leave a buffer rides there; the
  // uniform offset (soffset) is only used in range. Every step therefore
  // issues the same loads with no branch, and load counts stay exact.
  constexpr uint32_t kOob = 0x80000000u;
  auto k_of = [&](int s) { return (uint32_t)(kbeg + s * kSkBK); };

  // Weight stream: lane l loads the 32 codes [32h, 32h+32) of a step for
  // column l%32 (h = l/32) into a register ring kSkDepth steps deep.
  const uint32_t w_off = (uint32_t)((size_t)col * row_bytes + (size_t)half * WB);
  const uint32_t s_off =
      QUANT ? (uint32_t)(((size_t)col * p.gcols + ((32 * half) >> p.gshift)) * 2) : 0u;
  uint4 wreg[kSkDepth][WL];
  uint16_t sreg[kSkDepth];
  uint16_t qreg[kSkDepth];
  auto load_w = [&](int s, int d) {
    const bool in = s < nsteps;
    const uint32_t wo = in ? (uint32_t)((size_t)k_of(s) * (QUANT ? BITS : 16) / 8) : 0u;
#pragma unroll
    for (int i = 0; i < WL; ++i) { wreg[d][i] = sk_load16(wr, in ? w_off + 16 * i : kOob, wo); }
    if constexpr (QUANT) {
      const uint32_t so = in ? (k_of(s) >> p.gshift) * 2 : 0u;
      const uint32_t vo = in ? s_off : kOob;
      sreg[d] = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)vo, (int)so, 0);
      qreg[d] = __builtin_amdgcn_raw_buffer_load_b16(qr, (int)vo, (int)so, 0);
    }
  };

  // Activation stream: each thread loads XL 16 B chunks of the 128 x 64
  // tile into a register ring kSkDepth steps deep and writes them to LDS
  // one step before they are read. vmcnt retires a wave's loads in issue
  // order, so waiting for an activation step also waits for every weight
  // load issued before it: the activation loads therefore run as far ahead
  // as the weight loads, and each step issues them first.
  uint32_t x_off[XL];
  int x_lds[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int c = tid + NT * i;
    const int r = c >> 3;
    const int kc = c & 7;
    x_off[i] = (uint32_t)(((size_t)r * p.K + kc * 8) * 2);
    x_lds[i] = r * kSkLdsRow + kc * 8;
  }
  uint4 xreg[kSkDepth][XL];
  auto load_x = [&](int s, int slot) {
    const bool in = s < nsteps;
    const uint32_t kb = in ? k_of(s) * 2 : 0u;
#pragma unroll
    for (int i = 0; i < XL; ++i) { xreg[slot][i] = sk_load16(xr, in ? x_off[i] : kOob, kb); }
  };
  auto store_x = [&](int st, int slot) {
#pragma unroll
    for (int i = 0; i < XL; ++i) { *(uint4*)&lds_x[st][x_lds[i]] = xreg[slot][i]; }
  };

  // Fragment reads: tile i, slice j reads row 32i + l%32 at k = 32h + 8j.
  const uint16_t* a_base = &lds_x[0][0] + (lane & 31) * kSkLdsRow + 32 * half;
  auto read_a = [&](int st, int j, bf16x8* af) {
    const uint16_t* b = a_base + st * kSkRows * kSkLdsRow + 8 * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) { af[i] = *(const bf16x8*)(b + i * 32 * kSkLdsRow); }
  };

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[i][r] = 0.0f; }
  }

  // One step: slice 0's fragment reads, then the weight dequant (its VALU
  // work covers the LDS latency), then per slice 4 MFMAs with the next
  // slice's reads interleaved.
  auto compute = [&](int st, int d) {
    bf16x8 afr[2][4];
    bf16x8 bfr[4];
    read_a(st, 0, afr[0]);
    if constexpr (QUANT) {
      const float sc = bf16_to_f32(sreg[d]);
      const float qb = bf16_to_f32(qreg[d]);
      const uint32_t* words = (const uint32_t*)&wreg[d][0];
#pragma unroll
      for (int j = 0; j < 4; ++j) { bfr[j] = dequant8<BITS>(words + j * (BITS / 4), sc, qb); }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) { bfr[j] = __builtin_bit_cast(bf16x8, wreg[d][j]); }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, QUANT ? 20 * 4 : 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < 3) { read_a(st, j + 1, afr[(j + 1) & 1]); }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[j & 1][i], bfr[j], acc[i], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (j < 3) { __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); }
      }
    }
  };

  // Step s reads LDS stage s&1 and ring slot s%D; then it loads
  // activation step s+D and weight step s+D into that slot, writes
  // activation step s+1 (loaded three steps ago) to the other LDS stage,
  // and meets the other waves at the barrier, which publishes that stage
  // (the previous barrier guarantees every wave is done reading it). Up to
  // D-1 padded steps at the end compute zeros.
#pragma unroll
  for (int d = 0; d < kSkDepth; ++d) {
    load_x(d, d);
    load_w(d, d);
  }
  store_x(0, 0);
  __syncthreads();
  for (int s0 = 0; s0 < nsteps; s0 += kSkDepth) {
#pragma unroll
    for (int d = 0; d < kSkDepth; ++d) {
      const int s = s0 + d;
      compute(d & 1, d);
      load_x(s + kSkDepth, d);
      load_w(s + kSkDepth, d);
      store_x((d + 1) & 1, (d + 1) % kSkDepth);
      __syncthreads();
    }
  }

  // Accumulator layout of the 32x32 MFMA: lane l, register r holds row
  // 32i + 8(r/4) + 4(l/32) + r%4 of tile i, column l%32. Stores go through
  // buffer resources sized to the output: rows past M fall past the end,
  // and columns past N get an out-of-range per-lane offset, so masked
  // elements are dropped by the range check instead of branched around.
  const bool in_n = col < p.N;
  auto row_of = [&](int i, int r) { return 32 * i + 8 * (r >> 2) + 4 * half + (r & 3); };
  auto finish = [&](const f32x16* v) {
    const __amdgpu_buffer_rsrc_t yr = sk_rsrc(p.y, (size_t)p.M * p.N * 2);
    const float bv = in_n ? sk_bias(p.bias, p.bias_type, col) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float o = v[i][r] + bv;
        if (p.epilogue == kEpiGelu) { o = gelu_tanh(o); }
        const uint32_t vo = in_n ? (uint32_t)(((size_t)row_of(i, r) * p.N + col) * 2) : kOob;
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(o), yr, (int)vo, 0, 0);
      }
    }
  };
  if (p.splits == 1) {
    finish(acc);
    return;
  }

  const size_t plane = (size_t)p.M * p.N;
  {
    const __amdgpu_buffer_rsrc_t wr_p = sk_rsrc(p.partial + split * plane, plane * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t vo = in_n ? (uint32_t)(((size_t)row_of(i, r) * p.N + col) * 4) : kOob;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][r]), wr_p,
                                              (int)vo, 0, 0);
      }
    }
  }
  // Publish the partial, then count this split in.
  __threadfence();
  __syncthreads();
  if (tid == 0) { s_last = atomicAdd(&p.counters[tn], 1) == p.splits - 1; }
  __syncthreads();
  if (!s_last) { return; }
  __threadfence();
  // Sum the partials in split order (this workgroup's own included, read
  // back like the others, so the order never depends on who arrived
  // last). Each split's plane is its own buffer resource: rows past M fall
  // past its end and columns past N get an out-of-range per-lane offset,
  // so the 64 loads per lane and split carry no branch, are issued
  // together, and the reduction costs `splits` round trips.
  f32x16 sum[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { sum[i][r] = 0.0f; }
  }
  for (int t = 0; t < p.splits; ++t) {
    const __amdgpu_buffer_rsrc_t pr = sk_rsrc(p.partial + t * plane, plane * 4);
    f32x16 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t vo = in_n ? (uint32_t)(((size_t)row_of(i, r) * p.N + col) * 4) : kOob;
        v[i][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, (int)vo, 0, 0));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) { sum[i] += v[i]; }
  }
  finish(sum);
  if (tid == 0) { p.counters[tn] = 0; }
}

template <int NW>
hipError_t launch_nw(const SkParams& kp, int bits, int tiles_n, hipStream_t stream)
{
  const dim3 grid((unsigned)tiles_n, (unsigned)kp.splits, 1);
  const dim3 block(NW * 64);
  switch (bits) {
    case 8: hipLaunchKernelGGL((skinny_kernel<NW, 8>), grid, block, 0, stream, kp); break;
    case 4: hipLaunchKernelGGL((skinny_kernel<NW, 4>), grid, block, 0, stream, kp); break;
    default: hipLaunchKernelGGL((skinny_kernel<NW, 16>), grid, block, 0, stream, kp); break;
  }
  return hipGetLastError();
}

int sk_ilog2(int v)
{
  int s = 0;
  while ((1 << s) < v) { ++s; }
  return s;
}

}  // namespace

SkinnyPlan plan_skinny(int M, int N, int K, int cu_count)
{
  (void)M;
  SkinnyPlan plan;
  // Column tiles of 32*waves; prefer 4 waves (the activation tile is then
  // shared by 128 columns) and split K until about one workgroup per CU,
  // keeping at least 4 steps of 64 per split.
  plan.waves = 4;
  const int tiles = (N + 32 * plan.waves - 1) / (32 * plan.waves);
  const int max_split = std::max(1, K / 256);
  int s = std::max(1, std::min(max_split, (cu_count + tiles - 1) / tiles));
  int chunk = ((K + s - 1) / s + kSkBK - 1) / kSkBK * kSkBK;
  s = (K + chunk - 1) / chunk;
  plan.splits = s;
  plan.k_chunk = chunk;
  plan.tiles_n = tiles;
  plan.workspace_bytes = s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
  plan.counter_count = s > 1 ? tiles : 0;
  return plan;
}

hipError_t launch_skinny(const GemmDesc& d, const SkinnyPlan& plan, float* partial,
                         int* counters, hipStream_t stream)
{
  SkParams kp;
  kp.x = d.x;
  kp.w = d.w;
  kp.scales = d.scales;
  kp.qbias = d.qbias;
  kp.bias = d.bias;
  kp.y = d.y;
  kp.partial = partial;
  kp.counters = counters;
  kp.M = d.M;
  kp.N = d.N;
  kp.K = d.K;
  kp.gshift = d.bits == 16 ? 0 : sk_ilog2(d.group);
  kp.gcols = d.bits == 16 ? 0 : d.K / d.group;
  kp.k_chunk = plan.k_chunk;
  kp.splits = plan.splits;
  kp.bias_type = d.bias != nullptr ? d.bias_type : kBiasNone;
  kp.epilogue = d.epilogue;
  switch (plan.waves) {
    case 1: return launch_nw<1>(kp, d.bits, plan.tiles_n, stream);
    case 2: return launch_nw<2>(kp, d.bits, plan.tiles_n, stream);
    default: return launch_nw<4>(kp, d.bits, plan.tiles_n, stream);
  }
}

}  // namespace ltx25
