// The skinny quantized linear on gfx950, for M <= 128 rows (the audio
// stream's ~126 tokens): y = x . dequant(W)^T (+ bias) (+ GELU).
//
// These GEMMs sit near the bf16 ridge (about 256 FLOP per weight byte
// against a ridge of about 300) and each moves only 5-20 MB, so what
// decides their speed is how much of the weight stream is in flight
// against a loaded memory latency of 2-3 us. The layout:
//
//   - A workgroup owns 128 output columns (4 waves x 32) and one K range
//     (k_chunk, 256 or 512) of all rows. Its activation slab, 128 rows x
//     k_chunk bf16, is loaded ONCE into LDS by direct global-to-LDS loads,
//     behind a single barrier; the main loop then has no barrier at all.
//   - Each wave streams only its own 32 weight columns, straight into
//     registers in the MFMA operand layout, kSkDepth = 8 K steps (of 64)
//     ahead. Lane l holds column l%32 and, per step, the 32 codes
//     [32h, 32h+32) (h = l/32); MFMA slice j uses codes [32h+8j, +8), and
//     the activation fragments use the same permutation of K, which the
//     dot product allows. Every weight element is dequantized exactly once,
//     in registers, w = bf16(fma(scale, q, zero point)), right in front of
//     v_mfma_f32_32x32x16_bf16 (four 32-row tiles per wave).
//   - K is split over `splits` workgroups. Each wave writes its f32
//     partial 128 x 32 block and counts in on that block's own counter; the
//     wave that arrives last sums the partials in split order, adds the
//     bias, applies GELU and rounds once to bf16. The result is
//     deterministic, the linear is one launch, and the reductions are
//     spread over as many CUs as there are 32-column blocks. The last wave
//     resets its counter, so the counters are zero again after the launch.
//
// Reference semantics: MetalOps::linear(QWeight) (src/ltx25-metal-ops.cc:
// 531-569) over the affine_dequant weight, then ltx_bias_add.
#include "common.h"

#include <algorithm>

namespace ltx25 {
namespace {

typedef uint32_t __attribute__((address_space(3))) lds_u32;

constexpr int kSkRows = 128;              // rows per workgroup
constexpr int kSkBK = 64;                 // K per step
constexpr int kSkDepth = 8;               // weight steps in flight per wave
constexpr int kSkWaves = 4;               // waves (32 columns each) per workgroup
constexpr int kSysCoherent = 17;          // buffer cache policy sc0 | sc1
constexpr uint32_t kOob = 0x80000000u;    // a per-lane offset past every buffer

struct SkParams {
  const uint16_t* x;
  const void* w;
  const uint16_t* scales;
  const uint16_t* qbias;
  const void* bias;
  uint16_t* y;
  float* partial;        // [splits][M][N] f32
  int* counters;         // [tiles_n * kSkWaves], zero between launches
  int M, N, K;
  int gshift, gcols;
  int k_chunk, splits;   // k_chunk is 256 or 512
  int bias_type, epilogue;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, size_t bytes)
{
  // Raw buffer: the range check on the per-lane offset returns zeros (and
  // drops stores) past `bytes` without a memory access.
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

template <int BITS>
__global__ void __launch_bounds__(kSkWaves * 64)
skinny_kernel(SkParams p)
{
  constexpr bool QUANT = BITS != 16;
  constexpr int WB = QUANT ? 32 * BITS / 8 : 64;   // weight bytes per lane per step
  constexpr int WL = WB / 16;                       // 16 B loads per lane per step

  // The activation slab: 128 rows of k_chunk bf16 (512 B or 1 KB), rows
  // unpadded so that direct loads (64 lanes x 16 B = 1 KB contiguous) fill
  // it. The 16 B chunk c of row r sits at position c ^ (r & 15), so a
  // fragment read (16 rows, one chunk) hits 16 distinct bank groups.
  extern __shared__ __attribute__((aligned(1024))) uint16_t lds_x[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int tn = blockIdx.x;
  const int split = blockIdx.y;
  const int col = tn * 32 * kSkWaves + wave * 32 + (lane & 31);
  const bool in_n = col < p.N;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nsteps = (kend - kbeg) / kSkBK;
  const int rowb = p.k_chunk * 2;

  const size_t row_bytes = (size_t)p.K * (QUANT ? BITS : 16) / 8;
  const __amdgpu_buffer_rsrc_t xr = sk_rsrc(p.x, (size_t)p.M * p.K * 2);
  const __amdgpu_buffer_rsrc_t wr = sk_rsrc(p.w, (size_t)p.N * row_bytes);
  const __amdgpu_buffer_rsrc_t sr = sk_rsrc(p.scales, QUANT ? (size_t)p.N * p.gcols * 2 : 0);
  const __amdgpu_buffer_rsrc_t qr = sk_rsrc(p.qbias, QUANT ? (size_t)p.N * p.gcols * 2 : 0);

  // Weight ring: slot d holds step s (s % kSkDepth == d) from its load
  // until it is computed. Steps past nsteps, and columns past N, load with
  // an out-of-range per-lane offset: zeros, no memory access, and the zero
  // codes with zero scale and zero point add nothing. The uniform K offset
  // rides in soffset only when in range (the range check covers the
  // per-lane offset). Every step issues the same loads with no branch.
  const uint32_t w_off = (uint32_t)((size_t)col * row_bytes + (size_t)half * WB);
  const uint32_t s_off =
      QUANT ? (uint32_t)(((size_t)col * p.gcols + ((32 * half) >> p.gshift)) * 2) : 0u;
  uint4 wreg[kSkDepth][WL];
  uint16_t sreg[kSkDepth];
  uint16_t qreg[kSkDepth];
  // soffset must be wave-uniform (a per-lane value would make the compiler
  // loop over its distinct values), so it depends only on the step.
  auto load_w = [&](int s, int d) {
    const bool step_in = s < nsteps;
    const bool in = step_in && in_n;
    const uint32_t k = (uint32_t)(kbeg + s * kSkBK);
    const uint32_t wo = step_in ? (uint32_t)((size_t)k * (QUANT ? BITS : 16) / 8) : 0u;
#pragma unroll
    for (int i = 0; i < WL; ++i) { wreg[d][i] = sk_load16(wr, in ? w_off + 16 * i : kOob, wo); }
    if constexpr (QUANT) {
      const uint32_t so = step_in ? (k >> p.gshift) * 2 : 0u;
      const uint32_t vo = in ? s_off : kOob;
      sreg[d] = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)vo, (int)so, 0);
      qreg[d] = __builtin_amdgcn_raw_buffer_load_b16(qr, (int)vo, (int)so, 0);
    }
  };

#pragma unroll
  for (int d = 0; d < kSkDepth; ++d) { load_w(d, d); }

  // The slab: 1 KB direct load g covers LDS bytes [1024 g, 1024 g + 1024);
  // lane i lands at byte 16 i of it, i.e. row r, position pos, and fetches
  // the row's chunk pos ^ (r & 15). Chunks past this split's K range (the
  // last split) or rows past M read as zero.
  {
    const int n_loads = kSkRows * rowb / 1024;
    const int per_wave = n_loads / kSkWaves;
    for (int q = 0; q < per_wave; ++q) {
      const int g = wave * per_wave + q;
      const int byte = 1024 * g + 16 * lane;
      const int r = byte / rowb;
      const int c = ((byte % rowb) / 16) ^ (r & 15);
      const int k = kbeg + 8 * c;
      const uint32_t vo = k < kend ? (uint32_t)(((size_t)r * p.K + k) * 2) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_u32*)(lds_x + 512 * g), 16, (int)vo,
                                               0, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Fragment offsets: tile i, slice j of step s reads row 32i + l%32, chunk
  // 8s + 4h + j, stored at position (8s + 4h + j) ^ (row & 15); since the
  // XOR only touches the low 4 bits, step s adds 256 B per pair of steps
  // and its parity picks one of two offset sets.
  const int rsw = lane & 15;
  const int arow_b = (lane & 31) * rowb;
  int a_off[2][4];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
#pragma unroll
    for (int j = 0; j < 4; ++j) { a_off[par][j] = arow_b + 16 * ((8 * par + 4 * half + j) ^ rsw); }
  }
  const char* slab = (const char*)lds_x;

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[i][r] = 0.0f; }
  }

  // One step: dequantize the slot's 32 codes into four B fragments, then
  // 4 slices x 4 row tiles of MFMAs with the A fragments read one slice
  // ahead.
  auto compute = [&](int s, int d) {
    bf16x8 bfr[4];
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
    const char* base = slab + 256 * (s >> 1);
    const int par = d & 1;
    bf16x8 afr[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      afr[0][i] = *(const bf16x8*)(base + a_off[par][0] + i * 32 * rowb);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          afr[(j + 1) & 1][i] = *(const bf16x8*)(base + a_off[par][j + 1] + i * 32 * rowb);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[j & 1][i], bfr[j], acc[i], 0, 0, 0);
      }
    }
  };

  // Up to kSkDepth - 1 padded steps at the end compute zeros.
  for (int s0 = 0; s0 < nsteps; s0 += kSkDepth) {
#pragma unroll
    for (int d = 0; d < kSkDepth; ++d) {
      const int s = s0 + d;
      compute(s, d);
      load_w(s + kSkDepth, d);
    }
  }

  // Accumulator layout of the 32x32 MFMA: lane l, register r holds row
  // 32i + 8(r/4) + 4(l/32) + r%4 of tile i, column l%32. Stores go through
  // buffer resources sized to the output: rows past M fall past the end,
  // and columns past N get an out-of-range per-lane offset, so masked
  // elements are dropped by the range check instead of branched around.
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

  // Publish this wave's partial block, then count in on the block's
  // counter. The partial stores write through to memory (system-coherent
  // cache policy) and are waited for before the atomic; the last wave reads
  // the partials back with the same policy, bypassing the caches that are
  // not coherent across XCDs. (An agent-scope fence pair would instead
  // write back and invalidate the whole L2 in every wave.)
  const size_t plane = (size_t)p.M * p.N;
  {
    const __amdgpu_buffer_rsrc_t pw = sk_rsrc(p.partial + split * plane, plane * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t vo = in_n ? (uint32_t)(((size_t)row_of(i, r) * p.N + col) * 4) : kOob;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][r]), pw, (int)vo, 0,
                                              kSysCoherent);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  int* counter = p.counters + tn * kSkWaves + wave;
  int before = 0;
  if (lane == 0) {
    before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  before = __builtin_amdgcn_readfirstlane(before);
  if (before != p.splits - 1) { return; }

  // Last wave of the block: sum the partials in split order (its own read
  // back like the others, so the order never depends on who arrived last).
  // Each split's 64 values per lane are loaded together, so the reduction
  // costs `splits` round trips.
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
        v[i][r] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(pr, (int)vo, 0, kSysCoherent));
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) { sum[i] += v[i]; }
  }
  finish(sum);
  if (lane == 0) { *counter = 0; }
}

// The slab is dynamic LDS of up to 128 KB; a kernel may use more than
// 64 KB of it only once the limit is raised for that kernel.
template <int BITS>
hipError_t launch_one(const SkParams& kp, dim3 grid, size_t lds, hipStream_t stream)
{
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&skinny_kernel<BITS>),
      hipFuncAttributeMaxDynamicSharedMemorySize, kSkRows * 512 * 2);
  if (attr != hipSuccess) { return attr; }
  hipLaunchKernelGGL((skinny_kernel<BITS>), grid, dim3(kSkWaves * 64), lds, stream, kp);
  return hipGetLastError();
}

hipError_t launch_bits(const SkParams& kp, int bits, int tiles_n, hipStream_t stream)
{
  const dim3 grid((unsigned)tiles_n, (unsigned)kp.splits, 1);
  const size_t lds = (size_t)kSkRows * kp.k_chunk * 2;
  switch (bits) {
    case 8: return launch_one<8>(kp, grid, lds, stream);
    case 4: return launch_one<4>(kp, grid, lds, stream);
    default: return launch_one<16>(kp, grid, lds, stream);
  }
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
  SkinnyPlan plan;
  plan.waves = kSkWaves;
  const int tiles = (N + 32 * kSkWaves - 1) / (32 * kSkWaves);
  // K splits of 512, or of 256 while that still leaves at most two
  // workgroups per CU (the slab is then 64 KB and two share a CU).
  const int chunk = (long)tiles * ((K + 255) / 256) <= 2L * cu_count ? 256 : 512;
  const int s = (K + chunk - 1) / chunk;
  plan.splits = s;
  plan.k_chunk = chunk;
  plan.tiles_n = tiles;
  plan.workspace_bytes = s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
  plan.counter_count = s > 1 ? tiles * kSkWaves : 0;
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
  return launch_bits(kp, d.bits, plan.tiles_n, stream);
}

}  // namespace ltx25
