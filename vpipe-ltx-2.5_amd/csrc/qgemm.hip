// The quantized linear on gfx950: y = x . dequant(W)^T (+ bias) (+ GELU).
//
// One kernel template serves every weight format (w8 / w4 group-affine
// codes, or dense bf16) and both tile shapes:
//
//   tall   BM x BN = 256 x 256, 8 waves in 2 x 4, 128 x 64 per wave
//          (the video GEMMs, thousands of tokens); two waves per SIMD,
//          so one wave's LDS / barrier / load waits are covered by the
//          other's MFMAs
//   mid    BM x BN = 128 x 128, 4 waves in 2 x 2, 64 x 64 per wave,
//          with split-K across workgroups (more than 128 tokens but fewer
//          256 x 256 tiles than CUs, and the calls of at most 128 tokens
//          whose weight is too large for the M <= 128 kernel of skinny.hip,
//          which takes the audio GEMMs)
//
// Per K step of 64 (one w8g64 group):
//   - X rows stream from HBM as 16-byte loads into registers, then to LDS;
//   - weight codes stream as 16-byte loads (16 u8 codes or 32 u4 codes),
//     are dequantized ONCE per workgroup in registers,
//     w = bf16(fma(scale, q, qbias)), and land in LDS as bf16;
//   - each wave reads 32x16 bf16 fragments from LDS and issues
//     v_mfma_f32_32x32x16_bf16 with f32 accumulation.
// The next step's global loads are issued before the current step's MFMAs
// and land in the other LDS stage afterwards (two stages, one barrier per
// step). The bias add (f32 or bf16) and GELU-tanh are fused into the
// epilogue, ahead of the single rounding to bf16; with split-K the
// epilogue runs in a reduction kernel that sums the f32 partials in a
// fixed order, so results are deterministic.
//
// Reference semantics: MetalOps::linear(QWeight) (src/ltx25-metal-ops.cc:
// 531-569) computes the same product through affine_dequant + dense_gemm_mma
// (or affine_qmm_steel), then a separate ltx_bias_add pass.
#include "common.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace ltx25 {
namespace {

// Wave grid of the 256 x 256 tile.
constexpr int kTallWM = 2;
constexpr int kTallWN = 4;
// Width of the small tile (128 rows; four waves, 2 x 2 at 128 columns or
// 4 x 1 at 64).
constexpr int kMidBN = 128;
constexpr int kBK = 64;             // K per main-loop step (bf16 activations)
// BITS value of the int8 x int8 -> int32 GEMM (the int8 tier): both
// operands are int8 rows, 128 of K per step in the same 128-byte LDS rows.
constexpr int kI8Ops = 1;
constexpr int kLdsRow = kBK + 8;    // bf16 per LDS row: 144 B pitch keeps
                                    // the 16 B fragment reads conflict-free

struct KParams {
  const uint16_t* x;
  const uint16_t* x2;      // FOLD: columns [kx, K) of the activation, [M][K - kx]
  int wn;                  // weight rows in memory (<= N); rows past them read as zeros
  int kx;                  // FOLD: columns of x (a multiple of kBK); else K
  const int8_t* xq;        // int8 activations (kI8Ops)
  const float* sx;         // per-row activation scales (kI8Ops)
  const float* sw;         // per-column weight scales (kI8Ops)
  int32_t* acc_out;        // optional raw int32 accumulators (kI8Ops)
  const uint8_t* wq;       // codes as bytes (bits 8 or 4), or int8 weights
  const uint16_t* wd;      // dense bf16 weight (bits 16)
  const uint16_t* scales;
  const uint16_t* qbias;
  const void* bias;
  uint16_t* y;
  const uint16_t* y_in;    // accumulate source (may alias y), or null
  float* partial;          // [splits][M][N] when split
  int M, N, K;
  int gshift;              // log2(group)
  int gcols;               // K / group
  int k_chunk;
  int bias_type;
  int epilogue;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p,
                                                           size_t bytes)
{
  // Raw buffer resource: loads at offsets past `bytes` return zeros, which
  // is how rows past M and N are handled without branches.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)(uint32_t)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r,
                                            uint32_t voff, uint32_t soff)
{
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r,
                                              uint32_t voff, uint32_t soff)
{
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}

// Instruction-issue pattern for one scheduling region of NM MFMAs: after
// each MFMA, one LDS read while any of the NR remain, then this gap's share
// of the NG global loads and NV VALU ops, and an LDS write every other gap
// over the last 2*NW gaps (the writes depend on the VALU work before them).
// Masks: 0x008 MFMA, 0x100 LDS read, 0x200 LDS write, 0x020 VMEM read,
// 0x002 VALU.
template <int I, int NM, int NR, int NW, int NV, int NG>
__device__ __forceinline__ void interleave_gap()
{
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  constexpr int r = I < NR ? 1 : 0;
  constexpr int g = (I + 1) * NG / NM - I * NG / NM;
  constexpr int v = (I + 1) * NV / NM - I * NV / NM;
  constexpr int w0 = NM - 2 * NW > 0 ? NM - 2 * NW : 0;
  constexpr int w = (I >= w0 && ((I - w0) & 1) == 0 && (I - w0) / 2 < NW) ? 1 : 0;
  if constexpr (r > 0) { __builtin_amdgcn_sched_group_barrier(0x100, r, 0); }
  if constexpr (g > 0) { __builtin_amdgcn_sched_group_barrier(0x020, g, 0); }
  if constexpr (v > 0) { __builtin_amdgcn_sched_group_barrier(0x002, v, 0); }
  if constexpr (w > 0) { __builtin_amdgcn_sched_group_barrier(0x200, w, 0); }
}

template <int NM, int NR, int NW, int NV, int NG, int... I>
__device__ __forceinline__ void interleave_seq(std::integer_sequence<int, I...>)
{
  (interleave_gap<I, NM, NR, NW, NV, NG>(), ...);
}

template <int NM, int NR, int NW, int NV, int NG>
__device__ __forceinline__ void interleave()
{
  interleave_seq<NM, NR, NW, NV, NG>(std::make_integer_sequence<int, NM>{});
}

template <int BM, int BN, int WM, int WN, int BITS, bool SPLIT, int NS = 0, bool FOLD = false>
__global__ void __launch_bounds__(WM * WN * 64)
qgemm_kernel(KParams p)
{
  constexpr int NT = WM * WN * 64;                   // threads
  constexpr int WTM = BM / WM;
  constexpr int WTN = BN / WN;
  constexpr int FM = WTM / 32;
  constexpr int FN = WTN / 32;
  constexpr int A_LD = BM * 8 / NT;                  // 16 B chunks / thread
  constexpr int A_RSTEP = NT / 8;
  constexpr bool I8 = BITS == kI8Ops;
  constexpr bool QUANT = BITS == 8 || BITS == 4;     // group-affine codes
  constexpr int SK = I8 ? 2 * kBK : kBK;             // K elements per step
  constexpr int XB = I8 ? 1 : 2;                     // bytes per activation
  constexpr int B_CPR = QUANT ? kBK * BITS / 8 / 16 : 8;  // chunks/row
  constexpr int B_LD = BN * B_CPR / NT;
  constexpr int B_RSTEP = NT / B_CPR;
  constexpr int CPC = QUANT ? 128 / BITS : 8;        // codes per chunk (16 B in LDS units)
  static_assert(A_LD >= 1 && B_LD >= 1, "tile too small for the thread count");

  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][BN * kLdsRow];
  // The epilogue's per-column bias (as f32) and, for the int8 GEMM, per-column
  // and per-row scales, staged during the prologue so that the epilogue does
  // not wait on global loads.
  __shared__ float lds_ep[2 * BN + BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;

  int tm, tn;
  map_tile(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int split = SPLIT ? (int)blockIdx.y : 0;
  const int kbeg = split * p.k_chunk;
  const int kend = min(p.K, kbeg + p.k_chunk);
  const int nsteps = kend > kbeg ? (kend - kbeg) / SK : 0;

  const int a_c = tid & 7;
  const int a_r = tid >> 3;
  const int b_c = tid % B_CPR;
  const int b_r = tid / B_CPR;

  // Buffer resources and per-thread byte offsets, fixed for the whole loop;
  // each step adds a uniform K offset (an SGPR).
  const size_t wrow_bytes = (size_t)p.K * (QUANT ? BITS : (I8 ? 8 : 16)) / 8;
  // FOLD: the activation is [x | x2], x with kx columns, x2 with K - kx
  const int kx = FOLD ? p.kx : p.K;
  const __amdgpu_buffer_rsrc_t xr =
      make_rsrc(I8 ? (const void*)p.xq : (const void*)p.x, (size_t)p.M * kx * XB);
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(QUANT || I8 ? (const void*)p.wq : (const void*)p.wd, (size_t)p.wn * wrow_bytes);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(p.scales, (size_t)p.N * p.gcols * 2);
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(p.qbias, (size_t)p.N * p.gcols * 2);
  uint32_t a_off[A_LD];
  uint32_t b_off[B_LD];
  uint32_t s_off[B_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    a_off[i] = (uint32_t)((size_t)(m0 + a_r + A_RSTEP * i) * kx * XB + a_c * 16);
  }
  const int kx2 = FOLD ? p.K - kx : 0;
  const __amdgpu_buffer_rsrc_t xr2 = make_rsrc(p.x2, FOLD ? (size_t)p.M * kx2 * XB : 0);
  uint32_t a_off2[FOLD ? A_LD : 1];
  if constexpr (FOLD) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      a_off2[i] = (uint32_t)((size_t)(m0 + a_r + A_RSTEP * i) * kx2 * XB + a_c * 16);
    }
  }
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const size_t n = (size_t)(n0 + b_r + B_RSTEP * i);
    b_off[i] = (uint32_t)(n * wrow_bytes + b_c * 16);
    s_off[i] = QUANT ? (uint32_t)((n * p.gcols + ((b_c * CPC) >> p.gshift)) * 2) : 0u;
  }

  uint4 areg[A_LD];
  uint4 breg[B_LD];
  uint16_t sraw[B_LD];
  uint16_t qraw[B_LD];

  auto load_a = [&](int k) {
    if constexpr (FOLD) {
      // The step's K range lies in one part. Selects, not a branch: a
      // branch would split the step's scheduling regions (the issue
      // pattern of interleave<> holds within one basic block).
      const bool second = k >= kx;
      const __amdgpu_buffer_rsrc_t r = second ? xr2 : xr;
      const uint32_t so = (uint32_t)(second ? k - kx : k) * XB;
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        areg[i] = buf_load16(r, second ? a_off2[i] : a_off[i], so);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) { areg[i] = buf_load16(xr, a_off[i], (uint32_t)k * XB); }
    }
  };
  auto load_b = [&](int k) {
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      breg[i] = buf_load16(wr, b_off[i], (uint32_t)k * (QUANT ? BITS : (I8 ? 8 : 16)) / 8);
      if constexpr (QUANT) {
        const uint32_t so = (uint32_t)(k >> p.gshift) * 2;
        sraw[i] = buf_load2(sr, s_off[i], so);
        qraw[i] = buf_load2(qr, s_off[i], so);
      }
    }
  };
  auto load_regs = [&](int k) {
    load_a(k);
    load_b(k);
  };

  auto store_a = [&](int st) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      *(uint4*)&lds_a[st][(a_r + A_RSTEP * i) * kLdsRow + a_c * 8] = areg[i];
    }
  };

  // Weight rows [lo, hi) of this thread's B_LD chunks: dequantize (for
  // codes) and write to LDS stage `st`.
  auto store_b_rows = [&](int st, int lo, int hi) {
#pragma unroll
    for (int i = lo; i < hi; ++i) {
      uint16_t* dst = &lds_b[st][(b_r + B_RSTEP * i) * kLdsRow + b_c * CPC];
      if constexpr (!QUANT) {
        *(uint4*)dst = breg[i];
      } else if constexpr (BITS == 8) {
        const uint32_t wv[4] = {breg[i].x, breg[i].y, breg[i].z, breg[i].w};
        const float s = bf16_to_f32(sraw[i]), b = bf16_to_f32(qraw[i]);
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t v = wv[j];
          o[2 * j] = pack_bf16x2(fmaf(s, (float)(v & 0xffu), b),
                                 fmaf(s, (float)((v >> 8) & 0xffu), b));
          o[2 * j + 1] = pack_bf16x2(fmaf(s, (float)((v >> 16) & 0xffu), b),
                                     fmaf(s, (float)(v >> 24), b));
        }
        *(uint4*)dst = make_uint4(o[0], o[1], o[2], o[3]);
        *(uint4*)(dst + 8) = make_uint4(o[4], o[5], o[6], o[7]);
      } else {
        // w4: code 8j+s sits at bits 4s of word j. Even codes are the low
        // nibbles of each byte, odd codes the high nibbles.
        const uint32_t wv[4] = {breg[i].x, breg[i].y, breg[i].z, breg[i].w};
        const float s = bf16_to_f32(sraw[i]), b = bf16_to_f32(qraw[i]);
        uint32_t o[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = wv[j] & 0x0f0f0f0fu;
          const uint32_t hi = (wv[j] >> 4) & 0x0f0f0f0fu;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            o[4 * j + t] =
                pack_bf16x2(fmaf(s, (float)((lo >> (8 * t)) & 0xffu), b),
                            fmaf(s, (float)((hi >> (8 * t)) & 0xffu), b));
          }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          *(uint4*)(dst + 8 * t) =
              make_uint4(o[4 * t], o[4 * t + 1], o[4 * t + 2], o[4 * t + 3]);
        }
      }
    }
  };

  auto store_b = [&](int st) { store_b_rows(st, 0, B_LD); };

  using AccT = std::conditional_t<I8, i32x16, f32x16>;
  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { acc[i][j][r] = 0; }
    }
  }
  // Accumulate into an existing output (the LoRA delta's second GEMM): the
  // accumulators start from y_in, in the MFMA layout (block (i, j), lane l,
  // registers 4g..4g+3: row 32 i + l % 32, four consecutive columns from
  // 32 j + 8 g + 4 (l / 32)), so the K loop adds the products to it and the
  // epilogue rounds once. These loads overlap the operand prologue's.
  if constexpr (!I8 && !SPLIT) {
    if (p.y_in != nullptr) {
      const int lrow0 = lane & 31;
      const int lcol0 = (lane >> 5) * 4;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * (BM / WM) + i * 32 + lrow0;
        if (m >= p.M) { continue; }
        const uint16_t* yrow = p.y_in + (size_t)m * p.N;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * (BN / WN) + j * 32 + g * 8 + lcol0;
            if ((p.N & 3) == 0 && n + 3 < p.N) {
              const uint2 o = *(const uint2*)(yrow + n);
              acc[i][j][4 * g + 0] = __uint_as_float(o.x << 16);
              acc[i][j][4 * g + 1] = __uint_as_float(o.x & 0xffff0000u);
              acc[i][j][4 * g + 2] = __uint_as_float(o.y << 16);
              acc[i][j][4 * g + 3] = __uint_as_float(o.y & 0xffff0000u);
            } else {
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                acc[i][j][4 * g + t] = n + t < p.N ? bf16_to_f32(yrow[n + t]) : 0.0f;
              }
            }
          }
        }
      }
    }
  }

  // Fragment registers, double-buffered across the four 16-deep K slices
  // of a step: slice kk+1 is read from LDS while slice kk's MFMAs run.
  bf16x8 afr[2][FM];
  bf16x8 bfr[2][FN];
  const int a_frag = (wm * WTM + (lane & 31)) * kLdsRow + (lane >> 5) * 8;
  const int b_frag = (wn * WTN + (lane & 31)) * kLdsRow + (lane >> 5) * 8;

  auto read_frags = [&](int st, int kk, int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      afr[buf][i] = *(const bf16x8*)(lds_a[st] + a_frag + i * 32 * kLdsRow + kk * 16);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      bfr[buf][j] = *(const bf16x8*)(lds_b[st] + b_frag + j * 32 * kLdsRow + kk * 16);
    }
  };
  auto mfma_all = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (I8) {
          // 32 int8 of K per lane pair: the same 16 bytes a bf16 fragment holds
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
              __builtin_bit_cast(i32x4, bfr[buf][j]), __builtin_bit_cast(i32x4, afr[buf][i]),
              acc[i][j], 0, 0, 0);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[buf][j], afr[buf][i],
                                                             acc[i][j], 0, 0, 0);
        }
      }
    }
  };

  // One K step from LDS stage s&1, in four 16-deep slices. Interleaved with
  // the slices' MFMAs it writes step s+1 (already in registers) to the other
  // stage -- X tiles as they are in slice 0, weight tiles dequantized in
  // slices 1 and 2 -- and fetches step s+2 into the registers just freed
  // (X in slice 1, weights in slice 2), so each global load has about a
  // step to land. Every slice also reads the next slice's fragments, so the
  // fragment registers are double-buffered. The step's one barrier sits
  // before the last slice, whose fragments are already in registers; the
  // next step's first fragments are read under that slice's MFMAs.
  //
  // Each slice is its own scheduling region (sched_barrier) with an explicit
  // issue pattern (interleave<>): one MFMA per gap, the fragment reads in the
  // first gaps, the VALU dequant and global loads spread over all gaps, the
  // LDS writes in the second half. Left to itself the scheduler clusters
  // the reads after the MFMAs that free their registers, and the wave then
  // waits on LDS latency with the matrix pipe idle.
  constexpr int kMf = FM * FN;
  constexpr int kRd = FM + FN;
  constexpr int kB1 = B_LD / 2;
  constexpr int kValuChunk = !QUANT ? 0 : (BITS == 8 ? 42 : 86);
  constexpr int kWrChunk = !QUANT ? 1 : (BITS == 8 ? 2 : 4);
  auto step = [&](int s, auto do_store, auto do_load, int ld) {
    constexpr bool kStore = decltype(do_store)::value;
    constexpr bool kLoad = decltype(do_load)::value;
    constexpr int kGlB = QUANT ? 3 * B_LD : B_LD;
    const int st = s & 1;
    const int nst = st ^ 1;
    read_frags(st, 1, 1);
    mfma_all(0);
    if constexpr (kStore) { store_a(nst); }
    interleave<kMf, kRd, kStore ? A_LD : 0, 0, 0>();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(st, 2, 0);
    mfma_all(1);
    if constexpr (kStore) { store_b_rows(nst, 0, kB1); }
    if constexpr (kLoad) { load_a(kbeg + ld * SK); }
    interleave<kMf, kRd, kStore ? kB1 * kWrChunk : 0, kStore ? kB1 * kValuChunk : 0,
               kLoad ? A_LD : 0>();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(st, 3, 1);
    mfma_all(0);
    if constexpr (kStore) { store_b_rows(nst, kB1, B_LD); }
    if constexpr (kLoad) { load_b(kbeg + ld * SK); }
    interleave<kMf, kRd, kStore ? (B_LD - kB1) * kWrChunk : 0,
               kStore ? (B_LD - kB1) * kValuChunk : 0, kLoad ? kGlB : 0>();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if constexpr (kStore) { read_frags(nst, 0, 0); }
    mfma_all(1);
    interleave<kMf, kStore ? kRd : 0, 0, 0, 0>();
    __builtin_amdgcn_sched_barrier(0);
  };

  if constexpr (NS > 0) {
    // A split-K slice of exactly NS steps, fully unrolled, with the loads
    // kRing steps ahead of their LDS store (a register ring of kRing slots)
    // instead of one: under load a dependent memory round trip costs about
    // as much as five steps of this tile's MFMAs, so a one-step lookahead
    // stalls every other step. Step t lives in slot t % kRing.
    constexpr int kRing = 4;
    uint4 ar[kRing][A_LD];
    uint4 br[kRing][B_LD];
    uint16_t sr[kRing][B_LD];
    uint16_t qr[kRing][B_LD];
    auto to_slot = [&](int t) {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) { ar[t % kRing][i] = areg[i]; }
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        br[t % kRing][i] = breg[i];
        sr[t % kRing][i] = sraw[i];
        qr[t % kRing][i] = qraw[i];
      }
    };
    auto from_slot = [&](int t) {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) { areg[i] = ar[t % kRing][i]; }
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        breg[i] = br[t % kRing][i];
        sraw[i] = sr[t % kRing][i];
        qraw[i] = qr[t % kRing][i];
      }
    };
    load_regs(kbeg);
    store_a(0);
    store_b(0);
#pragma unroll
    for (int t = 1; t <= kRing && t < NS; ++t) {
      load_regs(kbeg + t * SK);
      to_slot(t);
    }
    __syncthreads();
    read_frags(0, 0, 0);
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      if (t + 1 < NS) { from_slot(t + 1); }
      if (t + 1 < NS && t + 1 + kRing < NS) {
        step(t, std::true_type{}, std::true_type{}, t + 1 + kRing);
        to_slot(t + 1 + kRing);
      } else if (t + 1 < NS) {
        step(t, std::true_type{}, std::false_type{}, 0);
      } else {
        step(t, std::false_type{}, std::false_type{}, 0);
      }
    }
  } else if (nsteps > 0) {
    // Two LDS stages; the last two steps are peeled so that the
    // steady-state body has no branches.
    load_regs(kbeg);
    // the epilogue's operands, fetched under the first operand loads
    float ep_v[(2 * BN + BM + NT - 1) / NT];
    if constexpr (!SPLIT) {
#pragma unroll
      for (int u = 0; u < (2 * BN + BM + NT - 1) / NT; ++u) {
        const int e = tid + u * NT;
        float v = 0.0f;
        if (e < BN) {
          const int n = n0 + e;
          v = n < p.N ? load_bias(p.bias, p.bias_type, n) : 0.0f;
        } else if (e < 2 * BN) {
          const int n = n0 + e - BN;
          v = I8 && n < p.N ? p.sw[n] : 0.0f;
        } else if (e < 2 * BN + BM) {
          const int m = m0 + e - 2 * BN;
          v = I8 && m < p.M ? p.sx[m] : 0.0f;
        }
        ep_v[u] = v;
      }
    }
    store_a(0);
    store_b(0);
    if constexpr (!SPLIT) {
#pragma unroll
      for (int u = 0; u < (2 * BN + BM + NT - 1) / NT; ++u) {
        const int e = tid + u * NT;
        if (e < 2 * BN + BM) { lds_ep[e] = ep_v[u]; }
      }
    }
    if (nsteps > 1) { load_regs(kbeg + SK); }
    __syncthreads();
    read_frags(0, 0, 0);
    int s = 0;
    for (; s + 2 < nsteps; ++s) { step(s, std::true_type{}, std::true_type{}, s + 2); }
    if (s + 1 < nsteps) {
      step(s, std::true_type{}, std::false_type{}, 0);
      ++s;
    }
    step(s, std::false_type{}, std::false_type{}, 0);
  }

  // Accumulator layout. The MFMAs take the weight fragment as their first
  // operand, so block (i, j) holds the transposed 32x32 product: lane l,
  // register r is row m = 32 i + l % 32 of the wave's sub-tile and column
  // n = 32 j + 8 (r / 4) + 4 (l / 32) + r % 4 -- registers 4g..4g+3 are four
  // consecutive columns of one row.
  const int lrow = lane & 31;
  const int lcol = (lane >> 5) * 4;
  if constexpr (SPLIT) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WTM + i * 32 + lrow;
      if (m >= p.M) { continue; }
      float* prow = p.partial + ((size_t)split * p.M + m) * p.N;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * WTN + j * 32 + g * 8 + lcol;
          const f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                           acc[i][j][4 * g + 3]};
          if ((p.N & 3) == 0 && n + 3 < p.N) {
            *(f32x4*)(prow + n) = v;
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              if (n + t < p.N) { prow[n + t] = v[t]; }
            }
          }
        }
      }
    }
  } else {
    // Bias and epilogue in f32, one rounding to bf16 into an LDS copy of
    // the tile (rows [0, BM/2) in the X stages, the rest in the weight
    // stages), then the tile leaves as 16-byte row segments.
    constexpr int EP = BN + 8;   // bf16 per staged row (16-byte pad)
    static_assert((BM / 2) * EP <= 2 * BM * kLdsRow && (BM / 2) * EP <= 2 * BN * kLdsRow,
                  "the staged output tile must fit the operand stages");
    uint16_t* const stage_lo = &lds_a[0][0];
    uint16_t* const stage_hi = &lds_b[0][0];
    constexpr int CPR = BN / 8;   // 16-byte chunks per row
    const bool vec_rows = (p.N & 7) == 0;
    __syncthreads();   // every wave is done reading the operand tiles
    // the GELU choice made once, outside the unrolled staging loop (a
    // runtime test inside it became a scalar branch per group of outputs)
    auto stage_tile = [&](auto gelu) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float bv[4][4];
        float swv[4][4];   // int8 GEMM: per-column weight scales
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int n = n0 + wn * WTN + j * 32 + g * 8 + lcol + t;
            const int c = wn * WTN + j * 32 + g * 8 + lcol + t;
            bv[g][t] = n < p.N ? lds_ep[c] : 0.0f;
            swv[g][t] = I8 && n < p.N ? lds_ep[BN + c] : 0.0f;
          }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int r = wm * WTM + i * 32 + lrow;
          uint16_t* srow = r < BM / 2 ? stage_lo + r * EP : stage_hi + (r - BM / 2) * EP;
          const int m = m0 + r;
          const float sxm = I8 && m < p.M ? lds_ep[2 * BN + r] : 0.0f;
          if constexpr (I8) {
            // the raw int32 accumulators, when asked for (bit-exact checks)
            if (p.acc_out != nullptr && m < p.M) {
              int32_t* arow = p.acc_out + (size_t)m * p.N;
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn * WTN + j * 32 + g * 8 + lcol;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                  if (n + t < p.N) { arow[n + t] = acc[i][j][4 * g + t]; }
                }
              }
            }
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float v[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              if constexpr (I8) {
                // y = bf16(fma(float(acc), sx[m] * sw[n], bias[n])), that order
                v[t] = fmaf((float)acc[i][j][4 * g + t], sxm * swv[g][t], bv[g][t]);
              } else {
                v[t] = acc[i][j][4 * g + t] + bv[g][t];
              }
            }
            if constexpr (decltype(gelu)::value) {
#pragma unroll
              for (int t = 0; t < 4; ++t) { v[t] = gelu_tanh(v[t]); }
            }
            *(uint2*)(srow + wn * WTN + j * 32 + g * 8 + lcol) =
                make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
          }
        }
      }
    };
    if (p.epilogue == kEpiGelu) {
      stage_tile(std::true_type{});
    } else {
      stage_tile(std::false_type{});
    }
    __syncthreads();
#pragma unroll 4
    for (int q = tid; q < BM * CPR; q += NT) {
      const int r = q / CPR;
      const int c = (q % CPR) * 8;
      const int m = m0 + r;
      const int n = n0 + c;
      if (m >= p.M || n >= p.N) { continue; }
      const uint16_t* srow = r < BM / 2 ? stage_lo + r * EP : stage_hi + (r - BM / 2) * EP;
      const uint4 v = *(const uint4*)(srow + c);
      uint16_t* dst = p.y + (size_t)m * p.N + n;
      if (vec_rows && n + 8 <= p.N) {
        // non-temporal: the tile is not read again by this launch (measured
        // +0.5% on the FFN GEMMs, whose stores leave in one chip-wide burst)
        __builtin_nontemporal_store(__builtin_bit_cast(i32x4, v), (i32x4*)dst);
      } else {
        const uint16_t e[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y,
                               (uint16_t)(v.y >> 16), (uint16_t)v.z, (uint16_t)(v.z >> 16),
                               (uint16_t)v.w, (uint16_t)(v.w >> 16)};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if (n + t < p.N) { dst[t] = e[t]; }
        }
      }
    }
  }
}

// Sum the split-K partials in split order, then bias, epilogue, bf16. The
// partials of up to kRedBatch splits, the bias and y_in are loaded before any
// is summed, so a thread waits for one memory round trip per batch, not one
// per split (a loop of dependent loads waited for each in turn).
constexpr int kRedBatch = 8;

__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float* partial, int splits, const void* bias,
                     int bias_type, int epilogue, const uint16_t* y_in, uint16_t* y, int M,
                     int N)
{
  const size_t total = (size_t)M * N;
  const size_t i0 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= total) { return; }
  const size_t plane = total;
  if ((N & 3) == 0 && i0 + 4 <= total) {
    // No branch around a partial's load (the wait counting then serializes
    // them): splits past the last re-read the last one, and are not added.
    // The first batch is issued before the bias and y_in loads, whose
    // branches on the bias type would otherwise be waited for first.
    f32x4 v[kRedBatch];
#pragma unroll
    for (int j = 0; j < kRedBatch; ++j) {
      v[j] = *(const f32x4*)(partial + (size_t)min(j, splits - 1) * plane + i0);
    }
    // one branch per operand, its four loads inside it
    const int n = (int)(i0 % (size_t)N);
    float b4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float yi[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias_type == kBiasF32) {
      const float* const bf = (const float*)bias + n;
#pragma unroll
      for (int t = 0; t < 4; ++t) { b4[t] = bf[t]; }
    } else if (bias_type == kBiasBf16) {
      const uint16_t* const bh = (const uint16_t*)bias + n;
#pragma unroll
      for (int t = 0; t < 4; ++t) { b4[t] = bf16_to_f32(bh[t]); }
    }
    if (y_in != nullptr) {
#pragma unroll
      for (int t = 0; t < 4; ++t) { yi[t] = bf16_to_f32(y_in[i0 + t]); }
    }
    // the sum in split order: split 0, then + split 1, + split 2, ...
    f32x4 s = v[0];
#pragma unroll
    for (int j = 1; j < kRedBatch; ++j) {
      if (j < splits) { s += v[j]; }
    }
    for (int k0 = kRedBatch; k0 < splits; k0 += kRedBatch) {
#pragma unroll
      for (int j = 0; j < kRedBatch; ++j) {
        v[j] = *(const f32x4*)(partial + (size_t)min(k0 + j, splits - 1) * plane + i0);
      }
#pragma unroll
      for (int j = 0; j < kRedBatch; ++j) {
        if (k0 + j < splits) { s += v[j]; }
      }
    }
    float o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float v = s[t] + b4[t];
      if (y_in != nullptr) { v += yi[t]; }
      if (epilogue == kEpiGelu) { v = gelu_tanh(v); }
      o[t] = v;
    }
    uint2 packed = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
    *(uint2*)(y + i0) = packed;
    return;
  }
  for (size_t i = i0; i < i0 + 4 && i < total; ++i) {
    float v = partial[i];
    for (int k = 1; k < splits; ++k) { v += partial[(size_t)k * plane + i]; }
    v += load_bias(bias, bias_type, (int)(i % (size_t)N));
    if (y_in != nullptr) { v += bf16_to_f32(y_in[i]); }
    if (epilogue == kEpiGelu) { v = gelu_tanh(v); }
    y[i] = f32_to_bf16(v);
  }
}

// Steps of the fully unrolled split-K slice (the audio shapes' K / 512).
constexpr int kSplitSteps = 8;

template <int BM, int BN, int WM, int WN, int BITS, bool SPLIT, bool FOLD = false>
hipError_t launch_cfg(const KParams& kp, int splits, hipStream_t stream)
{
  if constexpr (BITS == 16 && !FOLD) {
    if (kp.x2 != nullptr) { return launch_cfg<BM, BN, WM, WN, BITS, SPLIT, true>(kp, splits, stream); }
  }
  const dim3 grid((unsigned)(kp.tiles_m * kp.tiles_n), (unsigned)splits, 1);
  if constexpr (SPLIT && BITS != kI8Ops && BM == 128) {
    if (kp.k_chunk == kSplitSteps * kBK && kp.K % kp.k_chunk == 0) {
      hipLaunchKernelGGL((qgemm_kernel<BM, BN, WM, WN, BITS, SPLIT, kSplitSteps, FOLD>), grid,
                         dim3(WM * WN * 64), 0, stream, kp);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((qgemm_kernel<BM, BN, WM, WN, BITS, SPLIT, 0, FOLD>), grid,
                     dim3(WM * WN * 64), 0, stream, kp);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_tile(const KParams& kp, int bits, int splits,
                       hipStream_t stream)
{
  const bool split = splits > 1;
  switch (bits) {
    case 8:
      return split ? launch_cfg<BM, BN, WM, WN, 8, true>(kp, splits, stream)
                   : launch_cfg<BM, BN, WM, WN, 8, false>(kp, splits, stream);
    case 4:
      // 32 w4 codes per 16-byte chunk: a tile narrower than 128 columns
      // has fewer chunks per step than threads
      if constexpr (BN * kBK * 4 / 8 / 16 >= WM * WN * 64) {
        return split ? launch_cfg<BM, BN, WM, WN, 4, true>(kp, splits, stream)
                     : launch_cfg<BM, BN, WM, WN, 4, false>(kp, splits, stream);
      } else {
        return hipErrorInvalidValue;
      }
    default:
      return split ? launch_cfg<BM, BN, WM, WN, 16, true>(kp, splits, stream)
                   : launch_cfg<BM, BN, WM, WN, 16, false>(kp, splits, stream);
  }
}

int ilog2(int v)
{
  int s = 0;
  while ((1 << s) < v) { ++s; }
  return s;
}

}  // namespace

GemmPlan plan_gemm(int M, int N, int K, int bits, int cu_count, int force)
{
  GemmPlan plan;
  plan.cu_count = cu_count;
  if ((force == 0 || force == 3) && plan_skinny(M, N, K, bits, cu_count, plan)) { return plan; }
  const long tall_tiles = (long)((M + 255) / 256) * ((N + 255) / 256);
  // a forced M <= 128 kernel that cannot take the shape leaves the choice
  // to the planner
  if (force == 1 || ((force == 0 || force == 3) && M > 128 && tall_tiles >= cu_count)) {
    plan.tile = 0;
    plan.splits = 1;
    plan.k_chunk = K;
    return plan;
  }
  plan.tile = 1;
  const long tiles = (long)((M + 127) / 128) * ((N + kMidBN - 1) / kMidBN);
  // Split K until the workgroups cover the CUs once, with at least 512 of K
  // per split: each split writes a full f32 partial of the output. A sweep
  // over M = 256..2048, K = 2048 / 4096, N = 2048..16384 measured this
  // 0-28% faster than covering them twice (e.g. 33 vs 43 us at M = 1024,
  // K = 2048, N = 4096; 49 vs 66 us at M = 320, K = 2048, N = 16384).
  const long want = (1L * cu_count + tiles - 1) / tiles;
  const int max_split = std::max(1, K / 512);
  int s = (int)std::min<long>(std::max<long>(want, 1), max_split);
  int chunk = ((K + s - 1) / s + kBK - 1) / kBK * kBK;
  s = (K + chunk - 1) / chunk;
  plan.splits = s;
  plan.k_chunk = chunk;
  plan.workspace_bytes = s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
  return plan;
}

hipError_t launch_i8_gemm(const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                          const void* bias, int bias_type, int epilogue, uint16_t* y, int32_t* acc,
                          int M, int K, int N, hipStream_t stream)
{
  KParams kp = {};
  kp.xq = xq;
  kp.sx = sx;
  kp.sw = sw;
  kp.acc_out = acc;
  kp.wq = (const uint8_t*)wq;
  kp.bias = bias;
  kp.bias_type = bias != nullptr ? bias_type : kBiasNone;
  kp.epilogue = epilogue;
  kp.y = y;
  kp.M = M;
  kp.N = N;
  kp.wn = N;
  kp.K = K;
  kp.k_chunk = K;
  int dev = 0;
  int cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    cus = 256;
  }
  // the tall tile when it fills the GPU, else 128 x 128
  const bool fills = (long)((M + 255) / 256) * ((N + 255) / 256) >= cus;
  if (fills && tall_i8_takes(M, N, K)) {
    return launch_tall_i8(xq, sx, wq, sw, bias, kp.bias_type, epilogue, y, acc, M, K, N, stream);
  }
  if (fills) {
    kp.tiles_m = (M + 255) / 256;
    kp.tiles_n = (N + 255) / 256;
    return launch_cfg<256, 256, kTallWM, kTallWN, kI8Ops, false>(kp, 1, stream);
  }
  kp.tiles_m = (M + 127) / 128;
  kp.tiles_n = (N + 127) / 128;
  return launch_cfg<128, 128, 2, 2, kI8Ops, false>(kp, 1, stream);
}

hipError_t launch_splitk_reduce(const float* partial, int splits, const void* bias, int bias_type,
                                int epilogue, const uint16_t* y_in, uint16_t* y, int M, int N,
                                hipStream_t stream)
{
  const size_t total = (size_t)M * N;
  const unsigned blocks = (unsigned)((total + 1023) / 1024);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partial, splits,
                     bias, bias != nullptr ? bias_type : kBiasNone, epilogue, y_in, y, M, N);
  return hipGetLastError();
}

hipError_t launch_gemm(const GemmDesc& d, const GemmPlan& plan,
                       float* workspace, hipStream_t stream)
{
  if (d.x2 != nullptr &&
      (plan.tile == 2 || d.bits != 16 || d.kx <= 0 || d.kx >= d.K || d.kx % kBK != 0)) {
    return hipErrorInvalidValue;   // the two-part activation: dense weights, MFMA tiles
  }
  if (plan.tile == 2 && d.wn > 0 && d.wn < d.N) {
    return hipErrorInvalidValue;   // the M <= 128 kernel reads all N weight rows
  }
  if (plan.tile == 2) { return launch_skinny(d, plan, workspace, stream); }
  if (tall_dense_takes(d, plan) || tall_w8_takes(d, plan)) { return launch_tall_dense(d, stream); }
  KParams kp = {};
  kp.x = d.x;
  kp.x2 = d.x2;
  kp.kx = d.x2 != nullptr ? d.kx : d.K;
  kp.wn = d.wn > 0 && d.wn < d.N ? d.wn : d.N;
  kp.wq = (const uint8_t*)d.w;
  kp.wd = (const uint16_t*)d.w;
  kp.scales = d.scales;
  kp.qbias = d.qbias;
  kp.bias = d.bias;
  kp.y = d.y;
  kp.y_in = d.y_in;
  kp.partial = workspace;
  kp.M = d.M;
  kp.N = d.N;
  kp.K = d.K;
  kp.gshift = d.bits == 16 ? 0 : ilog2(d.group);
  kp.gcols = d.bits == 16 ? 0 : d.K / d.group;
  kp.k_chunk = plan.k_chunk;
  kp.bias_type = d.bias != nullptr ? d.bias_type : kBiasNone;
  kp.epilogue = d.epilogue;
  const int bm = plan.tile == 0 ? 256 : 128;
  const int bn = plan.tile == 0 ? 256 : kMidBN;
  kp.tiles_m = (d.M + bm - 1) / bm;
  kp.tiles_n = (d.N + bn - 1) / bn;

  hipError_t e = plan.tile == 0
                     ? launch_tile<256, 256, kTallWM, kTallWN>(kp, d.bits, plan.splits, stream)
                     : launch_tile<128, kMidBN, 2 * 128 / kMidBN, kMidBN / 64>(
                           kp, d.bits, plan.splits, stream);
  if (e != hipSuccess || plan.splits <= 1) { return e; }
  return launch_splitk_reduce(workspace, plan.splits, kp.bias, kp.bias_type, d.epilogue, d.y_in,
                              d.y, d.M, d.N, stream);
}

}  // namespace ltx25
