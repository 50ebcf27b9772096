// The 256 x 256 GEMM tile on the 16-row MFMAs, in three operand modes:
//   - bf16: y = x . w^T (+ bias) (+ GELU) on v_mfma_f32_16x16x32_bf16, for
//     the dequant-once arm of the quantized linear (the weight expanded to
//     bf16 once per call), for dense weights, and for the LoRA fold's
//     two-part activation [x | r];
//   - int8: the int8 tier's GEMM, int8 x int8 -> exact int32 on
//     v_mfma_i32_16x16x64_i8, 128 of K per step in the same 128-byte row
//     segments (so every fragment offset is the bf16 mode's), epilogue
//     y = bf16(epi(fma(float(acc), sx[m] * sw[n], bias[n] or +0))) in that
//     order, as the template's int8 mode computes it;
//   - w8: u8 codes (groups of 64 or 32) dequantized in registers once per
//     workgroup before the LDS write, with the expansion kernel's
//     arithmetic, so its results equal the bf16 mode's over the expansion
//     bit for bit (tall_w8_kernel, below).
//
// bf16 and int8: tall_kernel, an 8-wave ping-pong schedule.
//   - Waves 0-3 (group 0) own output rows 0..127, waves 4-7 (group 1) rows
//     128..255, each wave 64 columns: 8 x 4 blocks of 16 x 16, 128 f32 /
//     int32 accumulators per lane. Wave w and w + 4 share a SIMD.
//   - The two groups alternate, phase by phase, between a compute cluster
//     (the 64 MFMAs of one 64-deep K step on fragments already in
//     registers, at wave priority 1) and a memory cluster (the 24 fragment
//     reads for its next compute cluster, then its share of the operand
//     loads). A workgroup barrier ends every phase; group 1 runs one phase
//     behind group 0, so each SIMD always has one wave issuing MFMAs while
//     the other feeds it.
//   - Operands go straight from global memory into LDS (buffer_load ...
//     lds, 16 bytes per lane, one instruction = 8 rows x 128 bytes). Rows
//     are 128 bytes with the 16-byte pieces XOR-swizzled by row % 8: the
//     16x16x32 fragment reads (16 rows x 4 pieces) are then free of bank
//     conflicts (measured on the MI355X with SQ_LDS_BANK_CONFLICT: 0 cycles
//     per read; a swizzle by 2 ((row / 4) % 4) cost 4, none 12).
//   - X rows 0..127 are read only by group 0 and rows 128..255 only by
//     group 1, so X has two stages per half and the weight, read by both
//     groups, three (32 + 32 + 96 KB = the 160 KB of LDS). Group 0 loads
//     the X half group 1 reads and group 1 the X half group 0 reads; each
//     wave also loads 4 of the 32 weight load instructions of a step. Each
//     group issues its loads at the start of its memory cluster, so every
//     load has three or more phases (about 1.5 us) to land. The exact vmcnt
//     each wave waits for is derived per phase below.
//   - Per step and CU the fragment reads move 192 KB through LDS and the
//     loads 64 KB into it (measured costs ~4.6 ns per 1 KB read, ~1.9 ns per
//     1 KB load interleaved with reads): ~1 us of LDS time against ~1.1 us
//     of MFMA time, which is what holds this 8-wave tile below the MFMA
//     peak.
//   - Epilogue: bias (and the int8 scales) read from global memory, GELU,
//     one rounding to bf16, staged in LDS, 16-byte row stores.
//   Against the previous register-fed schedule (tall_w8_kernel's, with
//   bf16 operands) on the FFN GEMMs: 798 vs 830 us (up, GELU) and 720 vs
//   752 us (down), bit-identical (interleaved best-of-15 on one MI355X).
//
// Reference semantics: MetalOps::dequant_mma_ -> dense_mma_
// (src/ltx25-metal-ops.cc:467-502, 342-465), then bias_add (:568); the int8
// mode is the tier under dense_mma_ (I8GemmContext::gemm, :386-391).
#include "common.h"

#include <type_traits>
#include <utility>

namespace ltx25 {
namespace {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kThreads = 512;
constexpr int kSB = 128;                     // bytes of each row per K step
constexpr int kBK = 64;                      // bf16 per step (the int8 mode: 128 int8)
constexpr int kEP = kBN + 8;                 // bf16 per staged output row

constexpr int kModeBf16 = 0;
constexpr int kModeI8 = 1;
constexpr int kModeW8 = 2;

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t __attribute__((address_space(3))) lds_u32;

struct TallParams {
  const void* x;           // bf16 [M][K] or int8 [M][K]; with x2: bf16 [M][kx]
  const void* x2;          // the two-part activation's columns [kx, K), bf16 [M][K - kx]
  int kx;                  // columns of x when x2 is set (a multiple of 64)
  const void* w;           // bf16 [N][K] or int8 [N][K] (w8: u8 codes [N][K])
  const void* bias;
  const float* sx;         // int8 mode: per-row activation scales
  const float* sw;         // int8 mode: per-column weight scales
  int32_t* acc_out;        // int8 mode, optional: the raw int32 accumulators
  const uint16_t* scales;  // w8 mode: bf16 [N][K / group]
  const uint16_t* qbias;   // w8 mode: bf16 [N][K / group]
  int gshift, gcols;       // w8 mode: log2(group), K / group
  uint16_t* y;
  const uint16_t* y_in;    // bf16 mode without x2, optional: the accumulators start from it
  int M, N, K;             // K in elements
  int wn;                  // rows of w in memory; rows past them read as zeros
  int bias_type, epilogue;
  int tiles_m, tiles_n;
  // the phase-stamp instantiation only (ltx25_probe_tall_phases): eight
  // words per wave at (tile * 8 + wave) * 8
  unsigned long long* stamps;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, size_t bytes)
{
  // loads past `bytes` return zeros: rows past M and past wn
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)(uint32_t)bytes,
                                           0x00020000);
}

// s_waitcnt vmcnt(n), the other counters left alone (n < 16)
#define LTX25_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0f70 | (n))
// s_waitcnt lgkmcnt(0)
#define LTX25_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xc07f)
// A phase stamp (the STAMPS instantiation): the shader clock, with the
// scheduler held on both sides so that the read stays where the source puts it
#define LTX25_TSTAMP(var)                \
  if constexpr (STAMPS) {                \
    __builtin_amdgcn_sched_barrier(0);   \
    var = __builtin_amdgcn_s_memtime();  \
    __builtin_amdgcn_sched_barrier(0);   \
  }

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>): the
// index is a compile-time constant inside f
template <typename F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>)
{
  (f(std::integral_constant<int, I>{}), ...);
}

template <int N, typename F>
__device__ __forceinline__ void unroll(F&& f)
{
  unroll_seq(f, std::make_integer_sequence<int, N>{});
}

// The block's tile: XCD-grouped by map_tile, then the N-tiles relabelled
// tn -> 5 tn mod tiles_n (a bijection when 5 does not divide tiles_n): the
// tiles a round of workgroups finishes together then store scattered
// 512-byte segments of each output row, not runs of adjacent ones (1.9%
// faster on the 8160 x 4096 -> 16384 GEMM, 0.5% on 16384 -> 4096).
__device__ __forceinline__ void tile_of(const TallParams& p, int& m0, int& n0)
{
  int tm, tn;
  map_tile(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  if (p.tiles_n % 5 != 0) { tn = (tn * 5) % p.tiles_n; }
  m0 = tm * kBM;
  n0 = tn * kBN;
}

// ---- the ping-pong tile (bf16, int8) ----------------------------------------

// LDS: X stages 0, 1 (32 KB each: 256 rows x 128 bytes), then weight stages
// 0, 1, 2. The staged output tile of the epilogue reuses it.
constexpr int kOp = 256 * kSB;
constexpr int kXOff = 0;
constexpr int kWOff = 2 * kOp;
constexpr int kPPLds = 5 * kOp;
static_assert(kPPLds == 160 * 1024, "the stages fill the LDS");
static_assert(kBM * kEP * 2 <= kPPLds, "the staged tile fits the stages");

template <int MODE, bool FOLD, bool STAMPS = false>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
tall_kernel(TallParams p)
{
  static_assert(MODE == kModeBf16 || MODE == kModeI8, "w8 codes run tall_w8_kernel");
  static_assert(!FOLD || MODE == kModeBf16, "the two-part activation is a bf16-mode operand");
  static_assert(!STAMPS || !FOLD, "the phase stamps are built without the two-part activation");
  constexpr bool I8 = MODE == kModeI8;
  constexpr int kEB = I8 ? 1 : 2;   // bytes per element
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kPPLds];
  // phase stamps: shader clock at entry, step 0 landed, K loop done, output
  // staged in LDS, stores complete; 100 MHz clock at entry and at the end
  unsigned long long st[5] = {0, 0, 0, 0, 0};
  unsigned long long rt0 = 0;
  if constexpr (STAMPS) {
    __builtin_amdgcn_sched_barrier(0);
    rt0 = __builtin_amdgcn_s_memrealtime();
  }
  LTX25_TSTAMP(st[0])

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2;      // group: output rows 128 g .. 128 g + 127
  const int wn = wave & 3;      // output columns 64 wn .. 64 wn + 63
  int m0, n0;
  tile_of(p, m0, n0);
  const uint32_t row_bytes = (uint32_t)p.K * kEB;
  const int n = (int)(row_bytes / kSB);   // K steps

  // ---- loads. Instruction q (0..31) of an operand covers rows 8 q .. 8 q + 7
  // of the tile; lane l lands at byte 16 l of the instruction's 1 KB (row
  // 8 q + l / 8, slot l % 8) and fetches the row's piece (l % 8) ^ (row % 8),
  // a lane constant since 8 q is a multiple of 8. A wave of group 0 issues X
  // instructions 16 + 4 wn + i (the half group 1 reads), one of group 1
  // instructions 4 wn + i; wave w issues weight instructions 4 w + i.
  const uint32_t swz = (uint32_t)(((lane & 7) ^ ((lane >> 3) & 7)) * 16);
  const int xq = (g == 0 ? 16 : 0) + 4 * wn;
  const int xq_own = (g == 0 ? 0 : 16) + 4 * wn;   // the half the wave's group reads
  const int wq = 4 * wave;
  const uint32_t xrow = (uint32_t)(m0 + 8 * xq + (lane >> 3));
  const uint32_t xrow_own = (uint32_t)(m0 + 8 * xq_own + (lane >> 3));
  const uint32_t wrow = (uint32_t)(n0 + 8 * wq + (lane >> 3));
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (size_t)p.wn * row_bytes);
  // FOLD: the activation is [x | x2]; a step lies in one part, chosen by
  // uniform selects (rsrc, row pitch, step within the part)
  const int fsteps = FOLD ? p.kx / kBK : n;
  const uint32_t rb1 = FOLD ? (uint32_t)p.kx * 2u : row_bytes;
  const uint32_t rb2 = FOLD ? (uint32_t)(p.K - p.kx) * 2u : row_bytes;
  const __amdgpu_buffer_rsrc_t xr1 = make_rsrc(p.x, (size_t)p.M * rb1);
  const __amdgpu_buffer_rsrc_t xr2 = FOLD ? make_rsrc(p.x2, (size_t)p.M * rb2) : xr1;
  // Per-lane X offsets (row * pitch + piece) of each part, computed once:
  // with the part's pitch chosen per step inside the address, the compiler
  // redid the 64-bit multiply on every step (26 more instructions per step
  // in the fold's loop, 5.6% more cycles per K step).
  const uint32_t xv1 = xrow * rb1 + swz;
  const uint32_t xv1_own = xrow_own * rb1 + swz;
  const uint32_t xv2 = FOLD ? xrow * rb2 + swz : 0u;
  const uint32_t xv2_own = FOLD ? xrow_own * rb2 + swz : 0u;
  // `own`: the X half this wave's group reads (the prologue's step 0)
  auto load_x = [&](int s, bool own, int q0) {
    uint8_t* const base = lds + kXOff + (s & 1) * kOp + q0 * 1024;
    if (!FOLD || s < fsteps) {
      const uint32_t v0 = own ? xv1_own : xv1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr1, (lds_u32*)(base + i * 1024), 16,
                                                 (int)(v0 + 8u * i * rb1), s * kSB, 0, 0);
      }
    } else {
      const uint32_t v0 = own ? xv2_own : xv2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr2, (lds_u32*)(base + i * 1024), 16,
                                                 (int)(v0 + 8u * i * rb2), (s - fsteps) * kSB, 0,
                                                 0);
      }
    }
  };
  auto load_w = [&](int s, int wst) {
    uint8_t* const base = lds + kWOff + wst * kOp + wq * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_u32*)(base + i * 1024), 16,
                                               (int)((wrow + 8u * i) * row_bytes + swz), s * kSB, 0,
                                               0);
    }
  };

  // ---- fragments of a 16-row block b and a 64-byte K slice sl: lane l
  // holds row 16 b + l % 16, piece 4 sl + l / 16 (8 bf16 of a 16x16x32 MFMA,
  // 16 int8 of a 16x16x64 one), at slot piece ^ (l % 8)
  const int fo0 = (lane & 15) * kSB + ((((lane >> 4)) ^ (lane & 7)) * 16);
  const int fo1 = (lane & 15) * kSB + (((4 + (lane >> 4)) ^ (lane & 7)) * 16);
  const int xbase = kXOff + g * 128 * kSB;
  const int wbase = kWOff + wn * 64 * kSB;
  i32x4v afr[2][8], bfr[2][4];
  auto read_frags = [&](int xst, int wst) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const int fo = sl ? fo1 : fo0;
      const uint8_t* const sa = lds + xbase + xst * kOp + fo;
      const uint8_t* const sb = lds + wbase + wst * kOp + fo;
#pragma unroll
      for (int i = 0; i < 8; ++i) { afr[sl][i] = *(const i32x4v*)(sa + i * 16 * kSB); }
#pragma unroll
      for (int j = 0; j < 4; ++j) { bfr[sl][j] = *(const i32x4v*)(sb + j * 16 * kSB); }
    }
  };
  using AccT = std::conditional_t<I8, i32x4v, f32x4v>;
  AccT acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) { acc[i][j][r] = 0; }
    }
  }
  // Accumulate into an existing output (the LoRA pair's second GEMM,
  // y = bf16(y + r . B^T)): the accumulators start from y_in in their own
  // layout (block (i, j), lane l: row 16 i + l % 16 of the group's half,
  // four consecutive columns from 16 j + 4 (l / 16) of the wave's), so the
  // K loop adds the products to it and the epilogue rounds once, as the
  // template tile does. The loads are issued before any operand load, so
  // the hand-counted vmcnt waits below only ever wait longer for them.
  if constexpr (!I8 && !FOLD) {
    if (p.y_in != nullptr) {
      const int lrow = lane & 15;
      const int lcol = (lane >> 4) * 4;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int m = m0 + g * 128 + i * 16 + lrow;
        if (m >= p.M) { continue; }
        const uint16_t* const yrow = p.y_in + (size_t)m * p.N;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int nn = n0 + wn * 64 + j * 16 + lcol;
          if (nn >= p.N) { continue; }   // N % 8 == 0: all four columns or none
          const uint2 o = *(const uint2*)(yrow + nn);
          acc[i][j] = f32x4v{__uint_as_float(o.x << 16), __uint_as_float(o.x & 0xffff0000u),
                             __uint_as_float(o.y << 16), __uint_as_float(o.y & 0xffff0000u)};
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  auto compute = [&]() {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (I8) {
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bfr[sl][j], afr[sl][i], acc[i][j], 0, 0,
                                                             0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, bfr[sl][j]), __builtin_bit_cast(bf16x8, afr[sl][i]),
                acc[i][j], 0, 0, 0);
          }
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- prologue: step 0 whole (each wave its own X half's share and its
  // weight share), then the weight of step 1 and, from group 1, X rows
  // 0..127 of step 1 (group 0 sends rows 128..255 of step 1 in its M(0)).
  load_x(0, true, xq_own);
  load_w(0, 0);
  if (n > 1) {
    load_w(1, 1);
    if (g == 1) { load_x(1, false, xq); }
    // step 0 landed: group 0 leaves W(1) (4) in flight, group 1 W(1) and X(1) (8)
    if (g == 0) { LTX25_VMCNT(4); } else { LTX25_VMCNT(8); }
  } else {
    LTX25_VMCNT(0);
  }
  __builtin_amdgcn_s_barrier();
  LTX25_TSTAMP(st[1])
  if (g == 1) { __builtin_amdgcn_s_barrier(); }

  // ---- main loop. Group 0 runs M(s) in phase 2 s and C(s) in 2 s + 1, group
  // 1 one phase later (phase p ends with barrier p). Stages: X half h of
  // step t in X stage t % 2 (the half's readers finished step t - 2 two
  // phases before any wave could send step t), the weight of step t in
  // weight stage t % 3. Loads at the start of M(s): group 0 X rows
  // 128..255 of step s + 1, then its weight share of step s + 2; group 1 X
  // rows 0..127 and its weight share, both of step s + 2. Waits, each
  // before the barrier that precedes the first reader:
  //   group 0 end of M(s), s >= 1: its X(s) (in flight: W(s + 1), X(s + 1),
  //     W(s + 2));
  //   group 0 end of C(s): its W(s + 1) (in flight: X(s + 1), W(s + 2));
  //   group 1 end of M(s): its X(s + 1), W(s + 1) (in flight: X(s + 2),
  //     W(s + 2)).
  int wst = 0;   // s % 3
  for (int s = 0; s < n; ++s) {
    const int wst2 = wst == 0 ? 2 : wst - 1;   // (s + 2) % 3
    const bool m1 = s + 1 < n;
    const bool m2 = s + 2 < n;
    // memory cluster
    __builtin_amdgcn_sched_barrier(0);
    read_frags(s & 1, wst);
    if (g == 0) {
      if (m1) { load_x(s + 1, false, xq); }
      if (m2) { load_w(s + 2, wst2); }
    } else if (m2) {
      load_x(s + 2, false, xq);
      load_w(s + 2, wst2);
    }
    LTX25_LGKMCNT0();   // the fragments are in registers
    if (g == 0) {
      if (s >= 1) {
        if (m2) {
          LTX25_VMCNT(12);
        } else if (m1) {
          LTX25_VMCNT(8);
        } else {
          LTX25_VMCNT(0);
        }
      }
    } else if (m2) {
      LTX25_VMCNT(8);
    } else {
      LTX25_VMCNT(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // compute cluster
    compute();
    __builtin_amdgcn_sched_barrier(0);
    if (g == 0) {
      if (m2) {
        LTX25_VMCNT(8);
      } else if (m1) {
        LTX25_VMCNT(4);
      } else {
        LTX25_VMCNT(0);
      }
    }
    __builtin_amdgcn_s_barrier();
    wst = wst == 2 ? 0 : wst + 1;
  }
  if (g == 0) { __builtin_amdgcn_s_barrier(); }
  __syncthreads();   // every wave is done reading the operand stages
  LTX25_TSTAMP(st[2])

  // ---- epilogue. Accumulator block (i, j), lane l, register r (the MFMAs
  // take the weight fragment first): row 16 i + l % 16 of the wave's rows,
  // column 16 j + 4 (l / 16) + r of its columns -- four consecutive columns.
  const int lrow = lane & 15;
  const int lcol = (lane >> 4) * 4;
  uint16_t* const stage = (uint16_t*)lds;
  // The epilogue's operands -- bias, and the int8 mode's row and column
  // scales -- are loaded together before any is used, at indices clamped
  // into range (a column or row past the end is never stored): no branch
  // sits between the loads, so they are waited for once, not one by one.
  float b4s[4][4], sw4s[4][4], sxm[8];
  {
    int ncl[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int nn = n0 + wn * 64 + j * 16 + lcol + t;
        ncl[j][t] = nn < p.N ? nn : p.N - 1;
      }
    }
    if (p.bias_type == kBiasF32) {
      const float* const bf = (const float*)p.bias;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) { b4s[j][t] = bf[ncl[j][t]]; }
      }
    } else if (p.bias_type == kBiasBf16) {
      const uint16_t* const bh = (const uint16_t*)p.bias;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) { b4s[j][t] = bf16_to_f32(bh[ncl[j][t]]); }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) { b4s[j][t] = 0.0f; }
      }
    }
    if constexpr (I8) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) { sw4s[j][t] = p.sw[ncl[j][t]]; }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int m = m0 + g * 128 + i * 16 + lrow;
        sxm[i] = p.sx[m < p.M ? m : p.M - 1];
      }
      if (p.acc_out != nullptr) {
        // the raw int32 accumulators, when asked for (bit-exact checks);
        // N % 8 == 0, so the four columns are all in range
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int m = m0 + g * 128 + i * 16 + lrow;
            const int nn = n0 + wn * 64 + j * 16 + lcol;
            if (m < p.M && nn < p.N) {
              int32_t* arow = p.acc_out + (size_t)m * p.N + nn;
#pragma unroll
              for (int t = 0; t < 4; ++t) { arow[t] = acc[i][j][t]; }
            }
          }
        }
      }
    }
  }
  // The epilogue's choices are made once, outside the unrolled staging loop:
  // a runtime test per output became a scalar branch per output, which kept
  // the scheduler from interleaving outputs (and made it rematerialize the
  // GELU's constants per output). Without a bias no +0 is added. An
  // accumulator that starts at +0 is never -0 (x + (-x) rounds to +0), so
  // those bits are unchanged; one seeded from y_in = -0 whose products are
  // all -0 stays -0, as the reference's accumulate into y (lora_mma_'s
  // second GEMM, src/ltx25-metal-ops.cc:938-987) adds no bias either.
  auto stage_tile = [&](auto gelu, auto biased) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wn * 64 + j * 16 + lcol;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = g * 128 + i * 16 + lrow;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if constexpr (I8) {
            // y = bf16(fma(float(acc), sx[m] * sw[n], bias[n])), that order
            v[t] = fmaf((float)acc[i][j][t], sxm[i] * sw4s[j][t], b4s[j][t]);
          } else if constexpr (decltype(biased)::value) {
            v[t] = acc[i][j][t] + b4s[j][t];
          } else {
            v[t] = acc[i][j][t];
          }
          if constexpr (decltype(gelu)::value) { v[t] = gelu_tanh(v[t]); }
        }
        *(uint2*)(stage + r * kEP + c) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  };
  const bool biased = p.bias_type != kBiasNone;
  if (p.epilogue == kEpiGelu) {
    if (biased) {
      stage_tile(std::true_type{}, std::true_type{});
    } else {
      stage_tile(std::true_type{}, std::false_type{});
    }
  } else if (biased) {
    stage_tile(std::false_type{}, std::true_type{});
  } else {
    stage_tile(std::false_type{}, std::false_type{});
  }
  __syncthreads();
  LTX25_TSTAMP(st[3])
  constexpr int CPR = kBN / 8;   // 16-byte chunks per output row
#pragma unroll 4
  for (int q = tid; q < kBM * CPR; q += kThreads) {
    const int r = q / CPR;
    const int c = (q % CPR) * 8;
    const int m = m0 + r;
    const int nn = n0 + c;
    if (m >= p.M || nn >= p.N) { continue; }
    const uint4 v = *(const uint4*)(stage + r * kEP + c);
    // non-temporal: the tile is not read again by this launch
    __builtin_nontemporal_store(__builtin_bit_cast(i32x4, v), (i32x4*)(p.y + (size_t)m * p.N + nn));
  }
  if constexpr (STAMPS) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the stores have completed
    LTX25_TSTAMP(st[4])
    const unsigned long long rt1 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
    if (p.stamps != nullptr && lane == 0) {
      // HW_ID (CU, SH, SE of this wave) and XCC_ID, read from the hardware registers
      const unsigned long long hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
      const unsigned long long xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
      unsigned long long* o = p.stamps + ((size_t)blockIdx.x * 8 + wave) * 8;
#pragma unroll
      for (int i = 0; i < 5; ++i) { o[i] = st[i]; }
      o[5] = rt0;
      o[6] = rt1;
      o[7] = (xcc << 32) | hw;
    }
  }
}

// ---- the fused w8 tile: register-fed, 160-byte LDS rows ----------------------
//
//   - 8 waves in 2 x 4, 128 x 64 of the output per wave: 8 x 4 blocks of
//     16 x 16, 128 f32 accumulators per lane;
//   - a 64-deep K step is two 32-deep slices, each run in two halves of 16
//     MFMAs (A blocks 0..3, then 4..7); the next half's fragments are read
//     under the current half's MFMAs (A double-buffered per half, B per
//     slice: 64 registers);
//   - X rows arrive as whole 128-byte row segments (16-byte loads, 8 lanes
//     per row) in registers and are written a step later to one of two LDS
//     stages, in the third quarter of a step; each register is reloaded
//     right after its LDS write, which gives every load a step to land;
//   - each thread loads 16-byte runs of codes of two weight rows (4 lanes
//     per row's 64-code step) and each row's scale and zero point,
//     dequantizes them in registers exactly as the expansion kernel does
//     (fma(scale, q, zero point) in f32, one rounding to bf16) and writes
//     the 16 bf16 of each row to the row's 32-byte span of the stage;
//   - LDS rows are 160 bytes: a 16x16x32 fragment read covers 16 rows x 4
//     pieces of 16 bytes, and at this pitch those 64 pieces fall in distinct
//     banks. Two stages fill the 160 KB of LDS; the bias sits in the row
//     pads of the last 32 W rows of stage 1, which neither the operand rows
//     nor the staged output reach;
//   - one barrier per step; bias, GELU-tanh and one rounding to bf16 in the
//     epilogue, staged in LDS and stored as 16-byte row segments.
constexpr int kRow = kBK + 16;               // halfs per LDS row (160 bytes)
constexpr int kSide = 256 * kRow;            // one operand's rows in a stage
constexpr int kStage = 2 * kSide;
constexpr int kLd = 4;                       // 16-byte X loads per thread and step
constexpr int kLdsHalfs = 2 * kStage;        // 163840 bytes
static_assert(kBM * kEP <= kLdsHalfs, "the staged tile fits the stages");
// The bias in the 32-byte row pads of stage 1's last W rows (the operand
// rows use bytes 0..127 of a row; the staged output tile ends before them):
// bias value c at row 480 + c / 8, pad float c % 8.
constexpr int kPadRow(int first) { return kStage + first * kRow + kBK; }
static_assert(kPadRow(480) >= kBM * kEP, "the epilogue pads lie past the staged tile");

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
tall_w8_kernel(TallParams p)
{
  __shared__ __attribute__((aligned(16))) uint16_t lds[kLdsHalfs];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;
  const int wn = wave & 3;
  int m0, n0;
  tile_of(p, m0, n0);
  const uint32_t row_bytes = (uint32_t)p.K * 2u;
  const int nsteps = p.K / kBK;
  auto pad_at = [&](int first, int c) -> float* {
    return (float*)(lds + kPadRow(first) + (c / 8) * kRow) + (c & 7);
  };
  if (tid < kBN) {
    const int n = n0 + tid;
    *pad_at(480, tid) = n < p.N ? load_bias(p.bias, p.bias_type, n) : 0.0f;
  }

  // thread t loads rows t / 8 + 64 i of the X tile, 16-byte piece t % 8 of
  // the step's 128 bytes
  const int lr = tid >> 3;
  const int lc = tid & 7;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, (size_t)p.M * row_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (size_t)p.wn * (uint32_t)p.K);
  uint32_t xoff[kLd];
#pragma unroll
  for (int i = 0; i < kLd; ++i) {
    xoff[i] = (uint32_t)(m0 + lr + 64 * i) * row_bytes + (uint32_t)lc * 16u;
  }
  // thread t holds codes of weight rows t / 4 and t / 4 + 128, 16-byte
  // piece t % 4 of the step's 64 codes (4 lanes cover a row's segment), and
  // the scale and zero point of each piece's group
  const int cr = tid >> 2;
  const int cp = tid & 3;
  uint32_t coff[2], soff[2];
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(p.scales, (size_t)p.wn * p.gcols * 2);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(p.qbias, (size_t)p.wn * p.gcols * 2);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    coff[i] = (uint32_t)(n0 + cr + 128 * i) * (uint32_t)p.K + (uint32_t)cp * 16u;
    soff[i] = ((uint32_t)(n0 + cr + 128 * i) * (uint32_t)p.gcols +
               ((uint32_t)cp * 16u >> p.gshift)) * 2u;
  }
  const int gstep = (kBK >> p.gshift) * 2;   // bytes of a scale row per step
  uint4 creg[2];
  uint32_t sreg[2], breg[2];
  uint32_t dq[8];   // one row's 16 dequantized bf16
  auto load_c = [&](int s, int i) {
    creg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)coff[i], s * kBK, 0));
  };
  auto load_sb = [&](int s, int i) {
    sreg[i] = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)soff[i], s * gstep, 0);
    breg[i] = __builtin_amdgcn_raw_buffer_load_b16(br, (int)soff[i], s * gstep, 0);
  };
  // codes 2 h and 2 h + 1 of row i's piece
  auto dq_pair = [&](int i, int h) {
    const float sc = __builtin_bit_cast(float, sreg[i] << 16);
    const float zp = __builtin_bit_cast(float, breg[i] << 16);
    const uint32_t w = creg[i][h >> 1];
    const int sh = (h & 1) * 16;
    dq[h] = pack_bf16x2(fmaf(sc, (float)((w >> sh) & 0xffu), zp),
                        fmaf(sc, (float)((w >> (sh + 8)) & 0xffu), zp));
  };
  auto store_dq = [&](int st, int i, int hh) {
    *(uint4*)(lds + st * kStage + kSide + (cr + 128 * i) * kRow + cp * 16 + 8 * hh) =
        make_uint4(dq[4 * hh], dq[4 * hh + 1], dq[4 * hh + 2], dq[4 * hh + 3]);
  };
  const int dst = lr * kRow + lc * 8;
  uint4 xreg[kLd];
  auto load_x = [&](int s, int i) {
    xreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)xoff[i], s * kSB, 0));
  };
  auto store_x = [&](int st, int i) { *(uint4*)(lds + st * kStage + dst + 64 * i * kRow) = xreg[i]; };

  // fragments of a 16-row operand block b and a 64-byte K slice: lane l
  // holds row 16 b + l % 16, bytes 16 (l / 16) .. + 15 of the slice
  const int fa = (wm * 128 + (lane & 15)) * kRow + (lane >> 4) * 8;
  const int fb = kSide + (wn * 64 + (lane & 15)) * kRow + (lane >> 4) * 8;
  i32x4v afr[2][4];   // [half parity]: A blocks 4 h .. 4 h + 3
  i32x4v bfr[2][4];   // [slice parity]: the slice's 4 B blocks
  auto rd_a = [&](int st, int sl, int hh, int buf, int i) {
    afr[buf][i] = *(const i32x4v*)(lds + st * kStage + fa + (4 * hh + i) * 16 * kRow + sl * 32);
  };
  auto rd_b = [&](int st, int sl, int buf, int j) {
    bfr[buf][j] = *(const i32x4v*)(lds + st * kStage + fb + j * 16 * kRow + sl * 32);
  };
  f32x4v acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) { acc[i][j] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f}; }
  }
  auto mfma = [&](const i32x4v& b, const i32x4v& a, f32x4v c) -> f32x4v {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b),
                                                   __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
  };

  // prologue: step 0 into stage 0, step 1 into registers, the first fragments
#pragma unroll
  for (int i = 0; i < kLd; ++i) { load_x(0, i); }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    load_c(0, i);
    load_sb(0, i);
  }
#pragma unroll
  for (int i = 0; i < kLd; ++i) { store_x(0, i); }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int h = 0; h < 8; ++h) { dq_pair(i, h); }
    store_dq(0, i, 0);
    store_dq(0, i, 1);
  }
  if (nsteps > 1) {
    // Step 1's loads in the main loop's issue order (codes then scale and
    // zero point row by row, then X). The loop's wait counts also cover its
    // first iteration, so a prologue order that differs makes every
    // iteration wait for more loads than its own order needs.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      load_c(1, i);
      __builtin_amdgcn_sched_barrier(0);
      load_sb(1, i);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < kLd; ++i) {
      load_x(1, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rd_a(0, 0, 0, 0, i);
    rd_b(0, 0, 0, i);
  }

  // Step s reads stage s & 1 in four quarters (slice q / 2, half q % 2) of
  // 16 MFMAs. Fragment reads for later quarters: q0 A half 1 of slice 0 and
  // B of slice 1; q1 A half 0 of slice 1; q2 A half 1 of slice 1; q3 (after
  // the barrier) A half 0 and B of slice 0 of step s + 1. Writes of step
  // s + 1 to the other stage: the dequantized weight rows in q1, X in q2,
  // each register reloaded with step s + 2 in the gap after its write, so a
  // load has a whole step to land. The writes issue early enough to drain
  // before the barrier's lgkmcnt(0). Every instruction sits in its own gap
  // between MFMAs (the scheduling barriers hold the order).
  auto step = [&](int s, auto do_store, auto do_load) {
    constexpr bool kStore = decltype(do_store)::value;
    constexpr bool kLoad = decltype(do_load)::value;
    const int st = s & 1;
    const int nst = st ^ 1;
    unroll<4>([&](auto qq) {
      constexpr int q = decltype(qq)::value;
      constexpr int sl = q >> 1;
      constexpr int hh = q & 1;
      constexpr int abuf = q & 1;
      constexpr int bbuf = sl & 1;
      if constexpr (q == 3) {
        LTX25_LGKMCNT0();   // this wave's writes and reads done
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
      }
      unroll<16>([&](auto gg) {
        constexpr int g = decltype(gg)::value;
        constexpr int i = g / 4;
        constexpr int j = g % 4;
        acc[4 * hh + i][j] = mfma(bfr[bbuf][j], afr[abuf][i], acc[4 * hh + i][j]);
        if constexpr (q == 0 && g < 4) { rd_a(st, 0, 1, abuf ^ 1, g); }
        if constexpr (q == 0 && g >= 4 && g < 8) { rd_b(st, 1, 1, g - 4); }
        if constexpr (q == 1 && g < 4) { rd_a(st, 1, 0, abuf ^ 1, g); }
        if constexpr (q == 2 && g >= 8 && g < 12) { rd_a(st, 1, 1, abuf ^ 1, g - 8); }
        if constexpr (kStore && q == 3 && g < 4) { rd_a(nst, 0, 0, abuf ^ 1, g); }
        if constexpr (kStore && q == 3 && g >= 4 && g < 8) { rd_b(nst, 0, 0, g - 4); }
        // X writes at gaps 0, 2, 4, 6 of q2, reloads at 1, 3, 5, 7
        constexpr bool xwr_gap = g < 8 && (g & 1) == 0;
        constexpr bool xld_gap = g < 8 && (g & 1) == 1;
        constexpr int xi = g / 2;
        if constexpr (kStore && q == 2 && xwr_gap) { store_x(nst, xi); }
        if constexpr (kLoad && q == 2 && xld_gap) { load_x(s + 2, xi); }
        // row 0 dequantized in q0's second half, written in q1's first gaps;
        // row 1 dequantized in q1 gaps 4..11, written at 12 and 14; each
        // row's codes reloaded right after its writes
        if constexpr (kStore && q == 0 && g >= 8) { dq_pair(0, g - 8); }
        if constexpr (kStore && q == 1 && (g == 0 || g == 2)) { store_dq(nst, 0, g / 2); }
        if constexpr (kLoad && q == 1 && g == 1) { load_c(s + 2, 0); }
        if constexpr (kLoad && q == 1 && g == 3) { load_sb(s + 2, 0); }
        if constexpr (kStore && q == 1 && g >= 4 && g < 12) { dq_pair(1, g - 4); }
        if constexpr (kStore && q == 1 && (g == 12 || g == 14)) { store_dq(nst, 1, (g - 12) / 2); }
        if constexpr (kLoad && q == 1 && g == 13) { load_c(s + 2, 1); }
        if constexpr (kLoad && q == 1 && g == 15) { load_sb(s + 2, 1); }
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };
  // the last two steps are peeled: no loads past the end, no writes after it
  int s = 0;
  for (; s + 2 < nsteps; ++s) { step(s, std::true_type{}, std::true_type{}); }
  if (s + 1 < nsteps) {
    step(s, std::true_type{}, std::false_type{});
    ++s;
  }
  step(s, std::false_type{}, std::false_type{});
  __syncthreads();   // every wave is done reading the operand stages

  // epilogue (the accumulator layout of tall_kernel's)
  const int lrow = lane & 15;
  const int lcol = (lane >> 4) * 4;
  uint16_t* const stage = lds;
  // the GELU choice made once, outside the unrolled staging loop
  auto stage_tile = [&](auto gelu) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wn * 64 + j * 16 + lcol;
      const f32x4 b4 = *(const f32x4*)pad_at(480, c);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wm * 128 + i * 16 + lrow;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v[t] = acc[i][j][t] + b4[t];
          if constexpr (decltype(gelu)::value) { v[t] = gelu_tanh(v[t]); }
        }
        *(uint2*)(stage + r * kEP + c) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  };
  if (p.epilogue == kEpiGelu) {
    stage_tile(std::true_type{});
  } else {
    stage_tile(std::false_type{});
  }
  __syncthreads();
  constexpr int CPR = kBN / 8;
#pragma unroll 4
  for (int q = tid; q < kBM * CPR; q += kThreads) {
    const int r = q / CPR;
    const int c = (q % CPR) * 8;
    const int m = m0 + r;
    const int n = n0 + c;
    if (m >= p.M || n >= p.N) { continue; }
    const uint4 v = *(const uint4*)(stage + r * kEP + c);
    __builtin_nontemporal_store(__builtin_bit_cast(i32x4, v), (i32x4*)(p.y + (size_t)m * p.N + n));
  }
}

constexpr size_t kTwoGib = (size_t)1 << 31;
constexpr size_t kFourGib = (size_t)1 << 32;

hipError_t launch_tall(const TallParams& p, int mode, hipStream_t stream)
{
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
  if (p.stamps != nullptr) {
    // the phase-stamp instantiations (ltx25_probe_tall_phases)
    if (mode == kModeI8) {
      hipLaunchKernelGGL((tall_kernel<kModeI8, false, true>), grid, dim3(kThreads), 0, stream, p);
    } else if (mode == kModeBf16 && p.x2 == nullptr) {
      hipLaunchKernelGGL((tall_kernel<kModeBf16, false, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (mode == kModeI8) {
    hipLaunchKernelGGL((tall_kernel<kModeI8, false>), grid, dim3(kThreads), 0, stream, p);
  } else if (mode == kModeW8) {
    hipLaunchKernelGGL(tall_w8_kernel, grid, dim3(kThreads), 0, stream, p);
  } else if (p.x2 != nullptr) {
    hipLaunchKernelGGL((tall_kernel<kModeBf16, true>), grid, dim3(kThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((tall_kernel<kModeBf16, false>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

bool tall_dense_takes(const GemmDesc& d, const GemmPlan& plan)
{
  // The template keeps rows that are not whole 16-byte chunks and an
  // accumulating output beside the two-part activation or off 8-byte
  // alignment. The per-lane byte offsets are 32-bit, rows past the last
  // tile's end included.
  return plan.tile == 0 && plan.splits == 1 && d.bits == 16 &&
         (d.x2 == nullptr || (d.kx > 0 && d.kx < d.K && d.kx % kBK == 0)) &&
         (d.y_in == nullptr || (d.x2 == nullptr && ((uintptr_t)d.y_in & 7u) == 0)) &&
         d.N % 8 == 0 && d.K % kBK == 0 && d.K >= kBK &&
         (size_t)(d.M + kBM) * d.K * 2 < kFourGib && (size_t)(d.N + kBN) * d.K * 2 < kFourGib;
}

bool tall_w8_takes(const GemmDesc& d, const GemmPlan& plan)
{
  // w8 codes with groups of 64 or 32 on the 256 x 256 plan; the codes'
  // byte offsets are 32-bit like the activation's
  return plan.tile == 0 && plan.splits == 1 && d.bits == 8 && (d.group == 64 || d.group == 32) &&
         d.x2 == nullptr && d.y_in == nullptr && d.N % 8 == 0 && d.K % kBK == 0 && d.K >= kBK &&
         (size_t)(d.M + kBM) * d.K * 2 < kFourGib && (size_t)(d.N + kBN) * d.K < kFourGib;
}

hipError_t launch_tall_dense(const GemmDesc& d, hipStream_t stream, unsigned long long* stamps)
{
  if (d.bits == 8) {
    GemmPlan plan;
    plan.tile = 0;
    plan.splits = 1;
    if (d.M < 1 || !tall_w8_takes(d, plan) || (size_t)d.M * d.N * 2 >= kTwoGib) {
      return hipErrorInvalidValue;
    }
    TallParams p = {};
    p.x = d.x;
    p.w = d.w;
    p.scales = d.scales;
    p.qbias = d.qbias;
    p.gshift = d.group == 64 ? 6 : 5;
    p.gcols = d.K / d.group;
    p.bias = d.bias;
    p.y = d.y;
    p.M = d.M;
    p.N = d.N;
    p.K = d.K;
    p.wn = d.N;
    p.bias_type = d.bias != nullptr ? d.bias_type : kBiasNone;
    p.epilogue = d.epilogue;
    p.tiles_m = (d.M + kBM - 1) / kBM;
    p.tiles_n = (d.N + kBN - 1) / kBN;
    return launch_tall(p, kModeW8, stream);
  }
  if (d.M < 1 || d.N < 8 || d.N % 8 != 0 || d.K < kBK || d.K % kBK != 0 || d.bits != 16 ||
      (size_t)d.M * d.K * 2 >= kTwoGib || (size_t)d.N * d.K * 2 >= kTwoGib ||
      (size_t)d.M * d.N * 2 >= kTwoGib ||
      (d.x2 != nullptr && (d.kx <= 0 || d.kx >= d.K || d.kx % kBK != 0)) ||
      (d.y_in != nullptr && (d.x2 != nullptr || ((uintptr_t)d.y_in & 7u) != 0))) {
    return hipErrorInvalidValue;
  }
  TallParams p = {};
  p.x = d.x;
  p.x2 = d.x2;
  p.kx = d.x2 != nullptr ? d.kx : d.K;
  p.w = d.w;
  p.bias = d.bias;
  p.y = d.y;
  p.y_in = d.y_in;
  p.M = d.M;
  p.N = d.N;
  p.K = d.K;
  p.wn = d.wn > 0 && d.wn < d.N ? d.wn : d.N;
  p.bias_type = d.bias != nullptr ? d.bias_type : kBiasNone;
  p.epilogue = d.epilogue;
  p.tiles_m = (d.M + kBM - 1) / kBM;
  p.tiles_n = (d.N + kBN - 1) / kBN;
  p.stamps = stamps;
  return launch_tall(p, kModeBf16, stream);
}

bool tall_i8_takes(int M, int N, int K)
{
  // 128 of K per step; the same 32-bit offset bound as the bf16 mode
  return N % 8 == 0 && K % kSB == 0 && K >= kSB && (size_t)(M + kBM) * K < kFourGib &&
         (size_t)(N + kBN) * K < kFourGib;
}

hipError_t launch_tall_i8(const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                          const void* bias, int bias_type, int epilogue, uint16_t* y,
                          int32_t* acc, int M, int K, int N, hipStream_t stream,
                          unsigned long long* stamps)
{
  if (M < 1 || !tall_i8_takes(M, N, K) || (size_t)M * N * 2 >= kTwoGib) {
    return hipErrorInvalidValue;
  }
  TallParams p = {};
  p.x = xq;
  p.w = wq;
  p.sx = sx;
  p.sw = sw;
  p.acc_out = acc;
  p.bias = bias;
  p.y = y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.wn = N;
  p.bias_type = bias != nullptr ? bias_type : kBiasNone;
  p.epilogue = epilogue;
  p.tiles_m = (M + kBM - 1) / kBM;
  p.tiles_n = (N + kBN - 1) / kBN;
  p.stamps = stamps;
  return launch_tall(p, kModeI8, stream);
}

}  // namespace ltx25
