// The quantized linear for at most 128 tokens on gfx950 -- the audio
// stream's GEMMs (126 tokens) and any other call with M <= 128 whose weight
// needs at most 3 workgroups per CU (larger ones run on the 128 x 128 tile):
// y = x . dequant(W)^T (+ bias) (+ GELU) (+ y_in).
//
// At these shapes the activation slab X [M][K] is small (516 KB at
// K = 2048) and every XCD's L2 holds it after the first touch; the time is
// set by how fast each CU pulls X and its share of the weight. A 128-column
// tile with split-K reads 1/s of X per workgroup but writes s f32 partial
// outputs -- at 126 tokens as many bytes as the codes -- and needs a
// reduction launch. Here each workgroup owns a 32-column slice of the
// output and up to 2048 of K:
//   - the 8 waves split the workgroup's K into contiguous runs of 64-wide
//     chunks, so each X element and each weight code is read once per
//     workgroup;
//   - a chunk of X [128 rows][64] is loaded as 128-byte row segments
//     (8 lanes per row; a load instruction that touches 32 rows at 32 bytes
//     each moves 1.6x less per unit time from L2 on this GPU), written to
//     the wave's own LDS slot with an XOR swizzle and read back as MFMA
//     fragments: LDS is a transpose buffer, private to the wave, so the
//     K loop has no barriers;
//   - the wave's codes [32 rows][its K run] arrive once, as 256-byte (w8)
//     or 128-byte (w4) row segments, through the same slot, and stay in
//     registers; each chunk dequantizes its fragments in registers,
//     w = bf16(fma(scale, q, qbias)), the rule of every other route;
//     a dense bf16 weight (bits 16: unquantized checkpoints and the
//     dequant-once arm) is loaded per chunk straight into the fragment
//     layout, so both arms of that A/B switch sum in the same order;
//   - v_mfma_f32_32x32x16_bf16, weight fragment first, f32 accumulation;
//   - the 8 per-wave partial tiles are summed through LDS in wave order,
//     then bias, y_in and GELU-tanh in f32 and one rounding to bf16.
// With K > 2048 the workgroups split K (ceil(K / 2048) ways) and write f32
// partials that the split-K reduction sums in split order.
//
// Lane mapping of a chunk starting at k0: MFMA s (0..3) takes, in lane half
// h = lane / 32, the K values k0 + 32 h + 8 s + 0..7. Both operands use the
// same assignment, so the dot products are unchanged, and a lane's 32 codes
// of a chunk are one contiguous run.
//
// Reference semantics: MetalOps::linear(QWeight) (src/ltx25-metal-ops.cc:
// 531-569), the qmm route it takes below the matrix-core threshold
// (:550-564) included.
#include "common.h"

namespace ltx25 {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kCols = 32;            // output columns per workgroup
constexpr int kChunk = 64;           // K per chunk
constexpr int kMaxChunks = 4;        // chunks per wave: 2048 of K per workgroup
constexpr int kRows = 128;           // token rows (M <= 128)
constexpr int kMaxGroups = kWaves * kMaxChunks * kChunk / 32;   // groups per workgroup (g32)
// Per-wave LDS slot: the X chunk (128 rows x 128 B), the wave's codes
// (32 rows x 256 B at most) and, after the K loop, the wave's partial tile
// as 16 f32x4 runs of 64 lanes, each run padded to 68 entries so that the
// reduction's reads are conflict-free.
constexpr int kRedPitch = 68;
constexpr int kSlotBytes = 16 * kRedPitch * 16;   // 17408 >= 16384
constexpr int kUnitBytes = 64 * 128;              // X unit: 64 rows x 128 B
constexpr uint32_t kOob = 0x80000000u;            // past every buffer's range

typedef uint32_t __attribute__((address_space(3))) lds_u32;

struct SParams {
  const uint16_t* x;
  const uint8_t* wq;
  const uint16_t* scales;
  const uint16_t* qbias;
  const void* bias;
  const uint16_t* y_in;
  uint16_t* y;
  float* partial;           // [splits][M][N] when split
  int M, N, K;
  int gshift, gcols;
  int k_chunk;              // K per workgroup (multiple of 64)
  int bias_type, epilogue;
  // the phase-stamp build only (STAMPS): 10 words per wave, see below
  unsigned long long* stamps;
};

// Phase stamps (the STAMPS instantiation, for ltx25_probe_skinny_phases):
// the shader clock at a phase boundary, with the scheduler held on both
// sides so that the read stays where the source puts it.
#define LTX25_STAMP(var)                 \
  if constexpr (STAMPS) {                \
    __builtin_amdgcn_sched_barrier(0);   \
    var = __builtin_amdgcn_s_memtime();  \
    __builtin_amdgcn_sched_barrier(0);   \
  }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, size_t bytes)
{
  // loads at offsets past `bytes` return zeros (rows past M and N)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)(uint32_t)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
  const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

// Eight codes -> eight bf16 weights, w = bf16(fma(s, q, b)). w8: bytes of
// (lo, hi) in order; w4: the nibbles of `lo` in order (code c at bits 4c).
template <int BITS>
__device__ __forceinline__ bf16x8 dequant8(uint32_t lo, uint32_t hi, float s, float b)
{
  uint32_t o[4];
  if constexpr (BITS == 8) {
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      o[2 * j] = pack_bf16x2(fmaf(s, (float)(w[j] & 0xffu), b),
                             fmaf(s, (float)((w[j] >> 8) & 0xffu), b));
      o[2 * j + 1] = pack_bf16x2(fmaf(s, (float)((w[j] >> 16) & 0xffu), b),
                                 fmaf(s, (float)(w[j] >> 24), b));
    }
  } else {
    const uint32_t ev = lo & 0x0f0f0f0fu;          // codes 0, 2, 4, 6
    const uint32_t od = (lo >> 4) & 0x0f0f0f0fu;   // codes 1, 3, 5, 7
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      o[t] = pack_bf16x2(fmaf(s, (float)((ev >> (8 * t)) & 0xffu), b),
                         fmaf(s, (float)((od >> (8 * t)) & 0xffu), b));
    }
  }
  return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

template <int BITS, bool SPLIT, bool STAMPS = false>
__global__ void __launch_bounds__(kThreads)
skinny_kernel(SParams p)
{
  constexpr bool QUANT = BITS != 16;
  static_assert(2 * kUnitBytes <= kSlotBytes, "slot too small");

  __shared__ __attribute__((aligned(16))) uint8_t lds[kWaves * kSlotBytes];
  __shared__ float lds_bias[kCols];
  // the workgroup's scales and zero points [32 rows][groups of its K range]
  __shared__ uint16_t lds_sq[2][kCols * kMaxGroups];

  // phase stamps: shader clock at entry, codes in registers, scale block in
  // LDS, K loop done, partials summed, stores done; 100 MHz clock at entry
  // and at the end
  unsigned long long st[6] = {0, 0, 0, 0, 0, 0};
  unsigned long long rt0 = 0;
  if constexpr (STAMPS) {
    __builtin_amdgcn_sched_barrier(0);
    rt0 = __builtin_amdgcn_s_memrealtime();
  }
  LTX25_STAMP(st[0])

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (an SGPR): the LDS base of a direct-to-LDS load and every
  // buffer soffset below must be
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int l32 = lane & 31;
  uint8_t* const slot = lds + wave * kSlotBytes;

  const int n0 = blockIdx.x * kCols;
  const int split = SPLIT ? (int)blockIdx.y : 0;
  const int kbeg = split * p.k_chunk;
  const int nch = (min(p.K, kbeg + p.k_chunk) - kbeg) / kChunk;
  const int c_lo = nch * wave / kWaves;
  const int cnt = nch * (wave + 1) / kWaves - c_lo;  // 0..4 chunks for this wave
  const int kw0 = kbeg + c_lo * kChunk;

  if constexpr (!SPLIT) {
    if (tid < kCols) {
      const int n = n0 + tid;
      lds_bias[tid] = n < p.N ? load_bias(p.bias, p.bias_type, n) : 0.0f;
    }
  }

  const size_t wrow_bytes = (size_t)p.K * BITS / 8;   // bits 16: bf16 rows
  const __amdgpu_buffer_rsrc_t xr = rsrc(p.x, (size_t)p.M * p.K * 2);
  const __amdgpu_buffer_rsrc_t wr = rsrc(p.wq, (size_t)p.N * wrow_bytes);
  const __amdgpu_buffer_rsrc_t sr = rsrc(p.scales, (size_t)p.N * p.gcols * 2);
  const __amdgpu_buffer_rsrc_t qr = rsrc(p.qbias, (size_t)p.N * p.gcols * 2);

  // ---- the wave's weight, all chunks, in the fragment layout: lane (row
  // l32, half h) holds the codes of K values k0 + 32 h + 0..31 of each chunk
  // (32 B for w8, 16 B for w4, 64 B of bf16 for a dense weight). Chunks
  // past this wave's run load nothing (an offset past the buffer). Codes
  // arrive as whole row runs and are transposed through LDS (below); a
  // dense weight is loaded in the fragment layout directly.
  constexpr int WQ = QUANT ? (BITS == 8 ? 2 : 1) : 4;   // 16-byte loads per lane per chunk
  uint4 wv[kMaxChunks][WQ];
  // per-lane part of the offsets (row, half) in voffset, the chunk's K in soffset
  const uint32_t w_row = (uint32_t)((size_t)(n0 + l32) * wrow_bytes + 32 * h * BITS / 8);
  auto load_w = [&](int t) {
    const uint32_t kb = (uint32_t)((size_t)(kw0 + t * kChunk) * BITS / 8);
#pragma unroll
    for (int j = 0; j < WQ; ++j) { wv[t][j] = ld16(wr, t < cnt ? w_row + 16 * j : kOob, kb); }
  };
  // The workgroup's scale and zero-point block, [32 rows][ng groups], read
  // as contiguous row runs (consecutive threads, consecutive groups) and
  // staged in LDS: one 2-byte load per lane per row would touch 32 cache
  // lines per instruction.
  const int g_lo = kbeg >> p.gshift;
  const int ng = (nch * kChunk) >> p.gshift;
  constexpr int kSqLoads = kCols * kMaxGroups / kThreads;
  uint16_t sqv[2][kSqLoads];
  if constexpr (QUANT) {
#pragma unroll
    for (int i = 0; i < kSqLoads; ++i) {
      const int e = tid + i * kThreads;
      const int r = e / kMaxGroups;
      const int g = e % kMaxGroups;
      const uint32_t off =
          g < ng ? (uint32_t)(((size_t)(n0 + r) * p.gcols + g) * 2) : kOob;
      sqv[0][i] = __builtin_amdgcn_raw_buffer_load_b16(sr, (int)off, g_lo * 2, 0);
      sqv[1][i] = __builtin_amdgcn_raw_buffer_load_b16(qr, (int)off, g_lo * 2, 0);
    }
  }

  // ---- X: units of 64 rows x 64 K (8 KB: rows 64 hf.. of chunk t, u = 2t + hf),
  // loaded straight into LDS (buffer_load ... lds) through a 2-unit ring in
  // the wave's slot. One 1 KB load covers rows 8 i..8 i+7 of the unit; lane l
  // lands at byte 16 l of it (row 8 i + l / 8, position l % 8) and fetches the
  // row's 16-byte segment (l % 8) ^ ((row / 2) % 8), the swizzle that keeps
  // the fragment reads conflict-free. Rows past M read as zeros.
  const int nunits = 2 * cnt;
  auto load_unit = [&](int u) {
    const int t = u >> 1;
    const int hf = u & 1;
    lds_u32* dst = (lds_u32*)(slot + (u & 1) * kUnitBytes);
    const uint32_t soff = (uint32_t)(kw0 + t * kChunk) * 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r0 = 64 * hf + 8 * i;              // first row of this load
      // row r0 + l/8: swizzle (r/2) % 8 = (4 i + l/16) % 8 (r0 is a multiple of 8)
      const int sw = ((4 * i) + (lane >> 4)) & 7;
      const uint32_t vo = (uint32_t)((size_t)(r0 + (lane >> 3)) * p.K * 2 +
                                     (((lane & 7) ^ sw) * 16));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst + i * 256, 16, (int)vo, (int)soff, 0, 0);
    }
  };

  f32x16 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[mb][r] = 0.0f; }
  }

  // X unit 0 (L2) and the weight (HBM) are in flight together, and the
  // weight has landed before the K loop starts, so that the loop has no
  // loads into registers outstanding. (The compiler's wait counting does not
  // see direct-to-LDS loads: a register load still in flight inside the loop
  // would make it wait for the X units issued after it as well.)
  if (nunits > 0) { load_unit(0); }
  if constexpr (QUANT) {
    // The codes [32 rows][cnt * WB bytes] as WLPR 16-byte runs per row
    // (256 B per row for w8, 128 B for w4: a load instruction covers whole
    // rows), then through unit 1's LDS region, XOR-swizzled by row so that
    // both the writes and the fragment reads are conflict-free.
    constexpr int WB = kChunk * BITS / 8;
    constexpr int WROW = kMaxChunks * WB;
    constexpr int WLPR = WROW / 16;
    constexpr int WRPI = 64 / WLPR;
    constexpr int WNI = 32 / WRPI;
    static_assert(32 * WROW <= kUnitBytes, "the codes must fit one X unit region");
    const int c16 = lane % WLPR;
    uint4 wl[WNI];
#pragma unroll
    for (int i = 0; i < WNI; ++i) {
      const int r = i * WRPI + lane / WLPR;
      const uint32_t off = c16 * 16 < cnt * WB
                               ? (uint32_t)((size_t)(n0 + r) * wrow_bytes + c16 * 16)
                               : kOob;
      wl[i] = ld16(wr, off, (uint32_t)((size_t)kw0 * BITS / 8));
    }
    uint8_t* const wst = slot + kUnitBytes;
#pragma unroll
    for (int i = 0; i < WNI; ++i) {
      const int r = i * WRPI + lane / WLPR;
      const int sw = BITS == 8 ? (r & 15) : ((r >> 1) & 7);
      *(uint4*)(wst + r * WROW + ((c16 ^ sw) * 16)) = wl[i];
    }
    const int sw = BITS == 8 ? (l32 & 15) : ((l32 >> 1) & 7);
#pragma unroll
    for (int t = 0; t < kMaxChunks; ++t) {
#pragma unroll
      for (int j = 0; j < WQ; ++j) {
        const int s16 = (t * WB + 32 * h * BITS / 8) / 16 + j;
        wv[t][j] = *(const uint4*)(wst + l32 * WROW + ((s16 ^ sw) * 16));
      }
    }
    // the region is unit 1's: its reads have returned before unit 1 lands
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    LTX25_STAMP(st[1])
  } else {
    // The empty asm statements are the weight's first use, and so the point
    // where the compiler waits for it.
#pragma unroll
    for (int t = 0; t < kMaxChunks; ++t) { load_w(t); }
#pragma unroll
    for (int t = 0; t < kMaxChunks; ++t) {
#pragma unroll
      for (int j = 0; j < WQ; ++j) {
        i32x4 v = __builtin_bit_cast(i32x4, wv[t][j]);
        asm volatile("" : "+v"(v));
        wv[t][j] = __builtin_bit_cast(uint4, v);
      }
    }
  }
  if (nunits > 1) { load_unit(1); }
  if constexpr (QUANT) {
#pragma unroll
    for (int i = 0; i < kSqLoads; ++i) {
      const int e = tid + i * kThreads;
      lds_sq[0][e] = sqv[0][i];
      lds_sq[1][e] = sqv[1][i];
    }
  }
  __syncthreads();   // the scale block is in LDS
  LTX25_STAMP(st[2])

  // fragment reads: unit row 32 j + l32 (block mb = 2 hf + j), 16-byte
  // segment 4 h + s, stored at (4 h + s) ^ ((l32 / 2) % 8)
  const int fsw = (l32 >> 1) & 7;
  bf16x8 wf[4];   // the current chunk's weight fragments
#pragma unroll
  for (int u = 0; u < 2 * kMaxChunks; ++u) {
    if (u < nunits) {
      const int t = u >> 1;
      const int hf = u & 1;
      // Unit u has landed once at most unit u+1's 8 loads are outstanding
      // (loads complete in issue order).
      if (u + 1 < nunits) {
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      const uint8_t* src = slot + (u & 1) * kUnitBytes;
      bf16x8 xf[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
          xf[j][sp] = *(const bf16x8*)(src + (32 * j + l32) * 128 + (((4 * h + sp) ^ fsw) * 16));
        }
      }
      // the slot is free once the reads have returned; refill it with unit u+2
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (u + 2 < nunits) { load_unit(u + 2); }
      if (hf == 0) {
        // dequantize chunk t (group of K value k0 + 32 h, relative to the
        // workgroup's first group); VALU work under the X stream
        const int gi = l32 * kMaxGroups + ((kw0 + t * kChunk + 32 * h) >> p.gshift) - g_lo;
        const float sc = QUANT ? bf16_to_f32(lds_sq[0][gi]) : 0.0f;
        const float qb = QUANT ? bf16_to_f32(lds_sq[1][gi]) : 0.0f;
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
          if constexpr (!QUANT) {
            wf[sp] = __builtin_bit_cast(bf16x8, wv[t][sp]);
          } else if constexpr (BITS == 8) {
            const uint4 c = wv[t][sp >> 1];
            wf[sp] = dequant8<8>((sp & 1) ? c.z : c.x, (sp & 1) ? c.w : c.y, sc, qb);
          } else {
            const uint4 c = wv[t][0];
            const uint32_t v = sp == 0 ? c.x : sp == 1 ? c.y : sp == 2 ? c.z : c.w;
            wf[sp] = dequant8<4>(v, 0u, sc, qb);
          }
        }
      }
#pragma unroll
      for (int sp = 0; sp < 4; ++sp) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[2 * hf + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[sp], xf[j][sp],
                                                                    acc[2 * hf + j], 0, 0, 0);
        }
      }
    }
  }
  // every wave is done reading its X slots before the slots hold partial tiles
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  LTX25_STAMP(st[3])

  // ---- the 8 partial tiles, summed through LDS in wave order. Block mb,
  // registers 4g..4g+3 of lane l: row 32 mb + l % 32, columns
  // 8 g + 4 (l / 32) + 0..3 of the slice.
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 v = {acc[mb][4 * g], acc[mb][4 * g + 1], acc[mb][4 * g + 2], acc[mb][4 * g + 3]};
      *(f32x4*)(slot + ((mb * 4 + g) * kRedPitch + lane) * 16) = v;
    }
  }
  __syncthreads();
  LTX25_STAMP(st[4])

  // thread -> row m (0..127), 8 columns 8 nq .. 8 nq + 7
  const int m = tid >> 2;
  const int nq = tid & 3;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) { v[j] = 0.0f; }
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const f32x4 a = *(const f32x4*)(lds + w * kSlotBytes +
                                      (((m >> 5) * 4 + nq) * kRedPitch + (m & 31) + 32 * hh) * 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[4 * hh + j] += a[j]; }
    }
  }
  if (m < p.M) {
    const int n = n0 + 8 * nq;
    if constexpr (SPLIT) {
      float* prow = p.partial + ((size_t)split * p.M + m) * p.N;
      if ((p.N & 3) == 0 && n + 8 <= p.N) {
        *(f32x4*)(prow + n) = f32x4{v[0], v[1], v[2], v[3]};
        *(f32x4*)(prow + n + 4) = f32x4{v[4], v[5], v[6], v[7]};
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (n + j < p.N) { prow[n + j] = v[j]; }
        }
      }
    } else {
      const uint16_t* yin = p.y_in != nullptr ? p.y_in + (size_t)m * p.N : nullptr;
      uint16_t* yrow = p.y + (size_t)m * p.N;
      const bool vec = (p.N & 7) == 0 && n + 8 <= p.N;
      if (yin != nullptr) {
        if (vec) {
          const uint4 o = *(const uint4*)(yin + n);
          const uint32_t e[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[2 * j] += __uint_as_float(e[j] << 16);
            v[2 * j + 1] += __uint_as_float(e[j] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (n + j < p.N) { v[j] += bf16_to_f32(yin[n + j]); }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] += lds_bias[8 * nq + j];
        if (p.epilogue == kEpiGelu) { v[j] = gelu_tanh(v[j]); }
      }
      if (vec) {
        *(uint4*)(yrow + n) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                         pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (n + j < p.N) { yrow[n + j] = f32_to_bf16(v[j]); }
        }
      }
    }
  }
  if constexpr (STAMPS) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the stores have completed
    LTX25_STAMP(st[5])
    const unsigned long long rt1 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
    if (p.stamps != nullptr && lane == 0) {
      // HW_ID (CU, SH, SE of this wave) and XCC_ID, read from the hardware registers
      const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
      const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
      unsigned long long* o =
          p.stamps + ((size_t)(blockIdx.y * gridDim.x + blockIdx.x) * kWaves + wave) * 10;
#pragma unroll
      for (int i = 0; i < 6; ++i) { o[i] = st[i]; }
      o[6] = rt0;
      o[7] = rt1;
      o[8] = hw;
      o[9] = xcc;
    }
  }
}

}  // namespace

bool plan_skinny(int M, int N, int K, int bits, int cu_count, GemmPlan& plan)
{
  constexpr size_t kTwoGib = (size_t)1 << 31;
  if (M < 1 || M > kRows || (bits != 8 && bits != 4 && bits != 16) || K < kChunk ||
      K % kChunk != 0 || N < 1 || (size_t)kRows * K * 2 >= kTwoGib ||
      (size_t)N * K * bits / 8 >= kTwoGib || (size_t)M * N * 2 >= kTwoGib) {
    return false;
  }
  const int chunks = K / kChunk;
  constexpr int kPerGroup = kWaves * kMaxChunks;
  int s = (chunks + kPerGroup - 1) / kPerGroup;
  const int per = (chunks + s - 1) / s;
  s = (chunks + per - 1) / per;
  // Every 32-column workgroup reads all of X from L2: past about three
  // workgroups per CU (a large N x K weight) that stream costs more than the
  // 128 x 128 tile's partials (measured, M = 16..126: that tile is faster
  // from 1024 workgroups, e.g. 62 vs 72 us at K = 4096, N = 16384).
  if ((long)((N + kCols - 1) / kCols) * s > 3L * cu_count) { return false; }
  plan.tile = 2;
  plan.splits = s;
  plan.k_chunk = per * kChunk;
  plan.workspace_bytes = s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
  return true;
}

hipError_t launch_skinny(const GemmDesc& d, const GemmPlan& plan, float* workspace,
                         hipStream_t stream, unsigned long long* stamps)
{
  if (plan.tile != 2 || d.M < 1 || d.M > kRows || (d.bits != 8 && d.bits != 4 && d.bits != 16) ||
      (stamps != nullptr && d.bits != 8) || d.K % kChunk != 0 ||
      plan.k_chunk % kChunk != 0 || plan.k_chunk > kWaves * kMaxChunks * kChunk ||
      (long)plan.splits * plan.k_chunk < d.K || (plan.splits > 1 && workspace == nullptr)) {
    return hipErrorInvalidValue;
  }
  SParams p = {};
  p.x = d.x;
  p.wq = (const uint8_t*)d.w;
  p.scales = d.scales;
  p.qbias = d.qbias;
  p.bias = d.bias;
  p.bias_type = d.bias != nullptr ? d.bias_type : kBiasNone;
  p.epilogue = d.epilogue;
  p.y_in = d.y_in;
  p.y = d.y;
  p.partial = workspace;
  p.M = d.M;
  p.N = d.N;
  p.K = d.K;
  int gs = 0;
  while ((1 << gs) < d.group) { ++gs; }
  p.gshift = d.bits == 16 ? 0 : gs;
  p.gcols = d.bits == 16 ? 0 : d.K / d.group;
  p.k_chunk = plan.k_chunk;
  p.stamps = stamps;
  const dim3 grid((unsigned)((d.N + kCols - 1) / kCols), (unsigned)plan.splits, 1);
  const bool split = plan.splits > 1;
  if (stamps != nullptr) {
    // the phase-stamp instantiation (w8 only), for the probe entry point
    if (split) {
      hipLaunchKernelGGL((skinny_kernel<8, true, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((skinny_kernel<8, false, true>), grid, dim3(kThreads), 0, stream, p);
    }
  } else if (d.bits == 8) {
    if (split) {
      hipLaunchKernelGGL((skinny_kernel<8, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((skinny_kernel<8, false>), grid, dim3(kThreads), 0, stream, p);
    }
  } else if (d.bits == 16) {
    if (split) {
      hipLaunchKernelGGL((skinny_kernel<16, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((skinny_kernel<16, false>), grid, dim3(kThreads), 0, stream, p);
    }
  } else {
    if (split) {
      hipLaunchKernelGGL((skinny_kernel<4, true>), grid, dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((skinny_kernel<4, false>), grid, dim3(kThreads), 0, stream, p);
    }
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split) { return e; }
  return launch_splitk_reduce(workspace, plan.splits, d.bias, p.bias_type, d.epilogue, d.y_in,
                              d.y, d.M, d.N, stream);
}

}  // namespace ltx25
