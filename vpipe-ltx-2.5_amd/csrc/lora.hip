// The low-rank adapter delta on gfx950: y[M][N] += (x[M][K] . A^T) . B^T,
// with A bf16 [rank][K] and B bf16 [N][rank] in the [out][in] order every
// weight here uses.
//
// Replaces MetalOps::lora_add (src/ltx25-metal-ops.cc:989-1004) and its
// matrix-core pair lora_mma_ (:940-987). The reference's portable form is
// three passes (linear into r, linear into d, add d into y) and its
// matrix-core pair two (r, then an accumulate into y). Here it is ONE
// kernel per 32-token row block:
//
//   phase 1  r[32][rank] = bf16(x . A^T). The four waves split K and add
//            their f32 partials through LDS in wave order (deterministic),
//            and the last wave rounds r to bf16 into LDS, as the reference
//            rounds r into its bf16 scratch.
//   phase 2  y = bf16(f32(y) + r . B^T) for the workgroup's columns: the
//            accumulator is seeded from y and stored once, so the delta is
//            never materialised (the reference's `_acc` tile does the same).
//
// Both phases run v_mfma_f32_32x32x16_bf16 in the transposed form
// (C = A_frag . x_frag^T, then C = B_frag . r_frag^T) so the accumulator
// holds four consecutive output columns per lane and y moves as 8-byte
// vectors. Phase 2 streams y once in and once out; x is read once per
// column split and A, B stay L2-resident.
//
// The rank handled by one launch is at most kLoraMaxRank; the host runs a
// larger adapter as several launches over column slices of A and B.
//
// With many tokens the host computes r = bf16(x . A^T) once with the dense
// GEMM instead (phase 1 here re-reads x and all of A for every column split
// of a row block) and the kernel runs phase 2 only, reading its 32 rows of
// r from that buffer (`r_in`, [M][rank], rank % 8 == 0).

#include <type_traits>

#include "common.h"

namespace ltx25 {
namespace {

constexpr int kLoraRows = 32;
constexpr int kLoraWaves = 4;
constexpr int kLoraThreads = kLoraWaves * 64;
constexpr int kYsRow = 128 + 8;   // bf16 per row of a y staging tile (16 B pad)

struct LoraParams {
  const uint16_t* r_in;  // precomputed r [M][rank] (phase 2 only), or null
  const uint16_t* x;
  const uint16_t* a;  // this pass's first row of A
  const uint16_t* b;  // this pass's first column of B
  uint16_t* y;
  int M, K, N;
  int rank;     // adapter columns in this pass, <= kLoraMaxRank
  int ldb;      // row stride of B in elements (the adapter's full rank)
  int n_split;  // columns of y per workgroup along grid.y, multiple of 32
};

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer resource over `bytes` bytes: a load at an offset past the end
// returns zeros and a store there is dropped, so out-of-range lanes need no
// branch (a branch around a load makes the compiler wait for every
// outstanding load where the paths join, which would drain the pipelines
// below). Offsets are 32-bit: the host takes this path only for operands
// under 2 GiB.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, size_t bytes)
{
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)(uint32_t)bytes, 0x00020000);
}

// Eight bf16 of row `row`, columns k..k+7, of a row-major matrix with
// `rows` x `cols` valid elements and row stride `ld`; zero outside.
// Vector form: cols % 8 == 0 and 16-byte aligned rows, so a chunk is
// wholly inside or wholly outside; one 16-byte buffer load.
__device__ __forceinline__ bf16x8 frag8v(__amdgpu_buffer_rsrc_t r, int row, int rows, int k,
                                         int cols, int ld)
{
  const uint32_t off = (row < rows && k < cols) ? (uint32_t)(row * ld + k) * 2u : kOob;
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Element-wise form for any shape and 2-byte alignment.
__device__ __forceinline__ bf16x8 frag8s(const uint16_t* p, int row, int rows, int k, int cols,
                                         long ld)
{
  i32x4 v = {0, 0, 0, 0};
  if (row < rows) {
    const uint16_t* q = p + (size_t)row * ld;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (k + 2 * i < cols) ? q[k + 2 * i] : 0u;
      const uint32_t hi = (k + 2 * i + 1 < cols) ? q[k + 2 * i + 1] : 0u;
      v[i] = (int)(lo | (hi << 16));
    }
  }
  return __builtin_bit_cast(bf16x8, v);
}

// RB = 32-column blocks of rank this instance covers (rank <= 32 * RB);
// PRE_R: r comes from p.r_in instead of phase 1.
template <int RB, bool VEC, bool PRE_R>
__global__ __launch_bounds__(kLoraThreads) void lora_kernel(LoraParams p)
{
  constexpr int RP = 32 * RB;        // rank padded to the MFMA block
  constexpr int RS = RP + 8;         // bf16 per LDS row of r (16-byte pad)
  constexpr int FS = RP + 4;         // f32 per LDS row of the partials
  __shared__ __attribute__((aligned(16))) float red[RB >= 4 ? 4 : kLoraRows * FS];
  __shared__ __attribute__((aligned(16))) uint16_t rl[kLoraRows * RS];
  // per-wave y staging tiles of the vector path (unused by the other)
  __shared__ __attribute__((aligned(16))) uint16_t ystage[VEC ? kLoraWaves * kLoraRows * kYsRow : 8];

  const int lane = threadIdx.x & 63;
  // wave-uniform (an SGPR), so that the loop bounds below are too
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int m0 = blockIdx.x * kLoraRows;
  const auto rx = rsrc(p.x, (size_t)p.M * p.K * 2);
  const auto ra = rsrc(p.a, (size_t)p.rank * p.K * 2);
  const auto rbm = rsrc(p.b, ((size_t)(p.N - 1) * p.ldb + ((p.rank + 7) & ~7)) * 2);
  const auto ry = rsrc(p.y, (size_t)p.M * p.N * 2);
  auto xfrag = [&](int k) {
    if constexpr (VEC) { return frag8v(rx, m0 + l32, p.M, k, p.K, p.K); }
    else { return frag8s(p.x, m0 + l32, p.M, k, p.K, p.K); }
  };
  auto afrag = [&](int rb, int k) {
    if constexpr (VEC) { return frag8v(ra, rb * 32 + l32, p.rank, k, p.K, p.K); }
    else { return frag8s(p.a, rb * 32 + l32, p.rank, k, p.K, p.K); }
  };

  if constexpr (PRE_R) {
    // r's rows m0..m0+31, columns 0..RP-1 (zero past rank and M) -> rl, as
    // 16-byte chunks: rank % 8 == 0, so a chunk is wholly inside or outside
    const auto rr = rsrc(p.r_in, (size_t)p.M * p.rank * 2);
    constexpr int kCh = RP / 8;
    for (int e = threadIdx.x; e < kLoraRows * kCh; e += kLoraThreads) {
      const int row = e / kCh;
      const int col = (e % kCh) * 8;
      const uint32_t off = (m0 + row < p.M && col < p.rank)
                               ? (uint32_t)((m0 + row) * p.rank + col) * 2u
                               : kOob;
      *(i32x4*)(rl + row * RS + col) = __builtin_amdgcn_raw_buffer_load_b128(rr, (int)off, 0, 0);
    }
    __syncthreads();
  } else {
    // ---- phase 1: r^T[i][m] = sum_k A[i][k] x[m][k] ---------------------------
    // Narrow adapters (RB < 4) split K over the four waves and add the
    // partials through LDS in wave order; wide ones split the rank blocks
    // (RB / 4 per wave, each over all of K), so every wave owns its columns of
    // r and no reduction is needed. Either way the K steps of 16 run through
    // a ring of D1 register slots: slot d holds one step's fragments and is
    // refilled with the step D1 ahead as soon as its MFMAs have been issued.
    // A step past the end loads zeros (k = K is outside every row) and its
    // MFMAs add zeros: the ring's body has no exit, so the compiler's waits
    // stay one slot deep (an early exit from the body made it drain every
    // load before each MFMA).
    constexpr bool kRankSplit = RB >= 4;
    constexpr int RBW = kRankSplit ? RB / kLoraWaves : RB;   // rank blocks per wave
    constexpr int D1 = kRankSplit ? 4 : 8 / RB;
    const int rb0 = kRankSplit ? wave * RBW : 0;
    f32x16 acc[RBW];
  #pragma unroll
    for (int rb = 0; rb < RBW; ++rb) {
  #pragma unroll
      for (int r = 0; r < 16; ++r) { acc[rb][r] = 0.0f; }
    }
    const int steps = (p.K + 15) / 16;
    const int nloc = kRankSplit ? steps : (steps - wave + kLoraWaves - 1) / kLoraWaves;
    auto kstep = [&](int j) {
      if (j >= nloc) { return p.K; }
      return (kRankSplit ? j : wave + j * kLoraWaves) * 16 + hi * 8;
    };
    bf16x8 xf[D1];
    bf16x8 af[D1][RBW];
  #pragma unroll
    for (int d = 0; d < D1; ++d) {
      const int k = kstep(d);
      xf[d] = xfrag(k);
  #pragma unroll
      for (int rb = 0; rb < RBW; ++rb) { af[d][rb] = afrag(rb0 + rb, k); }
    }
    for (int j0 = 0; j0 < nloc; j0 += D1) {
  #pragma unroll
      for (int d = 0; d < D1; ++d) {
        const int kn = kstep(j0 + d + D1);
        const bf16x8 xc = xf[d];
        xf[d] = xfrag(kn);
  #pragma unroll
        for (int rb = 0; rb < RBW; ++rb) {
          acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[d][rb], xc, acc[rb], 0, 0, 0);
          af[d][rb] = afrag(rb0 + rb, kn);
        }
      }
    }

    // Lane l, register r of block rb holds r^T[i][m] with m = l & 31 and
    // i = 32 rb + 8 (r / 4) + 4 (l / 32) + r % 4; r lands in rl[m][i] as bf16.
    auto put_r = [&](int rb, int g, f32x4 v) {
      uint2 o;
      o.x = pack_bf16x2(v[0], v[1]);
      o.y = pack_bf16x2(v[2], v[3]);
      *(uint2*)(rl + l32 * RS + rb * 32 + g * 8 + hi * 4) = o;
    };
    if constexpr (kRankSplit) {
  #pragma unroll
      for (int rb = 0; rb < RBW; ++rb) {
  #pragma unroll
        for (int g = 0; g < 4; ++g) {
          put_r(rb0 + rb, g, f32x4{acc[rb][4 * g], acc[rb][4 * g + 1], acc[rb][4 * g + 2],
                                   acc[rb][4 * g + 3]});
        }
      }
      __syncthreads();
    } else {
      // waves add in order 0..3 through LDS; the last rounds to bf16
      for (int w = 0; w < kLoraWaves; ++w) {
        if (wave == w) {
  #pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
  #pragma unroll
            for (int g = 0; g < 4; ++g) {
              float* dst = red + l32 * FS + rb * 32 + g * 8 + hi * 4;
              f32x4 v = {acc[rb][4 * g], acc[rb][4 * g + 1], acc[rb][4 * g + 2],
                         acc[rb][4 * g + 3]};
              if (w > 0) { v += *(const f32x4*)dst; }
              if (w < kLoraWaves - 1) {
                *(f32x4*)dst = v;
              } else {
                put_r(rb, g, v);
              }
            }
          }
        }
        __syncthreads();
      }
    }
  }

  // ---- phase 2: y^T[n][m] = y^T[n][m] + sum_j B[n][j] r[m][j] -----------
  const int ksteps = (p.rank + 15) / 16;
  const int row = m0 + l32;
  const bool row_ok = row < p.M;
  const int n_lo = blockIdx.y * p.n_split;
  const int n_hi = min(p.N, n_lo + p.n_split);
  uint16_t* yrow = p.y + (size_t)row * p.N;
  if constexpr (VEC) {
    // Super blocks of 128 columns (four 32-column MFMA blocks), dealt
    // round-robin to the waves. A super block's y tile (32 rows x 256 B)
    // moves between HBM and a per-wave LDS tile as whole row segments (16
    // lanes per row, 16 B each) and between LDS and the accumulators in the
    // MFMA layout. Its HBM loads are issued kDy super blocks ahead. B's
    // fragments rotate per 32-column block: slot s is refilled with the
    // next block's rank step s as soon as its MFMA has been issued.
    constexpr int KS = 2 * RB;                      // 16-deep rank steps
    constexpr int kSb = 4;                          // MFMA blocks per super block
    constexpr int kSbStride = kLoraWaves * kSb * 32;
    // Four super blocks of y in flight for ranks up to 64 (5-7 us less on
    // an 8160 x 16384 y at ranks 8-64); above that the two extra slots'
    // 32 VGPRs each would halve the waves per SIMD, so two.
    constexpr int kDy = RB <= 2 ? 4 : 2;
    // B's rows are zero-padded to a multiple of 8 (the host pads a copy when
    // the adapter's rank is not), so an 8-column chunk below rank8 is whole.
    const int rank8 = (p.rank + 7) & ~7;
    uint16_t* ys = ystage + wave * (kLoraRows * kYsRow);
    const int lr = lane >> 4;         // row within a group of 4 (HBM side)
    const int lc = (lane & 15) * 8;   // column of this lane's 16 B (HBM side)
    auto yoff16 = [&](int sb, int i) {
      const int r = m0 + 4 * i + lr;
      const int n = sb + lc;
      return (r < p.M && n < n_hi) ? (uint32_t)(r * p.N + n) * 2u : kOob;
    };
    // B fragments in NB banks: block cb of a super block uses bank cb % NB,
    // and a bank's slot s is refilled with the block NB ahead.
    constexpr int NB = RB <= 2 ? 4 : (RB <= 8 ? 2 : 1);
    i32x4 yv[kDy][8];
    bf16x8 bf[NB][KS];
    const int sb0 = n_lo + wave * kSb * 32;
#pragma unroll
    for (int d = 0; d < kDy; ++d) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        yv[d][i] = __builtin_amdgcn_raw_buffer_load_b128(ry, (int)yoff16(sb0 + d * kSbStride, i),
                                                         0, 0);
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        bf[b][s] = frag8v(rbm, sb0 + b * 32 + l32, n_hi, s * 16 + hi * 8, rank8, p.ldb);
      }
    }
    for (int base = sb0; base < n_hi; base += kDy * kSbStride) {
#pragma unroll
      for (int d = 0; d < kDy; ++d) {
        const int sb = base + d * kSbStride;
        if (sb >= n_hi) { break; }
        // HBM rows -> LDS tile, then this slot's next loads
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          *(i32x4*)(ys + (4 * i + lr) * kYsRow + lc) = yv[d][i];
          yv[d][i] = __builtin_amdgcn_raw_buffer_load_b128(
              ry, (int)yoff16(sb + kDy * kSbStride, i), 0, 0);
        }
#pragma unroll
        for (int cb = 0; cb < kSb; ++cb) {
          const int nxt = cb + NB < kSb ? sb + (cb + NB) * 32 : sb + kSbStride + (cb + NB - kSb) * 32;
          uint16_t* yt = ys + l32 * kYsRow + cb * 32 + hi * 4;
          f32x16 c;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const u32x2 v = *(const u32x2*)(yt + g * 8);
            c[4 * g + 0] = __uint_as_float(v.x << 16);
            c[4 * g + 1] = __uint_as_float(v.x & 0xffff0000u);
            c[4 * g + 2] = __uint_as_float(v.y << 16);
            c[4 * g + 3] = __uint_as_float(v.y & 0xffff0000u);
          }
#pragma unroll
          for (int s = 0; s < KS; ++s) {
            if (s < ksteps) {
              const bf16x8 rfr = *(const bf16x8*)(rl + l32 * RS + s * 16 + hi * 8);
              c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[cb % NB][s], rfr, c, 0, 0, 0);
            }
            bf[cb % NB][s] = frag8v(rbm, nxt + l32, n_hi, s * 16 + hi * 8, rank8, p.ldb);
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            u32x2 o;
            o.x = pack_bf16x2(c[4 * g + 0], c[4 * g + 1]);
            o.y = pack_bf16x2(c[4 * g + 2], c[4 * g + 3]);
            *(u32x2*)(yt + g * 8) = o;
          }
        }
        // LDS tile -> HBM rows
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const i32x4 o = *(const i32x4*)(ys + (4 * i + lr) * kYsRow + lc);
          __builtin_amdgcn_raw_buffer_store_b128(o, ry, (int)yoff16(sb, i), 0, 0);
        }
      }
    }
  } else {
    for (int nb = n_lo + wave * 32; nb < n_hi; nb += kLoraWaves * 32) {
      f32x16 c;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + hi * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c[4 * g + e] = (row_ok && n + e < n_hi) ? bf16_to_f32(yrow[n + e]) : 0.0f;
        }
      }
      for (int s = 0; s < ksteps; ++s) {
        const int k = s * 16 + hi * 8;
        const bf16x8 bfr = frag8s(p.b, nb + l32, n_hi, k, p.rank, p.ldb);
        const bf16x8 rfr = *(const bf16x8*)(rl + l32 * RS + k);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr, rfr, c, 0, 0, 0);
      }
      if (row_ok) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = nb + g * 8 + hi * 4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e < n_hi) { yrow[n + e] = f32_to_bf16(c[4 * g + e]); }
          }
        }
      }
    }
  }
}

template <int RB>
hipError_t launch_rb(const LoraParams& p, bool vec, dim3 grid, hipStream_t stream)
{
  if (p.r_in != nullptr) {
    lora_kernel<RB, true, true><<<grid, kLoraThreads, 0, stream>>>(p);
  } else if (vec) {
    lora_kernel<RB, true, false><<<grid, kLoraThreads, 0, stream>>>(p);
  } else {
    lora_kernel<RB, false, false><<<grid, kLoraThreads, 0, stream>>>(p);
  }
  return hipGetLastError();
}

// dst[r * ld_dst + c] = c < cols ? src[r][c] : 0 for c < width (width and
// ld_dst multiples of 8): an adapter matrix with its rank padded, so the
// vector paths can load it, or written into a wider matrix's last columns
// (the folded linear's weight tail). One
// thread per 8 destination elements (one 16-byte store); the source side
// reads 16 bytes at once when its row start and stride allow it.
__global__ void lora_pad_kernel(const uint16_t* __restrict__ src, int rows, int cols,
                                int ld_src, uint16_t* __restrict__ dst, int ld_dst, int width)
{
  const size_t chunks = (size_t)width / 8;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * chunks) { return; }
  const size_t r = i / chunks;
  const int c = (int)(i % chunks) * 8;
  const uint16_t* s = src + r * (size_t)ld_src + c;
  uint4 v;
  if (c + 8 <= cols && ((uintptr_t)s & 15u) == 0) {
    v = *(const uint4*)s;
  } else {
    uint32_t w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t lo = c + 2 * t < cols ? s[2 * t] : 0u;
      const uint32_t hi = c + 2 * t + 1 < cols ? s[2 * t + 1] : 0u;
      w[t] = lo | (hi << 16);
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  *(uint4*)(dst + r * (size_t)ld_dst + c) = v;
}

// ---- the adapter merged into the dequant-once expansion ----------------
//   W'[n][k] = bf16(fma(scale, code, zero point) + sum_{i < rank} B[n][i] A[i][k])
// The linear then runs over W' at its own K. (x . A^T) . B^T = x . (B . A)^T,
// so this is the adapter of the reference's lora_add
// (src/ltx25-metal-ops.cc:989-1004) applied to the weight instead of the
// output: no r GEMM, and no extra K in the linear. One rounding to bf16 per
// weight element, where the reference rounds r = x . A^T and the output.
//
// One workgroup expands kMgTiles tiles of 64 rows x 128 columns of W (w8
// codes), stacked along N:
//   1. A's columns k0..k0+127 (rank rows, zero rows up to R) are staged
//      transposed in LDS once, so each MFMA fragment of A is one 16-byte
//      read;
//   2. per tile, wave w owns rows 16 w..16 w+15: D = B[rows][0..R) .
//      A[0..R)[k0..k0+127] on v_mfma_f32_16x16x32_bf16 (B's fragment
//      first, eight 16-column blocks, R / 32 MFMAs each) goes to the wave's
//      own LDS rows as f32;
//   3. the wave reads its rows back as runs of 8, dequantizes four runs per
//      lane, adds D and rounds once: one 16-byte store per run.
// Each wave reads back only what it wrote, so the tiles need no barrier.
// The next tile's codes, scales, zero points and B fragments are loaded
// before the current tile's MFMAs; the tiles are unrolled, so every wait
// is exact (a loop around register-carried loads makes the compiler wait
// for all of them at its head).
constexpr int kMgRows = 64;
constexpr int kMgCols = 128;
constexpr int kMgTiles = 4;
constexpr int kMgThreads = 256;
constexpr int kMgRuns = 16 * kMgCols / 8 / 64;   // runs of 8 per lane per tile: 4
constexpr int kMgDp = kMgCols + 4;               // f32 per LDS row of D
constexpr int kMgMaxRank = kMergeMaxRank;         // the widest instantiation

// R: the rank rounded up to 32 or 64. Wider adapters would re-read a wider
// transposed A slice from LDS for every 16 rows of W: at R = 480 the kernel
// took 253 us at the FFN up shape, LDS-bound, where the extra-K fold costs
// 155 us, so the host takes the merge up to rank 64 only.
template <int R>
__global__ __launch_bounds__(kMgThreads) void dequant_merge_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ qbias, int gshift, int gcols, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ b, int rank, int ldb, uint16_t* __restrict__ out, int N, int K)
{
  constexpr int AP = R + 8;   // bf16 per LDS row of A^T (16-byte pad keeps rows aligned)
  __shared__ __attribute__((aligned(16))) float dl[kMgRows * kMgDp];
  __shared__ __attribute__((aligned(16))) uint16_t at[kMgCols * AP];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int k0 = blockIdx.x * kMgCols;
  const int nb = blockIdx.y * kMgRows * kMgTiles + 16 * wave;   // the wave's first row, tile 0
  float* const dw = dl + 16 * wave * kMgDp;                      // the wave's 16 rows of D
  const auto rb = rsrc(b, (size_t)N * ldb * 2);

  // run j of a lane in a tile: the wave's row rr, columns cc .. cc + 7
  auto run_row = [&](int j) { return (lane + 64 * j) / (kMgCols / 8); };
  auto run_col = [&](int j) { return ((lane + 64 * j) % (kMgCols / 8)) * 8; };
  uint2 cv[2][kMgRuns];
  float sv[2][kMgRuns], bv[2][kMgRuns];
  i32x4 bf[2][R / 32];
  auto load_tile = [&](int buf, int tt) {
    const int n_w = nb + tt * kMgRows;
#pragma unroll
    for (int j = 0; j < kMgRuns; ++j) {
      const int n = n_w + run_row(j);
      const int nc = n < N ? n : N - 1;
      const int k = k0 + run_col(j);
      cv[buf][j] = *(const uint2*)(codes + (size_t)nc * K + k);
      const int g = k >> gshift;
      sv[buf][j] = bf16_to_f32(scales[(size_t)nc * gcols + g]);
      bv[buf][j] = bf16_to_f32(qbias[(size_t)nc * gcols + g]);
    }
    // B's fragment: row n_w + lane % 16, adapter columns 32 c + 8 (lane / 16) .. + 7
    // (B's columns from rank up to ldb are zeros)
    const int n = n_w + (lane & 15);
#pragma unroll
    for (int c = 0; c < R / 32; ++c) {
      const int i = 32 * c + 8 * (lane >> 4);
      const uint32_t off = (n < N && i < rank) ? (uint32_t)(n * ldb + i) * 2u : kOob;
      bf[buf][c] = __builtin_amdgcn_raw_buffer_load_b128(rb, (int)off, 0, 0);
    }
  };
  load_tile(0, 0);

  // 1. at[kk][i] = A[i][k0 + kk], zero for i >= rank: R / 16 pieces of 16
  // bytes per thread, loaded in batches of up to 8 before any is written (a
  // load-then-write loop waited for each load in turn)
  const auto ra = rsrc(a, (size_t)rank * K * 2);
  constexpr int kPieces = R * (kMgCols / 8) / kMgThreads;
  constexpr int kBatch = kPieces % 8 == 0 ? 8 : kPieces % 6 == 0 ? 6 : kPieces < 8 ? kPieces : 1;
  static_assert(kPieces % kBatch == 0, "whole batches of A pieces");
#pragma unroll
  for (int b0 = 0; b0 < kPieces; b0 += kBatch) {
    i32x4 v[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int p = tid + (b0 + q) * kMgThreads;
      const int i = p / (kMgCols / 8);
      const int kk = (p % (kMgCols / 8)) * 8;
      const uint32_t off = i < rank ? (uint32_t)(i * K + k0 + kk) * 2u : kOob;
      v[q] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)off, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int p = tid + (b0 + q) * kMgThreads;
      const int i = p / (kMgCols / 8);
      const int kk = (p % (kMgCols / 8)) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        at[(kk + 2 * e) * AP + i] = (uint16_t)((uint32_t)v[q][e] & 0xffffu);
        at[(kk + 2 * e + 1) * AP + i] = (uint16_t)((uint32_t)v[q][e] >> 16);
      }
    }
  }
  __syncthreads();

#pragma unroll
  for (int tt = 0; tt < kMgTiles; ++tt) {
    const int cur = tt & 1;
    if (tt + 1 < kMgTiles) { load_tile(cur ^ 1, tt + 1); }
    // 2. D[4 (lane / 16) + t][16 kb + lane % 16] of the wave's rows. The
    // eight blocks' accumulators are independent, so the rank chunks run
    // outermost and consecutive MFMAs never wait on each other; A's
    // fragments for chunk c + 1 are read from LDS while chunk c's MFMAs run
    // (the order held by scheduling barriers: read just before its MFMA,
    // each fragment's LDS latency stalled the wave).
    constexpr int KB = kMgCols / 16;
    f32x4 d[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) { d[kb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f}; }
    i32x4 af[2][KB];
    auto read_a = [&](int slot, int c) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        af[slot][kb] = *(const i32x4*)(at + (16 * kb + (lane & 15)) * AP + 32 * c +
                                       8 * (lane >> 4));
      }
    };
    read_a(0, 0);
#pragma unroll
    for (int c = 0; c < R / 32; ++c) {
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < R / 32) { read_a((c + 1) & 1, c + 1); }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        d[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, bf[cur][c]),
                                                        __builtin_bit_cast(bf16x8, af[c & 1][kb]),
                                                        d[kb], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < kMgCols / 16; ++kb) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        dw[(4 * (lane >> 4) + t) * kMgDp + 16 * kb + (lane & 15)] = d[kb][t];
      }
    }
    // 3. W' = bf16(fma(s, code, z) + D), one 16-byte store per run
    const int n_w = nb + tt * kMgRows;
#pragma unroll
    for (int j = 0; j < kMgRuns; ++j) {
      const int rr = run_row(j);
      const int cc = run_col(j);
      const f32x4 d0 = *(const f32x4*)(dw + rr * kMgDp + cc);
      const f32x4 d1 = *(const f32x4*)(dw + rr * kMgDp + cc + 4);
      const float dd[8] = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
      uint32_t o[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t w = h < 2 ? cv[cur][j].x : cv[cur][j].y;
        const int sh = (h & 1) * 16;
        o[h] = pack_bf16x2(fmaf(sv[cur][j], (float)((w >> sh) & 0xffu), bv[cur][j]) + dd[2 * h],
                           fmaf(sv[cur][j], (float)((w >> (sh + 8)) & 0xffu), bv[cur][j]) +
                               dd[2 * h + 1]);
      }
      const int n = n_w + rr;
      if (n < N) { *(uint4*)(out + (size_t)n * K + k0 + cc) = make_uint4(o[0], o[1], o[2], o[3]); }
    }
  }
}

}  // namespace

// The merge takes w8 codes, K % 128 == 0, rank up to kMgMaxRank, B's row
// stride ldb a multiple of 8 (its columns from rank to ldb zero), A and B
// 16-byte aligned and every operand under 2 GiB (32-bit buffer offsets).
bool dequant_merge_takes(int bits, int N, int K, int rank, int ldb, const void* a, const void* b)
{
  const size_t lim = (size_t)1 << 31;
  return bits == 8 && N > 0 && K > 0 && K % kMgCols == 0 && rank > 0 && rank <= kMgMaxRank &&
         ldb >= rank && ldb % 8 == 0 && ((uintptr_t)a & 15u) == 0 &&
         ((uintptr_t)b & 15u) == 0 && (size_t)rank * K * 2 < lim && (size_t)N * ldb * 2 < lim &&
         (size_t)N * K * 2 < lim;
}

hipError_t launch_dequant_merge(const uint8_t* codes, const uint16_t* scales,
                                const uint16_t* qbias, int group, const uint16_t* a,
                                const uint16_t* b, int rank, int ldb, uint16_t* out, int N,
                                int K, hipStream_t stream)
{
  if (!dequant_merge_takes(8, N, K, rank, ldb, a, b) || (group != 32 && group != 64)) {
    return hipErrorInvalidValue;
  }
  const int gshift = group == 64 ? 6 : 5;
  const int rows = kMgRows * kMgTiles;
  const dim3 grid((unsigned)(K / kMgCols), (unsigned)((N + rows - 1) / rows));
  auto go = [&](auto r) {
    constexpr int R = decltype(r)::value;
    dequant_merge_kernel<R><<<grid, kMgThreads, 0, stream>>>(codes, scales, qbias, gshift,
                                                             K / group, a, b, rank, ldb, out, N, K);
  };
  if (rank <= 32) {
    go(std::integral_constant<int, 32>{});
  } else {
    go(std::integral_constant<int, 64>{});
  }
  return hipGetLastError();
}

hipError_t launch_lora_pad(const uint16_t* src, int rows, int cols, int ld_src, uint16_t* dst,
                           int ld_dst, hipStream_t stream, int width)
{
  if (width == 0) { width = ld_dst; }
  if (ld_dst % 8 != 0 || width % 8 != 0 || width > ld_dst || ((uintptr_t)dst & 15u) != 0) {
    return hipErrorInvalidValue;
  }
  const size_t n = (size_t)rows * (width / 8);
  if (n == 0) { return hipSuccess; }
  lora_pad_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(src, rows, cols, ld_src, dst,
                                                                     ld_dst, width);
  return hipGetLastError();
}

// Column split along grid.y. Every split recomputes phase 1 for its row
// block (x and all of A again), so a wide adapter gets just enough
// workgroups to cover the CUs once; a narrow one, whose phase 2 is bound by
// y traffic and wants waves in flight, gets two per CU. Never fewer than
// 1024 columns per workgroup.
int lora_splits(int M, int N, int rank, int cu_count, bool pre_r)
{
  const int mtiles = (M + kLoraRows - 1) / kLoraRows;
  const int per_cu = rank > 128 && !pre_r ? 1 : 2;
  const int want = per_cu * cu_count / mtiles;
  const int cap = (N + 1023) / 1024;
  return want < 1 ? 1 : (want < cap ? want : cap);
}

hipError_t launch_lora(const uint16_t* x, const uint16_t* a, const uint16_t* b,
                       uint16_t* y, int M, int K, int N, int rank, int ldb,
                       bool vec, int cu_count, hipStream_t stream, const uint16_t* r_in)
{
  if (rank <= 0 || rank > kLoraMaxRank) { return hipErrorInvalidValue; }
  if (r_in != nullptr && (!vec || rank % 8 != 0)) { return hipErrorInvalidValue; }
  const int splits = lora_splits(M, N, rank, cu_count, r_in != nullptr);
  int n_split = (N + splits - 1) / splits;
  // whole super-block strides (4 waves x 128 columns) where N allows
  const int quantum = N >= 512 ? 512 : 32;
  n_split = (n_split + quantum - 1) / quantum * quantum;
  const int gy = (N + n_split - 1) / n_split;
  LoraParams p{r_in, x, a, b, y, M, K, N, rank, ldb, n_split};
  const dim3 grid((unsigned)((M + kLoraRows - 1) / kLoraRows), (unsigned)gy);
  const int rb = (rank + 31) / 32;
  if (rb <= 1) { return launch_rb<1>(p, vec, grid, stream); }
  if (rb <= 2) { return launch_rb<2>(p, vec, grid, stream); }
  if (rb <= 4) { return launch_rb<4>(p, vec, grid, stream); }
  if (rb <= 8) { return launch_rb<8>(p, vec, grid, stream); }
  return launch_rb<16>(p, vec, grid, stream);
}

}  // namespace ltx25
