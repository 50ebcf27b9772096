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

#include "common.h"

namespace ltx25 {
namespace {

constexpr int kLoraRows = 32;
constexpr int kLoraWaves = 4;
constexpr int kLoraThreads = kLoraWaves * 64;

struct LoraParams {
  const uint16_t* x;
  const uint16_t* a;  // this pass's first row of A
  const uint16_t* b;  // this pass's first column of B
  uint16_t* y;
  int M, K, N;
  int rank;     // adapter columns in this pass, <= kLoraMaxRank
  int ldb;      // row stride of B in elements (the adapter's full rank)
  int n_split;  // columns of y per workgroup along grid.y, multiple of 32
};

// Eight bf16 of row `row`, columns k..k+7, of a row-major matrix with
// `rows` x `cols` valid elements and row stride `ld`; zero outside. VEC
// requires cols % 8 == 0 and 16-byte aligned rows, so a chunk is either
// wholly inside or wholly outside.
template <bool VEC>
__device__ __forceinline__ bf16x8 frag8(const uint16_t* p, int row, int rows,
                                        int k, int cols, long ld)
{
  i32x4 v = {0, 0, 0, 0};
  if constexpr (VEC) {
    if (row < rows && k < cols) { v = *(const i32x4*)(p + (size_t)row * ld + k); }
  } else {
    if (row < rows) {
      const uint16_t* q = p + (size_t)row * ld;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (k + 2 * i < cols) ? q[k + 2 * i] : 0u;
        const uint32_t hi = (k + 2 * i + 1 < cols) ? q[k + 2 * i + 1] : 0u;
        v[i] = (int)(lo | (hi << 16));
      }
    }
  }
  return __builtin_bit_cast(bf16x8, v);
}

// RB = 32-column blocks of rank this instance covers (rank <= 32 * RB).
template <int RB, bool VEC>
__global__ __launch_bounds__(kLoraThreads) void lora_kernel(LoraParams p)
{
  constexpr int RP = 32 * RB;        // rank padded to the MFMA block
  constexpr int RS = RP + 8;         // bf16 per LDS row of r (16-byte pad)
  constexpr int FS = RP + 4;         // f32 per LDS row of the partials
  __shared__ __attribute__((aligned(16))) float red[kLoraRows * FS];
  __shared__ __attribute__((aligned(16))) uint16_t rl[kLoraRows * RS];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int m0 = blockIdx.x * kLoraRows;

  // ---- phase 1: r^T[i][m] = sum_k A[i][k] x[m][k], K split over waves ----
  f32x16 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc[rb][r] = 0.0f; }
  }
  // K steps of 16, dealt round-robin to the waves; U steps' fragments are
  // loaded before their MFMAs so several loads are in flight per wave.
  // A step past the end loads zeros (k = K is outside every row).
  constexpr int U = RB <= 2 ? 4 : (RB <= 4 ? 2 : 1);
  const int steps = (p.K + 15) / 16;
  const int nloc = (steps - wave + kLoraWaves - 1) / kLoraWaves;
  for (int j = 0; j < nloc; j += U) {
    bf16x8 xf[U];
    bf16x8 af[U][RB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = j + u < nloc ? (wave + (j + u) * kLoraWaves) * 16 + hi * 8 : p.K;
      xf[u] = frag8<VEC>(p.x, m0 + l32, p.M, k, p.K, p.K);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        af[u][rb] = frag8<VEC>(p.a, rb * 32 + l32, p.rank, k, p.K, p.K);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u][rb], xf[u], acc[rb], 0, 0, 0);
      }
    }
  }

  // Lane l, register r of block rb holds r^T[i][m] with m = l & 31 and
  // i = 32 rb + 8 (r / 4) + 4 (l / 32) + r % 4. Waves add in order 0..3;
  // the last rounds to bf16 into rl[m][i].
  for (int w = 0; w < kLoraWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int i = rb * 32 + g * 8 + hi * 4;
          float* dst = red + l32 * FS + i;
          f32x4 v = {acc[rb][4 * g], acc[rb][4 * g + 1], acc[rb][4 * g + 2],
                     acc[rb][4 * g + 3]};
          if (w > 0) { v += *(const f32x4*)dst; }
          if (w < kLoraWaves - 1) {
            *(f32x4*)dst = v;
          } else {
            uint2 o;
            o.x = pack_bf16x2(v[0], v[1]);
            o.y = pack_bf16x2(v[2], v[3]);
            *(uint2*)(rl + l32 * RS + i) = o;
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- phase 2: y^T[n][m] = y^T[n][m] + sum_j B[n][j] r[m][j] -----------
  const int ksteps = (p.rank + 15) / 16;
  const int row = m0 + l32;
  const bool row_ok = row < p.M;
  const int n_lo = blockIdx.y * p.n_split;
  const int n_hi = min(p.N, n_lo + p.n_split);
  for (int nb = n_lo + wave * 32; nb < n_hi; nb += kLoraWaves * 32) {
    f32x16 c;
    uint16_t* yrow = p.y + (size_t)row * p.N;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = nb + g * 8 + hi * 4;
      if constexpr (VEC) {
        uint2 v = {0u, 0u};
        if (row_ok && n < n_hi) { v = *(const uint2*)(yrow + n); }
        c[4 * g + 0] = __uint_as_float(v.x << 16);
        c[4 * g + 1] = __uint_as_float(v.x & 0xffff0000u);
        c[4 * g + 2] = __uint_as_float(v.y << 16);
        c[4 * g + 3] = __uint_as_float(v.y & 0xffff0000u);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          c[4 * g + e] = (row_ok && n + e < n_hi) ? bf16_to_f32(yrow[n + e]) : 0.0f;
        }
      }
    }
    for (int s = 0; s < ksteps; ++s) {
      const int k = s * 16 + hi * 8;
      const bf16x8 bfr = frag8<VEC>(p.b, nb + l32, n_hi, k, p.rank, p.ldb);
      const bf16x8 rfr = *(const bf16x8*)(rl + l32 * RS + k);
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr, rfr, c, 0, 0, 0);
    }
    if (row_ok) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + hi * 4;
        if constexpr (VEC) {
          if (n < n_hi) {
            uint2 o;
            o.x = pack_bf16x2(c[4 * g + 0], c[4 * g + 1]);
            o.y = pack_bf16x2(c[4 * g + 2], c[4 * g + 3]);
            *(uint2*)(yrow + n) = o;
          }
        } else {
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
  if (vec) {
    lora_kernel<RB, true><<<grid, kLoraThreads, 0, stream>>>(p);
  } else {
    lora_kernel<RB, false><<<grid, kLoraThreads, 0, stream>>>(p);
  }
  return hipGetLastError();
}

}  // namespace

// Column split along grid.y: enough workgroups to cover the CUs when the
// token count is small, but never fewer than 1024 columns per workgroup,
// because every split recomputes phase 1 for its row block.
int lora_splits(int M, int N, int cu_count)
{
  const int mtiles = (M + kLoraRows - 1) / kLoraRows;
  if (mtiles >= cu_count) { return 1; }
  const int want = (cu_count + mtiles - 1) / mtiles;
  const int cap = (N + 1023) / 1024;
  return want < cap ? want : cap;
}

hipError_t launch_lora(const uint16_t* x, const uint16_t* a, const uint16_t* b,
                       uint16_t* y, int M, int K, int N, int rank, int ldb,
                       bool vec, int cu_count, hipStream_t stream)
{
  if (rank <= 0 || rank > kLoraMaxRank) { return hipErrorInvalidValue; }
  const int splits = lora_splits(M, N, cu_count);
  int n_split = (N + splits - 1) / splits;
  n_split = (n_split + 31) / 32 * 32;
  const int gy = (N + n_split - 1) / n_split;
  LoraParams p{x, a, b, y, M, K, N, rank, ldb, n_split};
  const dim3 grid((unsigned)((M + kLoraRows - 1) / kLoraRows), (unsigned)gy);
  const int rb = (rank + 31) / 32;
  if (rb <= 1) { return launch_rb<1>(p, vec, grid, stream); }
  if (rb <= 2) { return launch_rb<2>(p, vec, grid, stream); }
  if (rb <= 4) { return launch_rb<4>(p, vec, grid, stream); }
  if (rb <= 8) { return launch_rb<8>(p, vec, grid, stream); }
  return launch_rb<16>(p, vec, grid, stream);
}

}  // namespace ltx25
