// Device-side helpers shared by the gfx950 kernels, and the internal
// launcher interface between the kernels and the C ABI layer (capi.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ltx25 {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h)
{
  return __uint_as_float((uint32_t)h << 16);
}

// Two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32,
// `lo` in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
  return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu);
}

// GELU, tanh approximation: 0.5 x (1 + tanh(u)) with
// u = sqrt(2/pi) (x + 0.044715 x^3), evaluated through the identity
// 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)) = 1 / (1 + 2^z),
// z = x (k1 + k3 x^2), k1 = -2 sqrt(2/pi) log2(e), k3 = 0.044715 k1:
// five VALU ops plus the hardware exp2 and reciprocal (each within about
// 1 ulp of f32, far inside the bf16 rounding that follows). Saturates at
// both ends: 2^z overflows to inf for large negative x, giving
// x * rcp(inf) = -0; for large positive x, 2^z = 0 and the result is x.
__device__ __forceinline__ float gelu_tanh(float x)
{
  constexpr float k1 = -2.302208198144325f;
  constexpr float k3 = -0.1029432395800235f;
  const float z = x * fmaf(k3, x * x, k1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

// ---- internal launcher interface ------------------------------------------

// Record `code` and a printf-style message as this thread's last error
// (what ltx25_last_error returns); returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Element type of a bias vector (matches LTX25_DT_* in the C header).
enum BiasType : int { kBiasNone = 0, kBiasBf16 = 1, kBiasF32 = 2 };
enum Epilogue : int { kEpiNone = 0, kEpiGelu = 1 };

// Workgroup id -> (tile_m, tile_n). Consecutive workgroup ids are dealt
// round-robin to the 8 XCDs, so the id is first remapped so that each XCD
// receives a contiguous range of tiles, then the range is walked in groups
// of 8 M-tiles: the workgroups an XCD runs at once share X and W tiles in
// that XCD's L2.
__device__ __forceinline__ void map_tile(int bid, int tiles_m, int tiles_n,
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

__device__ __forceinline__ float load_bias(const void* bias, int type, int n)
{
  if (type == kBiasBf16) { return bf16_to_f32(((const uint16_t*)bias)[n]); }
  if (type == kBiasF32) { return ((const float*)bias)[n]; }
  return 0.0f;
}

// One GEMM y[M][N] = x[M][K] . W[N][K]^T with W either group-affine codes
// (bits 8 or 4, `group` 32 or 64) or dense bf16 (bits 16).
struct GemmDesc {
  const uint16_t* x = nullptr;
  // A two-part activation (the LoRA fold, dense weights on the 256 x 256
  // and 128 x 128 tiles): columns [0, kx) of X are x [M][kx], columns
  // [kx, K) are x2 [M][K - kx]; kx a multiple of 64. Null x2: X = x [M][K].
  const uint16_t* x2 = nullptr;
  int kx = 0;
  // Rows of the weight present in memory (0: all N); rows past it read as
  // zeros (the 256 x 256 and 128 x 128 tiles). The fold's r GEMM reads A
  // [rank][K] as a [rk][K] weight this way.
  int wn = 0;
  const void* w = nullptr;          // u8/u32 codes, or bf16 dense
  const uint16_t* scales = nullptr;
  const uint16_t* qbias = nullptr;
  int bits = 8;                     // 8, 4, or 16 (= dense bf16)
  int group = 64;
  const void* bias = nullptr;
  int bias_type = kBiasNone;
  int epilogue = kEpiNone;
  uint16_t* y = nullptr;
  const uint16_t* y_in = nullptr;   // when set: y = bf16(acc + bias + y_in), y_in may be y
  int M = 0, N = 0, K = 0;
};

// The tile configuration a GEMM runs with, chosen on the host.
struct GemmPlan {
  int tile = 0;      // 0 = 256x256 (tall), 1 = 128x128 (mid), 2 = M <= 128 (skinny.hip)
  int splits = 1;    // split-K factor
  int k_chunk = 0;   // K elements per split (multiple of 64)
  size_t workspace_bytes = 0;   // f32 partials when splits > 1
  int cu_count = 256;           // CUs of the device planned for (persistent grids)
};

// `bits` is the weight format the GEMM reads: 8 or 4 (codes) or 16 (dense).
// `force` (the LTX25_TILE_* values): 0 the planner's choice; 1 the
// 256 x 256 tile; 2 the 128 x 128 split-K tile; 3 the M <= 128 kernel
// where it takes the shape, else the planner's choice.
GemmPlan plan_gemm(int M, int N, int K, int bits, int cu_count, int force = 0);
hipError_t launch_gemm(const GemmDesc& d, const GemmPlan& plan,
                       float* workspace, hipStream_t stream);
// The M <= 128 route (skinny.hip): 32 output columns per workgroup, K split
// between its 8 waves, and across workgroups above 2048. Fills `plan` and
// returns true when it takes the shape (up to 3 workgroups per CU).
bool plan_skinny(int M, int N, int K, int bits, int cu_count, GemmPlan& plan);
// `stamps` non-null (w8 only): the phase-stamp instantiation, ten words per
// wave at [(split * ceil(N / 32) + tile) * 8 + wave] * 10 (ltx25_probe_skinny_phases)
hipError_t launch_skinny(const GemmDesc& d, const GemmPlan& plan, float* workspace,
                         hipStream_t stream, unsigned long long* stamps = nullptr);
// The dense bf16 GEMM of the 256 x 256 tile on v_mfma_f32_16x16x32_bf16
// (tall.hip): the dequant-once arm and dense weights, also with the LoRA
// fold's two-part activation [x | r] (kx a multiple of 64), or with y_in
// (8-byte aligned, without the two-part activation); N % 8 == 0.
// launch_gemm routes there when it takes.
bool tall_dense_takes(const GemmDesc& d, const GemmPlan& plan);
// The same tile with w8 codes (groups of 64 or 32) dequantized in registers
// once per workgroup before the LDS write: bit-identical to the dense tile
// over the dequant-once expansion. launch_tall_dense runs either.
bool tall_w8_takes(const GemmDesc& d, const GemmPlan& plan);
// `stamps` non-null (bf16 without the two-part activation, or the int8
// launcher below): the phase-stamp instantiation, eight words per wave at
// (tile * 8 + wave) * 8 (ltx25_probe_tall_phases)
hipError_t launch_tall_dense(const GemmDesc& d, hipStream_t stream,
                             unsigned long long* stamps = nullptr);
// The int8 tier's GEMM on the same tile (tall.hip, v_mfma_i32_16x16x64_i8):
// N % 8 == 0, K a multiple of 128. launch_i8_gemm routes there when the
// 256 x 256 tiles fill the GPU and it takes the shape.
bool tall_i8_takes(int M, int N, int K);
hipError_t launch_tall_i8(const int8_t* xq, const float* sx, const int8_t* wq, const float* sw,
                          const void* bias, int bias_type, int epilogue, uint16_t* y,
                          int32_t* acc, int M, int K, int N, hipStream_t stream,
                          unsigned long long* stamps = nullptr);
// The no-allocation linear's split-K scratch (noalloc.hip): a fixed device
// array of kNoAllocScratchBytes per GPU. noalloc_scratch() returns the
// current device's copy, resolving its address on the first call there.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
hipError_t noalloc_scratch(void** out);
// Sums `splits` f32 partial planes [M][N] in split order, adds bias and
// y_in, applies the epilogue and rounds to bf16 once.
hipError_t launch_splitk_reduce(const float* partial, int splits, const void* bias, int bias_type,
                                int epilogue, const uint16_t* y_in, uint16_t* y, int M, int N,
                                hipStream_t stream);

// The low-rank adapter delta y += (x . A^T) . B^T (lora.hip). One launch
// covers at most kLoraMaxRank adapter columns: `a` points at the pass's
// first row of A [rank][K], `b` at its first column of B [N][ldb]. `vec`
// selects 16-byte operand loads (K % 8 == 0, ldb % 8 == 0, N % 8 == 0,
// aligned pointers, every operand under 2 GiB, and B's columns zero from
// `rank` up to the next multiple of 8).
// With `r_in` set ([M][rank] bf16, rank % 8 == 0, vector path only) the
// launch skips the x . A^T phase and reads r from it.
constexpr int kLoraMaxRank = 512;
int lora_splits(int M, int N, int rank, int cu_count, bool pre_r);
hipError_t launch_lora(const uint16_t* x, const uint16_t* a, const uint16_t* b,
                       uint16_t* y, int M, int K, int N, int rank, int ldb,
                       bool vec, int cu_count, hipStream_t stream,
                       const uint16_t* r_in = nullptr);
// B [rows][cols] (row stride ld_src) -> `width` columns of each dst row
// (row stride ld_dst; width 0 = ld_dst) with zeros past `cols`: the vector
// path's copy of an adapter whose rank is not a multiple of 8, and the
// folded linear's weight tail.
hipError_t launch_lora_pad(const uint16_t* src, int rows, int cols, int ld_src, uint16_t* dst,
                           int ld_dst, hipStream_t stream, int width = 0);
// The dequant-once expansion with the adapter merged in (lora.hip):
// out [N][K] = bf16(fma(scale, code, zero point) + B . A), A bf16
// [rank][K], B bf16 [N][ldb] (columns from rank to ldb zero).
// dequant_merge_takes: w8 codes, K % 128 == 0, rank at most kMergeMaxRank,
// ldb a multiple of 8, A and B 16-byte aligned, operands under 2 GiB;
// launch_dequant_merge refuses anything else (groups of 32 or 64).
constexpr int kMergeMaxRank = 64;
bool dequant_merge_takes(int bits, int N, int K, int rank, int ldb, const void* a, const void* b);
hipError_t launch_dequant_merge(const uint8_t* codes, const uint16_t* scales,
                                const uint16_t* qbias, int group, const uint16_t* a,
                                const uint16_t* b, int rank, int ldb, uint16_t* out, int N,
                                int K, hipStream_t stream);

hipError_t launch_bias_add(uint16_t* y, const void* bias, int bias_type,
                           int M, int N, hipStream_t stream);
hipError_t launch_gelu(const uint16_t* x, uint16_t* y, size_t n,
                       hipStream_t stream);
// y [tokens][heads][head_dim] bf16 *= 2 sigmoid(logits [tokens][heads] bf16), in place.
hipError_t launch_gate_heads(uint16_t* y, const uint16_t* logits, int heads, int tokens,
                             int head_dim, hipStream_t stream);
// codes -> bf16 [N][K] at output row stride ldo (0 = K); with `tail`,
// columns [K, ldo) of row n are tail [n][0, tail_cols) (row stride
// tail_ld) and zeros after them
hipError_t launch_dequant(const void* codes, const uint16_t* scales,
                          const uint16_t* qbias, int bits, int group,
                          uint16_t* out, int N, int K, hipStream_t stream, int ldo = 0,
                          const uint16_t* tail = nullptr, int tail_cols = 0, int tail_ld = 0);
hipError_t launch_quantize_affine(const float* w, uint32_t* codes,
                                  uint16_t* scales, uint16_t* qbias, int N,
                                  int K, int bits, int group,
                                  hipStream_t stream);
hipError_t launch_pack(const uint8_t* q, uint32_t* codes, int N, int K,
                       int bits, hipStream_t stream);
hipError_t launch_unpack(const uint32_t* codes, uint8_t* q, int N, int K,
                         int bits, hipStream_t stream);
hipError_t launch_f16_to_bf16(const uint16_t* in, uint16_t* out, size_t n,
                              hipStream_t stream);

hipError_t launch_i8_quantize_rows(const uint16_t* x, int8_t* q, float* s,
                                   int M, int K, hipStream_t stream);
hipError_t launch_i8_quantize_qweight(const void* codes,
                                      const uint16_t* scales,
                                      const uint16_t* qbias, int bits,
                                      int group, int8_t* q, float* s, int N,
                                      int K, hipStream_t stream);
// y = bf16(epilogue(fma(float(acc), sx[m] * sw[n], bias[n]))), epilogue
// kEpiNone or kEpiGelu (GELU-tanh in f32 before the one rounding).
hipError_t launch_i8_gemm(const int8_t* xq, const float* sx,
                          const int8_t* wq, const float* sw, const void* bias,
                          int bias_type, int epilogue, uint16_t* y, int32_t* acc,
                          int M, int K, int N, hipStream_t stream);

// Measurement probes (probes.hip): a streaming read of `bytes` (16-byte
// aligned, a multiple of 16) over `blocks` workgroups, one word per
// workgroup to `sink`; a stream of independent 16x16x32 bf16 MFMAs on zero
// or random register operands, 256 workgroups of 1 or 2 waves per SIMD.
hipError_t launch_probe_read(const void* src, size_t bytes, uint32_t* sink, int blocks,
                             hipStream_t stream);
hipError_t launch_probe_mfma(int iters, int random, int waves_per_simd, float* out,
                             hipStream_t stream);

}  // namespace ltx25
