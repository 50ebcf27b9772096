// The C ABI (include/ltx25_qlinear.h): argument validation, the dispatch
// policy between the tile shapes / split-K / int8 tier, and the grow-only
// scratch the split-K and int8 paths share.
//
// Validation runs before any HIP call, so malformed calls fail the same
// way on a host without a GPU. The reference reports shape errors at bind
// time and asserts in `linear`; here every entry point returns a code and
// leaves the message in ltx25_last_error().
#include "ltx25_qlinear.h"

#include "common.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

namespace {

thread_local std::string g_err;

int vfail(int code, const char* fmt, va_list ap)
{
  char buf[512];
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  g_err = buf;
  return code;
}

int fail(int code, const char* fmt, ...)
{
  va_list ap;
  va_start(ap, fmt);
  const int rc = vfail(code, fmt, ap);
  va_end(ap);
  return rc;
}

}  // namespace

namespace ltx25 {

int set_error(int code, const char* fmt, ...)
{
  va_list ap;
  va_start(ap, fmt);
  const int rc = vfail(code, fmt, ap);
  va_end(ap);
  return rc;
}

}  // namespace ltx25

namespace {

int hip_fail(hipError_t e, const char* what)
{
  return fail(LTX25_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;

// Per-device state: checked once, then the grow-only scratch.
struct DeviceState {
  bool checked = false;
  bool ok = false;
  int cu_count = 0;
  char arch[64] = {0};
  void* ws = nullptr;        // split-K f32 partials
  size_t ws_bytes = 0;
  void* i8 = nullptr;        // int8 tier operands: xq | sx | wq | sw
  size_t i8_bytes = 0;
  void* deq = nullptr;       // dequant-once arm: bf16 [N][K] expansion
  size_t deq_bytes = 0;
  void* lora_b = nullptr;    // LoRA B padded to a multiple of 8 columns
  size_t lora_b_bytes = 0;
  void* lora_mm = nullptr;   // LoRA GEMM pair: A padded | r | B padded
  size_t lora_mm_bytes = 0;
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];
// Process-wide switches (the reference keeps them per MetalOps; one set per
// process here), read on every call from any thread.
std::atomic<int> g_i8_on{0};
std::atomic<int> g_deq_once{LTX25_DEQUANT_ONCE_AUTO};
std::atomic<int> g_deq_min_m{LTX25_DEQUANT_ONCE_AUTO_MIN_M};

// Check (once per device) that the current device is gfx950.
int current_device(DeviceState** out)
{
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0) {
    int count = 0;
    (void)hipGetDeviceCount(&count);
    return fail(LTX25_E_NODEV, "no HIP device is visible (%s)",
                hipGetErrorString(e));
  }
  if (dev >= kMaxDevices) {
    return fail(LTX25_E_NODEV, "device index %d is out of range", dev);
  }
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& s = g_dev[dev];
  if (!s.checked) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) { return hip_fail(e, "hipGetDeviceProperties"); }
    std::snprintf(s.arch, sizeof s.arch, "%s", prop.gcnArchName);
    s.cu_count = prop.multiProcessorCount;
    s.ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    s.checked = true;
  }
  if (!s.ok) {
    return fail(LTX25_E_NODEV,
                "device %d is %s; these kernels are built for gfx950 only",
                dev, s.arch);
  }
  *out = &s;
  return LTX25_OK;
}

// Grow `*buf` to at least `need` bytes. The old buffer may still be read by
// work queued earlier, so the device is drained before it is released.
int grow(void** buf, size_t* cap, size_t need)
{
  if (*cap >= need) { return LTX25_OK; }
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) { return hip_fail(e, "hipDeviceSynchronize"); }
  if (*buf != nullptr) {
    (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
  }
  e = hipMalloc(buf, need);
  if (e != hipSuccess) {
    *buf = nullptr;
    return hip_fail(e, "hipMalloc (scratch)");
  }
  *cap = need;
  return LTX25_OK;
}

// The kernels move 16-byte vectors, so every tensor base must be 16-byte
// aligned (any allocator's base pointer is; a sliced view may not be).
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_aligned(const char* what, const void* p)
{
  if (p != nullptr && !aligned16(p)) {
    return fail(LTX25_E_INVAL, "%s (%p) is not 16-byte aligned", what, p);
  }
  return LTX25_OK;
}

bool bias_ok(const void* bias, int dt)
{
  if (bias == nullptr) { return dt == LTX25_DT_NONE || dt == LTX25_DT_BF16 || dt == LTX25_DT_F32; }
  return dt == LTX25_DT_BF16 || dt == LTX25_DT_F32;
}

int check_shape(int M, int K, int N)
{
  if (M <= 0 || K <= 0 || N <= 0) {
    return fail(LTX25_E_INVAL, "shape M=%d K=%d N=%d must be positive", M, K, N);
  }
  return LTX25_OK;
}

int check_qweight(const ltx25_qweight* w, int K)
{
  if (w == nullptr) { return fail(LTX25_E_INVAL, "weight is null"); }
  if (!w->quantized) {
    if (w->w == nullptr) { return fail(LTX25_E_INVAL, "dense weight `w` is null"); }
    return LTX25_OK;
  }
  if (w->codes == nullptr || w->scales == nullptr || w->qbias == nullptr) {
    return fail(LTX25_E_INVAL, "quantized weight has a null codes/scales/qbias");
  }
  if (w->bits != 8 && w->bits != 4) {
    return fail(LTX25_E_INVAL, "bits=%d; only 4 and 8 are packed", w->bits);
  }
  if (w->group != 64 && w->group != 32) {
    return fail(LTX25_E_INVAL, "group=%d; only 32 and 64 are packed", w->group);
  }
  if (K % w->group != 0) {
    return fail(LTX25_E_INVAL, "K=%d is not a multiple of the group %d", K, w->group);
  }
  return LTX25_OK;
}

int run_i8_linear(DeviceState* ds, hipStream_t st, const void* x,
                  const ltx25_qweight* w, const void* bias, int bias_dtype,
                  void* y, int M, int K, int N, int epilogue);

// Every operand a kernel addresses must stay under 2 GiB: the kernels form
// 32-bit buffer offsets (voffset + soffset) and a raw buffer's range is a
// 32-bit byte count. The reference declines the same operands for the same
// reason -- a wrapped offset computes wrong rows without any error
// (src/ltx25-metal-ops.cc:342-374). Here the activation and output are cut
// into row slabs that each stay under the limit; a weight at or over it is
// refused.
constexpr size_t kOperandMax = (size_t)1 << 31;

bool below_limit(size_t bytes) { return bytes < kOperandMax; }

size_t weight_bytes(int N, int K, int bits)
{
  return (size_t)N * (size_t)K * (size_t)bits / 8;
}

// Rows per launch so that X [rows][K] and Y [rows][N] (bf16) each stay
// under kOperandMax: all of M when they do, else a multiple of 256 rows.
int slab_rows(int M, int K, int N)
{
  const size_t widest = (size_t)(K > N ? K : N) * 2;
  const size_t rows = (kOperandMax - 1) / widest;
  if ((size_t)M <= rows) { return M; }
  return (int)(rows & ~(size_t)255);
}

std::atomic<int> g_tile{LTX25_TILE_AUTO};

// The route a linear takes, decided on the host before any device use.
struct LinearRoute {
  bool i8 = false;
  bool deq_once = false;
  int rows = 0;      // rows per launch
  int slabs = 1;
  ltx25::GemmPlan plan;   // of the first slab
  size_t scratch = 0;     // bytes of library scratch the call uses
};

int cu_count_hint()
{
  // the CU count of a device already checked, else the MI355X's
  for (int d = 0; d < kMaxDevices; ++d) {
    if (g_dev[d].checked && g_dev[d].ok) { return g_dev[d].cu_count; }
  }
  return 256;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t i8_scratch_bytes(int M, int K, int N)
{
  return align256((size_t)M * K) + align256((size_t)M * 4) + align256((size_t)N * K) +
         align256((size_t)N * 4);
}

// bits: 8 or 4 (codes) or 16 (a dense weight).
int plan_linear(int M, int K, int N, int bits, int cu_count, LinearRoute* r)
{
  if (!below_limit(weight_bytes(N, K, bits))) {
    return fail(LTX25_E_UNSUPPORTED,
                "the weight [%d][%d] at %d bits is %zu bytes; operands must stay under 2 GiB "
                "(32-bit buffer offsets)", N, K, bits, weight_bytes(N, K, bits));
  }
  r->i8 = ltx25_i8_takes(M, K, N) != 0;
  if (r->i8) {
    r->rows = M;
    r->slabs = 1;
    r->scratch = i8_scratch_bytes(M, K, N);
    return LTX25_OK;
  }
  r->deq_once = bits != 16 && ltx25_dequant_once_takes(M, K, N) != 0 &&
                below_limit(weight_bytes(N, K, 16));
  r->rows = slab_rows(M, K, N);
  if (r->rows <= 0) {
    return fail(LTX25_E_UNSUPPORTED, "K=%d N=%d: one row of X or Y is 2 GiB or more", K, N);
  }
  r->slabs = (M + r->rows - 1) / r->rows;
  const int gemm_bits = r->deq_once ? 16 : bits;
  r->plan = ltx25::plan_gemm(r->rows, N, K, gemm_bits, cu_count,
                             g_tile.load(std::memory_order_relaxed));
  r->scratch = r->plan.workspace_bytes + (r->deq_once ? (size_t)N * K * 2 : 0);
  return LTX25_OK;
}

// `noalloc`: the ltx25_linear_q_noalloc variant. It plans the same GEMM
// without the routes that need library scratch (the int8 tier, the
// dequant-once expansion) and puts split-K partials in the fixed device
// array of noalloc.hip, refusing a plan whose partials do not fit.
int run_linear(hipStream_t st, const void* x, const ltx25_qweight* w,
               const void* bias, int bias_dtype, void* y, int M, int K, int N,
               int epilogue, bool noalloc = false)
{
  if (x == nullptr || y == nullptr) { return fail(LTX25_E_INVAL, "x or y is null"); }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  rc = check_qweight(w, K);
  if (rc != LTX25_OK) { return rc; }
  if (!bias_ok(bias, bias_dtype)) {
    return fail(LTX25_E_INVAL, "bias dtype %d is not valid for a %s bias",
                bias_dtype, bias == nullptr ? "null" : "non-null");
  }
  if (epilogue != LTX25_EPI_NONE && epilogue != LTX25_EPI_GELU_TANH) {
    return fail(LTX25_E_INVAL, "unknown epilogue %d", epilogue);
  }
  if ((rc = check_aligned("x", x)) != LTX25_OK || (rc = check_aligned("y", y)) != LTX25_OK ||
      (rc = check_aligned("weight", w->quantized ? w->codes : w->w)) != LTX25_OK) {
    return rc;
  }
  if (K % 64 != 0) {
    return fail(LTX25_E_UNSUPPORTED,
                "K=%d: the MFMA kernels step K by 64; pad K to a multiple of 64", K);
  }
  const int bits = w->quantized ? w->bits : 16;
  LinearRoute route;
  rc = plan_linear(M, K, N, bits, cu_count_hint(), &route);
  if (rc != LTX25_OK) { return rc; }
  if (noalloc) {
    if (route.i8) {
      return fail(LTX25_E_UNSUPPORTED,
                  "the int8 tier takes M=%d K=%d N=%d and quantizes into library scratch; "
                  "the no-allocation linear cannot run it (ltx25_set_i8_gemm(0) turns it off)",
                  M, K, N);
    }
    // the in-register dequant: bit-identical to the dequant-once arm
    route.deq_once = false;
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  if (route.i8) { return run_i8_linear(ds, st, x, w, bias, bias_dtype, y, M, K, N, epilogue); }
  const int tile = g_tile.load(std::memory_order_relaxed);
  float* fixed_ws = nullptr;
  if (noalloc) {
    // every slab's plan must fit the fixed scratch before anything launches
    // (the slabs are `rows` tall except a shorter last one)
    const int last = M - (route.slabs - 1) * route.rows;
    const size_t need =
        std::max(ltx25::plan_gemm(route.rows, N, K, bits, ds->cu_count, tile).workspace_bytes,
                 ltx25::plan_gemm(last, N, K, bits, ds->cu_count, tile).workspace_bytes);
    if (need > ltx25::kNoAllocScratchBytes) {
      return fail(LTX25_E_UNSUPPORTED,
                  "M=%d K=%d N=%d: the split-K partials need %zu bytes; the no-allocation "
                  "linear's scratch holds %zu", M, K, N, need, ltx25::kNoAllocScratchBytes);
    }
    if (need > 0) {
      void* p = nullptr;
      const hipError_t e = ltx25::noalloc_scratch(&p);
      if (e != hipSuccess) { return hip_fail(e, "hipGetSymbolAddress (no-allocation scratch)"); }
      fixed_ws = (float*)p;
    }
  }

  ltx25::GemmDesc d;
  d.w = w->quantized ? w->codes : w->w;
  d.scales = (const uint16_t*)w->scales;
  d.qbias = (const uint16_t*)w->qbias;
  d.bits = bits;
  d.group = w->quantized ? w->group : 64;
  if (route.deq_once) {
    // The dequant-once arm: expand W into the grow-only bf16 scratch, then
    // the same GEMM tile over the dense copy. The expansion is bit-identical
    // to the in-register dequant, so both arms produce the same bits.
    std::lock_guard<std::mutex> lk(g_mu);
    rc = grow(&ds->deq, &ds->deq_bytes, (size_t)N * K * 2);
    if (rc != LTX25_OK) { return rc; }
    const hipError_t e = ltx25::launch_dequant(w->codes, (const uint16_t*)w->scales,
                                               (const uint16_t*)w->qbias, w->bits,
                                               w->group, (uint16_t*)ds->deq, N, K, st);
    if (e != hipSuccess) { return hip_fail(e, "dequant-once launch"); }
    d.w = ds->deq;
    d.scales = nullptr;
    d.qbias = nullptr;
    d.bits = 16;
    d.group = 64;
  }
  d.bias = bias;
  d.bias_type = bias != nullptr ? bias_dtype : ltx25::kBiasNone;
  d.epilogue = epilogue;
  d.N = N;
  d.K = K;
  for (int m0 = 0; m0 < M; m0 += route.rows) {
    d.M = M - m0 < route.rows ? M - m0 : route.rows;
    d.x = (const uint16_t*)x + (size_t)m0 * K;
    d.y = (uint16_t*)y + (size_t)m0 * N;
    const ltx25::GemmPlan plan = ltx25::plan_gemm(d.M, N, K, d.bits, ds->cu_count, tile);
    float* ws = nullptr;
    if (noalloc) {
      ws = fixed_ws;
    } else if (plan.workspace_bytes > 0) {
      std::lock_guard<std::mutex> lk(g_mu);
      rc = grow(&ds->ws, &ds->ws_bytes, plan.workspace_bytes);
      if (rc != LTX25_OK) { return rc; }
      ws = (float*)ds->ws;
    }
    const hipError_t e = ltx25::launch_gemm(d, plan, ws, st);
    if (e != hipSuccess) { return hip_fail(e, "qgemm launch"); }
  }
  return LTX25_OK;
}

// The int8 tier inside `linear`: quantize the activation per token and the
// weight per output channel for THIS call (the reference's tier keeps no
// persistent weight copy either, src/ltx25-metal-ops.h:810-816), then the
// int8 GEMM with the fused dequant epilogue.
int run_i8_linear(DeviceState* ds, hipStream_t st, const void* x,
                  const ltx25_qweight* w, const void* bias, int bias_dtype,
                  void* y, int M, int K, int N, int epilogue)
{
  // (plan_linear has checked that M * K, N * K and M * N * 2 stay under
  // 2 GiB for this tier)
  const size_t xq_b = align256((size_t)M * K);
  const size_t sx_b = align256((size_t)M * 4);
  const size_t wq_b = align256((size_t)N * K);
  const size_t sw_b = align256((size_t)N * 4);
  char* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    const int rc = grow(&ds->i8, &ds->i8_bytes, xq_b + sx_b + wq_b + sw_b);
    if (rc != LTX25_OK) { return rc; }
    base = (char*)ds->i8;
  }
  int8_t* xq = (int8_t*)base;
  float* sx = (float*)(base + xq_b);
  int8_t* wq = (int8_t*)(base + xq_b + sx_b);
  float* sw = (float*)(base + xq_b + sx_b + wq_b);
  hipError_t e = ltx25::launch_i8_quantize_rows((const uint16_t*)x, xq, sx, M, K, st);
  if (e != hipSuccess) { return hip_fail(e, "i8 quantize (x)"); }
  if (w->quantized) {
    e = ltx25::launch_i8_quantize_qweight(w->codes, (const uint16_t*)w->scales,
                                          (const uint16_t*)w->qbias, w->bits,
                                          w->group, wq, sw, N, K, st);
  } else {
    e = ltx25::launch_i8_quantize_rows((const uint16_t*)w->w, wq, sw, N, K, st);
  }
  if (e != hipSuccess) { return hip_fail(e, "i8 quantize (w)"); }
  e = ltx25::launch_i8_gemm(xq, sx, wq, sw, bias, bias != nullptr ? bias_dtype : 0, epilogue,
                            (uint16_t*)y, nullptr, M, K, N, st);
  if (e != hipSuccess) { return hip_fail(e, "i8 gemm launch"); }
  return LTX25_OK;
}

// The LoRA delta as the reference's matrix-core pair (lora_mma_,
// src/ltx25-metal-ops.cc:938-987): r = bf16(x . A^T) on the dense GEMM, then
// y = bf16(y + r . B^T) on the dense GEMM with its accumulate epilogue. The
// rank is padded to a multiple of 64 (A's extra rows and B's extra columns
// zero, so r's extra columns are zero and add nothing). Taken from rank
// kLoraPairMinRank up, where the adapter's FLOPs outweigh re-reading y:
// below it the fused one-pass kernel, bound by y's traffic, is faster.
constexpr int kLoraPairMinRank = 96;
// From this many tokens a narrow adapter's r = x . A^T is computed once by
// the dense GEMM rather than per column split inside the fused kernel.
constexpr int kLoraRFirstMinM = 512;

// The LoRA routes' preconditions. Each is what its kernels need to be
// correct; the AUTO thresholds sit on top of them (lora_route).
bool lora_pair_ok(int M, int K, int N, int rank, const void* x, const void* y)
{
  const size_t rk = (size_t)((rank + 63) & ~63);
  return K % 64 == 0 && N % 8 == 0 && aligned16(x) && aligned16(y) &&
         below_limit((size_t)M * K * 2) && below_limit((size_t)M * N * 2) &&
         below_limit(rk * K * 2) && below_limit((size_t)N * rk * 2) &&
         below_limit((size_t)M * rk * 2);
}

// The fused kernel's vector path: 16-byte operand loads and 32-bit buffer
// offsets. B is copied with its rank padded to a multiple of 8 when it is
// not already (so b's alignment is not a condition).
bool lora_vec_ok(int M, int K, int N, int rank, const void* x, const void* a, const void* y)
{
  const int rank8 = (rank + 7) & ~7;
  return K % 8 == 0 && N % 8 == 0 && aligned16(x) && aligned16(a) && aligned16(y) &&
         below_limit((size_t)M * K * 2) && below_limit((size_t)M * N * 2) &&
         below_limit((size_t)rank * K * 2) && below_limit((size_t)N * rank8 * 2);
}

bool lora_rfirst_ok(int M, int K, int N, int rank, const void* x, const void* a, const void* y)
{
  return lora_vec_ok(M, K, N, rank, x, a, y) && K % 64 == 0 && rank % 8 == 0 &&
         rank <= ltx25::kLoraMaxRank && below_limit((size_t)M * rank * 2);
}

std::atomic<int> g_lora_force{LTX25_LORA_AUTO};

// The route ltx25_lora_add takes (LTX25_LORA_*), or -1 with the error set
// when a forced route cannot take the shape.
int lora_route(int M, int K, int N, int rank, const void* x, const void* a, const void* y)
{
  if (M <= 0 || K <= 0 || N <= 0 || rank <= 0) { return LTX25_LORA_NONE; }
  const int force = g_lora_force.load(std::memory_order_relaxed);
  if (force == LTX25_LORA_PAIR) {
    if (lora_pair_ok(M, K, N, rank, x, y)) { return LTX25_LORA_PAIR; }
    fail(LTX25_E_UNSUPPORTED, "the forced LoRA GEMM pair needs K %% 64 == 0, N %% 8 == 0, "
         "16-byte aligned x and y and operands under 2 GiB (M=%d K=%d N=%d rank=%d)",
         M, K, N, rank);
    return -1;
  }
  if (force == LTX25_LORA_RFIRST) {
    if (lora_rfirst_ok(M, K, N, rank, x, a, y)) { return LTX25_LORA_RFIRST; }
    fail(LTX25_E_UNSUPPORTED, "the forced r-first LoRA route needs the vector path, "
         "K %% 64 == 0 and rank %% 8 == 0, rank <= %d (M=%d K=%d N=%d rank=%d)",
         ltx25::kLoraMaxRank, M, K, N, rank);
    return -1;
  }
  if (force == LTX25_LORA_FUSED) { return LTX25_LORA_FUSED; }
  if (rank >= kLoraPairMinRank && M >= 256 && lora_pair_ok(M, K, N, rank, x, y)) {
    return LTX25_LORA_PAIR;
  }
  if (M >= kLoraRFirstMinM && lora_rfirst_ok(M, K, N, rank, x, a, y)) {
    return LTX25_LORA_RFIRST;
  }
  return LTX25_LORA_FUSED;
}

int lora_pair(DeviceState* ds, hipStream_t st, const void* x, const void* a, const void* b,
              void* y, void* r_caller, int M, int K, int N, int rank)
{
  const int rk = (rank + 63) & ~63;
  // A's rows past `rank` read as zeros (the GEMM's weight-row bound), so A
  // is copied only when it is not 16-byte aligned or the r GEMM plans the
  // M <= 128 kernel, which takes whole weights only; B gets zero columns up
  // to rk. The caller's r ([M][rank]) holds r when it has rk columns.
  const ltx25::GemmPlan r_plan = ltx25::plan_gemm(M, rk, K, 16, ds->cu_count);
  const bool pad_a = !aligned16(a) || (rk != rank && r_plan.tile == 2);
  const bool pad_b = rk != rank || !aligned16(b);
  const bool own_r = r_caller == nullptr || rk != rank || !aligned16(r_caller);
  const size_t a_bytes = pad_a ? align256((size_t)rk * K * 2) : 0;
  const size_t r_bytes = own_r ? align256((size_t)M * rk * 2) : 0;
  const size_t b_bytes = pad_b ? align256((size_t)N * rk * 2) : 0;
  char* base = nullptr;
  if (a_bytes + r_bytes + b_bytes > 0) {
    std::lock_guard<std::mutex> lk(g_mu);
    const int rc = grow(&ds->lora_mm, &ds->lora_mm_bytes, a_bytes + r_bytes + b_bytes);
    if (rc != LTX25_OK) { return rc; }
    base = (char*)ds->lora_mm;
  }
  const uint16_t* pa = (const uint16_t*)a;
  uint16_t* pr = own_r ? (uint16_t*)(base + a_bytes) : (uint16_t*)r_caller;
  const uint16_t* pb = (const uint16_t*)b;
  if (pad_a) {
    // A [rank][K] -> [rk][K]: one row of rank*K elements, zero-filled to rk*K
    const hipError_t e = ltx25::launch_lora_pad(pa, 1, rank * K, rank * K, (uint16_t*)base,
                                                rk * K, st);
    if (e != hipSuccess) { return hip_fail(e, "lora pad launch"); }
    pa = (const uint16_t*)base;
  }
  if (pad_b) {
    uint16_t* dst = (uint16_t*)(base + a_bytes + r_bytes);
    const hipError_t e = ltx25::launch_lora_pad(pb, N, rank, rank, dst, rk, st);
    if (e != hipSuccess) { return hip_fail(e, "lora pad launch"); }
    pb = dst;
  }
  for (int half = 0; half < 2; ++half) {
    ltx25::GemmDesc d;
    d.bits = 16;
    d.group = 64;
    d.M = M;
    if (half == 0) {
      d.x = (const uint16_t*)x;
      d.w = pa;
      d.wn = pad_a ? rk : rank;
      d.y = pr;
      d.N = rk;
      d.K = K;
    } else {
      d.x = pr;
      d.w = pb;
      d.y = (uint16_t*)y;
      d.y_in = (const uint16_t*)y;
      d.N = N;
      d.K = rk;
    }
    const ltx25::GemmPlan plan =
        half == 0 ? r_plan
                  : ltx25::plan_gemm(d.M, d.N, d.K, d.bits, ds->cu_count,
                                     g_tile.load(std::memory_order_relaxed));
    float* ws = nullptr;
    if (plan.workspace_bytes > 0) {
      std::lock_guard<std::mutex> lk(g_mu);
      const int rc = grow(&ds->ws, &ds->ws_bytes, plan.workspace_bytes);
      if (rc != LTX25_OK) { return rc; }
      ws = (float*)ds->ws;
    }
    const hipError_t e = ltx25::launch_gemm(d, plan, ws, st);
    if (e != hipSuccess) { return hip_fail(e, "lora gemm launch"); }
  }
  return LTX25_OK;
}

// The LoRA fold: the adapter rides inside the linear's own GEMM as extra K,
//   y = epi([x | r] . [W | B]^T + bias),  r = bf16(x . A^T),
// where W is the dequant-once expansion written with row stride K + rk
// (rk = rank rounded up to 64) and B fills the last rk columns of each row
// (zeros past `rank`), and r [M][rk] comes from the dense GEMM over A
// padded to rk zero rows. The delta costs the r GEMM and rk / K more of
// the linear, instead of a second pass over y (read + write). Rounding:
// one bf16 rounding of x . W^T + bias + r . B^T, where the reference's
// linear + lora_add round twice (src/ltx25-metal-ops.cc:940-1004); before
// the GELU, as the reference applies the adapter
// (src/ltx25-block-metal.cc:639-648).
// On w8 codes the adapter is merged into the expansion instead
// (ltx25::launch_dequant_merge): W' = bf16(W + B . A), then the linear runs
// at its own K over W'. (x . A^T) . B^T = x . (B . A)^T, so no r GEMM and no
// extra K; one rounding per weight element and one of the output. Taken up
// to rank 64 (kMergeMaxRank): above it the merge kernel is LDS-bound and
// the extra K costs less.
struct FoldPlan {
  bool takes = false;
  int rk = 0;
  int bits = 0;
  bool merge = false;        // the shape allows the merge (pointers checked at run time)
  ltx25::GemmPlan r_plan;
  ltx25::GemmPlan plan;
  ltx25::GemmPlan merge_plan;   // the linear over W' [N][K]
};

FoldPlan plan_fold(int M, int K, int N, int rank, int bits, int cu_count, const void* x,
                   const void* y)
{
  FoldPlan f;
  if (M <= 0 || K <= 0 || N <= 0 || rank <= 0 || (bits != 8 && bits != 4)) { return f; }
  if (K % 64 != 0 || N % 8 != 0 || (x != nullptr && !aligned16(x)) ||
      (y != nullptr && !aligned16(y))) {
    return f;
  }
  LinearRoute route;
  if (plan_linear(M, K, N, bits, cu_count, &route) != LTX25_OK) {
    g_err.clear();
    return f;
  }
  if (route.i8 || !route.deq_once || route.slabs != 1) { return f; }
  const int rk = (rank + 63) & ~63;
  const int kt = K + rk;
  if (!below_limit((size_t)N * kt * 2) || !below_limit((size_t)M * rk * 2) ||
      !below_limit((size_t)rk * K * 2) || !below_limit((size_t)M * K * 2) ||
      !below_limit((size_t)M * N * 2)) {
    return f;
  }
  const int tile = g_tile.load(std::memory_order_relaxed);
  f.plan = ltx25::plan_gemm(M, N, kt, 16, cu_count, tile);
  if (f.plan.tile == 2) { return f; }
  f.r_plan = ltx25::plan_gemm(M, rk, K, 16, cu_count);
  // the merge's shape rule (A's alignment and the group size are checked
  // at run time; B is copied with its rank padded to 8 when it needs to be)
  f.merge = ltx25::dequant_merge_takes(bits, N, K, rank, (rank + 7) & ~7, nullptr, nullptr);
  if (f.merge) {
    f.merge_plan = ltx25::plan_gemm(M, N, K, 16, cu_count, tile);
    f.merge = f.merge_plan.tile != 2;
  }
  f.rk = rk;
  f.bits = bits;
  f.takes = true;
  return f;
}

int run_fold(DeviceState* ds, hipStream_t st, const FoldPlan& f, const void* x,
             const ltx25_qweight* w, const void* bias, int bias_dtype, const void* a,
             const void* b, int rank, void* y, int M, int K, int N, int epilogue)
{
  if (f.merge && aligned16(a) && (w->group == 32 || w->group == 64)) {
    // W' = bf16(W + B . A), then y = epi(x . W'^T + bias); B is copied with
    // its rank padded to a multiple of 8 (zero columns) when its rows are not
    // whole 16-byte pieces
    const int rank8 = (rank + 7) & ~7;
    const bool pad_b = rank8 != rank || !aligned16(b);
    uint16_t* wd = nullptr;
    uint16_t* bp = nullptr;
    float* ws = nullptr;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      int rc = grow(&ds->deq, &ds->deq_bytes, (size_t)N * K * 2);
      if (rc != LTX25_OK) { return rc; }
      if (pad_b) {
        rc = grow(&ds->lora_mm, &ds->lora_mm_bytes, (size_t)N * rank8 * 2);
        if (rc != LTX25_OK) { return rc; }
        bp = (uint16_t*)ds->lora_mm;
      }
      if (f.merge_plan.workspace_bytes > 0) {
        rc = grow(&ds->ws, &ds->ws_bytes, f.merge_plan.workspace_bytes);
        if (rc != LTX25_OK) { return rc; }
        ws = (float*)ds->ws;
      }
      wd = (uint16_t*)ds->deq;
    }
    hipError_t e = hipSuccess;
    if (pad_b) {
      e = ltx25::launch_lora_pad((const uint16_t*)b, N, rank, rank, bp, rank8, st);
      if (e != hipSuccess) { return hip_fail(e, "fold: B pad launch"); }
    }
    e = ltx25::launch_dequant_merge(
        (const uint8_t*)w->codes, (const uint16_t*)w->scales, (const uint16_t*)w->qbias,
        w->group, (const uint16_t*)a, pad_b ? bp : (const uint16_t*)b, rank,
        pad_b ? rank8 : rank, wd, N, K, st);
    if (e != hipSuccess) { return hip_fail(e, "fold: merge launch"); }
    ltx25::GemmDesc d;
    d.x = (const uint16_t*)x;
    d.w = wd;
    d.bits = 16;
    d.group = 64;
    d.bias = bias;
    d.bias_type = bias != nullptr ? bias_dtype : ltx25::kBiasNone;
    d.epilogue = epilogue;
    d.y = (uint16_t*)y;
    d.M = M;
    d.N = N;
    d.K = K;
    e = ltx25::launch_gemm(d, f.merge_plan, ws, st);
    if (e != hipSuccess) { return hip_fail(e, "fold: gemm launch"); }
    return LTX25_OK;
  }
  const int rk = f.rk;
  const int kt = K + rk;
  // A [rank][K] is read as an [rk][K] weight whose rows past `rank` are
  // zeros (the buffer range stops at A's end); copied with zero rows only
  // when it is not 16-byte aligned or the r GEMM plans the M <= 128 kernel
  const bool pad_a = !aligned16(a) || f.r_plan.tile == 2;
  const size_t a_bytes = pad_a ? align256((size_t)rk * K * 2) : 0;
  const size_t r_bytes = align256((size_t)M * rk * 2);
  uint16_t* wd = nullptr;
  char* base = nullptr;
  float* ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = grow(&ds->deq, &ds->deq_bytes, (size_t)N * kt * 2);
    if (rc != LTX25_OK) { return rc; }
    rc = grow(&ds->lora_mm, &ds->lora_mm_bytes, a_bytes + r_bytes);
    if (rc != LTX25_OK) { return rc; }
    const size_t wsb = std::max(f.plan.workspace_bytes, f.r_plan.workspace_bytes);
    if (wsb > 0) {
      rc = grow(&ds->ws, &ds->ws_bytes, wsb);
      if (rc != LTX25_OK) { return rc; }
      ws = (float*)ds->ws;
    }
    wd = (uint16_t*)ds->deq;
    base = (char*)ds->lora_mm;
  }
  // r = bf16(x . A^T), then [W | B]: both ahead of the main GEMM on `st` (on
  // a second stream beside the expansion they were measured slower: the two
  // kernels slow each other and the fork / join costs ~19 us of gaps)
  const uint16_t* pa = (const uint16_t*)a;
  hipError_t e = hipSuccess;
  if (pad_a) {
    e = ltx25::launch_lora_pad(pa, 1, rank * K, rank * K, (uint16_t*)base, rk * K, st);
    if (e != hipSuccess) { return hip_fail(e, "fold: A pad launch"); }
    pa = (const uint16_t*)base;
  }
  uint16_t* r = (uint16_t*)(base + a_bytes);
  ltx25::GemmDesc rd;
  rd.x = (const uint16_t*)x;
  rd.w = pa;
  rd.bits = 16;
  rd.group = 64;
  rd.y = r;
  rd.M = M;
  rd.N = rk;
  rd.wn = pad_a ? rk : rank;
  rd.K = K;
  e = ltx25::launch_gemm(rd, f.r_plan, ws, st);
  if (e != hipSuccess) { return hip_fail(e, "fold: r gemm launch"); }
  // [W | B]: the expansion at row stride K + rk, B in each row's last rk columns
  e = ltx25::launch_dequant(w->codes, (const uint16_t*)w->scales, (const uint16_t*)w->qbias,
                            w->bits, w->group, wd, N, K, st, kt, (const uint16_t*)b, rank, rank);
  if (e != hipSuccess) { return hip_fail(e, "fold: dequant launch"); }
  // y = epi([x | r] . [W | B]^T + bias)
  ltx25::GemmDesc d;
  d.x = (const uint16_t*)x;
  d.x2 = r;
  d.kx = K;
  d.w = wd;
  d.bits = 16;
  d.group = 64;
  d.bias = bias;
  d.bias_type = bias != nullptr ? bias_dtype : ltx25::kBiasNone;
  d.epilogue = epilogue;
  d.y = (uint16_t*)y;
  d.M = M;
  d.N = N;
  d.K = kt;
  e = ltx25::launch_gemm(d, f.plan, ws, st);
  if (e != hipSuccess) { return hip_fail(e, "fold: gemm launch"); }
  return LTX25_OK;
}

// The reference's init-time route knobs (src/ltx25-metal-ops.cc:186-231) and
// the int8 tier's VPIPE_I8_GEMM, mapped onto this library's switches. Only
// variables that are set change a switch.
void apply_env_overrides()
{
  // the int8 tier sits under the matrix-core GEMM (src/ltx25-metal-ops.cc:
  // 386-391), so VPIPE_LTX25_NO_MMA below overrides VPIPE_I8_GEMM=1
  if (const char* e = std::getenv("VPIPE_I8_GEMM")) {
    if (std::strcmp(e, "0") == 0) { g_i8_on.store(0, std::memory_order_relaxed); }
    if (std::strcmp(e, "1") == 0) { g_i8_on.store(1, std::memory_order_relaxed); }
  }
  if (std::getenv("VPIPE_LTX25_NO_MMA") != nullptr) {
    g_deq_once.store(LTX25_DEQUANT_ONCE_OFF, std::memory_order_relaxed);
    g_i8_on.store(0, std::memory_order_relaxed);
  }
  if (std::getenv("VPIPE_LTX25_NO_DEQUANT_MMA") != nullptr) {
    g_deq_once.store(LTX25_DEQUANT_ONCE_OFF, std::memory_order_relaxed);
  }
  if (const char* e = std::getenv("VPIPE_LTX25_MMA_MIN_M")) {
    const int v = std::atoi(e);
    if (v > 0) { g_deq_min_m.store(v, std::memory_order_relaxed); }
  }
  if (const char* e = std::getenv("VPIPE_LTX25_MMA_TILE")) {
    const int v = std::atoi(e);
    if (v == 128) { g_tile.store(LTX25_TILE_MID, std::memory_order_relaxed); }
    if (v == 256 || v == 512) { g_tile.store(LTX25_TILE_TALL, std::memory_order_relaxed); }
  }
  if (std::getenv("VPIPE_LTX25_NO_LORA_MMA") != nullptr) {
    g_lora_force.store(LTX25_LORA_FUSED, std::memory_order_relaxed);
  }
}

}  // namespace

extern "C" {

int ltx25_init(void)
{
  apply_env_overrides();
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  // set-up of the no-allocation linear: this device's scratch address
  void* p = nullptr;
  const hipError_t e = ltx25::noalloc_scratch(&p);
  if (e != hipSuccess) { return hip_fail(e, "hipGetSymbolAddress (no-allocation scratch)"); }
  return LTX25_OK;
}

const char* ltx25_last_error(void) { return g_err.c_str(); }

int ltx25_quant_available(void)
{
  DeviceState* ds = nullptr;
  return current_device(&ds) == LTX25_OK ? 1 : 0;
}

int ltx25_linear_q(void* stream, const void* x, const ltx25_qweight* w,
                   const void* bias, int bias_dtype, void* y, int M, int K,
                   int N)
{
  return run_linear((hipStream_t)stream, x, w, bias, bias_dtype, y, M, K, N,
                    LTX25_EPI_NONE);
}

int ltx25_linear_q_ex(void* stream, const void* x, const ltx25_qweight* w,
                      const void* bias, int bias_dtype, void* y, int M, int K,
                      int N, int epilogue)
{
  return run_linear((hipStream_t)stream, x, w, bias, bias_dtype, y, M, K, N,
                    epilogue);
}

int ltx25_linear_q_noalloc(void* stream, const void* x, const ltx25_qweight* w,
                           const void* bias, int bias_dtype, void* y, int M, int K, int N,
                           int epilogue)
{
  return run_linear((hipStream_t)stream, x, w, bias, bias_dtype, y, M, K, N, epilogue, true);
}

size_t ltx25_noalloc_scratch_bytes(void) { return ltx25::kNoAllocScratchBytes; }

int ltx25_linear(void* stream, const void* x, const void* w_bf16,
                 const void* bias, int bias_dtype, void* y, int M, int K,
                 int N)
{
  ltx25_qweight w;
  std::memset(&w, 0, sizeof w);
  w.w = w_bf16;
  w.quantized = 0;
  return run_linear((hipStream_t)stream, x, &w, bias, bias_dtype, y, M, K, N,
                    LTX25_EPI_NONE);
}

int ltx25_bias_add(void* stream, void* y, const void* bias, int bias_dtype,
                   int M, int N)
{
  if (y == nullptr || bias == nullptr) { return fail(LTX25_E_INVAL, "y or bias is null"); }
  if (bias_dtype != LTX25_DT_BF16 && bias_dtype != LTX25_DT_F32) {
    return fail(LTX25_E_INVAL, "bias dtype %d is not bf16 or f32", bias_dtype);
  }
  if (M <= 0 || N <= 0) { return fail(LTX25_E_INVAL, "M=%d N=%d must be positive", M, N); }
  if (check_aligned("y", y) != LTX25_OK) { return LTX25_E_INVAL; }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_bias_add((uint16_t*)y, bias, bias_dtype, M, N,
                                              (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "bias_add launch");
}

int ltx25_gelu_tanh(void* stream, const void* x, void* y, size_t n)
{
  if (x == nullptr || y == nullptr) { return fail(LTX25_E_INVAL, "x or y is null"); }
  if (n == 0) { return LTX25_OK; }
  if (check_aligned("x", x) != LTX25_OK || check_aligned("y", y) != LTX25_OK) {
    return LTX25_E_INVAL;
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_gelu((const uint16_t*)x, (uint16_t*)y, n,
                                          (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "gelu launch");
}

int ltx25_gate_heads(void* stream, void* y, const void* logits, int heads, int tokens,
                     int head_dim)
{
  if (heads <= 0 || tokens <= 0 || head_dim <= 0) { return LTX25_OK; }
  if (y == nullptr || logits == nullptr) { return fail(LTX25_E_INVAL, "y or logits is null"); }
  if ((((uintptr_t)y | (uintptr_t)logits) & 1u) != 0) {
    return fail(LTX25_E_INVAL, "a bf16 tensor is not 2-byte aligned");
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_gate_heads((uint16_t*)y, (const uint16_t*)logits, heads,
                                                tokens, head_dim, (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "gate_heads launch");
}

int ltx25_dequant(void* stream, const ltx25_qweight* w, void* out_bf16, int N,
                  int K)
{
  if (out_bf16 == nullptr) { return fail(LTX25_E_INVAL, "out is null"); }
  if (N <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "N=%d K=%d must be positive", N, K); }
  int rc = check_qweight(w, K);
  if (rc != LTX25_OK) { return rc; }
  if (!w->quantized) { return fail(LTX25_E_INVAL, "dequant needs a quantized weight"); }
  if ((rc = check_aligned("codes", w->codes)) != LTX25_OK ||
      (rc = check_aligned("out", out_bf16)) != LTX25_OK) {
    return rc;
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_dequant(w->codes, (const uint16_t*)w->scales,
                                             (const uint16_t*)w->qbias, w->bits,
                                             w->group, (uint16_t*)out_bf16, N, K,
                                             (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "dequant launch");
}

int ltx25_set_dequant_once(int mode)
{
  if (mode != LTX25_DEQUANT_ONCE_OFF && mode != LTX25_DEQUANT_ONCE_ON &&
      mode != LTX25_DEQUANT_ONCE_AUTO) {
    return fail(LTX25_E_INVAL, "dequant-once mode %d is not OFF, ON or AUTO", mode);
  }
  g_deq_once.store(mode, std::memory_order_relaxed);
  return LTX25_OK;
}

int ltx25_dequant_once_takes(int M, int K, int N)
{
  const int mode = g_deq_once.load(std::memory_order_relaxed);
  if (mode == LTX25_DEQUANT_ONCE_OFF) { return 0; }
  if (M < 64 || N < 16 || K <= 0 || K % 64 != 0) { return 0; }
  return mode == LTX25_DEQUANT_ONCE_ON || M >= g_deq_min_m.load(std::memory_order_relaxed) ? 1
                                                                                           : 0;
}

int ltx25_lora_on_matrix_cores(int M, int K, int N, int rank)
{
  // the reference's question: does this shape take the matrix-core GEMM
  // pair (src/ltx25-metal-ops.cc:921-936)? Pointers as any allocator returns.
  const void* p = (const void*)(uintptr_t)256;
  return lora_route(M, K, N, rank, p, p, p) == LTX25_LORA_PAIR ? 1 : 0;
}

int ltx25_set_lora_matrix_cores(int on)
{
  g_lora_force.store(on != 0 ? LTX25_LORA_AUTO : LTX25_LORA_FUSED, std::memory_order_relaxed);
  return LTX25_OK;
}

int ltx25_set_lora_route(int route)
{
  if (route != LTX25_LORA_AUTO && route != LTX25_LORA_PAIR && route != LTX25_LORA_RFIRST &&
      route != LTX25_LORA_FUSED) {
    return fail(LTX25_E_INVAL, "LoRA route %d is not AUTO, PAIR, RFIRST or FUSED", route);
  }
  g_lora_force.store(route, std::memory_order_relaxed);
  return LTX25_OK;
}

int ltx25_lora_route(const void* x, const void* a, const void* b, const void* y, int M, int K,
                     int N, int rank, int* route)
{
  (void)b;
  if (route == nullptr) { return fail(LTX25_E_INVAL, "route is null"); }
  const int r = lora_route(M, K, N, rank, x, a, y);
  if (r < 0) { return LTX25_E_UNSUPPORTED; }
  *route = r;
  return LTX25_OK;
}

int ltx25_lora_add(void* stream, const void* x, const void* a, const void* b,
                   void* y, void* r, void* d, int M, int K, int N, int rank)
{
  (void)d;
  // The reference returns without encoding anything for an empty shape
  // (src/ltx25-metal-ops.cc:996).
  if (M <= 0 || K <= 0 || N <= 0 || rank <= 0) { return LTX25_OK; }
  if (x == nullptr || a == nullptr || b == nullptr || y == nullptr) {
    return fail(LTX25_E_INVAL, "x, a, b or y is null");
  }
  if ((((uintptr_t)x | (uintptr_t)a | (uintptr_t)b | (uintptr_t)y) & 1u) != 0) {
    return fail(LTX25_E_INVAL, "a bf16 tensor is not 2-byte aligned");
  }
  const int route = lora_route(M, K, N, rank, x, a, y);
  if (route < 0) { return LTX25_E_UNSUPPORTED; }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  if (route == LTX25_LORA_PAIR) {
    return lora_pair(ds, (hipStream_t)stream, x, a, b, y, r, M, K, N, rank);
  }
  const int rank8 = (rank + 7) & ~7;
  const bool vec = lora_vec_ok(M, K, N, rank, x, a, y);
  const uint16_t* pa = (const uint16_t*)a;
  const uint16_t* pb = (const uint16_t*)b;
  int ldb = rank;
  if (vec && (rank != rank8 || !aligned16(b))) {
    {
      std::lock_guard<std::mutex> lk(g_mu);
      const int rc2 = grow(&ds->lora_b, &ds->lora_b_bytes, (size_t)N * rank8 * 2);
      if (rc2 != LTX25_OK) { return rc2; }
    }
    const hipError_t e = ltx25::launch_lora_pad(pb, N, rank, rank, (uint16_t*)ds->lora_b, rank8,
                                                (hipStream_t)stream);
    if (e != hipSuccess) { return hip_fail(e, "lora pad launch"); }
    pb = (const uint16_t*)ds->lora_b;
    ldb = rank8;
  }
  if (route == LTX25_LORA_RFIRST) {
    // Many tokens: r = bf16(x . A^T) once with the dense GEMM (A is the
    // [rank][K] weight of that linear), then the fused kernel's second
    // phase reads it -- instead of recomputing x . A^T for every column
    // split of a row block. Same roundings (r rounded once to bf16).
    // r goes to the caller's buffer when it has one ([M][rank], 16-byte
    // aligned), else to the library's scratch
    uint16_t* rb = (uint16_t*)r;
    if (rb == nullptr || !aligned16(rb)) {
      std::lock_guard<std::mutex> lk(g_mu);
      const int rc2 = grow(&ds->lora_mm, &ds->lora_mm_bytes, (size_t)M * rank * 2);
      if (rc2 != LTX25_OK) { return rc2; }
      rb = (uint16_t*)ds->lora_mm;
    }
    ltx25::GemmDesc gd;
    gd.x = (const uint16_t*)x;
    gd.w = pa;
    gd.bits = 16;
    gd.group = 64;
    gd.y = rb;
    gd.M = M;
    gd.N = rank;
    gd.K = K;
    const ltx25::GemmPlan plan = ltx25::plan_gemm(M, rank, K, 16, ds->cu_count);
    float* ws = nullptr;
    if (plan.workspace_bytes > 0) {
      std::lock_guard<std::mutex> lk(g_mu);
      const int rc2 = grow(&ds->ws, &ds->ws_bytes, plan.workspace_bytes);
      if (rc2 != LTX25_OK) { return rc2; }
      ws = (float*)ds->ws;
    }
    hipError_t e = ltx25::launch_gemm(gd, plan, ws, (hipStream_t)stream);
    if (e != hipSuccess) { return hip_fail(e, "lora r gemm launch"); }
    e = ltx25::launch_lora((const uint16_t*)x, pa, pb, (uint16_t*)y, M, K, N, rank, ldb, vec,
                           ds->cu_count, (hipStream_t)stream, rb);
    if (e != hipSuccess) { return hip_fail(e, "lora launch"); }
    return LTX25_OK;
  }
  for (int c = 0; c < rank; c += ltx25::kLoraMaxRank) {
    const int rp = rank - c < ltx25::kLoraMaxRank ? rank - c : ltx25::kLoraMaxRank;
    const hipError_t e = ltx25::launch_lora((const uint16_t*)x, pa + (size_t)c * K, pb + c,
                                            (uint16_t*)y, M, K, N, rp, ldb, vec,
                                            ds->cu_count, (hipStream_t)stream);
    if (e != hipSuccess) { return hip_fail(e, "lora launch"); }
  }
  return LTX25_OK;
}

int ltx25_lora_fold_takes(int M, int K, int N, int rank, int bits)
{
  return plan_fold(M, K, N, rank, bits, cu_count_hint(), nullptr, nullptr).takes ? 1 : 0;
}

int ltx25_linear_q_lora(void* stream, const void* x, const ltx25_qweight* w, const void* bias,
                        int bias_dtype, const void* a, const void* b, int rank, void* y, int M,
                        int K, int N, int epilogue)
{
  hipStream_t st = (hipStream_t)stream;
  // argument checks before any device work on either path (the fallback
  // below writes y with the linear before it reaches its own epilogue)
  if (epilogue != LTX25_EPI_NONE && epilogue != LTX25_EPI_GELU_TANH) {
    return fail(LTX25_E_INVAL, "unknown epilogue %d", epilogue);
  }
  if (!bias_ok(bias, bias_dtype)) {
    return fail(LTX25_E_INVAL, "bias dtype %d is not valid for a %s bias", bias_dtype,
                bias == nullptr ? "null" : "non-null");
  }
  if (rank > 0 && (a == nullptr || b == nullptr)) { return fail(LTX25_E_INVAL, "a or b is null"); }
  if (rank < 0) { return fail(LTX25_E_INVAL, "rank %d is negative", rank); }
  if (rank == 0 || M <= 0 || K <= 0 || N <= 0) {
    return run_linear(st, x, w, bias, bias_dtype, y, M, K, N, epilogue);
  }
  if ((((uintptr_t)a | (uintptr_t)b) & 1u) != 0) {
    return fail(LTX25_E_INVAL, "a bf16 adapter matrix is not 2-byte aligned");
  }
  const int bits = w != nullptr && w->quantized ? w->bits : 16;
  FoldPlan f = plan_fold(M, K, N, rank, bits, cu_count_hint(), x, y);
  if (f.takes) {
    // the linear's own checks (shape, weight, bias, epilogue, alignment)
    // before any device use: a dry run of its plan
    if (x == nullptr || y == nullptr) { return fail(LTX25_E_INVAL, "x or y is null"); }
    int rc = check_qweight(w, K);
    if (rc != LTX25_OK) { return rc; }
    if ((rc = check_aligned("weight", w->codes)) != LTX25_OK) { return rc; }
    DeviceState* ds = nullptr;
    rc = current_device(&ds);
    if (rc != LTX25_OK) { return rc; }
    if (ds->cu_count != cu_count_hint()) {
      f = plan_fold(M, K, N, rank, bits, ds->cu_count, x, y);
    }
    if (f.takes) {
      return run_fold(ds, st, f, x, w, bias, bias_dtype, a, b, rank, y, M, K, N, epilogue);
    }
  }
  // The reference's order: the linear, the adapter on its output, then the
  // GELU (src/ltx25-block-metal.cc:639-645).
  int rc = run_linear(st, x, w, bias, bias_dtype, y, M, K, N, LTX25_EPI_NONE);
  if (rc != LTX25_OK) { return rc; }
  rc = ltx25_lora_add(stream, x, a, b, y, nullptr, nullptr, M, K, N, rank);
  if (rc != LTX25_OK) { return rc; }
  if (epilogue == LTX25_EPI_GELU_TANH) { return ltx25_gelu_tanh(stream, y, y, (size_t)M * N); }
  return LTX25_OK;
}

int ltx25_probe_read(void* stream, const void* src, size_t bytes, void* sink, int blocks)
{
  if (src == nullptr || sink == nullptr) { return fail(LTX25_E_INVAL, "src or sink is null"); }
  if (bytes == 0 || bytes % 16 != 0 || !aligned16(src)) {
    return fail(LTX25_E_INVAL, "bytes=%zu must be a positive multiple of 16 from a 16-byte "
                "aligned src", bytes);
  }
  if (blocks < 1 || blocks > 65535) { return fail(LTX25_E_INVAL, "blocks=%d is not in 1..65535", blocks); }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_probe_read(src, bytes, (uint32_t*)sink, blocks,
                                                (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "probe read launch");
}

int ltx25_probe_mfma(void* stream, int iters, int random, int waves_per_simd, void* out)
{
  if (out == nullptr) { return fail(LTX25_E_INVAL, "out is null"); }
  if (iters < 1 || (random != 0 && random != 1) || (waves_per_simd != 1 && waves_per_simd != 2)) {
    return fail(LTX25_E_INVAL, "iters=%d random=%d waves_per_simd=%d: iters > 0, random 0 or 1, "
                "waves_per_simd 1 or 2", iters, random, waves_per_simd);
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_probe_mfma(iters, random, waves_per_simd, (float*)out,
                                                (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "probe mfma launch");
}

int ltx25_probe_skinny_phases(void* stream, const void* x, const ltx25_qweight* w,
                              const void* bias, int bias_dtype, void* y, int M, int K, int N,
                              int k_chunk, void* stamps, size_t stamps_bytes, int* splits_out)
{
  if (x == nullptr || y == nullptr || stamps == nullptr || splits_out == nullptr) {
    return fail(LTX25_E_INVAL, "x, y, stamps or splits_out is null");
  }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  rc = check_qweight(w, K);
  if (rc != LTX25_OK) { return rc; }
  if (!w->quantized || w->bits != 8) {
    return fail(LTX25_E_UNSUPPORTED, "the phase stamps are built for w8 weights only");
  }
  if (!bias_ok(bias, bias_dtype)) {
    return fail(LTX25_E_INVAL, "bias dtype %d is not valid for a %s bias",
                bias_dtype, bias == nullptr ? "null" : "non-null");
  }
  if ((rc = check_aligned("x", x)) != LTX25_OK || (rc = check_aligned("y", y)) != LTX25_OK ||
      (rc = check_aligned("weight", w->codes)) != LTX25_OK) {
    return rc;
  }
  if (k_chunk < 0 || k_chunk % 64 != 0 || k_chunk > 2048) {
    return fail(LTX25_E_INVAL, "k_chunk=%d: 0, or a multiple of 64 up to 2048", k_chunk);
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  ltx25::GemmPlan plan;
  if (K % 64 != 0 || !ltx25::plan_skinny(M, N, K, 8, ds->cu_count, plan)) {
    return fail(LTX25_E_UNSUPPORTED, "M=%d K=%d N=%d is not on the M <= 128 route", M, K, N);
  }
  if (k_chunk > 0) {
    plan.k_chunk = k_chunk;
    plan.splits = (K + k_chunk - 1) / k_chunk;
    plan.workspace_bytes = plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
  }
  const size_t tiles = (size_t)(N + 31) / 32;
  const size_t need = (size_t)plan.splits * tiles * 8 * 10 * sizeof(unsigned long long);
  if (stamps_bytes < need) {
    return fail(LTX25_E_INVAL, "stamps_bytes=%zu; %d splits x %zu tiles need %zu", stamps_bytes,
                plan.splits, tiles, need);
  }
  float* ws = nullptr;
  if (plan.workspace_bytes > 0) {
    std::lock_guard<std::mutex> lk(g_mu);
    rc = grow(&ds->ws, &ds->ws_bytes, plan.workspace_bytes);
    if (rc != LTX25_OK) { return rc; }
    ws = (float*)ds->ws;
  }
  ltx25::GemmDesc d;
  d.x = (const uint16_t*)x;
  d.w = w->codes;
  d.scales = (const uint16_t*)w->scales;
  d.qbias = (const uint16_t*)w->qbias;
  d.bits = 8;
  d.group = w->group;
  d.bias = bias;
  d.bias_type = bias != nullptr ? bias_dtype : ltx25::kBiasNone;
  d.epilogue = ltx25::kEpiNone;
  d.y = (uint16_t*)y;
  d.M = M;
  d.N = N;
  d.K = K;
  *splits_out = plan.splits;
  const hipError_t e = ltx25::launch_skinny(d, plan, ws, (hipStream_t)stream,
                                            (unsigned long long*)stamps);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "skinny phase-stamp launch");
}

// bytes of the 256 x 256 tile's phase stamps: eight u64 per wave, 8 waves per tile
static size_t tall_stamp_bytes(int M, int N)
{
  return (size_t)((M + 255) / 256) * ((N + 255) / 256) * 8 * 8 * sizeof(unsigned long long);
}

int ltx25_probe_tall_phases(void* stream, const void* x, const void* w_bf16, const void* bias,
                            int bias_dtype, void* y, int M, int K, int N, int epilogue,
                            void* stamps, size_t stamps_bytes)
{
  if (x == nullptr || w_bf16 == nullptr || y == nullptr || stamps == nullptr) {
    return fail(LTX25_E_INVAL, "x, w, y or stamps is null");
  }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  if (!bias_ok(bias, bias_dtype)) {
    return fail(LTX25_E_INVAL, "bias dtype %d is not valid for a %s bias",
                bias_dtype, bias == nullptr ? "null" : "non-null");
  }
  if (epilogue != LTX25_EPI_NONE && epilogue != LTX25_EPI_GELU_TANH) {
    return fail(LTX25_E_INVAL, "unknown epilogue %d", epilogue);
  }
  if ((rc = check_aligned("x", x)) != LTX25_OK || (rc = check_aligned("y", y)) != LTX25_OK ||
      (rc = check_aligned("w", w_bf16)) != LTX25_OK) {
    return rc;
  }
  if (K % 64 != 0 || N % 8 != 0) {
    return fail(LTX25_E_UNSUPPORTED, "K=%d N=%d: the 256 x 256 tile takes K %% 64 == 0 and "
                "N %% 8 == 0", K, N);
  }
  if (stamps_bytes < tall_stamp_bytes(M, N)) {
    return fail(LTX25_E_INVAL, "stamps_bytes=%zu; M=%d N=%d need %zu", stamps_bytes, M, N,
                tall_stamp_bytes(M, N));
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  ltx25::GemmDesc d;
  d.x = (const uint16_t*)x;
  d.w = w_bf16;
  d.bits = 16;
  d.group = 64;
  d.bias = bias;
  d.bias_type = bias != nullptr ? bias_dtype : ltx25::kBiasNone;
  d.epilogue = epilogue;
  d.y = (uint16_t*)y;
  d.M = M;
  d.N = N;
  d.K = K;
  const hipError_t e = ltx25::launch_tall_dense(d, (hipStream_t)stream,
                                                (unsigned long long*)stamps);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "tall phase-stamp launch");
}

int ltx25_probe_tall_i8_phases(void* stream, const int8_t* xq, const float* sx, const int8_t* wq,
                               const float* sw, const void* bias, int bias_dtype, void* y,
                               int M, int K, int N, void* stamps, size_t stamps_bytes)
{
  if (xq == nullptr || sx == nullptr || wq == nullptr || sw == nullptr || y == nullptr ||
      stamps == nullptr) {
    return fail(LTX25_E_INVAL, "null pointer");
  }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  if (!bias_ok(bias, bias_dtype)) { return fail(LTX25_E_INVAL, "bad bias dtype %d", bias_dtype); }
  if ((rc = check_aligned("xq", xq)) != LTX25_OK || (rc = check_aligned("wq", wq)) != LTX25_OK) {
    return rc;
  }
  if (!ltx25::tall_i8_takes(M, N, K)) {
    return fail(LTX25_E_UNSUPPORTED, "M=%d K=%d N=%d: the int8 256 x 256 tile takes K %% 128 "
                "== 0 and N %% 8 == 0", M, K, N);
  }
  if (stamps_bytes < tall_stamp_bytes(M, N)) {
    return fail(LTX25_E_INVAL, "stamps_bytes=%zu; M=%d N=%d need %zu", stamps_bytes, M, N,
                tall_stamp_bytes(M, N));
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_tall_i8(xq, sx, wq, sw, bias,
                                             bias != nullptr ? bias_dtype : ltx25::kBiasNone,
                                             ltx25::kEpiNone, (uint16_t*)y, nullptr, M, K, N,
                                             (hipStream_t)stream, (unsigned long long*)stamps);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "tall i8 phase-stamp launch");
}

int ltx25_set_i8_gemm(int on)
{
  g_i8_on.store(on != 0 ? 1 : 0, std::memory_order_relaxed);
  return LTX25_OK;
}

int ltx25_i8_takes(int M, int K, int N)
{
  return g_i8_on.load(std::memory_order_relaxed) != 0 && M >= 1024 && K >= 1024 &&
                 K % 128 == 0 && N >= 16 && below_limit((size_t)M * K) &&
                 below_limit((size_t)N * K) && below_limit((size_t)M * N * 2)
             ? 1
             : 0;
}

int ltx25_set_tile(int tile)
{
  if (tile != LTX25_TILE_AUTO && tile != LTX25_TILE_TALL && tile != LTX25_TILE_MID &&
      tile != LTX25_TILE_SKINNY) {
    return fail(LTX25_E_INVAL, "tile %d is not AUTO, TALL, MID or SKINNY", tile);
  }
  g_tile.store(tile, std::memory_order_relaxed);
  return LTX25_OK;
}

int ltx25_linear_route(int M, int K, int N, int bits, ltx25_route* out)
{
  if (out == nullptr) { return fail(LTX25_E_INVAL, "out is null"); }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  if (bits != 4 && bits != 8 && bits != 16) {
    return fail(LTX25_E_INVAL, "bits=%d; 4 or 8 (codes) or 16 (dense)", bits);
  }
  if (K % 64 != 0) {
    return fail(LTX25_E_UNSUPPORTED,
                "K=%d: the MFMA kernels step K by 64; pad K to a multiple of 64", K);
  }
  LinearRoute r;
  rc = plan_linear(M, K, N, bits, cu_count_hint(), &r);
  if (rc != LTX25_OK) { return rc; }
  std::memset(out, 0, sizeof *out);
  out->i8 = r.i8 ? 1 : 0;
  out->dequant_once = r.deq_once ? 1 : 0;
  out->tile = r.i8 ? 0
                   : (r.plan.tile == 0 ? LTX25_TILE_TALL
                                       : r.plan.tile == 1 ? LTX25_TILE_MID : LTX25_TILE_SKINNY);
  out->splits = r.i8 ? 1 : r.plan.splits;
  out->slabs = r.slabs;
  out->slab_rows = r.rows;
  out->scratch_bytes = r.scratch;
  return LTX25_OK;
}

int ltx25_i8_quantize_rows(void* stream, const void* x_bf16, int8_t* q,
                           float* scale, int M, int K)
{
  if (x_bf16 == nullptr || q == nullptr || scale == nullptr) {
    return fail(LTX25_E_INVAL, "null pointer");
  }
  if (M <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "M=%d K=%d must be positive", M, K); }
  if (K % 8 != 0) { return fail(LTX25_E_UNSUPPORTED, "K=%d is not a multiple of 8", K); }
  if (check_aligned("x", x_bf16) != LTX25_OK || check_aligned("q", q) != LTX25_OK) {
    return LTX25_E_INVAL;
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_i8_quantize_rows((const uint16_t*)x_bf16, q, scale,
                                                      M, K, (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "i8 quantize launch");
}

int ltx25_i8_quantize_qweight(void* stream, const ltx25_qweight* w,
                              int8_t* wq, float* sw, int N, int K)
{
  if (wq == nullptr || sw == nullptr) { return fail(LTX25_E_INVAL, "null pointer"); }
  if (N <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "N=%d K=%d must be positive", N, K); }
  int rc = check_qweight(w, K);
  if (rc != LTX25_OK) { return rc; }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  hipError_t e;
  if (w->quantized) {
    // 16-byte code loads and int8 stores
    if (check_aligned("codes", w->codes) != LTX25_OK || check_aligned("wq", wq) != LTX25_OK) {
      return LTX25_E_INVAL;
    }
    e = ltx25::launch_i8_quantize_qweight(w->codes, (const uint16_t*)w->scales,
                                          (const uint16_t*)w->qbias, w->bits, w->group,
                                          wq, sw, N, K, (hipStream_t)stream);
  } else {
    if (K % 8 != 0) { return fail(LTX25_E_UNSUPPORTED, "K=%d is not a multiple of 8", K); }
    if (check_aligned("w", w->w) != LTX25_OK || check_aligned("wq", wq) != LTX25_OK) {
      return LTX25_E_INVAL;
    }
    e = ltx25::launch_i8_quantize_rows((const uint16_t*)w->w, wq, sw, N, K,
                                       (hipStream_t)stream);
  }
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "i8 weight quantize launch");
}

int ltx25_i8_gemm(void* stream, const int8_t* xq, const float* sx,
                  const int8_t* wq, const float* sw, const void* bias,
                  int bias_dtype, void* y, int32_t* acc_dbg, int M, int K,
                  int N)
{
  if (xq == nullptr || sx == nullptr || wq == nullptr || sw == nullptr || y == nullptr) {
    return fail(LTX25_E_INVAL, "null pointer");
  }
  int rc = check_shape(M, K, N);
  if (rc != LTX25_OK) { return rc; }
  if (!bias_ok(bias, bias_dtype)) { return fail(LTX25_E_INVAL, "bad bias dtype %d", bias_dtype); }
  if (K % 128 != 0) {
    return fail(LTX25_E_UNSUPPORTED, "K=%d: the int8 MFMA kernel steps K by 128", K);
  }
  if ((rc = check_aligned("xq", xq)) != LTX25_OK || (rc = check_aligned("wq", wq)) != LTX25_OK) {
    return rc;
  }
  DeviceState* ds = nullptr;
  rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_i8_gemm(xq, sx, wq, sw, bias,
                                             bias != nullptr ? bias_dtype : 0,
                                             ltx25::kEpiNone, (uint16_t*)y, acc_dbg, M, K, N,
                                             (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "i8 gemm launch");
}

int ltx25_pack_codes(void* stream, const uint8_t* q, uint32_t* codes, int N,
                     int K, int bits)
{
  if (q == nullptr || codes == nullptr) { return fail(LTX25_E_INVAL, "null pointer"); }
  if (N <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "N=%d K=%d must be positive", N, K); }
  if ((bits != 4 && bits != 8) || ((long)K * bits) % 32 != 0) {
    return fail(LTX25_E_INVAL, "bits=%d K=%d do not fill whole u32 words", bits, K);
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_pack(q, codes, N, K, bits, (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "pack launch");
}

int ltx25_unpack_codes(void* stream, const uint32_t* codes, uint8_t* q,
                       int N, int K, int bits)
{
  if (q == nullptr || codes == nullptr) { return fail(LTX25_E_INVAL, "null pointer"); }
  if (N <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "N=%d K=%d must be positive", N, K); }
  if ((bits != 4 && bits != 8) || ((long)K * bits) % 32 != 0) {
    return fail(LTX25_E_INVAL, "bits=%d K=%d do not fill whole u32 words", bits, K);
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_unpack(codes, q, N, K, bits, (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "unpack launch");
}

int ltx25_quantize_affine(void* stream, const float* w, void* codes,
                          void* scales, void* qbias, int N, int K, int bits,
                          int group)
{
  if (w == nullptr || codes == nullptr || scales == nullptr || qbias == nullptr) {
    return fail(LTX25_E_INVAL, "null pointer");
  }
  if (N <= 0 || K <= 0) { return fail(LTX25_E_INVAL, "N=%d K=%d must be positive", N, K); }
  if (bits != 4 && bits != 8) { return fail(LTX25_E_INVAL, "bits=%d; only 4 and 8", bits); }
  if (group != 32 && group != 64) { return fail(LTX25_E_INVAL, "group=%d; only 32 and 64", group); }
  if (K % group != 0) { return fail(LTX25_E_INVAL, "K=%d is not a multiple of group %d", K, group); }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_quantize_affine(w, (uint32_t*)codes, (uint16_t*)scales,
                                                     (uint16_t*)qbias, N, K, bits, group,
                                                     (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "quantize launch");
}

int ltx25_f16_to_bf16(void* stream, const void* in_f16, void* out_bf16,
                      size_t n)
{
  if (in_f16 == nullptr || out_bf16 == nullptr) { return fail(LTX25_E_INVAL, "null pointer"); }
  if (n == 0) { return LTX25_OK; }
  if (check_aligned("in", in_f16) != LTX25_OK || check_aligned("out", out_bf16) != LTX25_OK) {
    return LTX25_E_INVAL;
  }
  DeviceState* ds = nullptr;
  const int rc = current_device(&ds);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = ltx25::launch_f16_to_bf16((const uint16_t*)in_f16, (uint16_t*)out_bf16,
                                                 n, (hipStream_t)stream);
  return e == hipSuccess ? LTX25_OK : hip_fail(e, "f16_to_bf16 launch");
}

int ltx25_qweight_infer(int K, long scales_cols, long codes_cols, int* bits,
                        int* group)
{
  if (bits == nullptr || group == nullptr) { return fail(LTX25_E_INVAL, "null out-pointer"); }
  if (K <= 0 || scales_cols <= 0 || codes_cols <= 0) {
    return fail(LTX25_E_INVAL, "K=%d, scales cols=%ld, codes cols=%ld must be positive",
                K, scales_cols, codes_cols);
  }
  const long g = (long)K / scales_cols;
  const long b = codes_cols * 32 / (long)K;
  if ((g != 32 && g != 64) || (b != 4 && b != 8) || scales_cols * g != (long)K ||
      codes_cols * 32 != (long)K * b) {
    return fail(LTX25_E_INVAL,
                "shapes do not close: K=%d, scales cols=%ld, codes cols=%ld", K,
                scales_cols, codes_cols);
  }
  if (*group != 0 && *group != (int)g) {
    return fail(LTX25_E_INVAL, "packed at group %ld but the checkpoint already used group %d",
                g, *group);
  }
  *group = (int)g;
  *bits = (int)b;
  return LTX25_OK;
}

}  // extern "C"
