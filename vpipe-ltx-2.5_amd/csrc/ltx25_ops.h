// ltx25::Ops -- the reference plugin's op vocabulary for the quantized
// linear, over the C ABI in ltx25_qlinear.h.
//
// Mirrors ltx25::MetalOps (src/ltx25-metal-ops.h) member for member on this
// path: `init`, `linear` (dense and QWeight overloads), `bias_add`, `gelu`,
// `set_i8_gemm`, `i8_takes`, `quant_available`, and the QWeight type. The
// differences are the ones the platform forces: a hipStream_t stands where
// the ComputeEncoder stood, and device pointers where SharedBuffers stood.
//
// Error behaviour follows the reference: `init` returns false and fills
// `err`; the dispatch methods return void, as the reference's do, and a
// failure is held until the caller's `wait_ok` (the reference's callers
// learn of GPU failures at `wait_ok`, src/ltx25-dit.cc:1922-1933).
//
// Header-only: everything below compiles into the caller.
#pragma once

#include "ltx25_qlinear.h"

#include <hip/hip_runtime.h>

#include <string>

namespace ltx25 {

// One linear's weights, dense or group-affine quantized
// (src/ltx25-metal-ops.h:45-57).
struct QWeight {
  const void* w = nullptr;                 // dense bf16 [N][K]
  const void* codes = nullptr;             // u32 [N][K*bits/32]
  const void* scales = nullptr;            // bf16 [N][K/group]
  const void* qbias = nullptr;             // bf16 [N][K/group], zero point
  int bits = 0;
  int group = 0;
  bool quantized = false;

  bool empty() const noexcept
  {
    return quantized ? (codes == nullptr || scales == nullptr || qbias == nullptr)
                     : w == nullptr;
  }
};

class Ops {
public:
  // False (with `err` set) when no gfx950 device is current
  // (src/ltx25-metal-ops.h:64).
  bool init(std::string* err)
  {
    const int rc = ltx25_init();
    _ok = rc == LTX25_OK;
    if (!_ok && err != nullptr) { *err = ltx25_last_error(); }
    return _ok;
  }

  bool quant_available() const noexcept { return _ok && ltx25_quant_available() != 0; }

  // y[M][N] = x[M][K] @ W[N][K]^T (+ bias[N]), bias bf16 as in the
  // reference (src/ltx25-metal-ops.h:82-87).
  void linear(hipStream_t enc, const void* x, const void* w, const void* bias,
              void* y, int M, int K, int N) const
  {
    note(ltx25_linear(enc, x, w, bias, bias != nullptr ? LTX25_DT_BF16 : LTX25_DT_NONE, y,
                      M, K, N));
  }

  // The same over a weight that may be quantized (src/ltx25-metal-ops.h:
  // 100-105). The bias is fused into the GEMM epilogue.
  void linear(hipStream_t enc, const void* x, const QWeight& w, const void* bias,
              void* y, int M, int K, int N) const
  {
    const ltx25_qweight cw = to_c(w);
    note(ltx25_linear_q(enc, x, &cw, bias,
                        bias != nullptr ? LTX25_DT_BF16 : LTX25_DT_NONE, y, M, K, N));
  }

  // linear + GELU-tanh in one dispatch (the feed-forward's ff_in).
  void linear_gelu(hipStream_t enc, const void* x, const QWeight& w, const void* bias,
                   void* y, int M, int K, int N) const
  {
    const ltx25_qweight cw = to_c(w);
    note(ltx25_linear_q_ex(enc, x, &cw, bias,
                           bias != nullptr ? LTX25_DT_BF16 : LTX25_DT_NONE, y, M, K, N,
                           LTX25_EPI_GELU_TANH));
  }

  // y[M][N] += bias[N] (src/ltx25-metal-ops.h:297-300).
  void bias_add(hipStream_t enc, void* y, const void* bias, int M, int N) const
  {
    note(ltx25_bias_add(enc, y, bias, LTX25_DT_BF16, M, N));
  }

  void gelu(hipStream_t enc, const void* x, void* y, int n) const
  {
    note(ltx25_gelu_tanh(enc, x, y, (size_t)n));
  }

  // y[t][h][d] *= 2 sigmoid(logits[t][h]) (src/ltx25-metal-ops.cc:1089-1101).
  void gate_heads(hipStream_t enc, void* y, const void* logits, int heads, int tokens,
                  int head_dim) const
  {
    note(ltx25_gate_heads(enc, y, logits, heads, tokens, head_dim));
  }

  // y[M][N] += (x . a^T) . b^T (src/ltx25-metal-ops.h:107-133). `r` and `d`
  // keep the reference signature's caller scratch; the fused kernel uses
  // neither.
  void lora_add(hipStream_t enc, const void* x, const void* a, const void* b, void* y,
                void* r, void* d, int M, int K, int N, int rank) const
  {
    note(ltx25_lora_add(enc, x, a, b, y, r, d, M, K, N, rank));
  }
  bool lora_on_matrix_cores(int M, int K, int N, int rank) const noexcept
  {
    return ltx25_lora_on_matrix_cores(M, K, N, rank) != 0;
  }
  // A linear and its adapter as one call (the adapter before the GELU when
  // `gelu`): a call site's linear + lora_ pair (src/ltx25-block-metal.cc:
  // 428-436, 523-524, 639-648), folded into the GEMM where it can be.
  void linear_lora(hipStream_t enc, const void* x, const QWeight& w, const void* bias,
                   const void* a, const void* b, int rank, void* y, int M, int K, int N,
                   bool gelu = false) const
  {
    const ltx25_qweight cw = to_c(w);
    note(ltx25_linear_q_lora(enc, x, &cw, bias, bias != nullptr ? LTX25_DT_BF16 : LTX25_DT_NONE,
                             a, b, rank, y, M, K, N,
                             gelu ? LTX25_EPI_GELU_TANH : LTX25_EPI_NONE));
  }

  // The dequant-once arm (src/ltx25-metal-ops.cc:467-502): LTX25_DEQUANT_ONCE_*.
  void set_dequant_once(int mode) { note(ltx25_set_dequant_once(mode)); }

  // src/ltx25-metal-ops.h:151,157.
  void set_i8_gemm(bool on) { ltx25_set_i8_gemm(on ? 1 : 0); }
  bool i8_takes(int M, int K, int N) const noexcept { return ltx25_i8_takes(M, K, N) != 0; }

  // Commit-and-wait on the caller's side: drains `enc` and reports the
  // first dispatch failure since the last wait, or a device error.
  bool wait_ok(hipStream_t enc, std::string* err) const
  {
    const hipError_t e = hipStreamSynchronize(enc);
    if (!_failed && e == hipSuccess) { return true; }
    if (err != nullptr) {
      *err = _failed ? _err : std::string("hipStreamSynchronize: ") + hipGetErrorString(e);
    }
    _failed = false;
    _err.clear();
    return false;
  }

private:
  static ltx25_qweight to_c(const QWeight& w)
  {
    ltx25_qweight c;
    c.w = w.w;
    c.codes = w.codes;
    c.scales = w.scales;
    c.qbias = w.qbias;
    c.bits = w.bits;
    c.group = w.group;
    c.quantized = w.quantized ? 1 : 0;
    return c;
  }

  void note(int rc) const
  {
    if (rc != LTX25_OK && !_failed) {
      _failed = true;
      _err = ltx25_last_error();
    }
  }

  bool _ok = false;
  mutable bool _failed = false;
  mutable std::string _err;
};

}  // namespace ltx25
