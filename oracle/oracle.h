/*
 * CPU oracle for the w8g64 quantized linear and the int8 GEMM tier.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is
 * compared against. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. Nothing in the product path
 * links it, calls it or falls back to it.
 *
 * Each function restates one piece of the reference's semantics and cites
 * the reference file:line it follows (paths are into the
 * tgo-app-dev/vpipe-ltx-2.5 source tree). Plain C, single thread unless
 * the name says otherwise, built with -ffp-contract=off so every float
 * expression rounds exactly as written.
 *
 * Pinning (what checks each function against something other than itself;
 * the checks live in tests/test_oracle.py):
 *   orc_bf16_rne / orc_bf16_to_f32   torch's RNE float->bfloat16 cast, ties
 *                                    and specials included
 *   orc_f16_to_bf16                  numpy's IEEE half decoder + torch cast
 *   orc_pack_codes / orc_unpack      known words (LOW bits first) + round trip
 *   orc_quantize_affine              exact grid round trip, constant group,
 *                                    half-away rounding, clamp, error bound
 *   orc_dequant                      closed form fmaf(scale, q, bias)
 *   orc_linear_f32_omp               numpy float64 within the f32 bound of
 *                                    K products, thread-count invariant
 *   orc_fill_normal                  seeded determinism, Kolmogorov-Smirnov
 *                                    against N(0, 1), mean + stddev * z
 *   orc_linear_f64                   numpy float64 matmul, and bit-exact
 *                                    against the reference's own linear_
 *                                    (oracle/_ref, built from its sources)
 *   orc_gelu_tanh                    torch gelu(approximate="tanh") in f64,
 *                                    and bit-exact against the reference's
 *                                    stream_ff_ GELU (oracle/_ref)
 *   orc_bias_add_bf16                torch bf16 add of the same operands
 *   orc_gate_heads                   bit-exact against the reference's own
 *                                    attention_ gating (oracle/_ref, v = a
 *                                    constant, identity out-projection);
 *                                    float64 sigmoid within one bf16 ulp;
 *                                    logit 0 is the identity, +-large
 *                                    logits double / zero y
 *   orc_lora_add                     the reference test's own known answer
 *                                    (f64 over the unrounded draws, rel-L2
 *                                    < 2e-2), numpy float64 matmuls with the
 *                                    same bf16 rounding of r, A = 0 leaves y
 *                                    bit-identical, rank-1 outer product
 *   orc_i8_quantize_rows             numpy rint / absmax closed form
 *   orc_i8_gemm_i32                  numpy int64 matmul
 *   orc_i8_epilogue                  closed form via numpy float32 fma
 *   orc_i8_epilogue_ex               epilogue 0 equals orc_i8_epilogue; epilogue 1
 *                                    equals orc_i8_epilogue's f32 value through
 *                                    orc_gelu_tanh, then one bf16 rounding
 * Two dequantized weights appear. orc_quantize_affine's `deq` is the
 * reference test's CPU ground truth (scale * q, then + min: two f32
 * roundings, tests/ltx25-qlinear-test.cc:93-141). orc_dequant is
 * fmaf(scale, q, min) rounded once, then to bf16: the NORMATIVE weight of
 * every GPU route, which the routes reproduce bit for bit. The two differ
 * by at most one f32 ulp before the bf16 rounding; the GPU bars are set
 * against orc_dequant's weight.
 * Not pinned against the reference: the exact output bits of libvpipe's
 * GEMM kernels and of its I8GemmContext (not present in the reference
 * tree), so parity there is against the closed-form semantics above.
 */
#ifndef LTX25_ORACLE_H
#define LTX25_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---------------------------------------------------- */
uint16_t orc_bf16_rne(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n);
void orc_f16_to_bf16_n(const uint16_t* in_f16, uint16_t* out_bf16, size_t n);

/* ---- group-affine quantization (MLX layout) ---------------------------- */
int orc_quantize_affine(const float* w, int N, int K, int bits, int group,
                        uint32_t* codes, uint16_t* scales, uint16_t* biases,
                        float* deq);
int orc_pack_codes(const uint8_t* q, int N, int K, int bits, uint32_t* codes);
int orc_unpack_codes(const uint32_t* codes, int N, int K, int bits,
                     uint8_t* q);
int orc_dequant(const uint32_t* codes, const uint16_t* scales,
                const uint16_t* biases, int N, int K, int bits, int group,
                float* w_f32, uint16_t* w_bf16);

/* ---- linear, GELU, bias ------------------------------------------------ */
void orc_linear_f64(const float* x, const float* w, const float* bias, int M,
                    int K, int N, float* out);
void orc_linear_f64_d(const float* x, const float* w, const float* bias,
                      int M, int K, int N, double* out);
void orc_linear_f32_omp(const float* x, const float* w, const float* bias,
                        int M, int K, int N, float* out, int threads);
void orc_gelu_tanh(const float* in, float* out, size_t n);
void orc_gate_heads(uint16_t* y, const uint16_t* logits, int heads, int tokens, int head_dim);
void orc_bias_add_bf16(uint16_t* y, const uint16_t* bias, int M, int N);

/* ---- low-rank adapter delta --------------------------------------------- */
void orc_lora_add(const uint16_t* x, const uint16_t* a, const uint16_t* b,
                  uint16_t* y, int M, int K, int N, int rank);

/* ---- int8 tier ---------------------------------------------------------- */
void orc_i8_quantize_rows(const uint16_t* x_bf16, int M, int K, int8_t* q,
                          float* scale);
void orc_i8_gemm_i32(const int8_t* xq, const int8_t* wq, int M, int K, int N,
                     int32_t* acc);
void orc_i8_epilogue(const int32_t* acc, const float* sx, const float* sw,
                     const void* bias, int bias_dtype, int M, int N,
                     uint16_t* y);
void orc_i8_epilogue_ex(const int32_t* acc, const float* sx, const float* sw,
                        const void* bias, int bias_dtype, int epilogue, int M, int N,
                        uint16_t* y);

/* ---- seeded synthetic data --------------------------------------------- */
void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean,
                     float stddev);

#ifdef __cplusplus
}
#endif

#endif
