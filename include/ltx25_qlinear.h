/*
 * ltx25_qlinear.h -- C ABI of the MI355X (gfx950) w8g64 quantized linear
 * and int8 GEMM tier.
 *
 * This is the drop-in boundary for the reference plugin's op vocabulary
 * (tgo-app-dev/vpipe-ltx-2.5, src/ltx25-metal-ops.h). Each entry point names
 * the reference interface it replaces. Conventions, all mirroring the
 * reference's:
 *
 *   - Tensors are caller-owned DEVICE pointers (the reference's
 *     SharedBuffer handles). Nothing here takes ownership.
 *   - Every op is asynchronous on the caller's stream (a hipStream_t passed
 *     as `void*`; NULL is the default stream), as the reference's ops only
 *     ENCODE into the caller's ComputeEncoder and the caller commits and
 *     waits (src/ltx25-dit.cc:1908-1933).
 *   - Weights are PyTorch [N out][K in] (src/ltx25-metal-ops.h:80-81);
 *     activations X are [M][K] bf16, outputs Y are [M][N] bf16, row-major,
 *     densely packed. Tensors the kernels move as 16-byte vectors (X, Y,
 *     weights / codes, int8 operands, and the inputs and outputs of the
 *     elementwise ops) must be 16-byte aligned; a misaligned pointer is
 *     refused with LTX25_E_INVAL.
 *   - Return value: LTX25_OK (0) or an LTX25_E_* code; the message for the
 *     last failure on the calling thread is ltx25_last_error(). This stands
 *     in for the reference's `std::string* err` out-parameter.
 *   - Ops that keep scratch (split-K partials, int8 operands) grow it on
 *     demand and share it across calls, like the reference's `_w_deq` and
 *     `_i8` scratch (src/ltx25-metal-ops.h:805-809,822-824,843-845): calls
 *     must be serialised on one stream, as the reference's serial encoder
 *     serialises them.
 *
 * Bias conventions: `bias` is [N] and its element type is `bias_dtype`
 * (LTX25_DT_NONE with bias == NULL, LTX25_DT_BF16 as in the reference, or
 * LTX25_DT_F32). In the fused epilogue the bias is added in f32 before the
 * single rounding to bf16.
 */
#ifndef LTX25_QLINEAR_H
#define LTX25_QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- return codes -------------------------------------------------------- */
#define LTX25_OK 0
#define LTX25_E_INVAL 1        /* bad argument: null pointer, bad shape       */
#define LTX25_E_UNSUPPORTED 2  /* well-formed, but no kernel takes it          */
#define LTX25_E_HIP 3          /* the HIP runtime reported an error            */
#define LTX25_E_NODEV 4        /* no gfx950 device is visible                  */
#define LTX25_E_DECLINED 5     /* the int8 tier declined this shape            */

/* ---- element types for bias ------------------------------------------------ */
#define LTX25_DT_NONE 0
#define LTX25_DT_BF16 1
#define LTX25_DT_F32 2

/* ---- fused epilogues -------------------------------------------------------- */
#define LTX25_EPI_NONE 0
#define LTX25_EPI_GELU_TANH 1  /* y = gelu_tanh(x.W^T + bias), in f32 */

/* One linear's weight, dense or group-affine quantized.
 * Replaces `QWeight` (src/ltx25-metal-ops.h:45-57).
 *   quantized == 0: `w` is bf16 [N][K].
 *   quantized != 0: `codes` is u32 [N][K*bits/32], LOW bits first (for
 *   bits == 8 this is exactly little-endian u8 [N][K]); `scales` and
 *   `qbias` are bf16 [N][K/group]; dequantized w = scale * q + qbias.
 *   `qbias` is the quantization zero point, NOT the linear's bias. */
typedef struct ltx25_qweight {
  const void* w;
  const void* codes;
  const void* scales;
  const void* qbias;
  int bits;       /* 4 or 8 */
  int group;      /* 32 or 64 */
  int quantized;  /* 0 = dense bf16 `w` */
} ltx25_qweight;

/* ---- lifecycle ------------------------------------------------------------ */

/* Select and check the device (the current HIP device must be gfx950) and
 * set up kernel attributes. Idempotent. Every compute entry point calls it
 * on first use.
 * Replaces MetalOps::init (src/ltx25-metal-ops.h:64).
 *
 * Route overrides from the environment, the reference's init-time A/B
 * knobs (src/ltx25-metal-ops.cc:186-231; the i8 tier's VPIPE_I8_GEMM,
 * src/ltx25-metal-ops.cc:749-757). Every call reads them, before the device
 * check (so a host without a GPU can still plan routes), and applies the
 * ones that are SET onto the process-wide switches below; an unset variable
 * leaves its switch as it is:
 *   VPIPE_LTX25_NO_MMA          dequant-once OFF and the int8 tier off: every
 *                               quantized weight runs the fused
 *                               dequant-in-GEMM kernel (the reference's qmm)
 *   VPIPE_LTX25_NO_DEQUANT_MMA  dequant-once OFF
 *   VPIPE_LTX25_MMA_MIN_M=v     v > 0: AUTO takes the dequant-once arm from
 *                               M >= v (the reference's gate on that arm)
 *   VPIPE_LTX25_MMA_TILE=t      128: LTX25_TILE_MID; 256 or 512:
 *                               LTX25_TILE_TALL; other values ignored
 *   VPIPE_LTX25_NO_LORA_MMA     LoRA route FUSED (no matrix-core pair)
 *   VPIPE_I8_GEMM=0|1           the int8 tier off / on
 * The reference keeps these per MetalOps instance; here they are
 * process-wide, so a knob set around one ltx25_init stays in force until a
 * setter or a later ltx25_init changes it. */
int ltx25_init(void);

/* Message for the last failure on this thread ("" when none). */
const char* ltx25_last_error(void);

/* 1 when the quantized kernels are available on this device (after a
 * successful ltx25_init), else 0.
 * Replaces MetalOps::quant_available (src/ltx25-metal-ops.h:294). */
int ltx25_quant_available(void);

/* ---- the linear ------------------------------------------------------------- */

/* y[M][N] = x[M][K] . dequant(W)^T (+ bias[N]), bf16 out, f32 accumulate.
 * A dense weight goes to ltx25_linear. K must be a multiple of the group.
 * Replaces MetalOps::linear(enc, x, const QWeight&, bias*, y, M, K, N)
 * (src/ltx25-metal-ops.h:100-105; dispatch at src/ltx25-metal-ops.cc:531-569),
 * with the bias pass fused into the GEMM epilogue instead of a second
 * ltx_bias_add dispatch. */
int ltx25_linear_q(void* stream, const void* x, const ltx25_qweight* w,
                   const void* bias, int bias_dtype, void* y, int M, int K,
                   int N);

/* ltx25_linear_q with a fused epilogue (LTX25_EPI_*): the feed-forward's
 * ff_in + GELU-tanh as one kernel (src/ltx25-block-metal.cc:639-646 issues
 * them as linear, then gelu). */
int ltx25_linear_q_ex(void* stream, const void* x, const ltx25_qweight* w,
                      const void* bias, int bias_dtype, void* y, int M, int K,
                      int N, int epilogue);

/* ltx25_linear_q_ex that allocates nothing: no hipMalloc, hipFree or
 * allocating library call, on any call. No counterpart in the reference;
 * it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation). Same kernels and
 * the same output bits as ltx25_linear_q_ex with the int8 tier off (the
 * in-register dequant stands in for the dequant-once expansion, which
 * produces the same bits). Split-K partials go to a fixed device array of
 * ltx25_noalloc_scratch_bytes() per GPU, held until the process ends and
 * resolved per device by ltx25_init or on the first call there (the HIP
 * runtime places the array in device memory at that point: call
 * ltx25_init on each device before capture or the serving loop).
 * LTX25_E_UNSUPPORTED when the plan's partials exceed that size, or when
 * the int8 tier is on and takes the shape. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race; calls ordered on one stream do not. Nothing in the array
 * needs to start at zero: each split writes its whole partial. */
int ltx25_linear_q_noalloc(void* stream, const void* x, const ltx25_qweight* w,
                           const void* bias, int bias_dtype, void* y, int M, int K,
                           int N, int epilogue);

/* Bytes of the no-allocation linear's per-GPU scratch (32 MiB). */
size_t ltx25_noalloc_scratch_bytes(void);

/* Dense bf16 linear: y = x . w^T (+ bias). K must be a multiple of 64.
 * Replaces the dense MetalOps::linear (src/ltx25-metal-ops.h:82-87;
 * src/ltx25-metal-ops.cc:504-529). */
int ltx25_linear(void* stream, const void* x, const void* w_bf16,
                 const void* bias, int bias_dtype, void* y, int M, int K,
                 int N);

/* y[M][N] = bf16(f32(y) + f32(bias[n])), in place, bias bf16 or f32.
 * Replaces MetalOps::bias_add (src/ltx25-metal-ops.h:297-300) and the
 * ltx_bias_add kernel (src/ltx25-kernels.metal:1420-1441). */
int ltx25_bias_add(void* stream, void* y, const void* bias, int bias_dtype,
                   int M, int N);

/* y[i] = bf16(gelu_tanh(f32(x[i]))) over n elements; may run in place.
 * Replaces MetalOps::gelu / gelu_tanh_ff_f16 (src/ltx25-metal-ops.cc:
 * 1061-1070; CPU form src/ltx25-block-ref.cc:265-272). */
int ltx25_gelu_tanh(void* stream, const void* x, void* y, size_t n);

/* Per-head gating of an attention output, in place:
 * y[t][h*head_dim + d] = bf16(f32(y) * 2 / (1 + exp(-f32(logits[t][h])))),
 * y bf16 [tokens][heads*head_dim], logits bf16 [tokens][heads] (the
 * to_gate_logits linear's output). Non-positive sizes are a no-op. The
 * 16-byte path needs head_dim % 8 == 0 and a 16-byte aligned y.
 * Replaces MetalOps::gate_heads (src/ltx25-metal-ops.cc:1089-1101) and the
 * ltx_gate_heads kernel (src/ltx25-kernels.metal:85-103); CPU form
 * src/ltx25-block-ref.cc:113-125. */
int ltx25_gate_heads(void* stream, void* y, const void* logits, int heads, int tokens,
                     int head_dim);

/* Expand a quantized weight to bf16 [N][K]: w = bf16(fma(scale, q, qbias)).
 * Replaces the dequant-once arm, affine_dequant_w{4,8}g{32,64}
 * (src/ltx25-metal-ops.cc:467-502). */
int ltx25_dequant(void* stream, const ltx25_qweight* w, void* out_bf16,
                  int N, int K);

/* The dequant-once arm: expand W into a grow-only bf16 [N][K] scratch shared
 * across calls (the reference's `_w_deq`, src/ltx25-metal-ops.h:843-845),
 * then run the dense GEMM over it. The expansion equals the fused kernel's
 * in-register dequant, so both routes return the same bits; they differ in
 * speed and in 2 B per weight of extra traffic. The fused kernel
 * dequantizes each weight once per 256-row tile, so the arm wins on tall
 * GEMMs: measured on MI355X at the DiT's widths (4096 -> 4096 / 12288 /
 * 16384, 16384 -> 4096) it is 2-22% faster from M = 1536 up, 4-12% faster
 * at M = 1024 except for 4096 -> 16384 (8% slower there), and 5-13% slower
 * at M = 512.
 *   OFF   always the fused dequant-in-GEMM kernel
 *   ON    the arm whenever the dense tile takes the shape (M >= 64,
 *         N >= 16: the reference's mma_eligible_ floor,
 *         src/ltx25-metal-ops.cc:342-374)
 *   AUTO  (the default) the arm from M >= LTX25_DEQUANT_ONCE_AUTO_MIN_M
 *         (or from VPIPE_LTX25_MMA_MIN_M when ltx25_init found it set)
 * The reference takes its dequant_mma_ route first whenever it is eligible
 * (src/ltx25-metal-ops.cc:467-502, tried at :544); AUTO keeps that route
 * where it is the faster one on this hardware. */
#define LTX25_DEQUANT_ONCE_OFF 0
#define LTX25_DEQUANT_ONCE_ON 1
#define LTX25_DEQUANT_ONCE_AUTO 2
#define LTX25_DEQUANT_ONCE_AUTO_MIN_M 1024
int ltx25_set_dequant_once(int mode);

/* 1 when ltx25_linear_q would take the dequant-once arm for this shape
 * under the current mode (K must also be a multiple of 64; the bf16
 * expansion must stay under 2 GiB). Host-only. */
int ltx25_dequant_once_takes(int M, int K, int N);

/* ---- routing: what a linear runs on, and the A/B switch ------------------------ */

/* Tile families of the GEMM behind ltx25_linear / ltx25_linear_q:
 *   TALL    256 x 256 output tiles, all of K per workgroup (the video GEMMs)
 *   MID     128 x 128 tiles, K split across workgroups until they cover the
 *           CUs once, f32 partials summed in split order by a second launch
 *   SKINNY  at most 128 tokens: 32-column slices, K split between the 8
 *           waves (and across workgroups above K = 2048)
 * ltx25_set_tile forces one for every later linear and for the second GEMM
 * of the LoRA pair (AUTO restores the planner); a forced SKINNY falls back to the planner for shapes it cannot
 * take (M > 128). Results are deterministic for a given route; different
 * routes sum in different orders. Process-wide, like the reference's
 * VPIPE_LTX25_MMA_TILE override (src/ltx25-metal-ops.cc:193-231, read at
 * init there), which exists for the same A/B re-measurement. */
#define LTX25_TILE_AUTO 0
#define LTX25_TILE_TALL 1
#define LTX25_TILE_MID 2
#define LTX25_TILE_SKINNY 3
int ltx25_set_tile(int tile);

/* The route ltx25_linear_q (bits 4 / 8) or ltx25_linear (bits 16) takes
 * for a shape under the current switches. Host-only, no device use. */
typedef struct ltx25_route {
  int tile;            /* LTX25_TILE_TALL / MID / SKINNY; 0 for the int8 tier */
  int i8;              /* 1: the int8 tier (ltx25_set_i8_gemm) */
  int dequant_once;    /* 1: the weight is expanded to bf16 first */
  int splits;          /* split-K factor of each launch */
  int slabs;           /* launches over row slabs */
  int slab_rows;       /* rows per slab (M when one) */
  size_t scratch_bytes;/* library scratch the call uses */
} ltx25_route;

/* Operand size limit: the kernels address every operand with 32-bit buffer
 * offsets, so each operand of a launch must stay under 2 GiB. The
 * activation and output are cut into row slabs (multiples of 256 rows)
 * that do; a weight of 2 GiB or more is refused with LTX25_E_UNSUPPORTED
 * before any device use. The reference refuses the same operands for the
 * same reason (mma_eligible_, src/ltx25-metal-ops.cc:342-374). */
int ltx25_linear_route(int M, int K, int N, int bits, ltx25_route* out);

/* ---- the low-rank adapter delta ------------------------------------------------ */

/* y[M][N] += (x[M][K] . a[rank][K]^T) . b[N][rank]^T, all bf16, in place on
 * y: r = bf16(x . a^T) with f32 accumulation, then y = bf16(f32(y) + r . b^T)
 * with the accumulator seeded from y. Three routes, same arithmetic:
 * - rank >= 96, M >= 256, K % 64 == 0, N % 8 == 0, 16-byte aligned x and y:
 *   the reference's matrix-core pair -- r on the dense GEMM, then the dense
 *   GEMM again with its accumulators seeded from y; the rank is padded to a
 *   multiple of 64 (a's missing rows read as zeros; b copied with zero
 *   columns when needed, and a when it is not 16-byte aligned) in a
 *   grow-only scratch that also holds r;
 * - rank < 96 with M >= 512, K % 64 == 0, rank % 8 == 0 and the vector
 *   path's conditions (below): r on the dense GEMM into that scratch, then
 *   the fused kernel's y pass reading it;
 * - otherwise one fused kernel per 512 adapter columns (16-byte aligned x,
 *   a and y with K % 8 == 0 and N % 8 == 0 take its vector path; when the
 *   rank is not a multiple of 8, b is first copied with its rows
 *   zero-padded to one).
 * `r` ([M][rank] bf16) and `d` ([M][N]) are the reference signature's
 * caller scratch; either may be NULL. A 16-byte aligned `r` receives
 * r = bf16(x . a^T) on the r-first route, and on the pair when rank is a
 * multiple of 64, in place of the library's scratch; other routes leave it
 * untouched. `d` is neither read nor written. An empty
 * shape (any of M, K, N, rank <= 0) is a no-op, as in the reference.
 * Pointers need only bf16 (2-byte) alignment.
 * Replaces MetalOps::lora_add (src/ltx25-metal-ops.h:107-133;
 * src/ltx25-metal-ops.cc:989-1004) and its matrix-core pair (:940-987). */
int ltx25_lora_add(void* stream, const void* x, const void* a, const void* b,
                   void* y, void* r, void* d, int M, int K, int N, int rank);

/* The three LoRA routes (see ltx25_lora_add); NONE for an empty shape. */
#define LTX25_LORA_AUTO 0
#define LTX25_LORA_NONE 0
#define LTX25_LORA_PAIR 1    /* two dense GEMMs, the second seeded from y */
#define LTX25_LORA_RFIRST 2  /* r on the dense GEMM, then the fused y pass */
#define LTX25_LORA_FUSED 3   /* one fused kernel per 512 adapter columns */

/* 1 when ltx25_lora_add takes the GEMM pair for this shape (with
 * allocator-aligned pointers) under the current switches, else 0.
 * Replaces MetalOps::lora_on_matrix_cores (src/ltx25-metal-ops.h:134-139;
 * src/ltx25-metal-ops.cc:921-936). Host-only. */
int ltx25_lora_on_matrix_cores(int M, int K, int N, int rank);

/* Turn the GEMM pair off (0: every shape takes the one-pass fused kernel)
 * or back on (1: the planner's choice). The A/B hook of
 * MetalOps::set_lora_matrix_cores (src/ltx25-metal-ops.h:140-146).
 * Process-wide. */
int ltx25_set_lora_matrix_cores(int on);

/* Force one LoRA route for every later ltx25_lora_add (LTX25_LORA_AUTO
 * restores the planner). A forced route that cannot take a shape makes
 * that call fail with LTX25_E_UNSUPPORTED before any device use; FUSED
 * takes every shape. Process-wide. */
int ltx25_set_lora_route(int route);

/* The route ltx25_lora_add would take for these pointers and shape under
 * the current switches, in *route (LTX25_LORA_*). Pointers are only
 * inspected (alignment), never dereferenced. Host-only. */
int ltx25_lora_route(const void* x, const void* a, const void* b, const void* y, int M, int K,
                     int N, int rank, int* route);

/* A quantized linear with its adapter, in the reference's order --
 *   y = epilogue(x . dequant(W)^T + bias + bf16(x . A^T) . B^T),
 * the adapter added BEFORE the epilogue's GELU -- as one call.
 * Replaces the pair a block's call sites issue: MetalOps::linear(QWeight)
 * then MetalBlock::lora_ -> MetalOps::lora_add on the same output
 * (src/ltx25-block-metal.cc:428-436,523-524,639-648; ff_in's GELU after
 * both, :645). Where ltx25_lora_fold_takes says so (the dequant-once arm
 * of a quantized weight: M >= LTX25_DEQUANT_ONCE_AUTO_MIN_M under AUTO)
 * the adapter is folded into the linear's own GEMM:
 *   - w8 codes, rank up to 64, K % 128 == 0, a 16-byte aligned: merged
 *     into the expanded weight, W' = bf16(dequant(W) + B . A), then
 *     y = epi(x . W'^T + bias) at the linear's own K
 *     ((x . A^T) . B^T = x . (B . A)^T); one rounding per weight element
 *     and one of the output;
 *   - otherwise as rank-rounded-to-64 more K: y = epi([x | r] . [W | B]^T
 *     + bias), r = bf16(x . A^T), one rounding of the output;
 * where the reference rounds the linear and the delta separately.
 * Elsewhere it runs ltx25_linear_q, ltx25_lora_add, then ltx25_gelu_tanh
 * for LTX25_EPI_GELU_TANH. a is bf16 [rank][K], b bf16 [N][rank];
 * rank 0 is a plain linear. */
int ltx25_linear_q_lora(void* stream, const void* x, const ltx25_qweight* w, const void* bias,
                        int bias_dtype, const void* a, const void* b, int rank, void* y, int M,
                        int K, int N, int epilogue);

/* 1 when ltx25_linear_q_lora folds the adapter into the linear's GEMM for
 * this shape (bits 4 or 8: the weight's code width) under the current
 * switches, with allocator-aligned x and y, else 0. Host-only. */
int ltx25_lora_fold_takes(int M, int K, int N, int rank, int bits);

/* ---- the int8 tier ------------------------------------------------------------ */

/* Turn the int8 tier on (1) or off (0) for ltx25_linear / ltx25_linear_q.
 * Replaces MetalOps::set_i8_gemm (src/ltx25-metal-ops.h:151). */
int ltx25_set_i8_gemm(int on);

/* 1 when linear would take the int8 tier for this shape: the tier is on,
 * M >= 1024, K >= 1024, K % 128 == 0, N >= 16, and the int8 operands and
 * the output stay under 2 GiB. The tier composes with the GELU epilogue
 * (ltx25_linear_q_ex), as the reference's tier sits under every quantized
 * linear, ff_in included. Host-only, no device use.
 * Replaces MetalOps::i8_takes (src/ltx25-metal-ops.h:157; the reference's
 * gates are asserted at tests/ltx25-i8-gemm-test.cc:144-179). */
int ltx25_i8_takes(int M, int K, int N);

/* Per-row symmetric int8: scale[m] = absmax_k |x[m][k]| / 127,
 * q = clamp(rint(x / scale), -127, 127); an all-zero row gives scale 0 and
 * q 0. Serves activations per token and dense bf16 weights per output
 * channel. */
int ltx25_i8_quantize_rows(void* stream, const void* x_bf16, int8_t* q,
                           float* scale, int M, int K);

/* The same per-output-channel int8 quantization applied to the dequantized
 * values of a group-affine weight (bf16(fma(scale, q, qbias))), without
 * materialising the bf16 weight. */
int ltx25_i8_quantize_qweight(void* stream, const ltx25_qweight* w,
                              int8_t* wq, float* sw, int N, int K);

/* acc = xq[M][K] . wq[N][K]^T in int32, then
 * y = bf16(fma(float(acc), sx[m] * sw[n], bias[n] or +0)).
 * `acc_dbg` (int32 [M][N]) may be NULL; when given, the raw accumulators
 * are written too (for bit-exact checks). K must be a multiple of 128.
 * The GEMM under I8GemmContext::gemm (src/ltx25-metal-ops.cc:386-391). */
int ltx25_i8_gemm(void* stream, const int8_t* xq, const float* sx,
                  const int8_t* wq, const float* sw, const void* bias,
                  int bias_dtype, void* y, int32_t* acc_dbg, int M, int K,
                  int N);

/* ---- packed-weight format ------------------------------------------------------ */

/* u8 codes [N][K] -> u32 words [N][K*bits/32], LOW bits first, and back.
 * The packing of tests/ltx25-qlinear-test.cc:134-137. */
int ltx25_pack_codes(void* stream, const uint8_t* q, uint32_t* codes, int N,
                     int K, int bits);
int ltx25_unpack_codes(void* stream, const uint32_t* codes, uint8_t* q,
                       int N, int K, int bits);

/* Group-affine quantize f32 w [N][K] (MLX layout): per group, bias =
 * bf16(min), scale = bf16((max - min) / (2^bits - 1)),
 * q = clamp(lround((w - bias) / scale), 0, 2^bits - 1), 0 when scale == 0.
 * The producer of the packed tensors; restates the quantizer of
 * tests/ltx25-qlinear-test.cc:93-141 (vpipe's AffineQuantizer is not in the
 * reference tree). */
int ltx25_quantize_affine(void* stream, const float* w, void* codes,
                          void* scales, void* qbias, int N, int K, int bits,
                          int group);

/* F16 -> bf16 (RNE) of n elements; may run in place. The loader's
 * conversion of a checkpoint's F16 scales and biases
 * (src/ltx25-dit-weights.cc:230-278, refill in place at :305-334). */
int ltx25_f16_to_bf16(void* stream, const void* in_f16, void* out_bf16,
                      size_t n);

/* Recover bits and group of a packed linear from its tensor shapes, given
 * the K the architecture says it reads: group = K / scales_cols,
 * bits = codes_cols * 32 / K (codes counted in u32 words). Returns
 * LTX25_E_INVAL when the shapes do not close, or when *group is already
 * set (non-zero) and differs (a checkpoint must use one group size).
 * Host-only. Replaces need_q_'s shape inference
 * (src/ltx25-dit-weights.cc:352-403). */
int ltx25_qweight_infer(int K, long scales_cols, long codes_cols, int* bits,
                        int* group);

/* ---- the on-disk pack reader ------------------------------------------------------ */

/* An open .safetensors file: mapped read-only, header parsed on the host.
 * The device buffers it binds belong to it until ltx25_pack_close. */
typedef struct ltx25_pack ltx25_pack;

/* Open and parse a pack. No device work. Replaces the weight-set reads of
 * the reference's loader (src/ltx25-dit-weights.cc:170-190), which go
 * through vpipe's WeightSet. */
int ltx25_pack_open(const char* path, ltx25_pack** out);

/* Drain the device, free every buffer the pack bound, unmap, close. */
void ltx25_pack_close(ltx25_pack* pack);

/* A tensor's safetensors dtype ("U32", "F16", "BF16", "F32", ...), rank
 * and dims (up to 8). Host-only. LTX25_E_INVAL when the name is absent. */
int ltx25_pack_tensor(const ltx25_pack* pack, const char* name, char dtype[16],
                      int* ndim, long dims[8]);

/* A string from the header's __metadata__, or NULL. */
const char* ltx25_pack_metadata(const ltx25_pack* pack, const char* key);

/* A tensor as bf16 in device memory the pack owns: BF16 as stored, F16
 * converted on the device, F32 converted on the host, both with round to
 * nearest even; cached per name. Replaces get_as_bf16_
 * (src/ltx25-dit-weights.cc:230-278). */
int ltx25_pack_read_bf16(ltx25_pack* pack, void* stream, const char* name,
                         const void** dev_bf16, size_t* count);

/* Bind one linear that may be quantized. When NAME.scales and NAME.weight
 * are both 2-D (and K > 0) it is quantized: bits and group come from the
 * shapes (ltx25_qweight_infer), `*group` is set by the first quantized
 * linear and checked on every later one, the u32 codes are uploaded
 * untouched and NAME.scales / NAME.biases are read as bf16. Otherwise
 * NAME.weight is the dense weight, read as bf16. A missing tensor is named
 * in `miss` (when non-NULL and still empty). The result's pointers are
 * owned by the pack. Replaces need_q_ (src/ltx25-dit-weights.cc:352-403;
 * the bind entry point bind_qlinear, src/ltx25-dit-weights.h:170-175). */
int ltx25_pack_bind_qlinear(ltx25_pack* pack, void* stream, const char* name,
                            int K, int* group, ltx25_qweight* out, char* miss,
                            size_t miss_len);

/* 1 when the DiT quantizer packs this tensor: inside a block stack (name
 * contains "_blocks."), a 2-D float ".weight", not a norm or embedding,
 * and not one of the two 2-D floats that are not matrices ("scale_shift"
 * tables, the "to_gate_logits" per-head gate). Host-only. Restates the
 * selection of src/ltx25-quant-family.cc:44-71. */
int ltx25_pack_quantizable(const char* name, const char* dtype, int ndim);

/* ---- measurement probes -------------------------------------------------- */

/* No counterpart in the reference: the two ceilings this library's kernels
 * are measured against (bench.py --ceilings), shipped so that the figures
 * quoted beside the GEMMs can be reproduced from the library itself.
 *
 * Streaming read: `bytes` of device memory from `src` read once with
 * 16-byte loads by `blocks` workgroups of 256 threads, each on its own
 * contiguous span; one u32 per workgroup to `sink` (device, `blocks`
 * words). src 16-byte aligned, bytes a positive multiple of 16, blocks in
 * 1..65535. */
int ltx25_probe_read(void* stream, const void* src, size_t bytes, void* sink, int blocks);

/* MFMA stream: 256 workgroups of 1 or 2 waves per SIMD (`waves_per_simd`)
 * each issue 8 x `iters` independent v_mfma_f32_16x16x32_bf16 (16384 FLOP
 * each) on register operands, zero (`random` 0) or random bf16 of
 * magnitude ~1 (`random` 1). `out` (device, 256 floats) is written only in
 * the practically impossible case that a sum equals 1.2345. iters > 0. */
int ltx25_probe_mfma(void* stream, int iters, int random, int waves_per_simd, void* out);

/* Per-phase clock stamps of the M <= 128 kernel (the audio GEMMs' route):
 * one w8 linear y = x . dequant(w)^T (+ bias) with M <= 128, through the
 * same kernel as ltx25_linear_q's M <= 128 route, instantiated with stamps
 * (the instantiations linear runs carry none). k_chunk is the K per
 * workgroup: 0 for the planner's split, else a multiple of 64 up to 2048,
 * which forces ceil(K / k_chunk) splits (their f32 partials in the
 * library's workspace, then the split-K reduction launch, as in linear).
 * Lane 0 of each wave writes ten u64 to `stamps` (device) at
 * [(split * ceil(N / 32) + tile) * 8 + wave] * 10: the shader clock
 * (s_memtime) at entry, codes in registers, the workgroup's scale block in
 * LDS, K loop done, the eight partial tiles summed, stores complete; the
 * 100 MHz clock (s_memrealtime) at entry and at the end; the HW_ID and
 * XCC_ID registers. stamps_bytes must hold splits * ceil(N / 32) * 640
 * bytes; *splits_out (host) receives the splits. Operand rules as for
 * ltx25_linear_q; LTX25_E_UNSUPPORTED when the shape is not on the
 * M <= 128 route or the weight is not w8. */
int ltx25_probe_skinny_phases(void* stream, const void* x, const ltx25_qweight* w,
                              const void* bias, int bias_dtype, void* y, int M, int K, int N,
                              int k_chunk, void* stamps, size_t stamps_bytes, int* splits_out);

/* Per-phase clock stamps of the 256 x 256 tile (the FFN GEMMs' and the int8
 * tier's kernel), instantiated with stamps (the instantiations linear and
 * i8_gemm run carry none). ltx25_probe_tall_phases runs the dense bf16
 * GEMM y = epi(x . w^T + bias), w bf16 [N][K] (what the dequant-once
 * route's expansion writes), K % 64 == 0, N % 8 == 0;
 * ltx25_probe_tall_i8_phases the int8 GEMM of ltx25_i8_gemm (operand rules
 * as there), K % 128 == 0. Lane 0 of each wave writes eight u64 to `stamps`
 * (device) at (tile * 8 + wave) * 8, tile = the workgroup id: the shader
 * clock (s_memtime) at entry, step 0 landed, K loop done, the output tile
 * staged in LDS, stores complete; the 100 MHz clock (s_memrealtime) at
 * entry and at the end; (XCC_ID << 32) | HW_ID. stamps_bytes must hold
 * ceil(M / 256) * ceil(N / 256) * 512 bytes. */
int ltx25_probe_tall_phases(void* stream, const void* x, const void* w_bf16, const void* bias,
                            int bias_dtype, void* y, int M, int K, int N, int epilogue,
                            void* stamps, size_t stamps_bytes);
int ltx25_probe_tall_i8_phases(void* stream, const int8_t* xq, const float* sx, const int8_t* wq,
                               const float* sw, const void* bias, int bias_dtype, void* y,
                               int M, int K, int N, void* stamps, size_t stamps_bytes);

#ifdef __cplusplus
}
#endif

#endif /* LTX25_QLINEAR_H */
