/*
 * moe_oracle.h -- CPU restatement of the GPT-OSS MoE block of the reference
 * (Jayluci4/hip-kernels), used ONLY as the test checker and as the timed CPU
 * baseline.  Nothing in the product library links or calls this code.
 *
 * Every routine states the reference file:line whose arithmetic it restates.
 * Rounding points follow the reference: fp32 accumulation, bf16 logits,
 * bf16 gate_up, bf16 SwiGLU output, bf16 expert output, bf16 layer output.
 *
 * Summation order.  The reference's own kernels fix an order only per kernel
 * (gemv_bf16_kernel for the router, fused_mxfp4_gemv_kernel for M=1 experts,
 * hipBLASLt with an unpinned order for M>1).  This oracle fixes ONE order per
 * dot product and the GPU kernels of this build reproduce it bit for bit:
 *   - router logits: the reference gemv_bf16_kernel tree exactly
 *     (gemv_bf16.cu:40-130): 256 strided chains of 8-element chunks,
 *     64-lane xor butterfly, 4-warp sequential sum, + bias.
 *   - expert products (MXFP4): K is cut into P contiguous parts
 *     (P = orc_parts(K)), each part one ascending fmaf chain from +0,
 *     parts added sequentially, + bias.  This is this build's canonical
 *     order; orc_mxfp4_gemv_refkernel() restates the reference's
 *     fused_mxfp4_gemv_kernel order and is used to measure how far the two
 *     orders are apart and to check the restatement against the compiled
 *     reference kernel.
 * exp() is orc_expf(): Cody-Waite reduction + degree-7 Taylor polynomial in
 * fmaf (same method in the GPU kernels).  The reference calls device expf;
 * its last-ulp behaviour is not reproducible on a CPU, so those bits are
 * "parity unpinned" and covered by tolerance (see the test headers).
 */
#ifndef GPTOSS_MOE_ORACLE_H
#define GPTOSS_MOE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);            /* round-to-nearest-even, NaN kept quiet */
float    orc_e2m1(int code);                  /* fused_mxfp4_gemv.cu:27-36 */
float    orc_e8m0(int code);                  /* fused_mxfp4_gemv.cu:41-45 (code<<23) */
float    orc_expf(float x);
float    orc_swiglu(float g, float u, float alpha, float limit);   /* swiglu.cu:25-28,54-62 */
int      orc_parts(int K);                    /* number of contiguous K-parts of the canonical dot */

/* exp() selection for the SwiGLU/softmax paths: 0 = orc_expf (canonical),
 * 1 = libm expf (used only to quantify the exp-implementation spread). */
void     orc_set_exp_mode(int mode);

/* ---- router (gemv_bf16.cu:40-130) --------------------------------------- */
/* logits[t*E+e] = dot(x[t], W[e]) (+ b[e]) with the reference tree.  If
 * out_bf16 != NULL the bf16-rounded logit is written there (reference mode);
 * if out_f32 != NULL the fp32 logit is written there (BASELINE cfg-1 mode). */
void orc_router(const uint16_t* x, const uint16_t* W, const uint16_t* b,
                int T, int E, int H, uint16_t* out_bf16, float* out_f32);

/* ---- top-k softmax (topk_softmax.cu:47-216 v1, :221-375 v2) ------------- */
/* logits are fp32 (bf16 logits are widened by the caller).  variant 1 or 2
 * selects the softmax summation order; variant 0 = the reference launcher's
 * choice (v1 if T <= 8 else v2, topk_softmax.cu:399).  Fully degenerate
 * tokens (no finite logit above -FLT_MAX) get idx = lane, w = 1/k (the v2
 * rule, :339-346) in every variant; partially degenerate slots get idx -1,
 * weight 0.  Returns 0, or -1 if k is not 1, 2, 4 or 8. */
int orc_topk_softmax(const float* logits, int T, int E, int k, int variant,
                     int32_t* idx, float* w);

/* ---- dispatch / permute (moe_permute.cu:24-76, 184-236) ----------------- */
/* counts[E], offsets[E+1], gather_map[T*k] (-1 for slots with idx < 0),
 * perm_token[pos] = token of the slot placed at pos, active[E] (expert ids
 * with count > 0, ascending); returns n_active. */
int orc_plan(const int32_t* idx, int T, int k, int E,
             int32_t* counts, int32_t* offsets, int32_t* gather_map,
             int32_t* perm_token, int32_t* active);

/* ---- MXFP4 products -------------------------------------------------------
 * W is row-major MXFP4: packed[N][K/2] (low nibble = even k), scales[N][K/32]
 * (one e8m0 byte per 32 consecutive k), as fused_mxfp4_gemv.cu:13-15 and
 * weight_loader.cu:782-842.  x is bf16 [M][K]; xf (optional, may be NULL) is
 * the same input given as fp32 values (used for the SwiGLU output that the
 * down projection consumes). y = bf16(dot + bias). */
void orc_mxfp4_gemv(const uint16_t* x, const float* xf, int M,
                    const uint8_t* packed, const uint8_t* scales,
                    const uint16_t* bias, int N, int K, uint16_t* y);
/* Same product in the fused_mxfp4_gemv_kernel order (fused_mxfp4_gemv.cu:
 * 76-184): 256 threads x uint32 chunks, pair sums, butterfly, 4-warp sum. */
void orc_mxfp4_gemv_refkernel(const uint16_t* x, int M,
                              const uint8_t* packed, const uint8_t* scales,
                              const uint16_t* bias, int N, int K, uint16_t* y);
/* bf16 dequant of one MXFP4 matrix (mxfp4_dequant.cu:263-350 semantics with
 * the register decode rule code<<23 for the scale). */
void orc_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, int N, int K,
                       uint16_t* out);

/* ---- SwiGLU on interleaved gate/up rows (swiglu.cu:117-176) -------------- */
void orc_swiglu_rows(const uint16_t* gate_up, int M, int I, float alpha,
                     float limit, uint16_t* out);

/* ---- combine (moe_combine.cu:31-117) ------------------------------------- */
/* out[t] = bf16( fmaf-chain over k of w*y[gather_map] , then + residual ).
 * Slots with gather_map < 0 are skipped. residual may be NULL. */
void orc_combine(const uint16_t* y, const int32_t* gather_map, const float* w,
                 const uint16_t* residual, int T, int k, int H, uint16_t* out);

/* ---- whole layer (moe_layer.cu:1011-1549, general path semantics) --------- */
typedef struct {
  int H, E, k, I;
  float alpha, limit;
  int logits_fp32;        /* 0: bf16 logits (reference), 1: fp32 logits */
  int topk_variant;       /* 0 = launcher choice by T */
  /* Expert products and combine:
   *   0: this build's canonical order (K-part fmaf chains, bias before the
   *      one bf16 rounding, combine from 0 with the residual last);
   *   1: the reference's own dispatch, orders and rounding points, per
   *      active expert as moe_layer.cu chooses them:
   *      - one token (fast path, moe_layer.cu:1028-1098): fused_mxfp4_gemv
   *        order with no bias (fused_mxfp4_gemv.cu:93-183), the gate_up bias
   *        added in fp32 inside the SwiGLU (moe_layer.cu:303-362), the down
   *        bias after the bf16 rounding (:442-463), the combine from the
   *        residual (:479-497);
   *      - several tokens, a batch of 8 active experts that all hold one
   *        token (:1319-1368): fused_mxfp4_gemv with the bias inside;
   *      - one token in a mixed batch (:1409-1411, :1464-1466): gemv_bf16 over
   *        the dequantised weights (gemv_bf16.cu:40-130), then bias_add_rows
   *        (moe_layer.cu:171-183);
   *      - several tokens (hipBLASLt, :1413-1417): rounding points as the
   *        reference (bf16 product, then bias_add_rows) with the canonical
   *        order standing in for hipBLASLt's (not restated: not vendored);
   *      - combine (T > 1): moe_combine.cu:69-115, the residual last. */
  int expert_order;
} orc_cfg;

typedef struct {
  const uint16_t* router_w;   /* [E][H] */
  const uint16_t* router_b;   /* [E] or NULL */
  const uint8_t*  w1_packed;  /* [E][2I][H/2] */
  const uint8_t*  w1_scales;  /* [E][2I][H/32] */
  const uint16_t* w1_bias;    /* [E][2I] or NULL */
  const uint8_t*  w2_packed;  /* [E][H][I/2] */
  const uint8_t*  w2_scales;  /* [E][H][I/32] */
  const uint16_t* w2_bias;    /* [E][H] or NULL */
} orc_weights;

/* Optional intermediate outputs (any may be NULL). */
typedef struct {
  uint16_t* logits_bf16;  float* logits_f32;   /* [T][E] */
  int32_t* idx; float* w;                       /* [T][k] */
  int32_t* gather_map;                          /* [T*k] */
  uint16_t* gate_up;                            /* [T*k][2I] permuted order */
  uint16_t* act;                                /* [T*k][I]  permuted order */
  uint16_t* y;                                  /* [T*k][H]  permuted order */
} orc_trace;

/* nthreads <= 0 -> all hardware threads. */
void orc_moe_forward(const orc_cfg* cfg, const orc_weights* wt,
                     const uint16_t* x, const uint16_t* residual, int T,
                     uint16_t* out, orc_trace* trace, int nthreads);

/* The expert half with the routing given (idx, w: [T][k]), as the layer after
 * its top-k (moe_layer.cu:1196-1549).  trace->logits/idx/w are not written. */
void orc_moe_forward_routed(const orc_cfg* cfg, const orc_weights* wt,
                            const uint16_t* x, const uint16_t* residual, int T,
                            const int32_t* idx, const float* w,
                            uint16_t* out, orc_trace* trace, int nthreads);

/* RMSNorm (rmsnorm.cu:47-83 semantics with an IEEE 1/sqrt): out = bf16(x*inv*w) */
void orc_rmsnorm(const uint16_t* x, const uint16_t* w, int T, int H, float eps,
                 uint16_t* out);
/* fused_residual_rmsnorm_forward: s = r + d (fp32), sum_out = bf16(s) (may be
 * NULL), normed = bf16((s * inv) * w) with inv from the gemv-tree sum of s^2. */
void orc_residual_rmsnorm(const uint16_t* r, const uint16_t* d, const uint16_t* w, int T, int H, float eps,
                          uint16_t* normed, uint16_t* sum_out);

#ifdef __cplusplus
}
#endif
#endif
