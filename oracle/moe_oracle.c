/*
 * moe_oracle.c -- CPU restatement of the reference GPT-OSS MoE block.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels and
 * the timed CPU baseline of bench.py; the product library never links it.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, fmaf only where written).
 *
 * The header (moe_oracle.h) documents the summation orders.  Reference file
 * references below are relative to the reference repository root.
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------------ */
/* bf16 <-> f32                                                              */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round to nearest even; NaN -> quiet NaN with the sign kept.  This is the
 * rounding of __float2bfloat16 used at every bf16 store in the reference
 * (e.g. gemv_bf16.cu:127, swiglu.cu:170, moe_combine.cu:112). */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
    return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

static inline float bf(uint16_t h) { return orc_bf16_to_f32(h); }
static inline float rbf(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* ------------------------------------------------------------------------ */
/* MXFP4 decode (fused_mxfp4_gemv.cu:27-45, BUGFIX_REPORT.md:79-80)          */
/* ------------------------------------------------------------------------ */
float orc_e2m1(int code) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float m = mag[code & 7];
  return (code & 8) ? -m : m;
}

/* The register path of the reference shifts the code into the fp32 exponent
 * field: code 0 decodes to +0, 255 to +inf (fused_mxfp4_gemv.cu:42-44). */
float orc_e8m0(int code) { return u2f(((uint32_t)(code & 0xff)) << 23); }

static inline float mx_weight(const uint8_t* packed, const uint8_t* scales,
                              int K, int n, int k) {
  uint8_t byte = packed[(size_t)n * (K / 2) + (k >> 1)];
  int code = (k & 1) ? (byte >> 4) : (byte & 0xf);
  return orc_e2m1(code) * orc_e8m0(scales[(size_t)n * (K / 32) + (k >> 5)]);
}

/* ------------------------------------------------------------------------ */
/* exp: Cody-Waite range reduction x = n*ln2 + r, |r| <= ln2/2, then the     */
/* degree-7 Taylor polynomial of e^r in Horner form with fmaf, then          */
/* ldexpf(p, n).  Same operation sequence as gx_expf in the HIP kernels.     */
/* ------------------------------------------------------------------------ */
static int g_exp_mode = 0;
void orc_set_exp_mode(int mode) { g_exp_mode = mode; }

float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541015625f) return 0.0f;
  const float log2e = 1.44269502162933349609375f;        /* RN(1/ln 2) */
  const float ln2_hi = 0.693147182464599609375f;         /* RN(ln 2) */
  const float ln2_lo = -1.904654323148236e-09f;          /* RN(ln 2 - ln2_hi) */
  float n = rintf(x * log2e);
  float r = fmaf(-n, ln2_hi, x);
  r = fmaf(-n, ln2_lo, r);
  float p = 1.98412698e-4f;                /* 1/7! */
  p = fmaf(p, r, 1.38888889e-3f);          /* 1/6! */
  p = fmaf(p, r, 8.33333333e-3f);          /* 1/5! */
  p = fmaf(p, r, 4.16666667e-2f);          /* 1/4! */
  p = fmaf(p, r, 1.66666667e-1f);          /* 1/3! */
  p = fmaf(p, r, 0.5f);                    /* 1/2! */
  p = fmaf(p, r, 1.0f);                    /* 1/1! */
  p = fmaf(p, r, 1.0f);                    /* 1/0! */
  return ldexpf(p, (int)n);
}

static inline float oexp(float x) { return g_exp_mode ? expf(x) : orc_expf(x); }

/* GPT-OSS gate activation (swiglu.cu:25-28, 54-62):
 *   g = min(g, limit); u = clamp(u, -limit, limit);
 *   out = (u + 1) * (g / (1 + exp(-alpha*g))) */
float orc_swiglu(float g, float u, float alpha, float limit) {
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  float e = oexp((-alpha) * g);
  float glu = g / (1.0f + e);
  return (u + 1.0f) * glu;
}

/* ------------------------------------------------------------------------ */
/* Canonical expert dot: K/32 blocks cut into P contiguous parts.           */
/* ------------------------------------------------------------------------ */
int orc_parts(int K) {
  int nb = K / 32;
  for (int p = 6; p > 1; --p)
    if (nb % p == 0) return p;
  return 1;
}

/* dot over k in [k0, k1) of x * w(n, k): one ascending fmaf chain from +0. */
static inline float mx_chain(const float* xr, const uint8_t* packed,
                             const uint8_t* scales, int K, int n, int k0, int k1) {
  float acc = 0.0f;
  for (int k = k0; k < k1; ++k) acc = fmaf(xr[k], mx_weight(packed, scales, K, n, k), acc);
  return acc;
}

static float mx_dot_canonical(const float* xr, const uint8_t* packed,
                              const uint8_t* scales, int K, int n) {
  int P = orc_parts(K);
  int plen = K / P;
  float total = mx_chain(xr, packed, scales, K, n, 0, plen);
  for (int p = 1; p < P; ++p)
    total = total + mx_chain(xr, packed, scales, K, n, p * plen, (p + 1) * plen);
  return total;
}

void orc_mxfp4_gemv(const uint16_t* x, const float* xf, int M,
                    const uint8_t* packed, const uint8_t* scales,
                    const uint16_t* bias, int N, int K, uint16_t* y) {
  float* xr = (float*)malloc(sizeof(float) * (size_t)K);
  for (int m = 0; m < M; ++m) {
    for (int k = 0; k < K; ++k)
      xr[k] = xf ? xf[(size_t)m * K + k] : bf(x[(size_t)m * K + k]);
    for (int n = 0; n < N; ++n) {
      float v = mx_dot_canonical(xr, packed, scales, K, n);
      if (bias) v = v + bf(bias[n]);
      y[(size_t)m * N + n] = orc_f32_to_bf16(v);
    }
  }
  free(xr);
}

/* ------------------------------------------------------------------------ */
/* 64-lane xor butterfly: v[l] <- v[l] + v[l ^ m], m = 32..1 (the reduction */
/* of gemv_bf16.cu:29-38 and fused_mxfp4_gemv.cu:51-61).  All lanes end     */
/* with the same value; lane 0's is returned.                                */
/* ------------------------------------------------------------------------ */
static float butterfly64(float* v) {
  float t[64];
  for (int m = 32; m >= 1; m >>= 1) {
    for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ m];
    memcpy(v, t, sizeof(t));
  }
  return v[0];
}

/* Restatement of fused_mxfp4_gemv_kernel's per-row arithmetic
 * (fused_mxfp4_gemv.cu:93-183): thread tid takes uint32 chunks tid, tid+256,
 * ...; per chunk dot = 0 then per byte dot += (x0*w0 + x1*w1); acc += dot;
 * remainder bytes; butterfly per 64-lane warp; val = 0 + s0 + s1 + s2 + s3.
 * The products are exact in fp32, so FMA contraction of the pair sum cannot
 * change the result.  xr holds the bf16 inputs as fp32 values. */
static float mx_dot_refkernel(const float* xr, const uint8_t* packed, const uint8_t* scales,
                              int K, int n) {
  const int KH = K >> 1, KH4 = KH >> 2;
  float part[256];
  for (int tid = 0; tid < 256; ++tid) {
    float acc = 0.0f;
    for (int kb4 = tid; kb4 < KH4; kb4 += 256) {
      int kb = kb4 << 2, k0 = kb << 1;
      float dot = 0.0f;
      for (int b = 0; b < 4; ++b) {
        int k = k0 + 2 * b;
        float w0 = mx_weight(packed, scales, K, n, k);
        float w1 = mx_weight(packed, scales, K, n, k + 1);
        float pair = xr[k] * w0 + xr[k + 1] * w1;
        dot = dot + pair;
      }
      acc = acc + dot;
    }
    for (int kb = KH4 * 4 + tid; kb < KH; kb += 256) {
      int k0 = kb << 1;
      float pair = xr[k0] * mx_weight(packed, scales, K, n, k0) +
                   xr[k0 + 1] * mx_weight(packed, scales, K, n, k0 + 1);
      acc = acc + pair;
    }
    part[tid] = acc;
  }
  float val = 0.0f;
  for (int w = 0; w < 4; ++w) val = val + butterfly64(part + 64 * w);
  return val;
}

void orc_mxfp4_gemv_refkernel(const uint16_t* x, int M,
                              const uint8_t* packed, const uint8_t* scales,
                              const uint16_t* bias, int N, int K, uint16_t* y) {
  float* xr = (float*)malloc(sizeof(float) * (size_t)K);
  for (int m = 0; m < M; ++m) {
    for (int k = 0; k < K; ++k) xr[k] = bf(x[(size_t)m * K + k]);
    for (int n = 0; n < N; ++n) {
      float val = mx_dot_refkernel(xr, packed, scales, K, n);
      if (bias) val = val + bf(bias[n]);
      y[(size_t)m * N + n] = orc_f32_to_bf16(val);
    }
  }
  free(xr);
}

void orc_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, int N, int K,
                       uint16_t* out) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      out[(size_t)n * K + k] = orc_f32_to_bf16(mx_weight(packed, scales, K, n, k));
}

/* ------------------------------------------------------------------------ */
/* Router: gemv_bf16_kernel tree (gemv_bf16.cu:48-129).                      */
/* Thread tid chains fmaf over 8-element chunks tid, tid+256, ... then the  */
/* K%8 remainder elements tid, tid+256, ...; butterfly per warp; 4 warps    */
/* summed in order from 0; + bias in fp32.                                   */
/* ------------------------------------------------------------------------ */
static float gemv_tree(const uint16_t* a, const uint16_t* b, int K) {
  const int KV = K >> 3;
  float part[256];
  for (int tid = 0; tid < 256; ++tid) {
    float acc = 0.0f;
    for (int kv = tid; kv < KV; kv += 256)
      for (int i = 0; i < 8; ++i) {
        int k = (kv << 3) + i;
        acc = fmaf(bf(a[k]), bf(b[k]), acc);
      }
    for (int k = (KV << 3) + tid; k < K; k += 256) acc = fmaf(bf(a[k]), bf(b[k]), acc);
    part[tid] = acc;
  }
  float val = 0.0f;
  for (int w = 0; w < 4; ++w) val = val + butterfly64(part + 64 * w);
  return val;
}

/* gemv_bf16_kernel (gemv_bf16.cu:48-129) over the bf16 dequantisation of an
 * MXFP4 row (mxfp4_dequant.cu:263-350, bf16(e2m1 * (code << 23))): the
 * reference's product for an expert with one token inside a batch that also
 * holds experts with several (moe_layer.cu:1409-1411, 1464-1466).  Products
 * of bf16 values are exact in fp32, so the chains' fmaf equals the kernel's
 * multiply-add however it is contracted. */
static float mx_dot_gemv_tree(const float* xr, const uint8_t* packed, const uint8_t* scales, int K, int n) {
  const int KV = K >> 3;
  float part[256];
  for (int tid = 0; tid < 256; ++tid) {
    float acc = 0.0f;
    for (int kv = tid; kv < KV; kv += 256)
      for (int i = 0; i < 8; ++i) {
        int k = (kv << 3) + i;
        acc = fmaf(xr[k], rbf(mx_weight(packed, scales, K, n, k)), acc);
      }
    for (int k = (KV << 3) + tid; k < K; k += 256) acc = fmaf(xr[k], rbf(mx_weight(packed, scales, K, n, k)), acc);
    part[tid] = acc;
  }
  float val = 0.0f;
  for (int w = 0; w < 4; ++w) val = val + butterfly64(part + 64 * w);
  return val;
}

void orc_router(const uint16_t* x, const uint16_t* W, const uint16_t* b,
                int T, int E, int H, uint16_t* out_bf16, float* out_f32) {
  for (int t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e) {
      float v = gemv_tree(x + (size_t)t * H, W + (size_t)e * H, H);
      if (b) v = v + bf(b[e]);
      if (out_bf16) out_bf16[(size_t)t * E + e] = orc_f32_to_bf16(v);
      if (out_f32) out_f32[(size_t)t * E + e] = v;
    }
}

/* ------------------------------------------------------------------------ */
/* Top-k softmax (topk_softmax.cu).                                          */
/* ------------------------------------------------------------------------ */
static inline float sanitize(float v) {            /* topk_softmax.cu:47-52 */
  return ((f2u(v) & 0x7f800000u) == 0x7f800000u) ? -FLT_MAX : v;
}

/* The reference selects with a two-stage warp argmax whose comparator is
 * "greater value, or equal value and lower index" (:60-72) and whose lanes
 * start from (-FLT_MAX, -1) and only take a value strictly above -FLT_MAX
 * (:133-142).  That is exactly: the k largest visible logits (value >
 * -FLT_MAX) ordered by (value desc, index asc), padded with (-FLT_MAX, -1);
 * -0 and +0 compare equal. */
int orc_topk_softmax(const float* logits, int T, int E, int k, int variant,
                     int32_t* idx, float* w) {
  if (!(k == 1 || k == 2 || k == 4 || k == 8)) return -1;
  if (variant == 0) variant = (T <= 8) ? 1 : 2;
  for (int t = 0; t < T; ++t) {
    const float* lg = logits + (size_t)t * E;
    float vals[8] = {0};
    int ids[8] = {0};
    unsigned char* taken = (unsigned char*)calloc((size_t)E, 1);
    for (int s = 0; s < k; ++s) {
      float bv = -FLT_MAX;
      int bi = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        float v = sanitize(lg[e]);
        if (v > bv) { bv = v; bi = e; }      /* first index wins on ties */
      }
      if (bi >= 0) taken[bi] = 1;
      vals[s] = bv;
      ids[s] = bi;
    }
    free(taken);
    int32_t* oi = idx + (size_t)t * k;
    float* ow = w + (size_t)t * k;
    if (ids[0] == -1) {                       /* :339-346 degenerate token */
      for (int s = 0; s < k; ++s) { oi[s] = s; ow[s] = 1.0f / (float)k; }
      continue;
    }
    float mx = -FLT_MAX;
    for (int s = 0; s < k; ++s) if (vals[s] > mx) mx = vals[s];
    float ex[8];
    for (int s = 0; s < k; ++s) ex[s] = oexp(vals[s] - mx);
    float sum;
    if (variant == 1) {                       /* :199-204 sequential from 0 */
      sum = 0.0f;
      for (int s = 0; s < k; ++s) sum = sum + ex[s];
    } else {                                  /* :358-362 xor butterfly over k lanes */
      float v[8];
      for (int s = 0; s < k; ++s) v[s] = ex[s];
      for (int m = k / 2; m > 0; m >>= 1) {
        float tmp[8];
        for (int s = 0; s < k; ++s) tmp[s] = v[s] + v[s ^ m];
        memcpy(v, tmp, sizeof(float) * (size_t)k);
      }
      sum = v[0];
    }
    float inv = 1.0f / sum;
    for (int s = 0; s < k; ++s) {
      oi[s] = ids[s];
      ow[s] = (ids[s] < 0) ? 0.0f : ex[s] * inv;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Dispatch plan: histogram + exclusive scan (moe_permute.cu:24-76) and the  */
/* stable counting sort of moe_compute_gather_map_cpu (:184-236), ep = 1.   */
/* ------------------------------------------------------------------------ */
int orc_plan(const int32_t* idx, int T, int k, int E,
             int32_t* counts, int32_t* offsets, int32_t* gather_map,
             int32_t* perm_token, int32_t* active) {
  const int S = T * k;
  memset(counts, 0, sizeof(int32_t) * (size_t)E);
  for (int s = 0; s < S; ++s)
    if (idx[s] >= 0 && idx[s] < E) counts[idx[s]]++;
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t* pos = (int32_t*)calloc((size_t)E, sizeof(int32_t));
  for (int s = 0; s < S; ++s) {
    int e = idx[s];
    if (e < 0 || e >= E) { gather_map[s] = -1; continue; }
    int p = offsets[e] + pos[e]++;
    gather_map[s] = p;
    if (perm_token) perm_token[p] = s / k;
  }
  free(pos);
  int n = 0;
  for (int e = 0; e < E; ++e)
    if (counts[e] > 0) { if (active) active[n] = e; n++; }
  return n;
}

/* ------------------------------------------------------------------------ */
/* SwiGLU on interleaved rows [g0,u0,g1,u1,...] (swiglu.cu:117-176).         */
/* ------------------------------------------------------------------------ */
void orc_swiglu_rows(const uint16_t* gate_up, int M, int I, float alpha,
                     float limit, uint16_t* out) {
  for (int m = 0; m < M; ++m)
    for (int j = 0; j < I; ++j) {
      float g = bf(gate_up[(size_t)m * 2 * I + 2 * j]);
      float u = bf(gate_up[(size_t)m * 2 * I + 2 * j + 1]);
      out[(size_t)m * I + j] = orc_f32_to_bf16(orc_swiglu(g, u, alpha, limit));
    }
}

/* ------------------------------------------------------------------------ */
/* Combine (moe_combine.cu:69-115): accum = 0; accum += w_k * y_k (compiled  */
/* as fma); accum += residual; bf16.                                         */
/* ------------------------------------------------------------------------ */
void orc_combine(const uint16_t* y, const int32_t* gather_map, const float* w,
                 const uint16_t* residual, int T, int k, int H, uint16_t* out) {
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (int s = 0; s < k; ++s) {
        int g = gather_map[t * k + s];
        if (g < 0) continue;
        acc = fmaf(w[t * k + s], bf(y[(size_t)g * H + h]), acc);
      }
      if (residual) acc = acc + bf(residual[(size_t)t * H + h]);
      out[(size_t)t * H + h] = orc_f32_to_bf16(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: sum of squares with the gemv tree, inv = 1/sqrt(mean + eps),     */
/* out = bf16((x * inv) * w) (rmsnorm.cu:47-83 with IEEE sqrt and divide).   */
/* ------------------------------------------------------------------------ */
void orc_rmsnorm(const uint16_t* x, const uint16_t* w, int T, int H, float eps,
                 uint16_t* out) {
  for (int t = 0; t < T; ++t) {
    const uint16_t* xr = x + (size_t)t * H;
    float ss = gemv_tree(xr, xr, H);
    float mean = ss / (float)H;
    float inv = 1.0f / sqrtf(mean + eps);
    for (int h = 0; h < H; ++h)
      out[(size_t)t * H + h] = orc_f32_to_bf16((bf(xr[h]) * inv) * bf(w[h]));
  }
}

/* fused_residual_rmsnorm_forward (rmsnorm.cu:224-337): s = r + d in fp32,   */
/* sum_out = bf16(s); the sum of squares of the fp32 s with the gemv tree     */
/* (the order of orc_rmsnorm); inv = 1/sqrt(mean + eps) (IEEE);               */
/* normed = bf16((s * inv) * w).  With d = 0 this is orc_rmsnorm of r.        */
void orc_residual_rmsnorm(const uint16_t* r, const uint16_t* d, const uint16_t* w, int T, int H, float eps,
                          uint16_t* normed, uint16_t* sum_out) {
  float* s = (float*)malloc(sizeof(float) * (size_t)H);
  const int KV = H >> 3;
  for (int t = 0; t < T; ++t) {
    const size_t o = (size_t)t * H;
    for (int h = 0; h < H; ++h) {
      s[h] = bf(r[o + h]) + bf(d[o + h]);
      if (sum_out) sum_out[o + h] = orc_f32_to_bf16(s[h]);
    }
    float part[256];
    for (int tid = 0; tid < 256; ++tid) {
      float acc = 0.0f;
      for (int kv = tid; kv < KV; kv += 256)
        for (int i = 0; i < 8; ++i) {
          const float v = s[(kv << 3) + i];
          acc = fmaf(v, v, acc);
        }
      for (int k = (KV << 3) + tid; k < H; k += 256) acc = fmaf(s[k], s[k], acc);
      part[tid] = acc;
    }
    float ss = 0.0f;
    for (int wv = 0; wv < 4; ++wv) ss = ss + butterfly64(part + 64 * wv);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int h = 0; h < H; ++h) normed[o + h] = orc_f32_to_bf16((s[h] * inv) * bf(w[h]));
  }
  free(s);
}

/* ------------------------------------------------------------------------ */
/* Whole layer, multi-threaded over permuted slots.                          */
/* ------------------------------------------------------------------------ */
/* How the product of one active expert is computed (expert_order, see
 * moe_oracle.h). */
enum {
  XP_CANONICAL = 0,   /* this build's order: K-part chains, bias before the rounding */
  XP_FAST_ONE = 1,    /* T == 1 fast path: fused GEMV order, no bias inside the GEMV */
  XP_FUSED_BATCH = 2, /* fused GEMV with the bias inside (a batch of one-token experts) */
  XP_GEMV_DQ = 3,     /* gemv_bf16 over the dequantised weights, then bias_add_rows */
  XP_MULTI = 4        /* several tokens: canonical order, bf16, then bias_add_rows */
};

/* The reference's choice per active expert j (ascending expert ids): one token
 * takes the fast path (moe_layer.cu:1028); otherwise the active experts are
 * cut into batches of 8 in ascending order (:1282-1304), a batch whose experts
 * all hold one token runs the fused GEMV (:1319-1323), any other batch
 * dequantises and runs gemv_bf16 for its one-token experts and hipBLASLt for
 * the rest (:1409-1417). */
static void classify_experts(int T, const int32_t* offsets, const int32_t* active, int n_active, int8_t* klass) {
  enum { kBatch = 8 };
  for (int j0 = 0; j0 < n_active; j0 += kBatch) {
    const int j1 = j0 + kBatch < n_active ? j0 + kBatch : n_active;
    int all_one = 1;
    for (int j = j0; j < j1; ++j)
      if (offsets[active[j] + 1] - offsets[active[j]] != 1) all_one = 0;
    for (int j = j0; j < j1; ++j) {
      const int m = offsets[active[j] + 1] - offsets[active[j]];
      klass[j] = (int8_t)(T == 1 ? XP_FAST_ONE : all_one ? XP_FUSED_BATCH : m == 1 ? XP_GEMV_DQ : XP_MULTI);
    }
  }
}

/* One output of an expert matrix in the order its class uses; the bias goes
 * where that path adds it (b = NULL: no bias). */
static float expert_row(int klass, const float* xr, const uint8_t* P, const uint8_t* Sc, int K, int n,
                        const uint16_t* b, int bias_inside) {
  float v;
  switch (klass) {
    case XP_FAST_ONE:
    case XP_FUSED_BATCH: v = mx_dot_refkernel(xr, P, Sc, K, n); break;
    case XP_GEMV_DQ: v = mx_dot_gemv_tree(xr, P, Sc, K, n); break;
    default: v = mx_dot_canonical(xr, P, Sc, K, n); break;
  }
  if (b == NULL) return v;
  if (bias_inside) return v + bf(b[n]);   /* the GEMV's own epilogue (fused_mxfp4_gemv.cu:180) */
  return rbf(v) + bf(b[n]);               /* a bias kernel over the bf16 product (moe_layer.cu:171-183, 442-463) */
}

/* ------------------------------------------------------------------------ */
/* Whole layer, multi-threaded over permuted slots.                          */
/* ------------------------------------------------------------------------ */
typedef struct {
  const orc_cfg* cfg;
  const orc_weights* wt;
  const uint16_t* x;
  const int32_t* perm_token;
  const int32_t* offsets;
  const int32_t* active;
  const int8_t* klass;      /* [n_active] dispatch class per active expert */
  int n_active;
  int next;                 /* work counter (guarded by mu) */
  pthread_mutex_t mu;
  uint16_t* gate_up;        /* [S][2I] */
  uint16_t* act;            /* [S][I] */
  uint16_t* y;              /* [S][H] */
} layer_job;

/* One unit of work = one active expert of either phase. */
static void* layer_worker_w1(void* arg) {
  layer_job* J = (layer_job*)arg;
  const orc_cfg* c = J->cfg;
  const int H = c->H, I = c->I, N1 = 2 * I;
  float* xr = (float*)malloc(sizeof(float) * (size_t)H);
  for (;;) {
    pthread_mutex_lock(&J->mu);
    int j = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (j >= J->n_active) break;
    int e = J->active[j];
    const int kl = J->klass[j];
    const uint8_t* P = J->wt->w1_packed + (size_t)e * N1 * (H / 2);
    const uint8_t* Sc = J->wt->w1_scales + (size_t)e * N1 * (H / 32);
    const uint16_t* B = J->wt->w1_bias ? J->wt->w1_bias + (size_t)e * N1 : NULL;
    for (int pos = J->offsets[e]; pos < J->offsets[e + 1]; ++pos) {
      const uint16_t* xt = J->x + (size_t)J->perm_token[pos] * H;
      for (int h = 0; h < H; ++h) xr[h] = bf(xt[h]);
      uint16_t* gu = J->gate_up + (size_t)pos * N1;
      /* the fast path's GEMV has no bias: it is added inside the SwiGLU */
      const uint16_t* Bg = kl == XP_FAST_ONE ? NULL : B;
      const int inside = kl == XP_CANONICAL || kl == XP_FUSED_BATCH;
      for (int n = 0; n < N1; ++n) gu[n] = orc_f32_to_bf16(expert_row(kl, xr, P, Sc, H, n, Bg, inside));
      for (int i = 0; i < I; ++i) {
        float g = bf(gu[2 * i]), u = bf(gu[2 * i + 1]);
        if (kl == XP_FAST_ONE && B) {      /* moe_layer.cu:345-352: bias in fp32, no rounding before */
          g = g + bf(B[2 * i]);
          u = u + bf(B[2 * i + 1]);
        }
        J->act[(size_t)pos * I + i] = orc_f32_to_bf16(orc_swiglu(g, u, c->alpha, c->limit));
      }
    }
  }
  free(xr);
  return NULL;
}

static void* layer_worker_w2(void* arg) {
  layer_job* J = (layer_job*)arg;
  const orc_cfg* c = J->cfg;
  const int H = c->H, I = c->I;
  float* ar = (float*)malloc(sizeof(float) * (size_t)I);
  for (;;) {
    pthread_mutex_lock(&J->mu);
    int j = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (j >= J->n_active) break;
    int e = J->active[j];
    const int kl = J->klass[j];
    const uint8_t* P = J->wt->w2_packed + (size_t)e * H * (I / 2);
    const uint8_t* Sc = J->wt->w2_scales + (size_t)e * H * (I / 32);
    const uint16_t* B = J->wt->w2_bias ? J->wt->w2_bias + (size_t)e * H : NULL;
    const int inside = kl == XP_CANONICAL || kl == XP_FUSED_BATCH;
    for (int pos = J->offsets[e]; pos < J->offsets[e + 1]; ++pos) {
      for (int i = 0; i < I; ++i) ar[i] = bf(J->act[(size_t)pos * I + i]);
      for (int n = 0; n < H; ++n)
        J->y[(size_t)pos * H + n] = orc_f32_to_bf16(expert_row(kl, ar, P, Sc, I, n, B, inside));
    }
  }
  free(ar);
  return NULL;
}

static void run_pool(void* (*fn)(void*), layer_job* J, int nthreads) {
  J->next = 0;
  if (nthreads <= 1) { fn(J); return; }
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, fn, J);
  for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
  free(th);
}

/* The one-token fast path's combine (moe_layer.cu:479-497): from the
 * residual, then w_k * y_k in slot order (compiled as fma), bf16.  Slots
 * without an expert (index -1) are skipped. */
static void combine_fast_one(const uint16_t* y, const int32_t* gather_map, const float* w, const uint16_t* residual,
                             int k, int H, uint16_t* out) {
  for (int h = 0; h < H; ++h) {
    float acc = residual ? bf(residual[h]) : 0.0f;
    for (int s = 0; s < k; ++s) {
      int g = gather_map[s];
      if (g < 0) continue;
      acc = fmaf(w[s], bf(y[(size_t)g * H + h]), acc);
    }
    out[h] = orc_f32_to_bf16(acc);
  }
}

/* The expert half of the layer with the routing given (moe_layer.cu:
 * 1196-1549: permute, experts, combine); idx/w are [T][k]. */
static void moe_experts_combine(const orc_cfg* cfg, const orc_weights* wt, const uint16_t* x,
                                const uint16_t* residual, int T, const int32_t* idx, const float* w,
                                uint16_t* out, orc_trace* trace, int nthreads) {
  const int H = cfg->H, E = cfg->E, k = cfg->k, I = cfg->I, S = T * k;
  if (nthreads <= 0) nthreads = (int)sysconf(_SC_NPROCESSORS_ONLN);
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
  int32_t* gmap = (int32_t*)malloc(sizeof(int32_t) * (size_t)S);
  int32_t* ptok = (int32_t*)malloc(sizeof(int32_t) * (size_t)S);
  int32_t* active = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
  int n_active = orc_plan(idx, T, k, E, counts, offsets, gmap, ptok, active);
  int8_t* klass = (int8_t*)calloc((size_t)E, 1);
  if (cfg->expert_order == 1) classify_experts(T, offsets, active, n_active, klass);

  layer_job J;
  memset(&J, 0, sizeof(J));
  J.cfg = cfg; J.wt = wt; J.x = x; J.perm_token = ptok; J.offsets = offsets;
  J.active = active; J.n_active = n_active; J.klass = klass;
  pthread_mutex_init(&J.mu, NULL);
  J.gate_up = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * 2 * I);
  J.act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * I);
  J.y = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * H);
  run_pool(layer_worker_w1, &J, nthreads);
  run_pool(layer_worker_w2, &J, nthreads);
  pthread_mutex_destroy(&J.mu);

  if (cfg->expert_order == 1 && T == 1) combine_fast_one(J.y, gmap, w, residual, k, H, out);
  else orc_combine(J.y, gmap, w, residual, T, k, H, out);

  if (trace) {
    if (trace->gather_map) memcpy(trace->gather_map, gmap, sizeof(int32_t) * (size_t)S);
    if (trace->gate_up) memcpy(trace->gate_up, J.gate_up, sizeof(uint16_t) * (size_t)S * 2 * I);
    if (trace->act) memcpy(trace->act, J.act, sizeof(uint16_t) * (size_t)S * I);
    if (trace->y) memcpy(trace->y, J.y, sizeof(uint16_t) * (size_t)S * H);
  }
  free(J.gate_up); free(J.act); free(J.y);
  free(counts); free(offsets); free(gmap); free(ptok); free(active); free(klass);
}

void orc_moe_forward(const orc_cfg* cfg, const orc_weights* wt,
                     const uint16_t* x, const uint16_t* residual, int T,
                     uint16_t* out, orc_trace* trace, int nthreads) {
  if (T <= 0) return;
  const int H = cfg->H, E = cfg->E, k = cfg->k, S = T * k;

  float* lf = (float*)malloc(sizeof(float) * (size_t)T * E);
  uint16_t* lb = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * E);
  if (cfg->logits_fp32) {
    orc_router(x, wt->router_w, wt->router_b, T, E, H, NULL, lf);
  } else {
    orc_router(x, wt->router_w, wt->router_b, T, E, H, lb, NULL);
    for (size_t i = 0; i < (size_t)T * E; ++i) lf[i] = bf(lb[i]);
  }
  int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)S);
  float* w = (float*)malloc(sizeof(float) * (size_t)S);
  orc_topk_softmax(lf, T, E, k, cfg->topk_variant, idx, w);

  moe_experts_combine(cfg, wt, x, residual, T, idx, w, out, trace, nthreads);

  if (trace) {
    if (trace->logits_bf16 && !cfg->logits_fp32)
      memcpy(trace->logits_bf16, lb, sizeof(uint16_t) * (size_t)T * E);
    if (trace->logits_f32) memcpy(trace->logits_f32, lf, sizeof(float) * (size_t)T * E);
    if (trace->idx) memcpy(trace->idx, idx, sizeof(int32_t) * (size_t)S);
    if (trace->w) memcpy(trace->w, w, sizeof(float) * (size_t)S);
  }
  free(lf); free(lb); free(idx); free(w);
}

void orc_moe_forward_routed(const orc_cfg* cfg, const orc_weights* wt,
                            const uint16_t* x, const uint16_t* residual, int T,
                            const int32_t* idx, const float* w,
                            uint16_t* out, orc_trace* trace, int nthreads) {
  if (T <= 0) return;
  moe_experts_combine(cfg, wt, x, residual, T, idx, w, out, trace, nthreads);
}
