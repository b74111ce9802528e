// moe_device.h -- device-side helpers shared by the gfx950 MoE kernels.
//
// Every floating-point step here is an IEEE operation whose result is fixed
// by its inputs (add, mul, fma, divide, rint, ldexp), so the CPU oracle that
// performs the same sequence produces the same bits.  All HIP sources of this
// library are compiled with -ffp-contract=off; fused multiply-adds are written
// as __builtin_fmaf where the order of the reference needs them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gxmoe {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN with its sign and leading
// payload bits (the upper half of the input with the quiet bit set).  This is
// what gfx950's v_cvt_pk_bf16_f32 computes (checked on the device against
// the integer form  nan ? (u >> 16) | 0x40 : (u + 0x7fff + ((u >> 16) & 1))
// >> 16  over 4.2 M inputs: random bit patterns, every exponent with tie and
// near-tie mantissas, denormals, infinities and NaN payloads), so one
// instruction rounds two values.
typedef __bf16 gx_bf16x2_cvt __attribute__((ext_vector_type(2)));
typedef float gx_f32x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(gx_f32x2_cvt{lo, hi}, gx_bf16x2_cvt));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// e^x by Cody-Waite reduction x = n*ln2 + r (|r| <= ln2/2, two-constant
// split of ln 2 applied with fma) and the degree-7 Taylor polynomial of e^r
// in Horner form, scaled by 2^n with ldexp.
// NaN, overflow (inf) and underflow (0) are selected after the polynomial
// path rather than branched to (the same function, no divergent branch).
__device__ __forceinline__ float gx_expf(float x) {
  const float log2e = 1.44269502162933349609375f;
  const float ln2_hi = 0.693147182464599609375f;
  const float ln2_lo = -1.904654323148236e-09f;
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);  // keeps n an in-range int
  float n = __builtin_rintf(xc * log2e);
  float r = __builtin_fmaf(-n, ln2_hi, xc);
  r = __builtin_fmaf(-n, ln2_lo, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  float v = __builtin_ldexpf(p, static_cast<int>(n));
  // three independent selects (a nested conditional expression compiles to
  // exec-mask branches here)
  v = x < -103.97208404541015625f ? 0.0f : v;
  v = x > 88.72283935546875f ? __builtin_inff() : v;
  return x != x ? x : v;
}

// GPT-OSS clamped SwiGLU on one (gate, up) pair: gate clamped above at
// `limit`, up clamped to [-limit, limit], out = (up + 1) * gate * sigmoid(alpha*gate).
__device__ __forceinline__ float gx_swiglu(float g, float u, float alpha, float limit) {
  g = __builtin_fminf(g, limit);
  u = __builtin_fminf(__builtin_fmaxf(u, -limit), limit);
  float e = gx_expf((-alpha) * g);
  float glu = g / (1.0f + e);
  return (u + 1.0f) * glu;
}

// ---- activations as two e4m3 parts for the block-scaled products ----------
// A 32-element block with largest magnitude m is split as v = (hi + lo/32) s,
// s = 2^(e - 7), e = the exponent of m: |v / s| < 256 fits e4m3 (max 448),
// hi = RNE(v / s) and lo = RNE((v / s - hi) * 32).  For |v| >= 2^-13 m, hi is
// a normal e4m3 value (4 significant bits), so v / s - hi has at most four
// significant bits and lies on lo's grid: the split is exact.  (gfx950's
// v_cvt_pk_fp8_f32 encodes OCP e4m3 with round to nearest even.)

// e8m0 codes of s and of s / 32, packed as code(s) | code(s / 32) << 8, and
// 1 / s; m >= 0 (inf or NaN gives codes of 2^121 that fp8x2_quant4 pairs
// with NaN parts).  Blocks below 2^-114 take s = 2^-121 (their parts
// underflow, an error below 2^-120).
__device__ __forceinline__ uint32_t fp8x2_codes(float m, float& inv_s) {
  int e = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu) - 127;
  e = e < -114 ? -114 : e;
  inv_s = __uint_as_float(static_cast<uint32_t>(127 + 7 - e) << 23);
  return static_cast<uint32_t>(e + 120) | (static_cast<uint32_t>(e + 115) << 8);
}

// Four values of one block -> four hi bytes and four lo bytes (byte i =
// element i).  finite = false (the block holds inf or NaN): NaN parts.
__device__ __forceinline__ void fp8x2_quant4(float v0, float v1, float v2, float v3, float inv_s, bool finite,
                                             uint32_t& hi, uint32_t& lo) {
  const float a0 = v0 * inv_s, a1 = v1 * inv_s, a2 = v2 * inv_s, a3 = v3 * inv_s;  // exact: power-of-two scale
  uint32_t h = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a0, a1, 0, false));
  h = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a2, a3, static_cast<int>(h), true));
  const int hs = static_cast<int>(h);
  const float r0 = (a0 - __builtin_amdgcn_cvt_f32_fp8(hs, 0)) * 32.0f;  // exact residuals
  const float r1 = (a1 - __builtin_amdgcn_cvt_f32_fp8(hs, 1)) * 32.0f;
  const float r2 = (a2 - __builtin_amdgcn_cvt_f32_fp8(hs, 2)) * 32.0f;
  const float r3 = (a3 - __builtin_amdgcn_cvt_f32_fp8(hs, 3)) * 32.0f;
  uint32_t l = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(r0, r1, 0, false));
  l = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(r2, r3, static_cast<int>(l), true));
  hi = finite ? h : 0x7f7f7f7fu;
  lo = finite ? l : 0u;
}

// e8m0 scale byte -> fp32 by placing the code in the exponent field
// (code 0 -> +0, 255 -> +inf).
__device__ __forceinline__ float e8m0_to_f32(uint32_t code) {
  return __uint_as_float((code & 0xffu) << 23);
}

// Two e2m1 nibbles of byte `sel` of `packed` times `scale` into two floats
// (low nibble first), with the gfx950 scaled fp4 conversion.
template <int sel>
__device__ __forceinline__ void fp4x2_to_f32(uint32_t packed, float scale, float& lo, float& hi) {
  auto v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(packed, scale, sel);
  lo = v[0];
  hi = v[1];
}

// Decode 8 e2m1 values (one dword, low nibble first) with the e8m0 scale
// `code`.  For codes 1..254 the gfx950 scaled conversion returns
// e2m1 * 2^(code-127) exactly (denormal results included).  Codes 0 and 255
// are decoded as the reference's register path does (code << 23 as the
// scale: +0 and +inf, fused_mxfp4_gemv.cu:42-45): the conversion runs with
// scale 1 (exact e2m1 values) and the IEEE product with the scale follows.
__device__ __forceinline__ void decode8(uint32_t d, uint32_t code, float* w) {
  const float scale = e8m0_to_f32(code);
  const bool special = ((code & 0xffu) - 1u) >= 254u;
  const float cs = special ? 1.0f : scale;
  fp4x2_to_f32<0>(d, cs, w[0], w[1]);
  fp4x2_to_f32<1>(d, cs, w[2], w[3]);
  fp4x2_to_f32<2>(d, cs, w[4], w[5]);
  fp4x2_to_f32<3>(d, cs, w[6], w[7]);
  if (__builtin_expect(special, 0)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = w[j] * scale;
  }
}

// decode8 for a scale known to come from a code in 1..254 (scale = its
// e8m0_to_f32 value): the conversion alone is exact.
__device__ __forceinline__ void decode8_regular(uint32_t d, float scale, float* w) {
  fp4x2_to_f32<0>(d, scale, w[0], w[1]);
  fp4x2_to_f32<1>(d, scale, w[2], w[3]);
  fp4x2_to_f32<2>(d, scale, w[4], w[5]);
  fp4x2_to_f32<3>(d, scale, w[6], w[7]);
}

// True if any byte of `v` selected by `mask` (0xff per selected byte) is an
// e8m0 code outside 1..254 (0x00 or 0xff).
__device__ __forceinline__ bool has_special_code(uint32_t v, uint32_t mask) {
  const uint32_t x = (v & mask) | (0x01010101u & ~mask);  // unselected bytes read as code 1
  const uint32_t y = ~x;
  return (((x - 0x01010101u) & ~x & 0x80808080u) | ((y - 0x01010101u) & ~y & 0x80808080u)) != 0u;
}

typedef uint32_t gx_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 gx_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 gx_bf16x2 __attribute__((ext_vector_type(2)));

// Row r's 16 bytes of one tiled MXFP4 block (layout in moe_kernels.h), given
// p = &block[tiled_dword(r, 0)]: dword g is slot 16 g + r % 16, 64 dwords
// after dword g - 1.  Nontemporal: streamed weights are read once.
__device__ __forceinline__ gx_u32x4 load_row_block_nt(const uint32_t* p) {
  gx_u32x4 v;
  v[0] = __builtin_nontemporal_load(p);
  v[1] = __builtin_nontemporal_load(p + 64);
  v[2] = __builtin_nontemporal_load(p + 128);
  v[3] = __builtin_nontemporal_load(p + 192);
  return v;
}

__device__ __forceinline__ gx_u32x4 load_row_block(const uint32_t* p) {
  gx_u32x4 v;
  v[0] = p[0];
  v[1] = p[64];
  v[2] = p[128];
  v[3] = p[192];
  return v;
}

// Eight e2m1 values (one dword, low nibble first) times the e8m0 scale as
// bf16, for a scale from a code in 1..254: the gfx950 scaled conversion is
// exact (e2m1 x 2^(code-127) has at most two significant bits).
__device__ __forceinline__ gx_bf16x8 decode8_bf16(uint32_t d, float scale) {
  const gx_bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0);
  const gx_bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1);
  const gx_bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2);
  const gx_bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3);
  const gx_u32x4 w{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1), __builtin_bit_cast(uint32_t, p2),
                   __builtin_bit_cast(uint32_t, p3)};
  return __builtin_bit_cast(gx_bf16x8, w);
}

// decode8_bf16 for any code (a zero-extended byte).  Codes 0 and 255 follow
// the reference's register decode (scale code << 23: +0 and +inf, so +-0,
// +-inf and NaN for 0 x inf), built from the exact e2m1 values.
__device__ __forceinline__ gx_bf16x8 decode8_bf16_special(uint32_t d, uint32_t code) {
  const float scale = __uint_as_float(code << 23);
  float w[8];
  fp4x2_to_f32<0>(d, 1.0f, w[0], w[1]);
  fp4x2_to_f32<1>(d, 1.0f, w[2], w[3]);
  fp4x2_to_f32<2>(d, 1.0f, w[4], w[5]);
  fp4x2_to_f32<3>(d, 1.0f, w[6], w[7]);
  gx_bf16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = __builtin_bit_cast(__bf16, f32_to_bf16(w[j] * scale));
  return r;
}

// 64-lane xor butterfly sum: after it every lane holds the same value, the
// tree v[l] + v[l^m] for m = 32, 16, 8, 4, 2, 1.
__device__ __forceinline__ float wave_butterfly_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, kWave);
  return v;
}

// LDS-only work-group barrier: orders the LDS traffic of the waves without
// waiting for their global memory operations (a weight stream stays in
// flight; stores that no other wave of the launch reads need not complete).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace gxmoe
