// moe_route.hip -- router GEMV + top-k softmax + device routing plan (gfx950).
//
// Replaces the reference's router GEMV/GEMM (gemv_bf16.cu:40-130,
// cuda_utils.h:226-308), topk_softmax_forward (topk_softmax.cu:380-432),
// moe_permute_classify (moe_permute.cu:129-179) and the host gather map
// (moe_permute.cu:184-236, moe_layer.cu:1217-1234), with no host round trip:
//
//   logits_kernel      each wave computes whole logits (TT tokens x EPW
//                      experts) with the gemv_bf16_kernel summation tree
//                      (few tokens);
//   logits_lds_kernel  (many tokens) the same tree, chains of 64 pairs per
//                      lane, each pair's butterfly run in one lane after an
//                      LDS transpose;
//   topk_plan_kernel   (T <= kTopkPlanMaxT) one work-group of 16 waves selects
//                      every token's top-k and builds the plan from LDS;
//   logits_mfma_kernel (T > 64) the logits on the matrix cores, operands
//                      staged in LDS by direct loads;
//   topk16_kernel +    (larger T) top-k spread over the device, sixteen lanes
//   plan_kernel        a token (topk_kernel, a wave a token, when E % 4 != 0
//                      or the logits are unaligned), then the plan from the
//                      selections.
//
// Kernel boundaries order the stages: no values cross work-groups inside a
// launch, so there are no tickets, exchange buffers or cache maintenance.
//
// Lane reductions use the gfx950 cross-lane moves (v_permlane32_swap and
// v_permlane16_swap for lanes 32 and 16 apart, DPP row_shl within 16-lane
// rows) instead of LDS permutes: a reduction to lane 0 is 6 VALU steps.
#include <float.h>

#include <algorithm>
#include <type_traits>

#include "moe_device.h"
#include "moe_kernels.h"
#include "moe_stages.h"
#include "moe_topk.h"

namespace gxmoe {

namespace {

constexpr int kRouteThreads = 256;
constexpr int kPlanThreads = 1024;
constexpr int kTopkPlanMaxT = 256;  // tokens of the single-work-group top-k + plan

// Dispatch plan over the T*k slots of `idx` with NT threads: counts,
// exclusive offsets, a gather map that is stable in slot order (the counting
// sort of moe_permute.cu:184-236), the permuted token list, the ascending
// list of experts with at least one slot and the task records.  Slots with an
// index outside [0, E) get gather_map = -1 and are not dispatched.
//
// Wave w owns the contiguous slots [w C, (w + 1) C).  Pass 1 counts its
// slots per expert 64 at a time: lanes with equal experts find each other by
// ballots over the expert bits and the lowest adds the group's size (LDS
// operations of one wave execute in order, so no atomics and no barrier).
// A scan over the waves then gives each (wave, expert) its base, and pass 2
// walks the chunk again: position = offset[e] + base[w][e] + rank.  The
// barriers order LDS only: no wave reads another's global stores.
template <int NT, typename IdxFn>
__device__ void build_plan(IdxFn idx, int T, int k, int E, PlanBufs p) {
  constexpr int NW = NT / kWave;
  static_assert(NT >= kMaxExperts, "one thread per expert in the scan");
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_wc[NW][kMaxExperts];  // pass 1: per-wave counts; then per-wave bases
  __shared__ int s_aidx[kMaxExperts];
  __shared__ unsigned long long s_mask[kMaxExperts / kWave];
  __shared__ int s_wsum[kMaxExperts / kWave];
  const int tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  const int S = T * k;
  const int C = ((S + NW - 1) / NW + kWave - 1) / kWave * kWave;  // slots per wave, a multiple of 64
  const int s0 = min(S, warp * C), s1 = min(S, s0 + C);
  const int nws = C > 0 ? (S + C - 1) / C : 0;  // waves holding slots: the only nonzero counts

  // rank of this lane's slot among the 64 slots' equal experts and the
  // group mask (wave-uniform control flow)
  auto group = [&](int e, bool valid, unsigned long long& peers) -> int {
    peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {  // E <= 256
      const bool bit = valid && ((e >> b) & 1);
      const unsigned long long mb = __ballot(bit);
      peers &= bit ? mb : ~mb;
    }
    return __popcll(peers & ((1ull << lane) - 1ull));
  };

  for (int i = tid; i < nws * kMaxExperts; i += NT) (&s_wc[0][0])[i] = 0;
  lds_barrier();
  for (int b = s0; b < s1; b += kWave) {
    const int s = b + lane;
    const int e = s < s1 ? idx(s) : -1;
    const bool valid = e >= 0 && e < E;
    unsigned long long peers;
    const int rank = group(e, valid, peers);
    if (valid && rank == 0) s_wc[warp][e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
  lds_barrier();

  // per-wave bases within each expert, then the exclusive scan over experts
  // (E <= 256: one value per thread of waves 0..3)
  int c = 0, incl = 0;
  bool act = false;
  unsigned long long am = 0ull;
  if (tid < kMaxExperts) {  // wave-uniform
    if (tid < E) {
#pragma unroll 4
      for (int w = 0; w < nws; ++w) {
        const int v = s_wc[w][tid];
        s_wc[w][tid] = c;
        c += v;
      }
    }
    incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += o;
    }
    if (lane == 63) s_wsum[warp] = incl;
    act = (tid < E) && (c > 0);
    am = __ballot(act);
    if (lane == 0) s_mask[warp] = am;
  }
  lds_barrier();
  int nact = 0;
#pragma unroll
  for (int w = 0; w < kMaxExperts / kWave; ++w) nact += __popcll(s_mask[w]);
  if (tid < kMaxExperts) {
    int base = 0, abase = 0;
    for (int w = 0; w < warp; ++w) {
      base += s_wsum[w];
      abase += __popcll(s_mask[w]);
    }
    const int excl = base + incl - c;
    if (tid < E) {
      s_off[tid] = excl;
      p.counts[tid] = c;
      p.offsets[tid] = excl;
    }
    if (tid == E - 1) {
      s_off[E] = excl + c;
      p.offsets[E] = excl + c;
    }
    const int aidx = abase + __popcll(am & ((1ull << lane) - 1ull));
    if (act) {
      p.active[aidx] = tid;
      s_aidx[tid] = aidx;
      if (p.tasks) {
        int32_t* t = p.tasks + static_cast<size_t>(aidx) * kTaskInts;
        t[0] = tid;
        t[1] = excl;
        t[2] = c;
        t[3] = 0;
      }
    }
    if (p.tasks && tid < E && tid >= nact) p.tasks[static_cast<size_t>(tid) * kTaskInts] = -1;
  }
  if (tid == 0) *p.n_active = nact;
  lds_barrier();

  // pass 2: stable positions
  for (int b = s0; b < s1; b += kWave) {
    const int s = b + lane;
    const int e = s < s1 ? idx(s) : -1;
    const bool valid = e >= 0 && e < E;
    unsigned long long peers;
    const int rank = group(e, valid, peers);
    if (valid) {
      const int pos = s_off[e] + s_wc[warp][e] + rank;
      p.gather_map[s] = pos;
      p.perm_token[pos] = s / k;
      if (p.tasks && pos - s_off[e] < kTaskTokens)
        p.tasks[static_cast<size_t>(s_aidx[e]) * kTaskInts + 4 + (pos - s_off[e])] = s / k;
    } else if (s < s1) {
      p.gather_map[s] = -1;
    }
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) s_wc[warp][e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

// Logits of TT tokens x EPW experts per wave (work-group: 4 waves, 4 EPW
// consecutive experts) with the gemv_bf16_kernel tree (gemv_bf16.cu:57-129):
// logical thread tau = lane + 64 j (j = 0..3) chains fmaf over the 8-element
// chunks tau, tau + 256, ... in that order; the chains of wave j are summed
// by the xor-butterfly tree; the four wave sums are added in order from 0;
// + bias; bf16 (or fp32) rounding.  Lane l holds chain j of every (token,
// expert) pair of the wave in acc[t][e][j]; its chunk positions are
// c = l + 64 p, p = j + 4 r.  NCH > 0: every position is loaded before the
// first FMA (H <= 512 NCH); NCH == 0: any H, one position at a time.
template <int TT, int EPW, int NCH, bool F32>
__global__ __launch_bounds__(kRouteThreads) void logits_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ W,
                                                               const uint16_t* __restrict__ bias, int T, int E, int H,
                                                               void* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int e0 = (blockIdx.x * 4 + wv) * EPW;
  const int t0 = blockIdx.y * TT;
  if (e0 >= E) return;  // wave-uniform; the kernel has no barriers
  const int KV = H >> 3;
  float acc[TT][EPW][4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int e = 0; e < EPW; ++e)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][e][j] = 0.0f;
  // rows past T / E read row 0 (their results are not stored)
  const uint16_t* xr[TT];
  const uint16_t* wr[EPW];
#pragma unroll
  for (int t = 0; t < TT; ++t) xr[t] = x + static_cast<size_t>(t0 + t < T ? t0 + t : 0) * H;
#pragma unroll
  for (int e = 0; e < EPW; ++e) wr[e] = W + static_cast<size_t>(e0 + e < E ? e0 + e : 0) * H;
  auto fma_chunk = [&](int j, const uint4 (&xv)[TT], const uint4 (&wv4)[EPW]) __attribute__((always_inline)) {
    float wf[EPW][8];
#pragma unroll
    for (int e = 0; e < EPW; ++e) unpack_bf16x8(wv4[e], wf[e]);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float xf[8];
      unpack_bf16x8(xv[t], xf);
#pragma unroll
      for (int e = 0; e < EPW; ++e)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[t][e][j] = __builtin_fmaf(xf[i], wf[e][i], acc[t][e][j]);
    }
  };
  if constexpr (NCH > 0) {
    uint4 xv[NCH][TT], wv4[NCH][EPW];
#pragma unroll
    for (int q = 0; q < NCH; ++q) {
      const int c = min(lane + kWave * q, KV - 1);  // positions past KV load a valid chunk, unused
#pragma unroll
      for (int t = 0; t < TT; ++t) xv[q][t] = *reinterpret_cast<const uint4*>(xr[t] + c * 8);
#pragma unroll
      for (int e = 0; e < EPW; ++e) wv4[q][e] = *reinterpret_cast<const uint4*>(wr[e] + c * 8);
    }
#pragma unroll
    for (int q = 0; q < NCH; ++q)
      if (lane + kWave * q < KV) fma_chunk(q & 3, xv[q], wv4[q]);
  } else {
    for (int r = 0; kRouteThreads * r < KV; ++r) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = lane + kWave * j + kRouteThreads * r;
        if (c < KV) {
          uint4 xv[TT], wv4[EPW];
#pragma unroll
          for (int t = 0; t < TT; ++t) xv[t] = *reinterpret_cast<const uint4*>(xr[t] + c * 8);
#pragma unroll
          for (int e = 0; e < EPW; ++e) wv4[e] = *reinterpret_cast<const uint4*>(wr[e] + c * 8);
          fma_chunk(j, xv, wv4);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
#pragma unroll
    for (int e = 0; e < EPW; ++e) {
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) v = v + tree_sum_lane0(acc[t][e][j]);
      if (lane == 0 && t0 + t < T && e0 + e < E) {
        if (bias != nullptr) v = v + bf16_to_f32(bias[e0 + e]);
        const size_t o = static_cast<size_t>(t0 + t) * E + e0 + e;
        if constexpr (F32) reinterpret_cast<float*>(logits)[o] = v;
        else reinterpret_cast<uint16_t*>(logits)[o] = f32_to_bf16(v);
      }
    }
  }
}

// logits_kernel<TT, EPW, 6> with the residual RMSNorm of rmsnorm.cu:224-337
// in front: x is the residual stream.  Each wave forms s = x + delta (fp32)
// for its tokens from the chunks it holds (every chunk c = l + 64 q of the
// row, q < 6), the sum of squares of s with the router's tree (the chains
// and butterflies of the logits), inv = 1/sqrt(mean + eps) and the normed
// bf16 values the products then read.  Wave 0 of the work-groups of experts
// 0.. also writes normed and sum_out = bf16(s) for the experts' launches.
template <int TT, int EPW, bool F32>
__global__ __launch_bounds__(kRouteThreads) void logits_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ delta, const uint16_t* __restrict__ norm_w, float eps,
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ bias, int T, int E, int H,
    void* __restrict__ logits, uint16_t* __restrict__ normed, uint16_t* __restrict__ sum_out) {
  constexpr int NCH = 6;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int e0 = (blockIdx.x * 4 + wv) * EPW;
  const int t0 = blockIdx.y * TT;
  if (e0 >= E) return;  // wave-uniform; wave 0 of work-group 0 always has experts
  const int KV = H >> 3;
  const uint16_t* wr[EPW];
#pragma unroll
  for (int e = 0; e < EPW; ++e) wr[e] = W + static_cast<size_t>(e0 + e < E ? e0 + e : 0) * H;
  // rows past T read row 0 (their results are not stored)
  size_t rowo[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) rowo[t] = static_cast<size_t>(t0 + t < T ? t0 + t : 0) * H;
  uint4 xv[NCH][TT], dv[NCH][TT], wv4[NCH][EPW], nwv[NCH];
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int c = min(lane + kWave * q, KV - 1);  // positions past KV load a valid chunk, unused
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      xv[q][t] = *reinterpret_cast<const uint4*>(x + rowo[t] + c * 8);
      dv[q][t] = *reinterpret_cast<const uint4*>(delta + rowo[t] + c * 8);
    }
#pragma unroll
    for (int e = 0; e < EPW; ++e) wv4[q][e] = *reinterpret_cast<const uint4*>(wr[e] + c * 8);
    nwv[q] = *reinterpret_cast<const uint4*>(norm_w + c * 8);
  }
  auto sum8 = [&](int q, int t, float (&s8)[8]) __attribute__((always_inline)) {
    float a[8], b[8];
    unpack_bf16x8(xv[q][t], a);
    unpack_bf16x8(dv[q][t], b);
#pragma unroll
    for (int i = 0; i < 8; ++i) s8[i] = a[i] + b[i];
  };
  // sum of squares: chain j = q & 3 takes positions q = j, j + 4 in order
  float inv[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    float ssa[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < NCH; ++q)
      if (lane + kWave * q < KV) {
        float s8[8];
        sum8(q, t, s8);
#pragma unroll
        for (int i = 0; i < 8; ++i) ssa[q & 3] = __builtin_fmaf(s8[i], s8[i], ssa[q & 3]);
      }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) ss = ss + tree_sum_lane0(ssa[j]);
    ss = __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(ss)), 0)));
    inv[t] = 1.0f / __builtin_sqrtf(ss / static_cast<float>(H) + eps);
  }
  // normed chunks (bf16), replacing the x chunks; the designated wave stores them
  const bool writer = blockIdx.x == 0 && wv == 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    float wn[8];
    unpack_bf16x8(nwv[q], wn);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      float s8[8];
      sum8(q, t, s8);
      uint32_t o[4], so[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = f32_to_bf16((s8[2 * i] * inv[t]) * wn[2 * i]) |
               (static_cast<uint32_t>(f32_to_bf16((s8[2 * i + 1] * inv[t]) * wn[2 * i + 1])) << 16);
        so[i] = f32_to_bf16(s8[2 * i]) | (static_cast<uint32_t>(f32_to_bf16(s8[2 * i + 1])) << 16);
      }
      xv[q][t] = make_uint4(o[0], o[1], o[2], o[3]);
      const int c = lane + kWave * q;
      if (writer && c < KV && t0 + t < T) {
        *reinterpret_cast<uint4*>(normed + rowo[t] + c * 8) = xv[q][t];
        if (sum_out) *reinterpret_cast<uint4*>(sum_out + rowo[t] + c * 8) = make_uint4(so[0], so[1], so[2], so[3]);
      }
    }
  }
  float acc[TT][EPW][4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int e = 0; e < EPW; ++e)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][e][j] = 0.0f;
#pragma unroll
  for (int q = 0; q < NCH; ++q)
    if (lane + kWave * q < KV) {
      float wf[EPW][8];
#pragma unroll
      for (int e = 0; e < EPW; ++e) unpack_bf16x8(wv4[q][e], wf[e]);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        float xf[8];
        unpack_bf16x8(xv[q][t], xf);
#pragma unroll
        for (int e = 0; e < EPW; ++e)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[t][e][q & 3] = __builtin_fmaf(xf[i], wf[e][i], acc[t][e][q & 3]);
      }
    }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
#pragma unroll
    for (int e = 0; e < EPW; ++e) {
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) v = v + tree_sum_lane0(acc[t][e][j]);
      if (lane == 0 && t0 + t < T && e0 + e < E) {
        if (bias != nullptr) v = v + bf16_to_f32(bias[e0 + e]);
        const size_t o = static_cast<size_t>(t0 + t) * E + e0 + e;
        if constexpr (F32) reinterpret_cast<float*>(logits)[o] = v;
        else reinterpret_cast<uint16_t*>(logits)[o] = f32_to_bf16(v);
      }
    }
  }
}

// Logits of 8 tokens x 8 experts per work-group with the same tree, for
// many tokens.  Wave j is the reference's wave j: lane l chains fmaf over
// the chunks tau = l + 64 j, tau + 256, ... of all 64 (token, expert) pairs
// at once (each loaded chunk feeds 8 pairs); the chains then go through LDS
// so that lane p holds the 64 chains of pair p and runs the xor-butterfly
// tree of tree_sum_lane0 in registers (level m adds lane l + m into lane l,
// m = 32 .. 1); lane p of wave 0 adds the four wave sums in order from 0.
constexpr int kLdsTT = 8, kLdsEPW = 8;
template <bool F32, bool kHoldW>
__global__ __launch_bounds__(kRouteThreads, 2) void logits_lds_kernel(const uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ W,
                                                                      const uint16_t* __restrict__ bias, int T, int E,
                                                                      int H, void* __restrict__ logits) {
  constexpr int kPairs = kLdsTT * kLdsEPW;  // = kWave: one pair per lane in the tree phase
  static_assert(kPairs == kWave, "one pair per lane");
  __shared__ float red[4][kPairs][kWave + 1];  // [wave][pair][lane], padded: conflict-free rows and columns
  const int lane = threadIdx.x & 63;
  const int j = threadIdx.x >> 6;
  const int e0 = blockIdx.x * kLdsEPW;
  const int KV = H >> 3;
  // rows past T / E read row 0 (their results are not stored)
  const uint16_t* wr = W + static_cast<size_t>(e0 < E ? e0 : 0) * H;
  const int en = min(kLdsEPW, E - e0);
  auto load_w = [&](int c, uint4 (&wv4)[kLdsEPW]) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < kLdsEPW; ++e)
      wv4[e] = *reinterpret_cast<const uint4*>(wr + static_cast<size_t>(e < en ? e : 0) * H + c * 8);
  };
  // kHoldW (H <= 4096, so a chain has at most two chunks): the lane's chunks
  // of the 8 router rows, loaded once and held while the work-group walks
  // its token blocks (blockIdx.y, + gridDim.y, ...); otherwise one token
  // block per work-group with both operands loaded per chunk.
  uint4 wh[kHoldW ? 2 : 1][kLdsEPW];
  if constexpr (kHoldW) {
#pragma unroll
    for (int q = 0; q < 2; ++q) load_w(min(lane + kWave * j + kRouteThreads * q, KV - 1), wh[q]);
  }
  const int ntb = (T + kLdsTT - 1) / kLdsTT;
  for (int tb = blockIdx.y; tb < ntb; tb += kHoldW ? static_cast<int>(gridDim.y) : ntb) {
    const int t0 = tb * kLdsTT;
    float acc[kLdsTT][kLdsEPW];
#pragma unroll
    for (int t = 0; t < kLdsTT; ++t)
#pragma unroll
      for (int e = 0; e < kLdsEPW; ++e) acc[t][e] = 0.0f;
    const uint16_t* xr = x + static_cast<size_t>(t0 < T ? t0 : 0) * H;
    const int tn = min(kLdsTT, T - t0);
    auto load_x = [&](int c, uint4 (&xv)[kLdsTT]) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < kLdsTT; ++t)
        xv[t] = *reinterpret_cast<const uint4*>(xr + static_cast<size_t>(t < tn ? t : 0) * H + c * 8);
    };
    auto fma_chunk = [&](const uint4 (&xv)[kLdsTT], const uint4 (&wv4)[kLdsEPW]) __attribute__((always_inline)) {
      float wf[kLdsEPW][8];
#pragma unroll
      for (int e = 0; e < kLdsEPW; ++e) unpack_bf16x8(wv4[e], wf[e]);
#pragma unroll
      for (int t = 0; t < kLdsTT; ++t) {
        float xf[8];
        unpack_bf16x8(xv[t], xf);
#pragma unroll
        for (int e = 0; e < kLdsEPW; ++e)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[t][e] = __builtin_fmaf(xf[i], wf[e][i], acc[t][e]);
      }
    };
    // Chunks tau, tau + 256, ... in order.
    if constexpr (kHoldW) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int c = lane + kWave * j + kRouteThreads * q;
        if (c < KV) {
          uint4 xa[kLdsTT];
          load_x(c, xa);
          fma_chunk(xa, wh[q]);
        }
      }
    } else {
      for (int c = lane + kWave * j; c < KV; c += kRouteThreads) {
        uint4 xa[kLdsTT], wa[kLdsEPW];
        load_x(c, xa);
        load_w(c, wa);
        fma_chunk(xa, wa);
      }
    }
#pragma unroll
    for (int t = 0; t < kLdsTT; ++t)
#pragma unroll
      for (int e = 0; e < kLdsEPW; ++e) red[j][t * kLdsEPW + e][lane] = acc[t][e];
    __syncthreads();
    float cv[kWave];
#pragma unroll
    for (int l = 0; l < kWave; ++l) cv[l] = red[j][lane][l];
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1)
#pragma unroll
      for (int l = 0; l < m; ++l) cv[l] = cv[l] + cv[l + m];
    __syncthreads();  // every row read before the sums overwrite column 0
    red[j][lane][0] = cv[0];
    __syncthreads();
    if (j == 0) {
      const int t = lane / kLdsEPW, e = lane % kLdsEPW;
      float v = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) v = v + red[jj][lane][0];
      if (t < tn && e < en) {
        if (bias != nullptr) v = v + bf16_to_f32(bias[e0 + e]);
        const size_t o = static_cast<size_t>(t0 + t) * E + e0 + e;
        if constexpr (F32) reinterpret_cast<float*>(logits)[o] = v;
        else reinterpret_cast<uint16_t*>(logits)[o] = f32_to_bf16(v);
      }
    }
    if constexpr (kHoldW) __syncthreads();  // the sums are read before the next block's chains land in red
  }
}

// Top-k softmax of every token, one token per wave.
template <bool F32, int NV>
__global__ __launch_bounds__(kRouteThreads) void topk_kernel(const void* logits, int T, int E, int k, int variant,
                                                            int32_t* idx, float* w, int32_t* tpe) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (kRouteThreads / kWave) + (threadIdx.x >> 6);
  if (t >= T) return;
  float v[NV];
  load_token_logits<F32, NV>(logits, t, E, lane, v);
  topk_token<NV, !F32>(v, k, variant, idx + static_cast<size_t>(t) * k, w + static_cast<size_t>(t) * k, tpe, lane);
}

// Top-k softmax of every token, kTopkGroup = 16 lanes per token (four tokens
// a wave).  Lane g of a token holds experts 64 c + 4 g .. 64 c + 4 g + 3, one
// 16-byte (fp32) or 8-byte (bf16) load per c.  A round takes the largest of
// the lanes' 64-bit words select_key << 32 | ~expert (value descending, and
// among equal values the smallest expert: the order of select_topk), which the
// sixteen lanes agree on through four DPP exchanges (lane pairs, quads, the
// mirrored halves of eight lanes, of sixteen); words are distinct, so the
// winner clears itself by equality, and a round whose largest word is 0 (no
// finite logit left) yields the padding (-FLT_MAX, -1).  The selected value
// comes back from its key (-0 as +0, which no slot weight can tell apart:
// both give exp(0) against either as the maximum).  Same slots as
// topk_kernel.
//
// Work-group b takes 16 tokens of the 32-token block (b / 16) * 8 + b % 8,
// half (b / 8) % 2: the block whose logits the matrix-core router kernel
// wrote on the same XCD (b % 8), so they are read where they were written
// (measured 1.1 us less after that kernel at 4096 tokens).  Requires E % 4 ==
// 0, E <= 256 and logits aligned to the load width (the launcher checks).
constexpr int kTopkGroup = 16;
template <int Ctrl>
__device__ __forceinline__ uint64_t max_dpp_u64(uint64_t x) {
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(x)), Ctrl, 0xf, 0xf, true));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(x >> 32)), Ctrl, 0xf, 0xf, true));
  const uint64_t y = (static_cast<uint64_t>(hi) << 32) | lo;
  return y > x ? y : x;
}

template <bool F32, int NC>
__global__ __launch_bounds__(kRouteThreads) void topk16_kernel(const void* logits, int T, int E, int k, int variant,
                                                              int32_t* idx, float* w, int32_t* tpe) {
  const int b = static_cast<int>(blockIdx.x);
  const int tb = (b >> 4) * 8 + (b & 7);
  const int tblk = tb * 32 + ((b >> 3) & 1) * (kRouteThreads / kTopkGroup);
  if (tblk >= T) return;  // work-group-uniform
  const int t = tblk + static_cast<int>(threadIdx.x) / kTopkGroup;
  const int g = static_cast<int>(threadIdx.x) % kTopkGroup;
  const int tl = min(t, T - 1);  // lanes of tokens past T load a real row and write nothing
  uint64_t key[4 * NC];
  if constexpr (F32) {
    float4 r[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
      r[c] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(logits) + static_cast<size_t>(tl) * E +
                                              min(64 * c + 4 * g, E - 4));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float f[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 64 * c + 4 * g + i;
        const uint32_t sk = e < E ? select_key(sanitize_logit(f[i])) : 0u;
        key[4 * c + i] = sk == 0u ? 0ull : (static_cast<uint64_t>(sk) << 32) | static_cast<uint32_t>(~e);
      }
    }
  } else {
    uint2 r[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
      r[c] = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(logits) + static_cast<size_t>(tl) * E +
                                             min(64 * c + 4 * g, E - 4));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float f[4] = {__uint_as_float(r[c].x << 16), __uint_as_float(r[c].x & 0xffff0000u),
                          __uint_as_float(r[c].y << 16), __uint_as_float(r[c].y & 0xffff0000u)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 64 * c + 4 * g + i;
        const uint32_t sk = e < E ? select_key(sanitize_logit(f[i])) : 0u;
        key[4 * c + i] = sk == 0u ? 0ull : (static_cast<uint64_t>(sk) << 32) | static_cast<uint32_t>(~e);
      }
    }
  }
  float sel_v[kMaxTopK];
  int sel_i[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    sel_v[s] = -FLT_MAX;
    sel_i[s] = -1;
    if (s < k) {
      uint64_t best = key[0];
#pragma unroll
      for (int j = 1; j < 4 * NC; ++j) best = key[j] > best ? key[j] : best;
      best = max_dpp_u64<0xB1>(best);   // quad_perm [1,0,3,2]
      best = max_dpp_u64<0x4E>(best);   // quad_perm [2,3,0,1]
      best = max_dpp_u64<0x141>(best);  // row_half_mirror
      best = max_dpp_u64<0x140>(best);  // row_mirror
      const uint32_t kv = static_cast<uint32_t>(best >> 32);
      if (kv != 0u) {
        sel_v[s] = __uint_as_float((kv & 0x80000000u) ? (kv & 0x7fffffffu) : ~kv);
        sel_i[s] = static_cast<int>(~static_cast<uint32_t>(best));
      }
#pragma unroll
      for (int j = 0; j < 4 * NC; ++j) key[j] = key[j] == best ? 0ull : key[j];
    }
  }
  if (g != 0 || t >= T) return;
  write_slots(sel_v, sel_i, k, variant, idx + static_cast<size_t>(t) * k, w ? w + static_cast<size_t>(t) * k : nullptr,
              tpe);
}

// Top-k of all T <= kTopkPlanMaxT tokens (16 waves, tokens w, w + 16, ...),
// then the plan from the selections.  Each wave loads all its tokens' logits
// before it stores anything (gfx9 counts stores in vmcnt, so a load issued
// after a store waits for the store's completion), keeps the selections and
// weights in LDS and the work-group writes them out once.
template <bool F32, int NV>
__global__ __launch_bounds__(kPlanThreads) void topk_plan_kernel(const void* logits, int T, int E, int k,
                                                                int variant, int32_t* idx, float* w, PlanBufs p) {
  constexpr int kWaves = kPlanThreads / kWave;
  constexpr int kTPW = kTopkPlanMaxT / kWaves;  // tokens per wave
  __shared__ int32_t s_idx[kTopkPlanMaxT * kMaxTopK];
  __shared__ float s_w[kTopkPlanMaxT * kMaxTopK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float v[kTPW][NV];
#pragma unroll
  for (int i = 0; i < kTPW; ++i) {
    const int t = wv + kWaves * i;
    load_token_logits<F32, NV>(logits, t < T ? t : 0, E, lane, v[i]);  // rows past T read row 0, unused
  }
#pragma unroll
  for (int i = 0; i < kTPW; ++i) {
    const int t = wv + kWaves * i;
    if (t < T) topk_token<NV, !F32>(v[i], k, variant, s_idx + t * k, s_w + t * k, nullptr, lane);
  }
  __syncthreads();
  for (int q = threadIdx.x; q < T * k; q += kPlanThreads) {
    idx[q] = s_idx[q];
    w[q] = s_w[q];
  }
  build_plan<kPlanThreads>([&](int s) { return s_idx[s]; }, T, k, E, p);
}

// Top-k + plan for T <= 64 tokens with one lane per token (E <= 128, a
// multiple of 8): wave w sorts the 8 logits of experts 8w..8w+7 of its
// lane's token (a depth-6 sorting network), keeps the top K, and the lists
// of the E/8 slices meet in a 4-level tree of bitonic merges through LDS.
// Each lane then applies its token's softmax.  Every step is a few
// dependent instructions on all tokens at once, where one wave per token
// would chain k wave-wide reductions.  Entries: larger = earlier in the
// reference's order, 0 = not selectable; fp32 logits: key << 32 | 0xffff -
// expert; bf16 logits: the key's high half (which holds a bf16 value
// exactly) | 0xffff - expert, so a compare-exchange is one max and one min.
constexpr int kLaneTopkSlice = 8;
constexpr int kLaneTopkMaxT = kWave;

__device__ __forceinline__ void ce_desc(uint64_t& a, uint64_t& b) {
  const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
  a = hi;
  b = lo;
}
__device__ __forceinline__ void ce_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

template <bool F32, int K>
__global__ __launch_bounds__(kPlanThreads) void topk_plan_lanes_kernel(const void* logits, int T, int E, int variant,
                                                                      int32_t* idx, float* w, PlanBufs p) {
  using Entry = std::conditional_t<F32, uint64_t, uint32_t>;
  constexpr int kSlices = kPlanThreads / kWave;  // 16: up to 128 experts
  __shared__ Entry s_list[kSlices][kLaneTopkMaxT][K];
  __shared__ int32_t s_idx[kLaneTopkMaxT * K];
  __shared__ float s_w[kLaneTopkMaxT * K];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nsl = (E + kLaneTopkSlice - 1) / kLaneTopkSlice;
  const int t = lane;
  if (wv < nsl) {
    const int e0 = wv * kLaneTopkSlice;
    float v[kLaneTopkSlice];
    const size_t o = static_cast<size_t>(t < T ? t : 0) * E + e0;  // lanes past T read token 0, unused
    if constexpr (F32) {
      const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(logits) + o);
      const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(logits) + o + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(logits) + o);
      unpack_bf16x8(a, v);
    }
    Entry en[kLaneTopkSlice];
#pragma unroll
    for (int i = 0; i < kLaneTopkSlice; ++i) {
      const uint32_t key = select_key(sanitize_logit(v[i]));
      const uint32_t ix = static_cast<uint32_t>(0xffff - (e0 + i));
      if constexpr (F32) en[i] = key ? (static_cast<uint64_t>(key) << 32) | ix : 0ull;
      else en[i] = key ? (key & 0xffff0000u) | ix : 0u;
    }
    // optimal 19-comparator sorting network for 8 inputs (descending)
    ce_desc(en[0], en[2]); ce_desc(en[1], en[3]); ce_desc(en[4], en[6]); ce_desc(en[5], en[7]);
    ce_desc(en[0], en[4]); ce_desc(en[1], en[5]); ce_desc(en[2], en[6]); ce_desc(en[3], en[7]);
    ce_desc(en[0], en[1]); ce_desc(en[2], en[3]); ce_desc(en[4], en[5]); ce_desc(en[6], en[7]);
    ce_desc(en[2], en[4]); ce_desc(en[3], en[5]);
    ce_desc(en[1], en[4]); ce_desc(en[3], en[6]);
    ce_desc(en[1], en[2]); ce_desc(en[3], en[4]); ce_desc(en[5], en[6]);
#pragma unroll
    for (int i = 0; i < K; ++i) s_list[wv][t][i] = i < kLaneTopkSlice ? en[i < kLaneTopkSlice ? i : 0] : Entry{0};
  }
  __syncthreads();
  // merge tree: at width d, wave w merges slice lists 2dw and 2dw + d
  for (int d = 1; d < nsl; d <<= 1) {
    const int a = 2 * d * wv, b = a + d;
    if (b < nsl) {
      Entry c[K];
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const Entry x = s_list[a][t][i], y = s_list[b][t][K - 1 - i];
        c[i] = x > y ? x : y;
      }
#pragma unroll
      for (int h = K >> 1; h > 0; h >>= 1)
#pragma unroll
        for (int i = 0; i < K; ++i)
          if ((i & h) == 0) ce_desc(c[i], c[i + h]);
#pragma unroll
      for (int i = 0; i < K; ++i) s_list[a][t][i] = c[i];
    }
    __syncthreads();
  }
  if (wv == 0 && t < T) {
    float sel_v[kMaxTopK];
    int sel_i[kMaxTopK];
#pragma unroll
    for (int s2 = 0; s2 < kMaxTopK; ++s2) {
      sel_v[s2] = -FLT_MAX;
      sel_i[s2] = -1;
      if (s2 < K) {
        const Entry en = s_list[0][t][s2 < K ? s2 : 0];
        if (en) {
          if constexpr (F32) {
            const uint32_t key = static_cast<uint32_t>(en >> 32);
            sel_v[s2] = __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
          } else {
            sel_v[s2] = bf16_of_key(en);
          }
          sel_i[s2] = 0xffff - static_cast<int>(en & 0xffffu);
        }
      }
    }
    write_slots(sel_v, sel_i, K, variant, s_idx + t * K, s_w + t * K, nullptr);
  }
  __syncthreads();
  for (int q = threadIdx.x; q < T * K; q += kPlanThreads) {
    idx[q] = s_idx[q];
    w[q] = s_w[q];
  }
  build_plan<kPlanThreads>([&](int s2) { return s_idx[s2]; }, T, K, E, p);
}

// Top-k of T <= kSmallTopkMaxT tokens (wave t: token t, topk_token) and the
// plan of their T k <= 64 slots by wave 0 after one barrier.
template <bool F32, int NV>
__global__ __launch_bounds__(kSmallTopkMaxT * kWave) void topk_plan_small_kernel(const void* logits, int T, int E,
                                                                                 int k, int variant, int32_t* idx,
                                                                                 float* w, PlanBufs p) {
  __shared__ int32_t s_idx[kSmallTopkMaxT * kMaxTopK];
  __shared__ float s_w[kSmallTopkMaxT * kMaxTopK];
  __shared__ int32_t s_cnt[kMaxExperts], s_off[kMaxExperts], s_aidx[kMaxExperts];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (wv < T) {
    float v[NV];
    load_token_logits<F32, NV>(logits, wv, E, lane, v);
    topk_token<NV, !F32>(v, k, variant, s_idx + wv * k, s_w + wv * k, nullptr, lane);
  }
  __syncthreads();
  if (wv != 0) return;
  const int S = T * k;
  if (lane < S) {
    idx[lane] = s_idx[lane];
    w[lane] = s_w[lane];
  }
  plan_one_wave<NV>(s_idx, S, k, E, p, lane, s_cnt, s_off, s_aidx);
}

// The plan of many slots in three launches that use the whole device (the
// single work-group's plan_kernel is bound by one CU's throughput).  Slots
// are cut into chunks of kPlanChunkSlots; work-group b owns chunk b, its
// wave w the 256 slots from 1024 b + 256 w, ranked 64 at a time as
// build_plan does (ballots over the expert bits, no atomics).
//   plan_count_kernel  per (chunk, expert) counts
//   plan_scan_kernel   per expert: exclusive scan over the chunks (counts
//                      become chunk bases), then the scan over experts:
//                      counts, offsets, active list, task records
//   plan_place_kernel  per chunk: wave bases, stable positions, gather map,
//                      permuted tokens, task token lists
// Stable in slot order: position = offset[e] + (slots of e in earlier
// chunks) + (in earlier waves of the chunk) + (earlier in the wave).
constexpr int kChunkThreads = 256;
constexpr int kChunkWaves = kChunkThreads / kWave;
constexpr int kChunkWaveSlots = kPlanChunkSlots / kChunkWaves;

__device__ __forceinline__ int slot_group(int e, bool valid, int lane, unsigned long long& peers) {
  peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {  // E <= 256
    const bool bit = valid && ((e >> b) & 1);
    const unsigned long long mb = __ballot(bit);
    peers &= bit ? mb : ~mb;
  }
  return __popcll(peers & ((1ull << lane) - 1ull));
}

// s_wc[w][e] += slots of expert e in wave w's part of chunk b
__device__ __forceinline__ void chunk_wave_counts(const int32_t* __restrict__ idx, int S, int E, int b, int w,
                                                  int lane, int (*s_wc)[kMaxExperts]) {
  const int s0 = b * kPlanChunkSlots + w * kChunkWaveSlots;
  const int s1 = min(S, s0 + kChunkWaveSlots);
  int ev[kChunkWaveSlots / kWave];
#pragma unroll
  for (int i = 0; i < kChunkWaveSlots / kWave; ++i) {  // all loads in flight first
    const int s = s0 + kWave * i + lane;
    ev[i] = s < s1 ? idx[s] : -1;
  }
#pragma unroll
  for (int i = 0; i < kChunkWaveSlots / kWave; ++i) {
    const bool valid = ev[i] >= 0 && ev[i] < E;
    unsigned long long peers;
    const int rank = slot_group(ev[i], valid, lane, peers);
    if (valid && rank == 0) s_wc[w][ev[i]] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kChunkThreads) void plan_count_kernel(const int32_t* __restrict__ idx, int S, int E,
                                                                   int32_t* __restrict__ chunk) {
  __shared__ int s_wc[kChunkWaves][kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, b = blockIdx.x;
  for (int i = tid; i < kChunkWaves * kMaxExperts; i += kChunkThreads) (&s_wc[0][0])[i] = 0;
  lds_barrier();
  chunk_wave_counts(idx, S, E, b, w, lane, s_wc);
  lds_barrier();
  for (int e = tid; e < E; e += kChunkThreads) {
    int c = 0;
#pragma unroll
    for (int ww = 0; ww < kChunkWaves; ++ww) c += s_wc[ww][e];
    chunk[static_cast<size_t>(b) * E + e] = c;
  }
}

__global__ __launch_bounds__(kMaxExperts) void plan_scan_kernel(int NB, int E, int32_t* __restrict__ chunk,
                                                                PlanBufs p) {
  __shared__ unsigned long long s_mask[kMaxExperts / kWave];
  __shared__ int s_wsum[kMaxExperts / kWave];
  const int tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  int c = 0;
  if (tid < E) {
    int v[8];
    for (int b0 = 0; b0 < NB; b0 += 8) {  // eight chunk counts in flight at a time
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = b0 + u < NB ? chunk[static_cast<size_t>(b0 + u) * E + tid] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (b0 + u < NB) {
          chunk[static_cast<size_t>(b0 + u) * E + tid] = c;
          c += v[u];
        }
    }
  }
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == 63) s_wsum[warp] = incl;
  const bool act = tid < E && c > 0;
  const unsigned long long am = __ballot(act);
  if (lane == 0) s_mask[warp] = am;
  __syncthreads();
  int nact = 0, base = 0, abase = 0;
#pragma unroll
  for (int w = 0; w < kMaxExperts / kWave; ++w) {
    nact += __popcll(s_mask[w]);
    if (w < warp) {
      base += s_wsum[w];
      abase += __popcll(s_mask[w]);
    }
  }
  const int excl = base + incl - c;
  if (tid < E) {
    p.counts[tid] = c;
    p.offsets[tid] = excl;
    if (tid == E - 1) p.offsets[E] = excl + c;
  }
  const int aidx = abase + __popcll(am & ((1ull << lane) - 1ull));
  if (tid < E) chunk[static_cast<size_t>(NB) * E + tid] = act ? aidx : -1;
  if (act) {
    p.active[aidx] = tid;
    if (p.tasks) {
      int32_t* t = p.tasks + static_cast<size_t>(aidx) * kTaskInts;
      t[0] = tid;
      t[1] = excl;
      t[2] = c;
      t[3] = 0;
    }
  }
  if (p.tasks && tid < E && tid >= nact) p.tasks[static_cast<size_t>(tid) * kTaskInts] = -1;
  if (tid == 0) *p.n_active = nact;
}

__global__ __launch_bounds__(kChunkThreads) void plan_place_kernel(const int32_t* __restrict__ idx, int S, int k,
                                                                   int E, const int32_t* __restrict__ chunk,
                                                                   PlanBufs p) {
  __shared__ int s_wc[kChunkWaves][kMaxExperts];  // counts, then the waves' bases
  __shared__ int s_off[kMaxExperts], s_aidx[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, b = blockIdx.x;
  const int NB = (S + kPlanChunkSlots - 1) / kPlanChunkSlots;
  for (int i = tid; i < kChunkWaves * kMaxExperts; i += kChunkThreads) (&s_wc[0][0])[i] = 0;
  lds_barrier();
  chunk_wave_counts(idx, S, E, b, w, lane, s_wc);
  lds_barrier();
  for (int e = tid; e < E; e += kChunkThreads) {
    int base = chunk[static_cast<size_t>(b) * E + e];
#pragma unroll
    for (int ww = 0; ww < kChunkWaves; ++ww) {
      const int v = s_wc[ww][e];
      s_wc[ww][e] = base;
      base += v;
    }
    s_off[e] = p.offsets[e];
    s_aidx[e] = chunk[static_cast<size_t>(NB) * E + e];
  }
  lds_barrier();
  const int s0 = b * kPlanChunkSlots + w * kChunkWaveSlots;
  const int s1 = min(S, s0 + kChunkWaveSlots);
  int ev[kChunkWaveSlots / kWave];
#pragma unroll
  for (int i = 0; i < kChunkWaveSlots / kWave; ++i) {
    const int s = s0 + kWave * i + lane;
    ev[i] = s < s1 ? idx[s] : -1;
  }
#pragma unroll
  for (int i = 0; i < kChunkWaveSlots / kWave; ++i) {
    const int s = s0 + kWave * i + lane;
    const int e = ev[i];
    const bool valid = e >= 0 && e < E;
    unsigned long long peers;
    const int rank = slot_group(e, valid, lane, peers);
    if (valid) {
      const int r = s_wc[w][e] + rank;  // rank of the slot within its expert
      const int pos = s_off[e] + r;
      p.gather_map[s] = pos;
      p.perm_token[pos] = s / k;
      if (p.tasks && r < kTaskTokens) p.tasks[static_cast<size_t>(s_aidx[e]) * kTaskInts + 4 + r] = s / k;
    } else if (s < s1) {
      p.gather_map[s] = -1;
    }
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) s_wc[w][e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
}

// staged: the T k indices are copied to (dynamic) LDS first, so the ranking
// rounds of build_plan, separated by barriers, read LDS instead of waiting
// on global loads one round at a time.
constexpr int kPlanStageMaxSlots = 24 * 1024;  // 96 KiB of LDS
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int32_t* idx, int T, int k, int E, PlanBufs p,
                                                            int staged) {
  extern __shared__ int32_t d_idx[];
  if (staged) {
    // 16 loads in flight per thread before the first store (a plain loop
    // waits for each load in turn)
    constexpr int kBatch = 16;
    const int S = T * k;
    for (int s0 = threadIdx.x; s0 < S; s0 += kBatch * kPlanThreads) {
      int v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int s = s0 + u * kPlanThreads;
        v[u] = s < S ? idx[s] : 0;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int s = s0 + u * kPlanThreads;
        if (s < S) d_idx[s] = v[u];
      }
    }
    lds_barrier();
    build_plan<kPlanThreads>([&](int s) { return d_idx[s]; }, T, k, E, p);
  } else {
    build_plan<kPlanThreads>([&](int s) { return idx[s]; }, T, k, E, p);
  }
}

hipError_t launch_plan_kernel(const int32_t* idx, int T, int k, int E, PlanBufs plan, hipStream_t s,
                              const KernelTimer& timer) {
  const int S = T * k;
  if (plan.chunk != nullptr && S > kPlanChunkSlots) {  // three launches over the device
    const int NB = (S + kPlanChunkSlots - 1) / kPlanChunkSlots;
    gx_launch(plan_count_kernel, dim3(NB), dim3(kChunkThreads), 0, s, KernelTimer{timer.start, nullptr}, idx, S, E,
              plan.chunk);
    gx_launch(plan_scan_kernel, dim3(1), dim3(kMaxExperts), 0, s, KernelTimer{}, NB, E, plan.chunk, plan);
    gx_launch(plan_place_kernel, dim3(NB), dim3(kChunkThreads), 0, s, KernelTimer{nullptr, timer.stop}, idx, S, k,
              E, static_cast<const int32_t*>(plan.chunk), plan);
    return hipGetLastError();
  }
  const int staged = S <= kPlanStageMaxSlots ? 1 : 0;
  const size_t lds = staged ? static_cast<size_t>(S) * 4 : 0;
  if (lds > 0) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(plan_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  gx_launch(plan_kernel, dim3(1), dim3(kPlanThreads), lds, s, timer, idx, T, k, E, plan, staged);
  return hipGetLastError();
}

// Logits on the matrix cores (many tokens; the reference routes T > 1
// through hipBLASLt, cuda_utils.h:226-308, moe_layer.cu:1174-1185): bf16
// products, fp32 sums in v_mfma_f32_16x16x32_bf16's order, + bias.
//
// A work-group computes kMmTT = 32 tokens x kMmEE = 64 experts.  K goes in
// chunks of kMmKB = 4 blocks (128 elements, 256 bytes of each row), and wave
// j owns chain j: block j of every chunk, for the whole 32 x 64 tile.  So a
// logit is four chains of products (blocks j, j + 4, ...) in block order,
// added pairwise at the end, plus the bias: a token's logits depend on its
// own row only (batch-invariant), and every run gives the same bits.  The
// grid gives the expert slices of eight token blocks to one XCD, so a token
// row is read from HBM once per XCD.
//
// A chunk's rows (32 token rows, 64 router rows: 24 KiB) go straight from
// memory into one of kMmS = 6 LDS stages (buffer_load ... lds, 16 bytes a
// lane: each load fills 1 KiB of the stage, four rows), with the 16-byte
// piece c of row r at slot c ^ (r % 16), so the operand reads (16 rows at
// one piece) hit distinct banks; five chunks are in flight behind the one
// being multiplied.  Each piece is read once, by the wave of its chain: the
// LDS moves 24 KiB in and 24 KiB out per chunk, and no registers hold the
// ring.  One barrier per chunk, after the wave's own wait for the chunk.
// Loads past the last chunk read past the buffer end (zeros, no memory
// access); blocks of the last chunk past K are loaded but not multiplied.
// The four chains meet in LDS at the end.
//
// Measured on MI355X at 4096 tokens x 128 experts x 2880 (harness, back-to-
// back launches): 10.3-10.5 us for the logits (the gemv tree: 71 us).  The
// earlier forms, with the same bits: a register ring stored to two LDS
// stages by four waves that each read their operands for all four chains
// (a tile's router rows read by two waves, its token rows by four, and a
// wait on every read before each product): 16.0-16.7 us; the same with the
// reads of a chunk issued together: 13.5 us; eight waves: 12.5 us.  The
// work-group's chain of chunks sets the time (9.3 us at 256 tokens, where
// the chip is nearly idle): five chunks in flight per CU and their latency.
constexpr int kMmTT = 32, kMmEE = 64, kMmKB = 4, kMmS = 6;
constexpr int kMmWaves = kMmKB;                        // wave j: chain j (block j of every chunk)
constexpr int kMmThreads = kWave * kMmWaves;
constexpr int kMmRows = kMmTT + kMmEE;                 // rows of a chunk: tokens, then router rows
constexpr int kMmRowB = kMmKB * 64;                    // bytes of a row in a chunk
constexpr int kMmLpr = kMmRowB / 16;                   // lanes per row in a load (= pieces per row)
constexpr int kMmRpl = kWave / kMmLpr;                 // rows per load
constexpr int kMmLoads = kMmRows * kMmRowB / 1024 / kMmWaves;  // 1 KiB loads per wave and chunk
constexpr int kMmStage = kMmRows * kMmRowB;            // bytes of a chunk in LDS
constexpr int kMmTE = kMmEE / 16, kMmTF = kMmTT / 16;  // 16 x 16 tiles of a work-group: experts, tokens

// s_waitcnt vmcnt(N), the other counters untouched.
template <int N>
__device__ __forceinline__ void mm_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

template <bool F32>
__global__ __launch_bounds__(kMmThreads) void logits_mfma_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ W,
                                                                 const uint16_t* __restrict__ bias, int T, int E,
                                                                 int H, void* __restrict__ logits) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) void lds_void_t;
  static_assert(kMmLpr == 16 && kMmLoads * kMmWaves * 1024 == kMmStage && kMmTT % kMmRpl == 0,
                "16 pieces per row (the swizzle); the waves share a chunk's loads; a load's rows are all token rows "
                "or all router rows");
  static_assert(kMmS * kMmStage <= 160 * 1024 && kMmWaves * kMmTE * kMmTF * 1024 <= kMmS * kMmStage,
                "the ring fits the LDS; the chains' exchange fits the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kMmS * kMmStage];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int neh = (E + kMmEE - 1) / kMmEE;
  const int id = static_cast<int>(blockIdx.x);
  const int eh = (id >> 3) % neh;                  // expert slice
  const int tb = (id / (8 * neh)) * 8 + (id & 7);  // token block: the same id % 8 (XCD) for all slices
  const int t0 = tb * kMmTT, e0 = eh * kMmEE;
  if (t0 >= T) return;  // the grid is rounded up to whole groups of eight token blocks
  const int nb = H >> 5;
  const int nch = (nb + kMmKB - 1) / kMmKB;
  const int rowb = H * 2;  // bytes per row
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W), 0, E * rowb, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, T * rowb, 0x00020000);
  // Load i of wave w fills the chunk's KiB L = kMmLoads w + i: rows R =
  // kMmRpl L + l / kMmLpr, lane l landing at slot s = l % kMmLpr of its row.
  // Slot s holds the row's piece s ^ (R % 16), so the lane loads that piece.
  // Rows past T / E read the last row (their sums are not stored).
  int goff[kMmLoads];
#pragma unroll
  for (int i = 0; i < kMmLoads; ++i) {
    const int R = kMmRpl * (kMmLoads * w + i) + lane / kMmLpr;
    const int c = (lane % kMmLpr) ^ (R & 15);
    const int row = R < kMmTT ? min(t0 + R, T - 1) : min(e0 + R - kMmTT, E - 1);
    goff[i] = row * rowb + 16 * c;
  }
  auto issue = [&](int ch, int st) __attribute__((always_inline)) {
    const int so = ch < nch ? ch * kMmRowB : 0x40000000;  // past the last chunk: out of range (zeros, no access)
    uint8_t* sp = ring + st * kMmStage;
#pragma unroll
    for (int i = 0; i < kMmLoads; ++i) {
      const bool ux = kMmRpl * (kMmLoads * w + i) < kMmTT;  // wave-uniform: token rows or router rows
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ux ? xrs : wrs, (lds_void_t*)(sp + 1024 * (kMmLoads * w + i)), 16,
                                               goff[i], so, 0, 0);
    }
  };
  // The bias of the tiles this wave finishes (tiles w, w + kMmWaves, ...:
  // experts 16 g + 4 (l / 16) + r), loaded now, before the ring's loads: a
  // null bias is a buffer of no bytes (zeros, no access), so the loads are
  // unconditional and land long before the end.
  constexpr int kMmTilesPW = kMmTE * kMmTF / kMmWaves;
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(bias), 0,
                                                                       bias != nullptr ? E * 2 : 0, 0x00020000);
  uint16_t bias_raw[kMmTilesPW][4];
#pragma unroll
  for (int u = 0; u < kMmTilesPW; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = e0 + 16 * ((w + kMmWaves * u) / kMmTF) + 4 * (lane >> 4) + r;
      bias_raw[u][r] = __builtin_amdgcn_raw_buffer_load_b16(brs, 2 * min(e, E), 0, 0);  // e >= E: past the end
    }
  // acc[g][f]: chain w of experts 16 g .., tokens 16 f .. (the products of
  // blocks w, w + 4, ... in block order)
  f32x4_t acc[kMmTE][kMmTF];
#pragma unroll
  for (int g = 0; g < kMmTE; ++g)
#pragma unroll
    for (int f = 0; f < kMmTF; ++f) acc[g][f] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int r16 = lane & 15, q = lane >> 4;
  const int pz = 16 * ((4 * w + q) ^ r16);  // piece 4 w + q of a 16-aligned row + r16
  auto compute = [&](int st, int ch) __attribute__((always_inline)) {
    if (kMmKB * ch + w >= nb) return;  // the last chunk's blocks past K (wave-uniform)
    const uint8_t* sp = ring + st * kMmStage + pz;
    gx_bf16x8 a[kMmTE], b[kMmTF];
#pragma unroll
    for (int g = 0; g < kMmTE; ++g) a[g] = *reinterpret_cast<const gx_bf16x8*>(sp + (kMmTT + 16 * g + r16) * kMmRowB);
#pragma unroll
    for (int f = 0; f < kMmTF; ++f) b[f] = *reinterpret_cast<const gx_bf16x8*>(sp + (16 * f + r16) * kMmRowB);
#pragma unroll
    for (int g = 0; g < kMmTE; ++g)
#pragma unroll
      for (int f = 0; f < kMmTF; ++f) acc[g][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[g], b[f], acc[g][f], 0, 0, 0);
  };
  // Ring of kMmS stages: at chunk c, chunks c .. c + kMmS - 2 are in flight;
  // once the wave's loads of chunk c have landed (vmcnt) and every wave's
  // (the barrier, which also ends every wave's reads of chunk c - 1), the
  // stage of chunk c - 1 takes chunk c + kMmS - 1.
#pragma unroll
  for (int c = 0; c < kMmS - 1; ++c) issue(c, c);
  int st = 0;
  for (int c = 0; c < nch; ++c) {
    mm_wait_vm<(kMmS - 2) * kMmLoads>();
    __builtin_amdgcn_s_barrier();  // no fence: the wait above is the one this barrier needs
    issue(c + kMmS - 1, st == 0 ? kMmS - 1 : st - 1);
    compute(st, c);
    st = st == kMmS - 1 ? 0 : st + 1;
  }
  // The chains meet in LDS (after the trailing loads past the end have
  // landed): wave w writes its chain, then takes tiles w, w + 4, ... and
  // adds the four chains pairwise, then the bias.
  mm_wait_vm<0>();
  __syncthreads();
  f32x4_t* xch = reinterpret_cast<f32x4_t*>(ring);  // [chain][tile][lane]
#pragma unroll
  for (int g = 0; g < kMmTE; ++g)
#pragma unroll
    for (int f = 0; f < kMmTF; ++f) xch[(w * kMmTE * kMmTF + g * kMmTF + f) * kWave + lane] = acc[g][f];
  __syncthreads();
  static_assert(kMmKB == 4 && (kMmTE * kMmTF) % kMmWaves == 0, "four chains; whole tiles per wave");
#pragma unroll
  for (int u = 0; u < kMmTilesPW; ++u) {
    const int tile = w + kMmWaves * u, g = tile / kMmTF, f = tile % kMmTF;
    f32x4_t ch[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ch[j] = xch[(j * kMmTE * kMmTF + tile) * kWave + lane];
    // ch[j][r]: expert 16 g + 4 (l / 16) + r, token 16 f + l % 16
    const int eb = e0 + 16 * g + 4 * q;
    const int t = t0 + 16 * f + r16;
    if (t >= T) continue;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = ((ch[0][r] + ch[1][r]) + (ch[2][r] + ch[3][r])) + bf16_to_f32(bias_raw[u][r]);
    const size_t o = static_cast<size_t>(t) * E + eb;
    // one 16- (fp32) or 8-byte (bf16) store when the four logits are whole
    // and aligned to it (the C ABI does not require aligned logits)
    const bool vec = eb + 4 <= E && (E & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & (F32 ? 15 : 7)) == 0;
    if (vec) {
      if constexpr (F32) *reinterpret_cast<float4*>(reinterpret_cast<float*>(logits) + o) = make_float4(v[0], v[1], v[2], v[3]);
      else *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(logits) + o) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (eb + r < E) {
          if constexpr (F32) reinterpret_cast<float*>(logits)[o + r] = v[r];
          else reinterpret_cast<uint16_t*>(logits)[o + r] = f32_to_bf16(v[r]);
        }
    }
  }
}

constexpr int kNormFusedMaxT = 4;  // tokens up to which the residual RMSNorm runs inside the router
// Tokens above which the router's logits come from the matrix cores; up to
// it every logit follows the reference's gemv_bf16 tree (its T = 1 path).
constexpr int kMmMinT = 64;

// The matrix-core router applies: many tokens, whole 32-element blocks, and
// every offset inside a 32-bit buffer range.
bool mm_router_ok(const RouteArgs& a) {
  return a.T > kMmMinT && a.H % 32 == 0 &&
         static_cast<size_t>(a.T) * a.H * 2 < (size_t{1} << 30) && static_cast<size_t>(a.E) * a.H * 2 < (size_t{1} << 30);
}

template <bool F32>
hipError_t launch_logits(const RouteArgs& a, hipStream_t s, const KernelTimer& t) {
  // tokens per wave x experts per wave: more waves for few tokens (latency),
  // more reuse of each loaded row for many.  Up to H = 3072 the decode
  // shapes load every chunk up front.
  const bool upfront = (a.H >> 3) <= kWave * 6;
  if (a.norm_w != nullptr) {
    if (a.T <= kNormFusedMaxT && upfront) {
      // the norm fused into the router: each token's row is in registers.
      // Every wave recomputes its token's norm, which beats a launch of its
      // own only for a few tokens (measured: 1.5 us saved at 1 token, lost
      // from 8).
      gx_launch(logits_norm_kernel<1, 1, F32>, dim3((a.E + 3) / 4, a.T), dim3(kRouteThreads), 0, s, t, a.x, a.delta,
                a.norm_w, a.eps, a.W, a.b, a.T, a.E, a.H, a.logits, a.normed, a.sum_out);
      return hipGetLastError();
    }
    // more tokens: the norm first (its own launch), then the router on normed
    const hipError_t e = launch_residual_rmsnorm(a.x, a.delta, a.norm_w, a.normed, a.sum_out, a.T, a.H, a.eps, s);
    if (e != hipSuccess) return e;
    RouteArgs b = a;
    b.x = a.normed;
    b.norm_w = nullptr;
    return launch_logits<F32>(b, s, t);
  }
  // Measured (GPT-OSS-120B router, back-to-back launches, bf16 logits):
  // one token x one expert per wave at T = 8 / 16 / 32 takes 2.7 / 3.1 /
  // 3.8 us against 4.1 / 4.1 / 4.2 for 2 x 2; at T = 64, 2 tokens x 1
  // expert 5.15 against 5.3 for 2 x 2 and 5.4 for 1 x 1 (4 x 2 and 2 x 4
  // are slower everywhere).  Every mapping gives the same bits.
  if (a.T <= 32 && upfront) {
    gx_launch(logits_kernel<1, 1, 6, F32>, dim3((a.E + 3) / 4, a.T), dim3(kRouteThreads), 0, s, t, a.x, a.W, a.b,
              a.T, a.E, a.H, a.logits);
  } else if (a.T <= 64 && upfront) {
    gx_launch(logits_kernel<2, 1, 6, F32>, dim3((a.E + 3) / 4, (a.T + 1) / 2), dim3(kRouteThreads), 0, s, t, a.x, a.W,
              a.b, a.T, a.E, a.H, a.logits);
  } else if (a.T <= 8) {
    gx_launch(logits_kernel<1, 1, 0, F32>, dim3((a.E + 3) / 4, a.T), dim3(kRouteThreads), 0, s, t, a.x, a.W, a.b,
              a.T, a.E, a.H, a.logits);
  } else if (mm_router_ok(a)) {  // many tokens: the matrix cores
    const int neh = (a.E + kMmEE - 1) / kMmEE, ntb = (a.T + kMmTT - 1) / kMmTT;
    const int grid = ((ntb + 7) / 8) * 8 * neh;
    gx_launch(logits_mfma_kernel<F32>, dim3(grid), dim3(kMmThreads), 0, s, t, a.x, a.W, a.b, a.T, a.E, a.H,
              a.logits);
  } else {
    const int gx = (a.E + kLdsEPW - 1) / kLdsEPW, ntb = (a.T + kLdsTT - 1) / kLdsTT;
    if (a.H <= 8 * 2 * kRouteThreads) {  // every chain holds at most two chunks: router rows held across blocks
      // about two work-groups per CU of 256 (the kernel's occupancy), each walking token blocks
      const int gy = std::min(ntb, std::max(1, 512 / gx));
      gx_launch(logits_lds_kernel<F32, true>, dim3(gx, gy), dim3(kRouteThreads), 0, s, t, a.x, a.W, a.b, a.T, a.E,
                a.H, a.logits);
    } else {
      gx_launch(logits_lds_kernel<F32, false>, dim3(gx, ntb), dim3(kRouteThreads), 0, s, t, a.x, a.W, a.b, a.T,
                a.E, a.H, a.logits);
    }
  }
  return hipGetLastError();
}

}  // namespace

size_t route_scratch_bytes(int, int, int) { return 256; }

// Instantiations per NV = ceil(E / 64) values per lane.
template <bool F32>
void launch_topk_plan_t(const RouteArgs& a, int variant, hipStream_t s, const KernelTimer& t) {
  const int nv = (a.E + kWave - 1) / kWave;
  const void* lg = a.logits;
#define GX_TPK(NV_) gx_launch(topk_plan_kernel<F32, NV_>, dim3(1), dim3(kPlanThreads), 0, s, t, lg, a.T, a.E, a.k, \
                              variant, a.idx, a.w, a.plan)
  if (nv <= 1) GX_TPK(1);
  else if (nv == 2) GX_TPK(2);
  else if (nv == 3) GX_TPK(3);
  else GX_TPK(4);
#undef GX_TPK
}

template <bool F32>
void launch_topk_t(const void* logits, int T, int E, int k, int variant, int32_t* idx, float* w, int32_t* tpe,
                   hipStream_t s, const KernelTimer& t) {
  const int nv = (E + kWave - 1) / kWave;
  const uintptr_t width = F32 ? 16 : 8;  // bytes of one topk16_kernel load
  if (E % 4 == 0 && reinterpret_cast<uintptr_t>(logits) % width == 0) {
    const int ntb = (T + 31) / 32;
    const dim3 grid(((ntb + 7) / 8) * 16);
#define GX_T16(NC_) gx_launch(topk16_kernel<F32, NC_>, grid, dim3(kRouteThreads), 0, s, t, logits, T, E, k, variant, \
                              idx, w, tpe)
    if (nv <= 1) GX_T16(1);
    else if (nv == 2) GX_T16(2);
    else if (nv == 3) GX_T16(3);
    else GX_T16(4);
#undef GX_T16
    return;
  }
  const dim3 grid((T + 3) / 4);
#define GX_TK(NV_) gx_launch(topk_kernel<F32, NV_>, grid, dim3(kRouteThreads), 0, s, t, logits, T, E, k, variant, idx, \
                             w, tpe)
  if (nv <= 1) GX_TK(1);
  else if (nv == 2) GX_TK(2);
  else if (nv == 3) GX_TK(3);
  else GX_TK(4);
#undef GX_TK
}

hipError_t launch_route(const RouteArgs& a, hipStream_t s) {
  if (a.T <= 0) return hipSuccess;
  const int variant = (a.T <= 8) ? 1 : 2;  // topk_softmax.cu:399
  const bool plan = a.plan.counts != nullptr;
  const bool fused = plan && a.T <= kTopkPlanMaxT;
  if (a.logits_only) return a.logits_fp32 ? launch_logits<true>(a, s, a.timer) : launch_logits<false>(a, s, a.timer);
  const KernelTimer first{a.timer.start, nullptr}, last{nullptr, a.timer.stop};
  hipError_t err = a.logits_fp32 ? launch_logits<true>(a, s, first) : launch_logits<false>(a, s, first);
  if (err != hipSuccess) return err;
  if (fused && a.T <= kSmallTopkMaxT) {
    const void* lg = a.logits;
    const int nv = (a.E + kWave - 1) / kWave;
#define GX_TPS(F_, NV_) gx_launch(topk_plan_small_kernel<F_, NV_>, dim3(1), dim3(kWave * a.T), 0, s, last, lg, a.T, \
                                  a.E, a.k, variant, a.idx, a.w, a.plan)
    if (a.logits_fp32) {
      if (nv <= 1) GX_TPS(true, 1);
      else if (nv == 2) GX_TPS(true, 2);
      else if (nv == 3) GX_TPS(true, 3);
      else GX_TPS(true, 4);
    } else {
      if (nv <= 1) GX_TPS(false, 1);
      else if (nv == 2) GX_TPS(false, 2);
      else if (nv == 3) GX_TPS(false, 3);
      else GX_TPS(false, 4);
    }
#undef GX_TPS
    return hipGetLastError();
  }
  if (fused && a.T <= kLaneTopkMaxT && a.E <= kLaneTopkSlice * (kPlanThreads / kWave) && a.E % kLaneTopkSlice == 0) {
    const void* lg = a.logits;
#define GX_TPL(F_, K_) gx_launch(topk_plan_lanes_kernel<F_, K_>, dim3(1), dim3(kPlanThreads), 0, s, last, lg, a.T, \
                                 a.E, variant, a.idx, a.w, a.plan)
    if (a.logits_fp32) {
      if (a.k == 1) GX_TPL(true, 1);
      else if (a.k == 2) GX_TPL(true, 2);
      else if (a.k == 4) GX_TPL(true, 4);
      else GX_TPL(true, 8);
    } else {
      if (a.k == 1) GX_TPL(false, 1);
      else if (a.k == 2) GX_TPL(false, 2);
      else if (a.k == 4) GX_TPL(false, 4);
      else GX_TPL(false, 8);
    }
#undef GX_TPL
    return hipGetLastError();
  }
  if (fused) {
    if (a.logits_fp32) launch_topk_plan_t<true>(a, variant, s, last);
    else launch_topk_plan_t<false>(a, variant, s, last);
    return hipGetLastError();
  }
  const KernelTimer mid = plan ? KernelTimer{} : last;
  if (a.logits_fp32) launch_topk_t<true>(a.logits, a.T, a.E, a.k, variant, a.idx, a.w, nullptr, s, mid);
  else launch_topk_t<false>(a.logits, a.T, a.E, a.k, variant, a.idx, a.w, nullptr, s, mid);
  err = hipGetLastError();
  if (err != hipSuccess || !plan) return err;
  return launch_plan_kernel(static_cast<const int32_t*>(a.idx), a.T, a.k, a.E, a.plan, s, last);
}

hipError_t launch_topk(const void* logits, int logits_fp32, int T, int E, int k,
                       int32_t* idx, float* w, int32_t* tpe, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  const int variant = (T <= 8) ? 1 : 2;
  if (logits_fp32) launch_topk_t<true>(logits, T, E, k, variant, idx, w, tpe, s, KernelTimer{});
  else launch_topk_t<false>(logits, T, E, k, variant, idx, w, tpe, s, KernelTimer{});
  return hipGetLastError();
}

hipError_t launch_plan(const int32_t* idx, int T, int k, int E, PlanBufs plan, hipStream_t s,
                       const KernelTimer& timer) {
  if (T <= 0) return hipSuccess;
  return launch_plan_kernel(idx, T, k, E, plan, s, timer);
}

}  // namespace gxmoe
