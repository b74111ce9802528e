// moe_topk.h -- device helpers of the top-k softmax and the small-batch
// routing plan, shared by the router launches (moe_route.hip) and the
// decode gate_up kernel that routes a few tokens in its prologue
// (moe_decode.hip).
#pragma once

#include <float.h>

#include "moe_device.h"
#include "moe_kernels.h"

namespace gxmoe {
namespace {

constexpr int kSmallTopkMaxT = 8;  // tokens routed by one work-group without a plan launch

__device__ __forceinline__ float sanitize_logit(float v) {
  // topk_softmax.cu:47-52: NaN and +-Inf become -FLT_MAX.
  return ((__float_as_uint(v) & 0x7f800000u) == 0x7f800000u) ? -FLT_MAX : v;
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float* f) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(d[i] << 16);
    f[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
  }
}

// Lane l + 16 / l + 32 values into lane l (for l below 16 / 32), and DPP
// row_shl:m (lane l reads lane l + m of its 16-lane row).
__device__ __forceinline__ uint32_t from_plus32(uint32_t x) {
  return __builtin_amdgcn_permlane32_swap(x, x, false, false)[1];
}
__device__ __forceinline__ uint32_t from_plus16(uint32_t x) {
  return __builtin_amdgcn_permlane16_swap(x, x, false, false)[1];
}
template <int M>
__device__ __forceinline__ uint32_t from_plus_row(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x100 | M, 0xf, 0xf, true));
}

// The sum of the 64 lanes' values in the order of the xor butterfly of
// gemv_bf16.cu:95-100 (lanes 32 apart added first, then 16, 8, 4, 2, 1):
// lane 0 adds exactly the same pairs in the same order.  Valid in lane 0.
__device__ __forceinline__ float tree_sum_lane0(float v) {
  v = v + __uint_as_float(from_plus32(__float_as_uint(v)));
  v = v + __uint_as_float(from_plus16(__float_as_uint(v)));
  v = v + __uint_as_float(from_plus_row<8>(__float_as_uint(v)));
  v = v + __uint_as_float(from_plus_row<4>(__float_as_uint(v)));
  v = v + __uint_as_float(from_plus_row<2>(__float_as_uint(v)));
  v = v + __uint_as_float(from_plus_row<1>(__float_as_uint(v)));
  return v;
}

// Wave-uniform max / min of a per-lane u32.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, from_plus32(x));
  x = max(x, from_plus16(x));
  x = max(x, from_plus_row<8>(x));
  x = max(x, from_plus_row<4>(x));
  x = max(x, from_plus_row<2>(x));
  x = max(x, from_plus_row<1>(x));
  return __builtin_amdgcn_readfirstlane(x);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = min(x, from_plus32(x));
  x = min(x, from_plus16(x));
  x = min(x, from_plus_row<8>(x));
  x = min(x, from_plus_row<4>(x));
  x = min(x, from_plus_row<2>(x));
  x = min(x, from_plus_row<1>(x));
  return __builtin_amdgcn_readfirstlane(x);
}

// Selection key of a logit: larger key = earlier in the reference's order
// (value descending; -0 and +0 equal).  After sanitizing, -FLT_MAX is never
// selected (the reference compares strictly against -FLT_MAX,
// topk_softmax.cu:133-159) and gets key 0.
__device__ __forceinline__ uint32_t select_key(float v) {
  if (v == -FLT_MAX) return 0u;
  if (v == 0.0f) v = 0.0f;
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The bf16 value whose select_key has high half key >> 16 (+0 for -0):
// the inverse of select_key on bf16 values, which the key's high half holds
// exactly.
__device__ __forceinline__ float bf16_of_key(uint32_t key) {
  const uint32_t h = key >> 16;
  return __uint_as_float(((h & 0x8000u) ? (h & 0x7fffu) : (~h & 0xffffu)) << 16);
}

// Logits of one token as the lanes of a wave hold them: expert lane + 64 j
// (NV = ceil(E / 64) values per lane).  Every load reads an in-range
// expert and the ones past E are replaced afterwards, so the loads are all
// in flight before one wait (a conditional load compiles to a branch with
// its own wait).
template <bool F32, int NV>
__device__ __forceinline__ void load_token_logits(const void* logits, int t, int E, int lane, float (&v)[NV]) {
  float r[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const size_t o = static_cast<size_t>(t) * E + min(lane + kWave * j, E - 1);
    r[j] = F32 ? reinterpret_cast<const float*>(logits)[o] : bf16_to_f32(reinterpret_cast<const uint16_t*>(logits)[o]);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = lane + kWave * j >= E ? -FLT_MAX : r[j];
}

// Sum of the k selected exponentials in the reference's order: v1
// (topk_softmax.cu:199-204) adds them in slot order; v2 (topk_softmax.cu:
// 358-362) ends every lane of its butterfly with the tree t[s] + t[s ^ m],
// m = k/2 .. 1, whose value in slot 0 this returns.
template <int K>
__device__ __forceinline__ float slot_sum(const float* ex, int variant) {
  if (variant == 1) {
    float sum = 0.0f;
#pragma unroll
    for (int s = 0; s < K; ++s) sum = sum + ex[s];
    return sum;
  }
  float t[K];
#pragma unroll
  for (int s = 0; s < K; ++s) t[s] = ex[s];
#pragma unroll
  for (int m = K >> 1; m > 0; m >>= 1) {
    float u[K];
#pragma unroll
    for (int s = 0; s < K; ++s) u[s] = t[s] + t[s ^ m];
#pragma unroll
    for (int s = 0; s < K; ++s) t[s] = u[s];
  }
  return t[0];
}

// Softmax over the selected slots and the slot outputs (topk_softmax.cu:
// 160-215, 339-375): sel_i[0] == -1 means no finite logit at all (experts
// 0..k-1, weight 1/k); padded slots (index -1) get weight 0.  oi / ow are
// set for slots s < k.
// K is the compile-time k: straight-line code for the k slots.
template <int K>
__device__ __forceinline__ void slot_values_k(const float* sel_v, const int* sel_i, int variant, int* oi, float* ow) {
  if (sel_i[0] == -1) {
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      oi[s] = s;
      ow[s] = 1.0f / static_cast<float>(K);
    }
    return;
  }
  float mx = -FLT_MAX;
#pragma unroll
  for (int s = 0; s < K; ++s) mx = sel_v[s] > mx ? sel_v[s] : mx;
  float ex[K];
#pragma unroll
  for (int s = 0; s < K; ++s) ex[s] = gx_expf(sel_v[s] - mx);
  const float inv = 1.0f / slot_sum<K>(ex, variant);
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    oi[s] = sel_i[s];
    ow[s] = (s >= K || sel_i[s] < 0) ? 0.0f : ex[s < K ? s : 0] * inv;
  }
}

__device__ __forceinline__ void slot_values(const float* sel_v, const int* sel_i, int k, int variant, int* oi,
                                            float* ow) {
  switch (k) {
    case 1: slot_values_k<1>(sel_v, sel_i, variant, oi, ow); return;
    case 2: slot_values_k<2>(sel_v, sel_i, variant, oi, ow); return;
    case 4: slot_values_k<4>(sel_v, sel_i, variant, oi, ow); return;
    default: slot_values_k<8>(sel_v, sel_i, variant, oi, ow); return;
  }
}

// out_w null: the indices only (no softmax).
__device__ __forceinline__ void write_slots(const float* sel_v, const int* sel_i, int k, int variant, int32_t* out_idx,
                                            float* out_w, int32_t* tokens_per_expert) {
  int oi[kMaxTopK];
  float ow[kMaxTopK];
  if (out_w) {
    slot_values(sel_v, sel_i, k, variant, oi, ow);
  } else {
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) oi[s] = sel_i[0] == -1 ? s : sel_i[s];
  }
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    if (s < k) {
      out_idx[s] = oi[s];
      if (out_w) out_w[s] = ow[s];
      if (tokens_per_expert && oi[s] >= 0) atomicAdd(&tokens_per_expert[oi[s]], 1);
    }
  }
}

// The k selections of one token from the lanes' sanitized logits v
// (expert lane + 64 j).  Round s takes the largest visible key (value desc)
// and, among equal keys, the smallest expert index; a round with nothing
// visible yields (-FLT_MAX, -1), the reference's padding.  kPacked: the
// logits are bf16 values, whose selection key fits 16 bits, so key and
// (0xffff - index) share one 32-bit word and each round is one wave
// max-reduction instead of a max and an index min; the winning word also
// gives back the value (bf16_of_key) and clears itself by equality (words
// are distinct), so the round has no branch.  Wave-uniform results.
template <int NV, bool kPacked>
__device__ __forceinline__ void select_topk(const float (&v)[NV], int k, int lane, float (&sel_v)[kMaxTopK],
                                            int (&sel_i)[kMaxTopK]) {
  uint32_t key[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const uint32_t k32 = select_key(v[j]);  // for a bf16 value the low 16 bits are all equal
    key[j] = !kPacked || k32 == 0u ? k32
                                   : (k32 & 0xffff0000u) | static_cast<uint32_t>(0xffff - (lane + kWave * j));
  }
  if constexpr (kPacked) {
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) {
      sel_v[s] = -FLT_MAX;
      sel_i[s] = -1;
      if (s < k) {
        uint32_t best = key[0];
#pragma unroll
        for (int j = 1; j < NV; ++j) best = max(best, key[j]);
        const uint32_t W = wave_max_u32(best);
        sel_v[s] = W != 0u ? bf16_of_key(W) : -FLT_MAX;
        sel_i[s] = W != 0u ? 0xffff - static_cast<int>(W & 0xffffu) : -1;
#pragma unroll
        for (int j = 0; j < NV; ++j) key[j] = key[j] == W ? 0u : key[j];
      }
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    sel_v[s] = -FLT_MAX;
    sel_i[s] = -1;
    if (s < k) {
      uint32_t best = key[0];
#pragma unroll
      for (int j = 1; j < NV; ++j) best = max(best, key[j]);
      const uint32_t W = wave_max_u32(best);
      if (W != 0u) {
        uint32_t cand = 0xffffffffu;
#pragma unroll
        for (int j = NV - 1; j >= 0; --j)
          if (key[j] == W) cand = static_cast<uint32_t>(lane + kWave * j);
        const int I = static_cast<int>(wave_min_u32(cand));
        const int jj = I >> 6, ll = I & 63;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          if (j == jj) {
            sel_v[s] = __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(v[j])), ll)));
            if (lane == ll) key[j] = 0u;
          }
        }
        sel_i[s] = I;
      }
    }
  }
}

// Top-k of one token and the softmax over the selected k (topk_softmax.cu:
// 77-375), from the lanes' logits v (select_topk; kPacked for bf16 logits).
// Lane 0 writes the slot outputs (v1 sequential sum for variant 1, v2
// butterfly tree otherwise).  Control flow is wave-uniform.
template <int NV, bool kPacked = false>
__device__ __forceinline__ void topk_token(float (&v)[NV], int k, int variant, int32_t* out_idx, float* out_w,
                                           int32_t* tokens_per_expert, int lane) {
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = sanitize_logit(v[j]);
  float sel_v[kMaxTopK];
  int sel_i[kMaxTopK];
  select_topk<NV, kPacked>(v, k, lane, sel_v, sel_i);
  if (lane != 0) return;
  write_slots(sel_v, sel_i, k, variant, out_idx, out_w, tokens_per_expert);
}

// The plan of S <= 64 slots (values from LDS) built by one wave with no
// barrier: lane s holds slot s; its rank among equal experts comes from
// ballots over the expert bits; the counts go through LDS to the lanes that
// own the experts (lane l: experts NV l .. NV l + NV - 1), which add them up
// and take one wave scan of the packed (slots, active experts) sums for the
// offsets and the ascending active list.  Same outputs as build_plan,
// written to p unless p.counts is null.  With l_hdr, also the LDS task
// headers of a decode kernel: l_hdr[a] = {expert | count << 9, offset} for
// active expert a, and l_tok[pos] = token of permuted slot pos.  LDS
// accesses of one wave execute in order, so values written are read back
// without a wait.  Returns the number of active experts (every lane).
template <int NV>
__device__ __forceinline__ int plan_one_wave(const int32_t* s_idx, int S, int k, int E, PlanBufs p, int lane,
                                             int32_t* s_cnt, int32_t* s_off, int32_t* s_aidx,
                                             int2* l_hdr = nullptr, int32_t* l_tok = nullptr) {
  const bool gw = p.counts != nullptr;
  const int e = lane < S ? s_idx[lane] : -1;
  const bool valid = e >= 0 && e < E;
  unsigned long long peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {  // E <= 256
    const bool bit = valid && ((e >> b) & 1);
    const unsigned long long mb = __ballot(bit);
    peers &= bit ? mb : ~mb;
  }
  const int rank = __popcll(peers & ((1ull << lane) - 1ull));
#pragma unroll
  for (int j = 0; j < NV; ++j) s_cnt[NV * lane + j] = 0;
  __builtin_amdgcn_wave_barrier();
  if (valid && rank == 0) s_cnt[e] = __popcll(peers);
  __builtin_amdgcn_wave_barrier();
  // experts NV lane + j: counts, and one scan of (slots | active experts << 16)
  int c[NV];
  int csum = 0, asum = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int ex = NV * lane + j;
    c[j] = ex < E ? s_cnt[ex] : 0;
    csum += c[j];
    asum += c[j] > 0 ? 1 : 0;
  }
  const int packed = csum | (asum << 16);  // slots <= 64, experts <= 256
  int incl = packed;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  const int nact = __builtin_amdgcn_readlane(incl, kWave - 1) >> 16;
  int excl = (incl - packed) & 0xffff, aidx = (incl - packed) >> 16;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int ex = NV * lane + j;
    if (ex < E) {
      s_off[ex] = excl;
      if (gw) {
        p.counts[ex] = c[j];
        p.offsets[ex] = excl;
        if (ex == E - 1) p.offsets[E] = excl + c[j];
      }
      if (c[j] > 0) {
        s_aidx[ex] = aidx;
        if (l_hdr) l_hdr[aidx] = make_int2(ex | (c[j] << 9), excl);
        if (gw) {
          p.active[aidx] = ex;
          if (p.tasks) {
            int32_t* t = p.tasks + static_cast<size_t>(aidx) * kTaskInts;
            t[0] = ex;
            t[1] = excl;
            t[2] = c[j];
            t[3] = 0;
          }
        }
        ++aidx;
      }
    }
    excl += c[j];
  }
  if (gw) {
    if (lane == 0) *p.n_active = nact;
    if (p.tasks) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int r = lane + kWave * j;
        if (r < E && r >= nact) p.tasks[static_cast<size_t>(r) * kTaskInts] = -1;
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (valid) {
    const int pos = s_off[e] + rank;
    if (l_tok) l_tok[pos] = lane / k;
    if (gw) {
      p.gather_map[lane] = pos;
      p.perm_token[pos] = lane / k;
      if (p.tasks && rank < kTaskTokens) p.tasks[static_cast<size_t>(s_aidx[e]) * kTaskInts + 4 + rank] = lane / k;
    }
  } else if (lane < S && gw) {
    p.gather_map[lane] = -1;
  }
  return nact;
}

// One token with bf16 logits, routed and planned by one wave, for the
// decode gate_up prologue at T = 1, where every work-group of the launch
// routes the token.  Two parts: route_one_token_select gives the selections
// and the LDS task headers the work-group's items need;
// route_one_token_publish, called by work-groups without items, writes the
// plan for the later launches.  Together they give the
// outputs of topk_token followed by plan_one_wave (S = K slots).  Selection
// as select_topk<NV, true>.  The K selected experts are distinct (or -1
// padding, which only follows the valid ones), so every active expert
// holds one slot, and an expert's offset, its slot's permuted position and
// its active index are all the number of selected experts below it.
struct OneTokenRoute {
  float sel_v[kMaxTopK];  // selected logits, in selection order
  int sel_i[kMaxTopK];    // selected experts, -1: none
};

// Slot experts (experts 0..K-1 when no logit is finite, topk_softmax.cu:
// 160-215), their validity, positions and the active count; wave-uniform.
template <int K>
__device__ __forceinline__ int one_token_slots(const OneTokenRoute& r, int E, int (&oi)[K], bool (&ok)[K],
                                               int (&pos)[K]) {
  int nact = 0;
#pragma unroll
  for (int s = 0; s < K; ++s) {
    oi[s] = r.sel_i[0] == -1 ? s : r.sel_i[s];
    ok[s] = oi[s] >= 0 && oi[s] < E;
    nact += ok[s] ? 1 : 0;
  }
#pragma unroll
  for (int s = 0; s < K; ++s) {
    int q = 0;
#pragma unroll
    for (int t = 0; t < K; ++t) q += (ok[t] && oi[t] < oi[s]) ? 1 : 0;
    pos[s] = q;
  }
  return nact;
}

// The selections, and the LDS task headers in selection order: header s
// holds the s-th selected expert (count 1) and its position.  That is the
// plan's active order permuted, so a work-group's items cover the same
// (expert, tile) pairs and every output lands at its permuted slot.
// l_tok[position] = 0 (the one token).  Returns the number of active experts.
template <int NV, int K>
__device__ __forceinline__ int route_one_token_select(const float (&v_in)[NV], int E, int lane, int2* l_hdr,
                                                      int32_t* l_tok, OneTokenRoute& r) {
  float v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) v[j] = sanitize_logit(v_in[j]);
  select_topk<NV, true>(v, K, lane, r.sel_v, r.sel_i);
  int oi[K], pos[K];
  bool ok[K];
  const int nact = one_token_slots<K>(r, E, oi, ok, pos);
  if (lane < K) {
    int e = -1, q = 0;
    bool o = false;
#pragma unroll
    for (int s = 0; s < K; ++s)
      if (s == lane) {
        e = oi[s];
        o = ok[s];
        q = pos[s];
      }
    if (o) {
      l_hdr[lane] = make_int2(e | (1 << 9), q);
      l_tok[q] = 0;
    }
  }
  return nact;
}

template <int NV>
__device__ __forceinline__ int route_one_token_select_k(const float (&v)[NV], int k, int E, int lane, int2* l_hdr,
                                                        int32_t* l_tok, OneTokenRoute& r) {
  switch (k) {
    case 1: return route_one_token_select<NV, 1>(v, E, lane, l_hdr, l_tok, r);
    case 2: return route_one_token_select<NV, 2>(v, E, lane, l_hdr, l_tok, r);
    case 4: return route_one_token_select<NV, 4>(v, E, lane, l_hdr, l_tok, r);
    default: return route_one_token_select<NV, 8>(v, E, lane, l_hdr, l_tok, r);
  }
}

// The plan buffers p, written once by G >= 1 work-groups: work-group wg
// writes the entries of experts and task records wg, wg + G, ... (and
// offsets[E]), work-group 0 the per-slot arrays and the routing weights
// (softmax over the selected logits, computed there only).
template <int K>
__device__ __forceinline__ void route_one_token_publish(const OneTokenRoute& r, int E, int variant, PlanBufs p,
                                                        int wg, int G, int32_t* g_idx, float* g_w, int lane) {
  if (p.counts == nullptr) return;
  int oi[K], pos[K];
  bool ok[K];
  const int nact = one_token_slots<K>(r, E, oi, ok, pos);
  if (wg == 0) {
    int si[kMaxTopK];
    float ow[kMaxTopK];
    slot_values_k<K>(r.sel_v, r.sel_i, variant, si, ow);
    if (lane < K) {
      int e = -1, q = 0;
      bool o = false;
      float w = 0.0f;
#pragma unroll
      for (int s = 0; s < K; ++s)
        if (s == lane) {
          e = oi[s];
          w = ow[s];
          o = ok[s];
          q = pos[s];
        }
      g_idx[lane] = e;
      g_w[lane] = w;
      p.gather_map[lane] = o ? q : -1;
      if (o) p.perm_token[q] = 0;
    }
    if (lane == 0) *p.n_active = nact;
  }
  // expert (and task record) e = wg + G lane' for lanes with e <= E
  for (int e = wg + G * lane; e <= E; e += G * kWave) {
    int c = 0, off = 0, er = -1;
#pragma unroll
    for (int s = 0; s < K; ++s) {
      c += (ok[s] && oi[s] == e) ? 1 : 0;
      off += (ok[s] && oi[s] < e) ? 1 : 0;
      if (ok[s] && pos[s] == e) er = oi[s];
    }
    if (e == E) {
      p.offsets[E] = nact;
      continue;
    }
    p.counts[e] = c;
    p.offsets[e] = off;
    if (e < nact) {  // the e-th active expert
      p.active[e] = er;
      if (p.tasks) {
        int32_t* t = p.tasks + static_cast<size_t>(e) * kTaskInts;
        t[0] = er;
        t[1] = e;
        t[2] = 1;
        t[3] = 0;
        t[4] = 0;  // the slot's token
      }
    } else if (p.tasks) {
      p.tasks[static_cast<size_t>(e) * kTaskInts] = -1;
    }
  }
}

__device__ __forceinline__ void route_one_token_publish_k(const OneTokenRoute& r, int k, int E, int variant,
                                                          PlanBufs p, int wg, int G, int32_t* g_idx, float* g_w,
                                                          int lane) {
  switch (k) {
    case 1: route_one_token_publish<1>(r, E, variant, p, wg, G, g_idx, g_w, lane); return;
    case 2: route_one_token_publish<2>(r, E, variant, p, wg, G, g_idx, g_w, lane); return;
    case 4: route_one_token_publish<4>(r, E, variant, p, wg, G, g_idx, g_w, lane); return;
    default: route_one_token_publish<8>(r, E, variant, p, wg, G, g_idx, g_w, lane); return;
  }
}

}  // namespace
}  // namespace gxmoe
