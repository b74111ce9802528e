// moe_route.hip -- router GEMV + top-k softmax + device routing plan (gfx950).
//
// One launch replaces the reference's router GEMV/GEMM (gemv_bf16.cu:40-130,
// cuda_utils.h:226-308), topk_softmax_forward (topk_softmax.cu:380-432),
// moe_permute_classify (moe_permute.cu:129-179) and the host gather map
// (moe_permute.cu:184-236, moe_layer.cu:1217-1234), with no host round trip:
//
//   grid (ceil(E/4), ceil(T/8)), 256 threads.  Work-group (g, tg) computes
//   the logits of experts 4g..4g+3 for tokens 8tg..8tg+7 with the
//   gemv_bf16_kernel summation tree.  The last work-group to finish a token
//   group (atomic ticket) selects the top-k of its tokens; the last token
//   group to finish builds the plan (histogram, exclusive scan, stable
//   counting-sort gather map, permuted token list, active expert list); with
//   a single token group (T <= 8) the selecting work-group builds it from
//   LDS directly.  Values crossing work-groups go through write-through
//   exchange buffers (no L2 flush).  Tickets are reset by their last holder,
//   so the launch is replayable (hipGraph) without a memset.
#include <float.h>

#include "moe_device.h"
#include "moe_kernels.h"

namespace gxmoe {

namespace {

constexpr int kRouteThreads = 256;

__device__ __forceinline__ float sanitize_logit(float v) {
  // topk_softmax.cu:47-52: NaN and +-Inf become -FLT_MAX.
  return ((__float_as_uint(v) & 0x7f800000u) == 0x7f800000u) ? -FLT_MAX : v;
}

// Cross-work-group exchange without cache maintenance: agent-scope relaxed
// stores and loads write through / read past the per-XCD L2, so a writer
// that waits for its stores (vmcnt 0) before taking a ticket, and a reader
// that loads only after holding the last ticket, see each other's data.
__device__ __forceinline__ void st_xchg(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_xchg(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_xchg(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_xchg(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
__device__ __forceinline__ uint32_t take_ticket(uint32_t* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_ticket(uint32_t* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Logit loaders for the top-k: a user buffer (bf16 or fp32) or the fp32
// exchange row (already rounded as the logits are).
struct LogitsUser {
  const void* row;
  bool f32;
  __device__ float operator()(int e) const {
    return f32 ? reinterpret_cast<const float*>(row)[e] : bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[e]);
  }
};
struct LogitsXchg {
  const float* row;
  __device__ float operator()(int e) const { return ld_xchg(row + e); }
};

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float* f) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(d[i] << 16);
    f[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
  }
}

// Lane l's four logits (experts l, l+64, l+128, l+192); -FLT_MAX past E.
template <typename Loader>
__device__ __forceinline__ void load_token_logits(const Loader& load, int E, int lane, float (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int e = lane + 64 * j;
    v[j] = (e < E) ? load(e) : -FLT_MAX;
  }
}

// Top-k of one token by one wave from its lanes' logits v (as loaded by
// load_token_logits; sanitised here).  Each round takes the largest visible
// logit (> -FLT_MAX) by (value desc, index asc); a round with nothing visible
// yields (-FLT_MAX, -1), the reference's padding (topk_softmax.cu:133-159).
// Lane 0 then applies the softmax over the k selected values in the order of
// the reference variant (v1 sequential sum for T <= 8, v2 xor-butterfly sum
// otherwise).
__device__ __forceinline__ void topk_select(float (&v)[4], int k, int variant, int32_t* out_idx, float* out_w,
                                            int32_t* tokens_per_expert, int32_t* lds_idx, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = sanitize_logit(v[j]);
  float sel_v[kMaxTopK];
  int sel_i[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    sel_v[s] = -FLT_MAX;
    sel_i[s] = -1;
    if (s < k) {
      float bv = -FLT_MAX;
      int bi = -1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (v[j] > bv) { bv = v[j]; bi = lane + 64 * j; }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(bv, m, kWave);
        int oi = __shfl_xor(bi, m, kWave);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      sel_v[s] = bv;
      sel_i[s] = bi;
      if (bi >= 0 && (bi & 63) == lane) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if ((bi >> 6) == j) v[j] = -FLT_MAX;
      }
    }
  }
  if (lane != 0) return;
  if (sel_i[0] == -1) {  // topk_softmax.cu:339-346: no finite logit at all
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (s < k) {
        out_idx[s] = s;
        out_w[s] = 1.0f / static_cast<float>(k);
        if (lds_idx) lds_idx[s] = s;
      }
    if (tokens_per_expert)
      for (int s = 0; s < k; ++s) atomicAdd(&tokens_per_expert[s], 1);
    return;
  }
  float mx = -FLT_MAX;
  float ex[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s)
    if (s < k && sel_v[s] > mx) mx = sel_v[s];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) ex[s] = (s < k) ? gx_expf(sel_v[s] - mx) : 0.0f;
  float sum;
  if (variant == 1) {  // topk_softmax.cu:199-204
    sum = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (s < k) sum = sum + ex[s];
  } else {  // topk_softmax.cu:358-362, the tree every lane of the butterfly ends with
    float t[kMaxTopK];
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s) t[s] = ex[s];
    for (int m = k >> 1; m > 0; m >>= 1) {
      float u[kMaxTopK];
#pragma unroll
      for (int s = 0; s < kMaxTopK; ++s) u[s] = t[s] + t[s ^ m];
#pragma unroll
      for (int s = 0; s < kMaxTopK; ++s) t[s] = u[s];
    }
    sum = t[0];
  }
  float inv = 1.0f / sum;
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    if (s < k) {
      out_idx[s] = sel_i[s];
      out_w[s] = (sel_i[s] < 0) ? 0.0f : ex[s] * inv;
      if (lds_idx) lds_idx[s] = sel_i[s];
      if (tokens_per_expert && sel_i[s] >= 0) atomicAdd(&tokens_per_expert[sel_i[s]], 1);
    }
  }
}

template <typename Loader>
__device__ __forceinline__ void topk_one_token(const Loader& load, int E, int k, int variant,
                                               int32_t* out_idx, float* out_w,
                                               int32_t* tokens_per_expert, int32_t* lds_idx, int lane) {
  float v[4];
  load_token_logits(load, E, lane, v);
  topk_select(v, k, variant, out_idx, out_w, tokens_per_expert, lds_idx, lane);
}

// Block-wide (256 threads) dispatch plan over the T*k slots of `idx`:
// counts, exclusive offsets, a gather map that is stable in slot order (the
// counting sort of moe_permute.cu:184-236), the permuted token list and the
// ascending list of experts with at least one slot.  Slots with an index
// outside [0, E) get gather_map = -1 and are not dispatched.
template <typename IdxFn>
__device__ void build_plan(IdxFn idx, int T, int k, int E, PlanBufs p) {
  __shared__ int s_off[kMaxExperts + 1];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_run[kMaxExperts];
  __shared__ int s_wc[4][kMaxExperts];
  __shared__ int s_aidx[kMaxExperts];
  __shared__ unsigned long long s_mask[4];
  __shared__ int s_wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  const int S = T * k;

  // slot tid's expert is read once and reused by the rank pass below
  const int e_first = (tid < S) ? idx(tid) : -1;
  auto slot_expert = [&](int s) { return s == tid ? e_first : idx(s); };
  s_cnt[tid] = 0;
  s_run[tid] = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) s_wc[w][tid] = 0;
  __syncthreads();
  for (int s = tid; s < S; s += kRouteThreads) {
    int e = slot_expert(s);
    if (e >= 0 && e < E) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();

  // exclusive scan of the counts (E <= 256: one value per thread)
  const int c = (tid < E) ? s_cnt[tid] : 0;
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += o;
  }
  if (lane == 63) s_wsum[warp] = incl;
  const bool act = (tid < E) && (c > 0);
  const unsigned long long am = __ballot(act);
  if (lane == 0) s_mask[warp] = am;
  __syncthreads();
  int base = 0, abase = 0;
  for (int w = 0; w < warp; ++w) { base += s_wsum[w]; abase += __popcll(s_mask[w]); }
  const int excl = base + incl - c;
  if (tid < E) {
    s_off[tid] = excl;
    p.counts[tid] = c;
    p.offsets[tid] = excl;
  }
  if (tid == E - 1) { s_off[E] = excl + c; p.offsets[E] = excl + c; }
  const int aidx = abase + __popcll(am & ((1ull << lane) - 1ull));
  const int nact = __popcll(s_mask[0]) + __popcll(s_mask[1]) + __popcll(s_mask[2]) + __popcll(s_mask[3]);
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
  if (tid == 0) *p.n_active = nact;
  __syncthreads();

  // stable positions, 256 slots per round
  for (int r0 = 0; r0 < S; r0 += kRouteThreads) {
    const int s = r0 + tid;
    const int e = (s < S) ? slot_expert(s) : -1;
    const bool valid = (e >= 0 && e < E);
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const unsigned long long mb = __ballot(bit);
      peers &= bit ? mb : ~mb;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    if (valid && rank == 0) s_wc[warp][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pos = s_off[e] + s_run[e] + rank;
      for (int w = 0; w < warp; ++w) pos += s_wc[w][e];
      p.gather_map[s] = pos;
      p.perm_token[pos] = s / k;
      if (p.tasks && pos - s_off[e] < kTaskTokens)
        p.tasks[static_cast<size_t>(s_aidx[e]) * kTaskInts + 4 + (pos - s_off[e])] = s / k;
    } else if (s < S) {
      p.gather_map[s] = -1;
    }
    __syncthreads();
    if (tid < E) {
      s_run[tid] += s_wc[0][tid] + s_wc[1][tid] + s_wc[2][tid] + s_wc[3][tid];
#pragma unroll
      for (int w = 0; w < 4; ++w) s_wc[w][tid] = 0;
    }
    __syncthreads();
  }
}

// The H%8 tail of the router chains (gemv_bf16.cu:118-125), after the chunks.
__device__ __forceinline__ void router_tail(const uint16_t* xr, const RouteArgs& a, int e0, int KV, int tid,
                                            float (&acc)[kRouteExpertsPerGroup]) {
  const int H = a.H, E = a.E;
  for (int kk = KV * 8 + tid; kk < H; kk += kRouteThreads) {
    const float xs = bf16_to_f32(xr[kk]);
#pragma unroll
    for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee)
      if (e0 + ee < E) acc[ee] = __builtin_fmaf(xs, bf16_to_f32(a.W[static_cast<size_t>(e0 + ee) * H + kk]), acc[ee]);
  }
}

// Logits of one token with the gemv_bf16_kernel tree (gemv_bf16.cu:57-129):
// thread tid chains fmaf over 8-element chunks tid, tid+256, ... (NJ of
// them at most), then the H%8 tail.  xs_chunk(j) / ws_chunk(ee, j) give chunk
// tid + 256 j.
template <int NJ, typename XFn, typename WFn>
__device__ __forceinline__ void router_chains(XFn xs_chunk, WFn ws_chunk, const uint16_t* xr, const RouteArgs& a,
                                              int e0, int KV, int tid, float (&acc)[kRouteExpertsPerGroup]) {
  const int E = a.E;
#pragma unroll
  for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) acc[ee] = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (tid + kRouteThreads * j < KV) {
      float xs[8];
      unpack_bf16x8(xs_chunk(j), xs);
#pragma unroll
      for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) {
        if (e0 + ee < E) {
          float ws[8];
          unpack_bf16x8(ws_chunk(ee, j), ws);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[ee] = __builtin_fmaf(xs[i], ws[i], acc[ee]);
        }
      }
    }
  }
  router_tail(xr, a, e0, KV, tid, acc);
}

// NJ > 0: every thread holds at most NJ chunks (H <= 2048 * NJ); all of the
// work-group's router and token loads are issued before the first FMA.
// NJ == 0: any H, one chunk in flight at a time.
template <bool F32, int NJ>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  const int e0 = blockIdx.x * kRouteExpertsPerGroup;
  const int t0 = blockIdx.y * kRouteTokensPerGroup;
  const int tn = min(kRouteTokensPerGroup, a.T - t0);
  const int H = a.H, E = a.E;
  const int KV = H >> 3;
  __shared__ float red[kRouteTokensPerGroup][kRouteExpertsPerGroup][4];
  __shared__ uint32_t s_ticket;

  // Logits: per token, the chains of router_chains; xor butterfly per wave;
  // the 4 wave sums are added in order from 0.
  constexpr int kNJ = NJ > 0 ? NJ : 1;
  uint4 wv[kRouteExpertsPerGroup][kNJ];
  uint4 xv[kRouteTokensPerGroup][kNJ];
  if constexpr (NJ > 0) {
#pragma unroll
    for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int kv = tid + kRouteThreads * j;
        wv[ee][j] = (kv < KV && e0 + ee < E)
                        ? *reinterpret_cast<const uint4*>(a.W + static_cast<size_t>(e0 + ee) * H + kv * 8)
                        : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
    for (int tt = 0; tt < kRouteTokensPerGroup; ++tt)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int kv = tid + kRouteThreads * j;
        xv[tt][j] = (tt < tn && kv < KV)
                        ? *reinterpret_cast<const uint4*>(a.x + static_cast<size_t>(t0 + tt) * H + kv * 8)
                        : make_uint4(0, 0, 0, 0);
      }
  }
#pragma unroll
  for (int tt = 0; tt < kRouteTokensPerGroup; ++tt) {
    if (tt >= tn) break;
    const uint16_t* xr = a.x + static_cast<size_t>(t0 + tt) * H;
    float acc[kRouteExpertsPerGroup];
    if constexpr (NJ > 0) {
      router_chains<NJ>([&](int j) { return xv[tt][j]; }, [&](int ee, int j) { return wv[ee][j]; }, xr, a, e0, KV,
                        tid, acc);
    } else {
      for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) acc[ee] = 0.0f;
      for (int kv = tid; kv < KV; kv += kRouteThreads) {
        float xs[8];
        unpack_bf16x8(*reinterpret_cast<const uint4*>(xr + kv * 8), xs);
#pragma unroll
        for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) {
          if (e0 + ee < E) {
            float ws[8];
            unpack_bf16x8(*reinterpret_cast<const uint4*>(a.W + static_cast<size_t>(e0 + ee) * H + kv * 8), ws);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[ee] = __builtin_fmaf(xs[i], ws[i], acc[ee]);
          }
        }
      }
      router_tail(xr, a, e0, KV, tid, acc);
    }
#pragma unroll
    for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) acc[ee] = wave_butterfly_sum(acc[ee]);
    if (lane == 0) {
#pragma unroll
      for (int ee = 0; ee < kRouteExpertsPerGroup; ++ee) red[tt][ee][warp] = acc[ee];
    }
  }
  __syncthreads();
  if (tid < tn * kRouteExpertsPerGroup) {
    const int tt = tid / kRouteExpertsPerGroup, ee = tid % kRouteExpertsPerGroup, e = e0 + ee;
    if (e < E) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) v = v + red[tt][ee][w];
      if (a.b != nullptr) v = v + bf16_to_f32(a.b[e]);
      const size_t o = static_cast<size_t>(t0 + tt) * E + e;
      if constexpr (F32) {
        reinterpret_cast<float*>(a.logits)[o] = v;
      } else {
        const uint16_t h = f32_to_bf16(v);
        reinterpret_cast<uint16_t*>(a.logits)[o] = h;
        v = bf16_to_f32(h);
      }
      st_xchg(a.xchg_logits + o, v);
    }
  }

  // The last expert group of this token group selects the top-k.
  wait_stores();
  __syncthreads();
  if (tid == 0) s_ticket = take_ticket(&a.group_counter[blockIdx.y]);
  __syncthreads();
  if (s_ticket != gridDim.x - 1) return;
  if (tid == 0) reset_ticket(&a.group_counter[blockIdx.y]);
  const int variant = (a.T <= 8) ? 1 : 2;  // topk_softmax.cu:399
  const bool one_group = gridDim.y == 1;
  __shared__ int32_t s_idx[kRouteTokensPerGroup * kMaxTopK];
  // Wave w selects tokens w and w + 4; both rows' logits are loaded first.
  static_assert(kRouteTokensPerGroup == 8, "two tokens per wave");
  float lv[2][4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tt = warp + 4 * h;
    if (tt < tn) load_token_logits(LogitsXchg{a.xchg_logits + static_cast<size_t>(t0 + tt) * E}, E, lane, lv[h]);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tt = warp + 4 * h;
    if (tt < tn) {
      const int t = t0 + tt;
      topk_select(lv[h], a.k, variant, a.idx + static_cast<size_t>(t) * a.k, a.w + static_cast<size_t>(t) * a.k,
                  nullptr, one_group ? s_idx + tt * a.k : nullptr, lane);
      if (!one_group && lane == 0)
        for (int s2 = 0; s2 < a.k; ++s2)
          st_xchg(a.xchg_idx + static_cast<size_t>(t) * a.k + s2, a.idx[static_cast<size_t>(t) * a.k + s2]);
    }
  }
  if (a.plan.counts == nullptr) return;
  if (one_group) {  // T <= 8: this work-group holds every token's selection
    __syncthreads();
    build_plan([&](int s2) { return s_idx[s2]; }, a.T, a.k, E, a.plan);
    return;
  }

  // The last token group builds the plan over all T*k slots.
  wait_stores();
  __syncthreads();
  if (tid == 0) s_ticket = take_ticket(a.done_counter);
  __syncthreads();
  if (s_ticket != gridDim.y - 1) return;
  if (tid == 0) reset_ticket(a.done_counter);
  build_plan([&](int s2) { return ld_xchg(a.xchg_idx + s2); }, a.T, a.k, E, a.plan);
}

template <bool F32>
__global__ __launch_bounds__(kRouteThreads) void topk_kernel(const void* logits, int T, int E, int k,
                                                            int32_t* idx, float* w, int32_t* tpe) {
  const int lane = threadIdx.x & 63, warp = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + warp;
  if (t >= T) return;
  const void* row = F32 ? static_cast<const void*>(reinterpret_cast<const float*>(logits) + static_cast<size_t>(t) * E)
                        : static_cast<const void*>(reinterpret_cast<const uint16_t*>(logits) + static_cast<size_t>(t) * E);
  topk_one_token(LogitsUser{row, F32}, E, k, (T <= 8) ? 1 : 2, idx + static_cast<size_t>(t) * k,
                 w + static_cast<size_t>(t) * k, tpe, nullptr, lane);
}

__global__ __launch_bounds__(kRouteThreads) void plan_kernel(const int32_t* idx, int T, int k, int E,
                                                            PlanBufs p) {
  build_plan([&](int s) { return idx[s]; }, T, k, E, p);
}

}  // namespace

static size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

size_t route_scratch_bytes(int T, int E, int k) {
  const size_t groups = (static_cast<size_t>(T > 0 ? T : 1) + kRouteTokensPerGroup - 1) / kRouteTokensPerGroup;
  return align256((groups + 1) * 4) + align256(static_cast<size_t>(T) * E * 4) + align256(static_cast<size_t>(T) * k * 4);
}

void route_scratch_carve(void* scratch, int T, int E, int k, RouteArgs& a) {
  const size_t groups = (static_cast<size_t>(T > 0 ? T : 1) + kRouteTokensPerGroup - 1) / kRouteTokensPerGroup;
  char* p = static_cast<char*>(scratch);
  a.group_counter = reinterpret_cast<uint32_t*>(p);
  a.done_counter = a.group_counter + groups;
  p += align256((groups + 1) * 4);
  a.xchg_logits = reinterpret_cast<float*>(p);
  p += align256(static_cast<size_t>(T) * E * 4);
  a.xchg_idx = reinterpret_cast<int32_t*>(p);
}

hipError_t launch_route(const RouteArgs& a, hipStream_t s) {
  if (a.T <= 0) return hipSuccess;
  dim3 grid((a.E + kRouteExpertsPerGroup - 1) / kRouteExpertsPerGroup,
            (a.T + kRouteTokensPerGroup - 1) / kRouteTokensPerGroup);
  // chunks of 8 inputs per thread: 2 covers H <= 4096 (GPT-OSS: 2880)
  const int nj = ((a.H >> 3) + kRouteThreads - 1) / kRouteThreads;
  if (a.logits_fp32) {
    if (nj <= 1) gx_launch(route_kernel<true, 1>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
    else if (nj == 2) gx_launch(route_kernel<true, 2>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
    else gx_launch(route_kernel<true, 0>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
  } else {
    if (nj <= 1) gx_launch(route_kernel<false, 1>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
    else if (nj == 2) gx_launch(route_kernel<false, 2>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
    else gx_launch(route_kernel<false, 0>, grid, dim3(kRouteThreads), 0, s, a.timer, a);
  }
  return hipGetLastError();
}

hipError_t launch_topk(const void* logits, int logits_fp32, int T, int E, int k,
                       int32_t* idx, float* w, int32_t* tpe, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  dim3 grid((T + 3) / 4);
  if (logits_fp32)
    hipLaunchKernelGGL(topk_kernel<true>, grid, dim3(kRouteThreads), 0, s, logits, T, E, k, idx, w, tpe);
  else
    hipLaunchKernelGGL(topk_kernel<false>, grid, dim3(kRouteThreads), 0, s, logits, T, E, k, idx, w, tpe);
  return hipGetLastError();
}

hipError_t launch_plan(const int32_t* idx, int T, int k, int E, PlanBufs plan, hipStream_t s,
                       const KernelTimer& timer) {
  if (T <= 0) return hipSuccess;
  gx_launch(plan_kernel, dim3(1), dim3(kRouteThreads), 0, s, timer, idx, T, k, E, plan);
  return hipGetLastError();
}

}  // namespace gxmoe
