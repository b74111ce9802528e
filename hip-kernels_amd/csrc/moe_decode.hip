// moe_decode.hip -- decode-path MXFP4 expert products on the gfx950 matrix
// cores (the default decode path of the layer).
//
// Replaces fused_mxfp4_gemv_forward / _multi_forward (fused_mxfp4_gemv.cu:
// 76-310) with the bias kernels (moe_layer.cu:171-194, 442-473) and
// swiglu_forward (swiglu.cu:117-211) fused in, as issued per active expert
// by moe_layer.cu:1316-1487:
//
//   mc_stream_kernel<gated>    gate_up: + bias, bf16 gate/up, clamped SwiGLU,
//                              bf16 activations (permuted slot order)
//   mc_stream_kernel<!gated>   down: + bias, bf16 expert outputs
//
// Decode is HBM-bound: every touched expert's MXFP4 weights are read once
// and used by its few tokens.  The kernel is therefore a weight stream:
//
// * Work items are (active expert, 64-row tile) pairs of the routing plan's
//   task records; a work-group of P waves takes items v, v + G, ... (G = grid,
//   v the XCD-grouped block index, so one XCD's work-groups cover a
//   contiguous item range and share the items' token rows in their L2);
//   gate_up's last, partial round takes item r G + b (b the block index),
//   which spreads the round's items over the XCDs and CUs.
//   Wave p reduces over K-part p (nb / P blocks of 32); the P partial sums
//   meet in LDS and are added in part order (deterministic).
// * Per block, lane l issues one 16-byte nontemporal load of slot l of the
//   tiled KiB (moe_kernels.h): dword i is the A operand of the 16x16x32 bf16
//   product of sub-tile i (rows 16 i + l % 16, elements 8 (l/16) .. +7),
//   one dword of the block's slot-order scales (row 16 i + l % 16 in byte i),
//   and 16 bytes of its token column's activations (the B operand, shared by
//   the four sub-tiles).  Decode to bf16 is the scaled fp4 conversion
//   (exact for codes 1..254; experts holding code 0 or 255 take the exact
//   special-code decode).
// * Loads move through a ring of D blocks in VGPRs: consuming block i issues
//   block i + D, which past the end of the part is block i + D - nb/P of the
//   work-group's next step, so a wave's stream does not stop between items;
//   a missing next step reads fixed valid data (static wait counts).
// * Tokens: a step applies the tile to up to 16 NC of the expert's slots
//   (NC chunks of 16 token columns); larger experts take further steps.
//
// Numerics: products of bf16 activations and exactly decoded weights are
// exact; sums are fp32 in the matrix core's order and then in part order, so
// results differ from the canonical (exact VALU) order by fp32 rounding
// before the bf16 rounding, as the prefill path does.
#include <type_traits>

#include "moe_device.h"
#include "moe_kernels.h"
#include "moe_topk.h"

namespace gxmoe {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct McParams {
  const uint16_t* x;          // gate_up: token rows [T][K]; down: activation rows [S][K] (slot order)
  const uint8_t* wn;          // tiled nibbles, [E] x g.nib_bytes
  const uint8_t* ws;          // tiled scales, [E] x g.scale_bytes (slot-order region read)
  const uint16_t* bias;       // [E][N] or null
  const int32_t* tasks;       // [max_active][kTaskInts] task records
  const int32_t* n_active;    // [1]
  const int32_t* perm_token;  // [S] slot -> token (gate_up)
  const int32_t* special;     // [E] nonzero: the expert's scales hold code 0 or 255; null: any may
  uint16_t* out;              // gate_up: activations [S][N/2]; down: expert outputs [S][N]
  uint16_t* gate_up;          // [S][N] bf16 trace or null (gate_up only)
  uint32_t wn_bytes, ws_bytes, x_bytes;  // buffer extents (each < 2^32 - 2^16)
  int slots;                  // S = T * k (gate_up: slot -> token map length)
  int max_tasks;              // task records readable at tasks (>= *n_active)
  int bpp;                    // blocks per K-part: nb / P, a multiple of D
  float alpha, limit;
  TiledGeom g;
  // Routing in the gate_up prologue (kRoute): every work-group selects the
  // top-k of the r_T <= kSmallTopkMaxT tokens from the router's logits and
  // builds the plan in LDS; work-group 0 also writes r_idx, r_w and r_plan
  // for the launches after this one.
  const void* r_logits;
  int r_fp32, r_T, r_E, r_k, r_variant;
  int32_t* r_idx;
  float* r_w;
  PlanBufs r_plan;
};

constexpr int kLdsSlots = 1024;       // slot -> token map staged in LDS up to this many slots
constexpr int kBufWord3 = 0x00020000;  // raw buffer, dword data (gfx9 descriptor word 3)
constexpr int kNT = 2;                 // buffer load cache policy: nontemporal (streamed once)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), kBufWord3);
}

struct McStep {
  int valid, q, t, cg, e, off, M, sp;
};

// Byte offsets of one step's first block in the three buffers (wave-uniform)
// plus this lane's B-row offsets.  A missing step points past the end of
// every buffer with zero strides: its loads return zeros and touch no memory.
template <int NC>
struct McSrc {
  uint32_t a, s, b;          // soffset of block 0
  uint32_t astr, sstr, bstr; // bytes per block (0 for a missing step)
  uint32_t vb[NC];           // voffset of this lane's B row in chunk c
};

// kSpec: some expert's scales hold code 0 or 255, so each step checks its
// expert's flag (a variant launched only for such weights: the check costs
// registers in the block loop).  BPP: blocks per K-part when known at compile
// time (a step is then straight-line code, so the compiler's load waits see
// exactly which ring slot each block needs); 0 = a.bpp, a multiple of D.
// kRoute (gate_up, T <= kSmallTopkMaxT): the routing plan is made in the
// prologue (McParams r_*) instead of read from a plan launch.
// kStg (straight-line steps): operands each wave copies into LDS once per
// step, for its K-part, instead of loading them per block and lane.
//   1: the scales.  Per block a lane needs one dword of 16, so the per-lane
//      loads return 256 bytes for 64.
//   2: the scales and the input rows of columns 0 and 1 (at most 2 slots
//      per expert, one 16-token chunk).  The B loads would return 1 KiB per
//      block for one or two distinct 64-byte rows.
// With scales only, the next step's copy is loaded halfway through the step
// and written to LDS after its last block, when every LDS read of the step
// is issued.  With rows (one or two tokens, so mostly one item per
// work-group) a work-group given another item copies it with a full wait.
template <bool kGated, int P, int D, int NC, bool kSpec, int BPP, bool kRoute = false, int kStg = 0>
__global__ __launch_bounds__(P * kWave) void mc_stream_kernel(McParams a) {
  constexpr int kFr = 4 * NC;   // accumulator fragments: (sub-tile, chunk)
  constexpr int kTok = 16 * NC; // token columns per step
  constexpr int kRed = P > 1 ? P * kFr * kWave : 1;
  constexpr int kOwn = (kFr + P - 1) / P;  // fragments this wave finishes
  // the routing prologue's selections and plan scratch (ints), dead before
  // the epilogue's first use of red, live in red
  constexpr int kRouteInts = 2 * kSmallTopkMaxT * kMaxTopK + 3 * kMaxExperts;
  constexpr int kRedAll = kRoute && kRed * 4 < kRouteInts ? (kRouteInts + 3) / 4 : kRed;
  __shared__ int2 hdr[kMaxExperts];
  __shared__ f32x4 red[kRedAll];  // [P][kFr][64 lanes]
  __shared__ int32_t tok[kGated ? kLdsSlots : 1];  // slot -> token (gate_up, S <= kLdsSlots)
  constexpr bool kStageS = kStg >= 1, kStageB = kStg == 2;
  static_assert(kStg == 0 || (BPP > 0 && !kSpec), "staged operands: straight-line steps");
  static_assert(!kStageB || NC == 1, "staged rows: one chunk");
  // staged operands, per wave: the part's scales (and input rows 0 and 1),
  // kStgU4 16-byte words each (whole 64-lane loads)
  constexpr int kStgRows = kStageB ? 3 : 1;
  constexpr int kStgU4 = kStageS ? (BPP * 4 + kWave - 1) / kWave * kWave : 1;
  __shared__ gx_u32x4 stg[kStageS ? P * kStgRows * kStgU4 : 1];

  const TiledGeom& g = a.g;
  const int lane = threadIdx.x & 63;
  const int p = P > 1 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6) : 0;
  const int K = g.K, N = g.N, nb = g.nb, bpp = BPP > 0 ? BPP : a.bpp;
  const int ntiles = N / kTileRows;
  const int G = gridDim.x;  // a multiple of 8: block b runs on XCD b % 8
  const int vb = static_cast<int>(blockIdx.x);
  const int v = (vb & 7) * (G >> 3) + (vb >> 3);
  int nact;
  int4 hpre = make_int4(0, 0, 0, 0);
  OneTokenRoute r1;          // one-token routing
  bool r1_publish = false;   // held by wave 0 (one token, bf16 logits)
  if constexpr (kRoute) {
    static_assert(kGated && !kSpec, "the routing prologue is a gate_up variant for regular scale codes");
    // One token with bf16 logits: wave 0 selects it and writes the task
    // headers (route_one_token_select).  The plan for the later launches is
    // written by the work-groups past the items (the launch adds 8), so no
    // streaming wave issues a store before its epilogue (stores share the
    // load counter and would hold up the ring's first waits); without such
    // work-groups, by all after their items.
    // Otherwise wave w selects tokens w, w + P, ...
    // (topk_token, as the router's own small top-k launch does) and wave 0
    // then builds the plan.  Either way the plan's task headers and slot ->
    // token map land in LDS; every work-group computes the same plan and
    // the last one, which holds no item, also writes it (and idx, w) for the
    // later launches; only it computes the routing weights.
    int32_t* r_idx = reinterpret_cast<int32_t*>(red);
    float* r_w = reinterpret_cast<float*>(r_idx + kSmallTopkMaxT * kMaxTopK);
    int32_t* r_cnt = reinterpret_cast<int32_t*>(r_w + kSmallTopkMaxT * kMaxTopK);
    int32_t* r_off = r_cnt + kMaxExperts;
    int32_t* r_aidx = r_off + kMaxExperts;
    __shared__ int r_nact;
    // the plan writer of the multi-token path: the last work-group, which
    // holds no item unless the grid is capped at the resident work-groups
    const bool w0 = blockIdx.x == gridDim.x - 1;
    if (a.r_T == 1 && !a.r_fp32) {
      if (p == 0) {
        float lv[kMaxExperts / kWave];
        load_token_logits<false, kMaxExperts / kWave>(a.r_logits, 0, a.r_E, lane, lv);
        const int na = route_one_token_select_k<kMaxExperts / kWave>(lv, a.r_k, a.r_E, lane, hdr, tok, r1);
        if (lane == 0) r_nact = na;
        r1_publish = true;
      }
    } else {
      for (int t = p; t < a.r_T; t += P) {
        float lv[kMaxExperts / kWave];
        if (a.r_fp32) {
          load_token_logits<true, kMaxExperts / kWave>(a.r_logits, t, a.r_E, lane, lv);
          topk_token<kMaxExperts / kWave, false>(lv, a.r_k, a.r_variant, r_idx + t * a.r_k,
                                                 w0 ? r_w + t * a.r_k : nullptr, nullptr, lane);
        } else {
          load_token_logits<false, kMaxExperts / kWave>(a.r_logits, t, a.r_E, lane, lv);
          topk_token<kMaxExperts / kWave, true>(lv, a.r_k, a.r_variant, r_idx + t * a.r_k,
                                                w0 ? r_w + t * a.r_k : nullptr, nullptr, lane);
        }
      }
      __syncthreads();
      if (p == 0) {
        const int S = a.r_T * a.r_k;
        if (w0 && lane < S) {
          a.r_idx[lane] = r_idx[lane];
          a.r_w[lane] = r_w[lane];
        }
        const int na = plan_one_wave<kMaxExperts / kWave>(r_idx, S, a.r_k, a.r_E, w0 ? a.r_plan : PlanBufs{}, lane,
                                                          r_cnt, r_off, r_aidx, hdr, tok);
        if (lane == 0) r_nact = na;
      }
    }
    __syncthreads();
    nact = __builtin_amdgcn_readfirstlane(r_nact);
  } else {
    // The first task headers are read together with the active count (one
    // memory latency instead of two): records below max_tasks are in the
    // buffer, and those past the count are not used.
    if (static_cast<int>(threadIdx.x) < a.max_tasks)
      hpre = reinterpret_cast<const int4*>(a.tasks)[static_cast<size_t>(threadIdx.x) * (kTaskInts / 4)];
    nact = __builtin_amdgcn_readfirstlane(*a.n_active);
  }
  const int n_items = nact * ntiles;
  // Item of round r: r G + v while every work-group has one (r < kfull).
  // gate_up takes r G + vb in the last, partial round, whose items then
  // spread over the XCDs and over distinct CUs instead of filling the first
  // XCDs' ranges (two boxes, three interleaved pairs each: B=16 gate_up
  // 73.5-74.6 -> 71.3-73.0 us, B=64 148.4-153.7 -> 147.3-149.0, B=8 and 32
  // even); down keeps v there (at 64 and 32 tokens it measured 0.3-0.7 us
  // slower in block order, even at 8).
  const int kfull = n_items / G;
  auto round_item = [&](int r) { return r * G + (kGated && r >= kfull ? vb : v); };
  const int q0 = round_item(0);
  if (q0 >= n_items) {  // the whole work-group, before any further barrier
    if constexpr (kRoute)
      if (r1_publish)
        route_one_token_publish_k(r1, a.r_k, a.r_E, a.r_variant, a.r_plan, q0 - n_items, G - n_items, a.r_idx,
                                  a.r_w, lane);
    return;
  }

  if constexpr (!kRoute) {
    // Task headers: {expert | special << 8 | count << 9, offset}.  The
    // special flag is read only by the variant that branches on it.
    for (int i = threadIdx.x; i < nact; i += P * kWave) {
      const int4 h = i == static_cast<int>(threadIdx.x)
                         ? hpre
                         : reinterpret_cast<const int4*>(a.tasks)[static_cast<size_t>(i) * (kTaskInts / 4)];
      const int sp = !kSpec ? 0 : a.special ? (a.special[h.x] != 0) : 1;
      hdr[i] = make_int2(h.x | (sp << 8) | (h.z << 9), h.y);
    }
    // The next step's token ids are read while the weight stream is in
    // flight: from LDS they need no wait on the loads ahead of them (slots
    // <= kLdsSlots, checked at launch).
    if constexpr (kGated)
      for (int i = threadIdx.x; i < a.slots; i += P * kWave) tok[i] = a.perm_token[i];
    __syncthreads();
  }

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(a.wn, a.wn_bytes);
  const __amdgpu_buffer_rsrc_t rS = make_rsrc(a.ws, a.ws_bytes);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.x, a.x_bytes);
  const int lo16 = lane & 15, g16 = lane >> 4;
  const uint32_t voffA = static_cast<uint32_t>(lane) * 16, voffS = static_cast<uint32_t>(lo16) * 4;

  int qr = 1, qa = round_item(1);  // the next item and its round
  auto step_of = [&](int q, int cg) -> McStep {
    McStep s;
    s.valid = q < n_items;
    s.q = q;
    const int qq = s.valid ? q : 0;
    const int j = qq / ntiles;
    s.t = qq - j * ntiles;
    s.cg = cg;
    // LDS values are per-lane to the compiler: make the step scalar
    const int hx = __builtin_amdgcn_readfirstlane(hdr[j].x);
    s.e = hx & 0xff;
    s.sp = (hx >> 8) & 1;
    s.M = hx >> 9;
    s.off = __builtin_amdgcn_readfirstlane(hdr[j].y);
    return s;
  };
  auto next_of = [&](const McStep& s) -> McStep {
    if ((s.cg + 1) * kTok < s.M) return step_of(s.q, s.cg + 1);
    return step_of(qa, 0);
  };
  // Input rows of the B operand for this lane's column of each chunk:
  // gate_up gathers the slot's token, down reads the slot's activation row.
  // Columns past the expert's slots get -1: their B loads go past the end
  // of the buffer (zeros, no memory traffic) and their outputs are not
  // stored.
  auto rows_of = [&](const McStep& s, int (&row)[NC]) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int m = s.cg * kTok + 16 * c + lo16;
      const int slot = s.valid ? s.off + min(m, s.M - 1) : 0;
      if constexpr (kGated) row[c] = s.valid ? tok[slot] : 0;
      else row[c] = slot;
      if (s.valid && m >= s.M) row[c] = -1;
    }
  };
  auto src_of = [&](const McStep& s, const int (&row)[NC]) -> McSrc<NC> {
    McSrc<NC> r;
    const uint32_t blk0 = static_cast<uint32_t>(s.t * nb + p * bpp);
    r.a = s.valid ? static_cast<uint32_t>(s.e) * static_cast<uint32_t>(g.nib_bytes) + blk0 * 1024u : a.wn_bytes;
    r.s = s.valid ? static_cast<uint32_t>(s.e) * static_cast<uint32_t>(g.scale_bytes) +
                        static_cast<uint32_t>(g.mscale_off) + blk0 * 64u
                  : a.ws_bytes;
    r.b = s.valid ? static_cast<uint32_t>(p * bpp) * 64u : a.x_bytes;
    r.astr = s.valid ? 1024u : 0u;
    r.sstr = s.valid ? 64u : 0u;
    r.bstr = s.valid ? 64u : 0u;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      r.vb[c] = !s.valid     ? 0u
                : row[c] < 0 ? a.x_bytes
                             : static_cast<uint32_t>(row[c]) * static_cast<uint32_t>(K) * 2u + 16u * g16;
    return r;
  };

  gx_u32x4 ra[D];
  uint32_t rs[D];
  gx_u32x4 rb[D][NC];
  // kStg: this wave's staged words and the staged row of this lane's column
  gx_u32x4* const stg_w = stg + (kStageS ? p * kStgRows * kStgU4 : 0);
  int bcol = 0;
  // block blk's staged operands
  auto issue_lds = [&](int u, int blk) __attribute__((always_inline)) {
    if constexpr (kStageS) rs[u] = reinterpret_cast<const uint32_t*>(stg_w)[blk * 16 + lo16];
    if constexpr (kStageB) rb[u][0] = stg_w[(1 + bcol) * kStgU4 + blk * 4 + g16];
  };
  // lds: block blk belongs to the staged step (the next step's blocks read
  // their staged operands once that step is staged)
  auto issue = [&](int u, const McSrc<NC>& s, int blk, bool lds) __attribute__((always_inline)) {
    const uint32_t ub = static_cast<uint32_t>(blk);
    ra[u] = __builtin_amdgcn_raw_buffer_load_b128(rA, voffA, s.a + ub * s.astr, kNT);
    if constexpr (kStageS) {
      if (lds) issue_lds(u, blk);
    } else {
      rs[u] = __builtin_amdgcn_raw_buffer_load_b32(rS, voffS, s.s + ub * s.sstr, kNT);
    }
    if constexpr (!kStageB) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        rb[u][c] = __builtin_amdgcn_raw_buffer_load_b128(rB, s.vb[c], s.b + ub * s.bstr, 0);
    }
  };
  // The step's part of its scales (and of the input rows of its columns 0
  // and 1, which lanes 0 and 1 hold), loaded into registers (stage_load)
  // and written to this wave's words (stage_store).  A missing step reads
  // past the buffers: zeros, never used.
  constexpr int kStgLd = kStgU4 / kWave;
  struct Staged {
    gx_u32x4 w[kStgRows][kStageS ? kStgLd : 1];
    int bcol;
  };
  auto stage_load = [&](const McStep& s, const McSrc<NC>& src, const int (&row)[NC], Staged& st)
                        __attribute__((always_inline)) {
    if constexpr (kStageS) {
      const uint32_t part = static_cast<uint32_t>(p * bpp) * 64u;
#pragma unroll
      for (int q = 0; q < kStgLd; ++q) {
        const uint32_t o = static_cast<uint32_t>(q * kWave + lane) * 16u;
        st.w[0][q] = __builtin_amdgcn_raw_buffer_load_b128(rS, o, src.s, kNT);
        if constexpr (kStageB) {
          const int r0 = __builtin_amdgcn_readlane(row[0], 0), r1 = __builtin_amdgcn_readlane(row[0], 1);
          // a row past the columns (r < 0) reads past the buffer: zeros
          const uint32_t x0 =
              !s.valid || r0 < 0 ? a.x_bytes : static_cast<uint32_t>(r0) * static_cast<uint32_t>(K) * 2u + part;
          const uint32_t x1 =
              !s.valid || r1 < 0 ? a.x_bytes : static_cast<uint32_t>(r1) * static_cast<uint32_t>(K) * 2u + part;
          st.w[1][q] = __builtin_amdgcn_raw_buffer_load_b128(rB, o, x0, 0);
          st.w[2][q] = __builtin_amdgcn_raw_buffer_load_b128(rB, o, x1, 0);
        }
      }
      st.bcol = kStageB && s.valid ? min(lo16, min(s.M - s.cg * kTok, 2) - 1) : 0;
    }
  };
  auto stage_store = [&](const Staged& st) __attribute__((always_inline)) {
    if constexpr (kStageS) {
#pragma unroll
      for (int k = 0; k < kStgRows; ++k)
#pragma unroll
        for (int q = 0; q < kStgLd; ++q) stg_w[k * kStgU4 + q * kWave + lane] = st.w[k][q];
      bcol = st.bcol;
    }
  };

  McStep cur = step_of(q0, 0);
  McSrc<NC> cs;
  Staged st0;
  {
    int crow[NC];
    rows_of(cur, crow);
    cs = src_of(cur, crow);
    stage_load(cur, cs, crow, st0);  // ahead of the weights: the waits below then skip their loads
  }
  // the same load order as the steady state, so the waits for the first
  // step's blocks are as shallow as for every later step
#pragma unroll
  for (int u = 0; u < D; ++u) {
    issue(u, cs, u, false);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (kStageS) {
    stage_store(st0);
#pragma unroll
    for (int u = 0; u < D; ++u) issue_lds(u, u);
  }

  f32x4 acc[4][NC];
  for (;;) {
    const McStep nxt = next_of(cur);
    int nrow[NC];
    rows_of(nxt, nrow);  // token ids land long before the last group needs them
    // this step's bias for the fragments this wave finishes (issued ahead
    // of its uses in the epilogue): fragment f = j P + p, sub-tile f % 4
    uint2 braw[kOwn];
    {
      const int n0 = cur.t * kTileRows + 4 * g16;
#pragma unroll
      for (int j = 0; j < kOwn; ++j) {
        const int i = (j * P + p) & 3;
        braw[j] = a.bias ? *reinterpret_cast<const uint2*>(a.bias + static_cast<size_t>(cur.e) * N + n0 + 16 * i)
                         : make_uint2(0u, 0u);
      }
    }
    const int ncl = NC == 1 ? 1 : min(NC, (cur.M - cur.cg * kTok + 15) >> 4);  // chunks with a live column
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const McSrc<NC> ns = src_of(nxt, nrow);
    Staged stn;  // the next step's staged operands

    // The blocks of this step; the branch on the expert's special-code flag
    // is taken once per step, so the block loop itself has no branches.
    auto run = [&](auto SPC) __attribute__((always_inline)) {
      constexpr bool kSp = decltype(SPC)::value;
      auto consume = [&](int u) __attribute__((always_inline)) {
        const uint32_t sc = rs[u];
        gx_bf16x8 av[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t code = (sc >> (8 * i)) & 0xffu;
          if constexpr (kSp) av[i] = decode8_bf16_special(ra[u][i], code);
          else av[i] = decode8_bf16(ra[u][i], __uint_as_float(code << 23));
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (NC == 1 || c < ncl) {
            const gx_bf16x8 bv = __builtin_bit_cast(gx_bf16x8, rb[u][c]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv, acc[i][c], 0, 0, 0);
          }
        }
      };
      if constexpr (BPP > 0) {
        // block i refills its slot with block i + D, of the next step past the end
#pragma unroll
        for (int i = 0; i < BPP; ++i) {
          consume(i % D);
          if (i + D < BPP) issue(i % D, cs, i + D, true);
          else issue(i % D, ns, i + D - BPP, false);
          if (kStg == 1 && i == BPP / 2) stage_load(nxt, ns, nrow, stn);
          __builtin_amdgcn_sched_barrier(0);  // keep the ring order: one block decoded at a time
        }
      } else {
        for (int i0 = 0; i0 < bpp - D; i0 += D) {
#pragma unroll
          for (int u = 0; u < D; ++u) {
            consume(u);
            issue(u, cs, i0 + u + D, true);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        // last group: its refills are the next step's first D blocks
#pragma unroll
        for (int u = 0; u < D; ++u) {
          consume(u);
          issue(u, ns, u, false);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    if constexpr (kSpec) {
      if (cur.sp) run(std::true_type{});
      else run(std::false_type{});
    } else {
      run(std::false_type{});
    }
    if constexpr (kStg == 1) {
      // every LDS read of this step is issued: the next step's operands
      // replace them, and its first blocks (already in flight) read theirs
      stage_store(stn);
#pragma unroll
      for (int u = 0; u < D; ++u) issue_lds(u, u);
    }

    // Epilogue: fragment (i, c) of lane l is rows t*64 + 16 i + 4 (l/16) + r,
    // r = 0..3, of the step's column 16 c + l % 16.
    auto emit = [&](int i, int c, const uint2 bb, const f32x4& sum) __attribute__((always_inline)) {
      const int m = cur.cg * kTok + 16 * c + lo16;
      if (m >= cur.M) return;
      const size_t slot = static_cast<size_t>(cur.off) + m;
      const int n = cur.t * kTileRows + 16 * i + 4 * g16;
      uint16_t y[4];
      y[0] = f32_to_bf16(sum[0] + bf16_to_f32(static_cast<uint16_t>(bb.x)));
      y[1] = f32_to_bf16(sum[1] + bf16_to_f32(static_cast<uint16_t>(bb.x >> 16)));
      y[2] = f32_to_bf16(sum[2] + bf16_to_f32(static_cast<uint16_t>(bb.y)));
      y[3] = f32_to_bf16(sum[3] + bf16_to_f32(static_cast<uint16_t>(bb.y >> 16)));
      if constexpr (kGated) {
        // rows n, n+2 are gate (even), n+1, n+3 up (odd)
        const uint16_t a0 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[0]), bf16_to_f32(y[1]), a.alpha, a.limit));
        const uint16_t a1 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[2]), bf16_to_f32(y[3]), a.alpha, a.limit));
        *reinterpret_cast<uint32_t*>(a.out + slot * (N / 2) + n / 2) = a0 | (static_cast<uint32_t>(a1) << 16);
        if (a.gate_up)
          *reinterpret_cast<uint2*>(a.gate_up + slot * N + n) =
              make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
      } else {
        *reinterpret_cast<uint2*>(a.out + slot * N + n) =
            make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
      }
    };
    if constexpr (P == 1) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (NC == 1 || c < ncl)
#pragma unroll
          for (int i = 0; i < 4; ++i) emit(i, c, braw[4 * c + i], acc[i][c]);
    } else {
      // Partial sums through LDS; fragment f = 4 c + i is finished by wave
      // f % P, adding the parts in order.  One buffer (half the LDS of two,
      // so two 6-wave work-groups fit a CU): a second LDS-only barrier keeps
      // the next step's writes behind this step's reads.
      f32x4* rb0 = red;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) rb0[(p * kFr + 4 * c + i) * kWave + lane] = acc[i][c];
      lds_barrier();
#pragma unroll
      for (int j = 0; j < kOwn; ++j) {
        const int f = j * P + p;
        if (f < kFr && (f >> 2) < ncl) {
          f32x4 sum = rb0[f * kWave + lane];
#pragma unroll
          for (int pp = 1; pp < P; ++pp) sum = sum + rb0[(pp * kFr + f) * kWave + lane];
          emit(f & 3, f >> 2, braw[j], sum);
        }
      }
      if (nxt.valid) lds_barrier();  // work-group uniform
    }
    if (!nxt.valid) break;
    if constexpr (kStg == 2) {
      Staged sn;
      stage_load(nxt, ns, nrow, sn);
      stage_store(sn);
#pragma unroll
      for (int u = 0; u < D; ++u) issue_lds(u, u);
    }
    if (nxt.cg == 0) qa = round_item(++qr);  // nxt starts item qa
    cur = nxt;
    cs = ns;
  }
  // a grid capped at the resident work-groups may leave none idle: then
  // every work-group writes its share of the one-token plan here
  if constexpr (kRoute)
    if (r1_publish && G <= n_items)
      route_one_token_publish_k(r1, a.r_k, a.r_E, a.r_variant, a.r_plan, v, G, a.r_idx, a.r_w, lane);
}

// Per-expert flag: does the slot-order scale region hold code 0 or 255?
__global__ void special_scan_kernel(const uint8_t* __restrict__ ws, TiledGeom g, int E, int32_t* __restrict__ flags) {
  const size_t per = static_cast<size_t>(g.N) * g.nb / 16;  // 16-byte words per expert (N*nb is a multiple of 64)
  const size_t total = per * E;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t e = q / per, w = q % per;
    const uint4 v = reinterpret_cast<const uint4*>(ws + e * g.scale_bytes + g.mscale_off)[w];
    if (has_special_code(v.x, 0xffffffffu) || has_special_code(v.y, 0xffffffffu) ||
        has_special_code(v.z, 0xffffffffu) || has_special_code(v.w, 0xffffffffu))
      atomicOr(&flags[e], 1);
  }
}

constexpr int kDownOnePerCuSlots = 64;

template <bool kGated, int P, int D, int NC, bool kSpec, int BPP, bool kRoute = false, int kStg = 0>
hipError_t launch_mc_t(const McParams& p, int max_items, int num_cus, hipStream_t s, const KernelTimer& timer) {
  static const int per_cu = [] {  // resident work-groups per CU (a property of the kernel)
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, mc_stream_kernel<kGated, P, D, NC, kSpec, BPP, kRoute, kStg>,
                                                     P * kWave, 0) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  const int cus = num_cus > 0 ? num_cus : 256;
  const long resident = static_cast<long>(per_cu) * cus;
  long grid = max_items < resident ? max_items : resident;
  // The down product from kDownOnePerCuSlots slots on: one work-group per CU
  // (each of its waves on a SIMD of its own, fewer streams in flight).
  // Measured (GPT-OSS-120B, P=3, D=10, five resident per CU, per-dispatch
  // events): down at B=64 74.6-75.1 against 76.6-77.0 us, B=32 56.6-56.8
  // against 57.9-58.3, B=16 37.9-38.1 against 38.3-38.4 (four runs, two
  // boxes); B=48 even; at B=8 (32 slots) slower, 24.6 against 21.2.  Grids
  // of 512, 640 and 768 work-groups were no faster, 384 slower (88 us at
  // B=64); gate_up with one per CU was slower (150.5 against 147.5 us).
  if constexpr (!kGated)
    if (p.slots >= kDownOnePerCuSlots && grid > cus) grid = cus;
  grid = (grid + 7) & ~7L;  // a multiple of 8 for the XCD-grouped block order
  if constexpr (kRoute) grid += 8;  // work-groups past the items: they write the one-token plan
  McParams q = p;
  q.bpp = p.g.nb / P;
  gx_launch(mc_stream_kernel<kGated, P, D, NC, kSpec, BPP, kRoute, kStg>, dim3(static_cast<unsigned>(grid)),
            dim3(P * kWave), 0, s, timer, q);
  return hipGetLastError();
}

// The compiled launch shapes: (waves per work-group = K-parts, ring depth in
// blocks, 16-token chunks per step).  GPT-OSS (K = 2880, 90 blocks per row)
// runs straight-line steps of 90 / P blocks; other K take the generic block
// loop (P = 1, D dividing K / 32).
constexpr int kNbGptOss = 90;
#define GX_MC_SHAPES(X) \
  X(6, 15, 1)           \
  X(6, 5, 1)            \
  X(3, 10, 1)           \
  X(3, 15, 1)           \
  X(3, 5, 1)            \
  X(2, 9, 1)            \
  X(2, 15, 1)           \
  X(1, 9, 1)            \
  X(5, 9, 1)            \
  X(5, 18, 1)           \
  X(9, 10, 1)           \
  X(2, 9, 2)
#define GX_MC_GENERIC(X) \
  X(1, 4, 1)             \
  X(1, 3, 1)             \
  X(1, 2, 1)             \
  X(1, 1, 1)

bool shape_compiled(int nb, int P, int D, int NC) {
#define GX_MC_IS(p_, d_, nc_) \
  if (nb == kNbGptOss && P == p_ && D == d_ && NC == nc_) return true;
  GX_MC_SHAPES(GX_MC_IS)
#undef GX_MC_IS
#define GX_MC_IS(p_, d_, nc_) \
  if (P == p_ && D == d_ && NC == nc_ && nb % D == 0) return true;
  GX_MC_GENERIC(GX_MC_IS)
#undef GX_MC_IS
  return false;
}

template <bool kGated>
hipError_t launch_mc_shape(const McParams& p, int P, int D, int NC, int max_items, int num_cus, hipStream_t s,
                           const KernelTimer& timer) {
  if (p.g.nb == kNbGptOss) {
#define GX_MC_GO(p_, d_, nc_) \
  if (P == p_ && D == d_ && NC == nc_)  \
    return launch_mc_t<kGated, p_, d_, nc_, false, kNbGptOss / p_, false, 1>(p, max_items, num_cus, s, timer);
    GX_MC_SHAPES(GX_MC_GO)
#undef GX_MC_GO
  }
#define GX_MC_GO(p_, d_, nc_) \
  if (P == p_ && D == d_ && NC == nc_)  \
    return launch_mc_t<kGated, p_, d_, nc_, false, 0>(p, max_items, num_cus, s, timer);
  GX_MC_GENERIC(GX_MC_GO)
#undef GX_MC_GO
  return hipErrorInvalidValue;
}

// Shapes compiled with the routing prologue (used for one token): pick_shape's
// choice and the alternatives the tuning override may select.
#define GX_MC_ROUTE_SHAPES(X) \
  X(3, 5)                     \
  X(3, 10)                    \
  X(3, 15)                    \
  X(2, 9)                     \
  X(6, 5)                     \
  X(6, 15)                    \
  X(5, 9)                     \
  X(5, 18)                    \
  X(9, 10)

bool route_shape(int nb, int P, int D, int NC) {
  if (NC != 1) return false;
  if (nb == kNbGptOss) {
#define GX_MC_IS(p_, d_) \
  if (P == p_ && D == d_) return true;
    GX_MC_ROUTE_SHAPES(GX_MC_IS)
#undef GX_MC_IS
    return false;
  }
  return P == 1 && D >= 1 && D <= 4 && nb % D == 0;
}

hipError_t launch_mc_route(const McParams& p, int P, int D, int max_items, int num_cus, hipStream_t s,
                           const KernelTimer& timer) {
  if (p.g.nb == kNbGptOss) {
    // the default shape with staged operands (at most 2 tokens: 2 slots per expert)
    if (P == 3 && D == 5 && p.r_T <= 2)
      return launch_mc_t<true, 3, 5, 1, false, 30, true, 2>(p, max_items, num_cus, s, timer);
#define GX_MC_GO(p_, d_) \
  if (P == p_ && D == d_)                                                                                 \
    return launch_mc_t<true, p_, d_, 1, false, kNbGptOss / p_, true, 1>(p, max_items, num_cus, s, timer);
    GX_MC_ROUTE_SHAPES(GX_MC_GO)
#undef GX_MC_GO
  }
  if (P == 1 && D == 4) return launch_mc_t<true, 1, 4, 1, false, 0, true>(p, max_items, num_cus, s, timer);
  if (P == 1 && D == 3) return launch_mc_t<true, 1, 3, 1, false, 0, true>(p, max_items, num_cus, s, timer);
  if (P == 1 && D == 2) return launch_mc_t<true, 1, 2, 1, false, 0, true>(p, max_items, num_cus, s, timer);
  if (P == 1 && D == 1) return launch_mc_t<true, 1, 1, 1, false, 0, true>(p, max_items, num_cus, s, timer);
  return hipErrorInvalidValue;
}

// Default shape for nb blocks and S routed slots, measured on MI355X at the
// GPT-OSS-120B shape (graph-replayed steps at 1..64 tokens, 12 compiled
// shapes; most differ by a few percent): three K-parts with a 5-block ring
// up to 2 tokens and at 8, two parts with a 9-block ring for down at 4,
// three parts with a 10-block ring otherwise and from 16 tokens (1-2 % ahead of six parts with each
// wave's whole 15-block part in flight, in repeated runs at 16, 32 and 64).
// The same shape serves both products, except the down product of one token
// (k x 45 items, one per work-group), which takes the 10-block ring (B=1:
// 24.0 against 24.5 us per layer in three paired runs; from two tokens the
// shared shape is ahead).  At 9-16 slots (after the staged scales, three
// passes): gate_up takes three parts with the 10-block ring (16 slots: 26.0
// against 29.3 us; 12 slots: even), and so does down up to 12 slots (11.4
// against 12.9 us), while down at 13-16 slots keeps two parts with the
// 9-block ring (13.8 against 16.1 us).  gate_up keeps the 10-block ring up
// to 24 slots (20 slots: 31.0 against 35.8 us, 24: 34.4 against 38.5) and
// takes the 5-block ring only at 25-32 (28 slots: 38.9 against 39.9 us,
// 32: 40.4 against 41.6).
void pick_shape(int nb, int S, bool gated, int T, int& P, int& D, int& NC) {
  NC = 1;
  if (nb == kNbGptOss) {
    const bool ring5 = gated ? S <= 8 || (S > 24 && S <= 32) : S <= 8 || (S > 16 && S <= 32);
    if (!gated && T == 1) { P = 3; D = 10; }
    else if (ring5) { P = 3; D = 5; }
    else if (!gated && S > 12 && S <= 16) { P = 2; D = 9; }
    else { P = 3; D = 10; }
    return;
  }
  P = 1;
  D = nb % 4 == 0 ? 4 : nb % 3 == 0 ? 3 : nb % 2 == 0 ? 2 : 1;
}

hipError_t launch_mc(const ExpertArgs& a, bool gated, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g = gated ? tiled_geom(2 * a.I, a.H) : tiled_geom(a.H, a.I);
  McParams p{};
  p.x = gated ? a.x : a.act;
  p.wn = gated ? a.w1n : a.w2n;
  p.ws = gated ? a.w1s : a.w2s;
  p.bias = gated ? a.b1 : a.b2;
  p.tasks = a.plan.tasks;
  p.n_active = a.plan.n_active;
  p.perm_token = a.plan.perm_token;
  p.special = gated ? a.special1 : a.special2;
  p.out = gated ? a.act : a.y;
  p.gate_up = gated ? a.gate_up : nullptr;
  p.alpha = a.alpha;
  p.limit = a.limit;
  p.slots = a.T * a.k;
  p.max_tasks = a.max_active;
  p.g = g;
  if (p.slots > kLdsSlots) return hipErrorInvalidValue;  // decode_mc_supported() is false
  const size_t wn_bytes = g.nib_bytes * a.E, ws_bytes = g.scale_bytes * a.E;
  const size_t x_bytes = static_cast<size_t>(gated ? a.T : a.T * a.k) * g.K * 2;
  constexpr size_t kMaxBuf = 0xffff0000u;  // offsets + lane terms stay below 2^32
  if (wn_bytes > kMaxBuf || ws_bytes > kMaxBuf || x_bytes > kMaxBuf) return hipErrorInvalidValue;
  p.wn_bytes = static_cast<uint32_t>(wn_bytes);
  p.ws_bytes = static_cast<uint32_t>(ws_bytes);
  p.x_bytes = static_cast<uint32_t>(x_bytes);
  int P, D, NC;
  pick_shape(g.nb, a.T * a.k, gated, a.T, P, D, NC);
  const int* ov = a.mc_shape + (gated ? 0 : 3);
  if (ov[0] > 0 && shape_compiled(g.nb, ov[0], ov[1], ov[2])) {
    P = ov[0];
    D = ov[1];
    NC = ov[2];
  }
  const int max_items = a.max_active * (g.N / kTileRows);
  if (gated && a.route_logits != nullptr) {  // routing in the prologue (decode_route_in_w1 said yes)
    if (a.special_any1 || NC != 1 || a.T > kSmallTopkMaxT || !route_shape(g.nb, P, D, NC))
      return hipErrorInvalidValue;
    p.r_logits = a.route_logits;
    p.r_fp32 = a.route_fp32;
    p.r_T = a.T;
    p.r_E = a.E;
    p.r_k = a.k;
    p.r_variant = a.route_variant;
    p.r_idx = a.route_idx;
    p.r_w = a.route_w;
    p.r_plan = a.plan;
    return launch_mc_route(p, P, D, max_items, a.num_cus, s, a.timer);
  }
  if (gated ? a.special_any1 : a.special_any2)  // weights with e8m0 code 0 or 255: the checking variant
    return gated ? launch_mc_t<true, 1, 1, 1, true, 0>(p, max_items, a.num_cus, s, a.timer)
                 : launch_mc_t<false, 1, 1, 1, true, 0>(p, max_items, a.num_cus, s, a.timer);
  // down at one or two tokens whose experts are distinct (so at most 2 slots
  // per expert: the staged rows cover columns 0 and 1 only): the default
  // shapes with staged operands.  Caller-given indices may repeat an expert
  // within a token and take the per-lane B loads.
  if (!gated && a.T <= 2 && a.distinct_slots && g.nb == kNbGptOss && NC == 1 && P == 3) {
    if (D == 10) return launch_mc_t<false, 3, 10, 1, false, 30, false, 2>(p, max_items, a.num_cus, s, a.timer);
    if (D == 5) return launch_mc_t<false, 3, 5, 1, false, 30, false, 2>(p, max_items, a.num_cus, s, a.timer);
  }
  return gated ? launch_mc_shape<true>(p, P, D, NC, max_items, a.num_cus, s, a.timer)
               : launch_mc_shape<false>(p, P, D, NC, max_items, a.num_cus, s, a.timer);
}

}  // namespace

hipError_t launch_w1_mc(const ExpertArgs& a, hipStream_t s) { return launch_mc(a, true, s); }
hipError_t launch_w2_mc(const ExpertArgs& a, hipStream_t s) { return launch_mc(a, false, s); }

bool decode_shape_valid(int nb, int P, int D, int NC) { return shape_compiled(nb, P, D, NC); }

// Measured on MI355X (GPT-OSS-120B, graph-replayed steps, packed-key
// selection): up to two tokens the prologue's top-k and plan cost less than
// the launch they replace (B=2: 35.1 vs 36.2 us per layer); from four the
// waves' serial selections before the first weight load cost more (B=4:
// 57.8-58.5 vs 57.5, B=8: 79.7 vs 76.8 us).
constexpr int kRouteInW1MaxT = 2;

bool decode_route_in_w1(int T, int k, int E, int H, int I, const int* mc_shape) {
  if (T < 1 || T > kRouteInW1MaxT || T * k > kWave || E > kMaxExperts) return false;
  const TiledGeom g = tiled_geom(2 * I, H);
  int P, D, NC;
  pick_shape(g.nb, T * k, true, T, P, D, NC);
  if (mc_shape && mc_shape[0] > 0 && shape_compiled(g.nb, mc_shape[0], mc_shape[1], mc_shape[2])) {
    P = mc_shape[0];
    D = mc_shape[1];
    NC = mc_shape[2];
  }
  return route_shape(g.nb, P, D, NC);
}

bool decode_mc_supported(int T, int k, int E, int H, int I) {
  const TiledGeom g1 = tiled_geom(2 * I, H), g2 = tiled_geom(H, I);
  constexpr size_t kMaxBuf = 0xffff0000u;
  return T * k <= kLdsSlots && g1.nib_bytes * E <= kMaxBuf && g1.scale_bytes * E <= kMaxBuf &&
         g2.nib_bytes * E <= kMaxBuf && g2.scale_bytes * E <= kMaxBuf &&
         static_cast<size_t>(T) * k * I * 2 <= kMaxBuf && static_cast<size_t>(T) * H * 2 <= kMaxBuf;
}

hipError_t launch_special_scan(const uint8_t* ws, int N, int K, int E, int32_t* flags, hipStream_t s) {
  const TiledGeom g = tiled_geom(N, K);
  hipError_t err = hipMemsetAsync(flags, 0, sizeof(int32_t) * E, s);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(special_scan_kernel, dim3(1024), dim3(256), 0, s, ws, g, E, flags);
  return hipGetLastError();
}

}  // namespace gxmoe
