// moe_experts.hip -- decode-path MXFP4 expert products on gfx950.
//
// Replaces fused_mxfp4_gemv_forward / _multi_forward (fused_mxfp4_gemv.cu:
// 76-310), the bias kernels (moe_layer.cu:171-194, 442-473), swiglu_forward
// (swiglu.cu:117-211), moe_combine_forward (moe_combine.cu:31-117) and the
// per-batch host loop of moe_layer.cu:1316-1487 with three launches:
//
//   expert_stream_kernel<gated>   gate_up: + bias, bf16 gate/up, clamped
//                                 SwiGLU, bf16 activations
//   expert_stream_kernel<!gated>  down: + bias, bf16 expert outputs
//   combine8_kernel               out = bf16(sum_k w_k * y_k + residual)
//
// The stream kernel is persistent: at most two work-groups per CU walk the
// (active expert, tile group) items of the routing plan's task records, so
// the weights stream without a gap between items (see expert_stream_kernel).
//
// Memory layout (tiled MXFP4, built once by pack_nib/pack_scale; TiledGeom
// in moe_kernels.h): for each expert, each 64-row tile holds nb = K/32 blocks
// of one KiB; lane l's row block is the four dwords tiled_dword(l, 0..3) of
// it, so one wave's loads of block b cover one contiguous KiB.  Scales of
// each (tile, part, lane) are one contiguous group of `spad` bytes (bpp used).
//
// Arithmetic (the canonical expert dot): lane = row, wave = K-part; each
// lane runs one ascending fmaf chain over its part; the P part sums are added
// in part order; + bias; bf16.  The token activations are staged in LDS as
// fp32 and read as wave-wide broadcasts.
#include <float.h>

#include <type_traits>

#include "moe_device.h"
#include "moe_kernels.h"

namespace gxmoe {

TiledGeom tiled_geom(int N, int K) {
  TiledGeom g;
  g.N = N;
  g.K = K;
  g.nb = K / 32;
  g.parts = dot_parts(K);
  g.bpp = g.nb / g.parts;
  g.spad = (g.bpp + 3) & ~3;
  g.nib_bytes = static_cast<size_t>(N) * K / 2;
  g.mscale_off = static_cast<size_t>(N / kTileRows) * g.parts * kTileRows * g.spad;
  g.scale_bytes = g.mscale_off + static_cast<size_t>(N) * g.nb;
  return g;
}

namespace {

constexpr int kMaxBpp = 16;  // blocks per K-part handled by the unrolled loop

// LDS row length (elements) of one staged K-part: the exact part length for
// a compile-time block count, else room for kMaxBpp blocks; at least R*64 so
// the rows can hold the part sums.
template <int BPP, int R>
struct PartLen {
  static constexpr int kLen = (BPP ? BPP : kMaxBpp) * 32;
  static constexpr int kValue = kLen > R * kTileRows ? kLen : R * kTileRows;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per work-group LDS: each wave's staged activations (fp32, TC token rows of
// its K-part, which after the wave's dot hold its part sums), the packed
// header of every active-expert task record ({expert | count << 8, offset})
// and, for small batches, the slot -> token map.  Kept under a third of the
// CU's 160 KiB, so the compiler does not budget for fewer resident waves
// (which also sets the VGPR allocation it reports to the dispatcher).
template <int PK, int TC, int kTok>
struct StreamSmem {
  float x[kMaxParts][TC][PK];
  int2 hdr[kMaxExperts];
  int32_t tok[kTok];
};

// Activations of one token chunk for one wave's K-part: lane l moves 16-byte
// pieces l, l + 64, ... of the chunk's rows, the last valid piece standing in
// for those past the end, so every lane issues the same loads (the wait
// counts stay static).
template <int TC, int PK>
struct XSlots {
  static constexpr int kN = (TC * PK / 8 + kWave - 1) / kWave;
  uint4 v[kN];
};

// Chunk row m and piece c of slot i of this lane, for mc rows of nchunk pieces.
template <int TC>
__device__ __forceinline__ void slot_of(int i, int lane, int mc, int nchunk, int& m, int& c) {
  int q = lane + i * kWave;
  const int last = mc * nchunk - 1;
  q = q > last ? last : q;
  m = 0;
#pragma unroll
  for (int t = 1; t < TC; ++t) m += (q >= t * nchunk) ? 1 : 0;
  c = q - m * nchunk;
}

// Widen the loaded activations to fp32 into this wave's LDS rows and make
// them visible to the whole wave.  Lanes past the end write the clamped last
// piece again (same data, same place), so the stores need no branch.
template <int TC, int PK>
__device__ __forceinline__ void store_x(const XSlots<TC, PK>& xl, float (*sx)[PK], int mc, int nchunk, int lane) {
#pragma unroll
  for (int i = 0; i < XSlots<TC, PK>::kN; ++i) {
    int m, c;
    slot_of<TC>(i, lane, mc, nchunk, m, c);
    const uint4 v = xl.v[i];
    f32x4 lo, hi;
    lo[0] = __uint_as_float(v.x << 16); lo[1] = __uint_as_float(v.x & 0xffff0000u);
    lo[2] = __uint_as_float(v.y << 16); lo[3] = __uint_as_float(v.y & 0xffff0000u);
    hi[0] = __uint_as_float(v.z << 16); hi[1] = __uint_as_float(v.z & 0xffff0000u);
    hi[2] = __uint_as_float(v.w << 16); hi[3] = __uint_as_float(v.w & 0xffff0000u);
    *reinterpret_cast<f32x4*>(&sx[m][c * 8]) = lo;
    *reinterpret_cast<f32x4*>(&sx[m][c * 8 + 4]) = hi;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct StreamParams {
  const uint16_t* x;          // input rows: normed tokens [T][K] (gate_up) or activations [S][K] (down)
  const uint8_t* wn;          // tiled nibbles, [E] x g.nib_bytes
  const uint8_t* ws;          // tiled scales, [E] x g.scale_bytes
  const uint16_t* bias;       // [E][N] or null
  const int32_t* tasks;       // [max_active][kTaskInts] task records
  const int32_t* n_active;    // [1]
  const int32_t* perm_token;  // [S] token of each permuted slot (gate_up only)
  int slots;                  // S = T * top_k
  uint16_t* out;              // gate_up: SwiGLU activations [S][N/2]; down: expert outputs [S][N]
  uint16_t* gate_up;          // [S][N] bf16 trace or null (gate_up only)
  int max_active;
  float alpha, limit;
  TiledGeom g;                // [N, K] geometry
};

// One step of a work-group's stream: tile group tp (R tiles) of the j-th
// active expert, token chunk c.
struct Step {
  int valid, j, tp, c, e, off, M;
};

// The persistent expert stream.  Work-group b takes the items (j, tp) =
// b, b + G, ... of the n_active x ceil(tiles/R) item list (G = grid size) and
// each item's token chunks in order; each step applies the R tiles' weights
// to up to TC tokens.  Lane l of wave p owns row l of each tile and runs, per
// token, one ascending fmaf chain over K-part p (the canonical dot); the part
// sums are added in part order across the work-group, which then adds the
// bias and emits (gate_up: bf16 gate/up values, clamped SwiGLU on lane pairs,
// bf16 activations; down: bf16 expert outputs).
//
// Streaming: the weights of a step move through a ring of D blocks per row
// held in VGPRs; consuming block i issues block i + D, which past the end of
// the part is block i + D - part of the next step.  The next step's scales,
// activation pieces and token ids are issued during the current step, so a
// wave's loads never stop between steps; loads for a step that does not
// exist read a fixed valid location (static wait counts, no stray traffic).
template <int BPP, int R, int TC, int D, bool kGated, int kTok>
__global__ __launch_bounds__(kTileRows * kMaxParts) __attribute__((amdgpu_waves_per_eu(4)))
void expert_stream_kernel(StreamParams a) {
  constexpr int PK = PartLen<BPP, R>::kValue;
  static_assert(TC * R * kTileRows <= TC * PK, "part sums fit the staged rows");
  __shared__ __attribute__((aligned(16))) StreamSmem<PK, TC, kTok> sm;
  constexpr int kLoop = BPP ? BPP : kMaxBpp;
  constexpr int kD = D < kLoop ? D : kLoop;
  static_assert(kLoop % kD == 0, "ring depth must divide the part length");
  constexpr int kN = XSlots<TC, PK>::kN;
  const TiledGeom& g = a.g;
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bpp = BPP ? BPP : g.bpp;
  const int plen = bpp * 32, k0 = p * plen, nchunk = plen >> 3;
  const int K = g.K, N = g.N;
  const int ntiles = N / kTileRows;
  const int ntp = (ntiles + R - 1) / R;
  const int G = gridDim.x;
  const size_t tile_bytes = static_cast<size_t>(g.nb) * 1024;

  // First step straight from its task record.
  Step cur;
  cur.j = blockIdx.x / ntp;
  if (cur.j >= a.max_active) return;
  const int32_t* tk0 = a.tasks + static_cast<size_t>(cur.j) * kTaskInts;
  cur.e = tk0[0];
  if (cur.e < 0) return;
  cur.off = tk0[1];
  cur.M = tk0[2];
  cur.tp = blockIdx.x - cur.j * ntp;
  cur.c = 0;
  cur.valid = 1;

  // Task headers into LDS (issued first: their wait leaves the rest in flight).
  int4 hv = make_int4(-1, 0, 0, 0);
  if (static_cast<int>(threadIdx.x) < a.max_active)
    hv = reinterpret_cast<const int4*>(a.tasks)[static_cast<size_t>(threadIdx.x) * (kTaskInts / 4)];
  static_assert(kMaxExperts <= 256, "expert id packs into 8 bits");
  const int nact = *a.n_active;
  // Small batches stage the slot -> token map (S <= kTok) so the next step's
  // token ids are LDS reads rather than loads queued behind the weights.
  int tv = 0;
  if constexpr (kGated && kTok > 1)
    if (static_cast<int>(threadIdx.x) < a.slots) tv = a.perm_token[threadIdx.x];

  // Per-step addresses (dwords; a block is 256 of them).  An invalid step
  // points every load at fixed valid data (expert 0, tile 0, input row 0)
  // with a zero block stride.
  auto wsrc = [&](const Step& s, int r, int& stride) -> const uint32_t* {
    stride = s.valid ? 256 : 0;
    const int t = s.valid ? min(s.tp * R + r, ntiles - 1) : 0;
    const int pp = s.valid ? p : 0;
    const size_t eoff = s.valid ? static_cast<size_t>(s.e) * g.nib_bytes : 0;
    return reinterpret_cast<const uint32_t*>(a.wn + eoff + static_cast<size_t>(t) * tile_bytes) +
           static_cast<size_t>(pp) * bpp * 256 + tiled_dword(lane, 0);
  };
  auto ssrc = [&](const Step& s, int r) -> const uint32_t* {
    const int t = s.valid ? min(s.tp * R + r, ntiles - 1) : 0;
    const size_t eoff = s.valid ? static_cast<size_t>(s.e) * g.scale_bytes : 0;
    return reinterpret_cast<const uint32_t*>(a.ws + eoff +
                                             (static_cast<size_t>(t) * g.parts + p) * kTileRows * g.spad +
                                             static_cast<size_t>(lane) * g.spad);
  };
  auto load_sc = [&](const Step& s, uint32_t (&sc)[R][kMaxBpp / 4]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t* s32 = ssrc(s, r);
#pragma unroll
      for (int q = 0; q < (kLoop + 3) / 4; ++q)
        if (BPP || q * 4 < bpp) sc[r][q] = __builtin_nontemporal_load(s32 + q);
    }
  };
  // Row of activation slot i for step s; tok[i] is the slot's token (gate_up).
  auto row_of = [&](const Step& s, int i, int tok) -> const uint16_t* {
    if (!s.valid) return a.x;
    if constexpr (kGated) return a.x + static_cast<size_t>(tok) * K;
    int m, c;
    slot_of<TC>(i, lane, min(TC, s.M - s.c * TC), nchunk, m, c);
    return a.x + static_cast<size_t>(s.off + s.c * TC + m) * K;
  };
  auto issue_x = [&](const Step& s, const int (&tok)[kN], XSlots<TC, PK>& xl) {
    const int mc = s.valid ? min(TC, s.M - s.c * TC) : 1;
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      int m, c;
      slot_of<TC>(i, lane, mc, nchunk, m, c);
      xl.v[i] = *reinterpret_cast<const uint4*>(row_of(s, i, tok[i]) + k0 + c * 8);
    }
  };

  // Raw bf16 bias of row rr of step s's tile group (rows of a missing tile:
  // clamped, not emitted).  Each thread prefetches the bias of its own row
  // rt = tid % (R*64), converted only where it is used, so its wait never
  // covers the weight loads issued after it.
  auto bias_raw = [&](const Step& s, int rr) -> uint16_t {
    if (a.bias == nullptr || !s.valid) return 0;
    const int row = min(s.tp * R * kTileRows + rr, N - 1);
    return a.bias[static_cast<size_t>(s.e) * N + row];
  };
  const int rt = static_cast<int>(threadIdx.x) % (R * kTileRows);
  uint16_t braw = bias_raw(cur, rt);

  // Prologue: the first step's scales, activations and first kD blocks.
  uint32_t sc[R][kMaxBpp / 4];
  load_sc(cur, sc);
  int tok[kN];
  if constexpr (kGated) {
    // the first chunk's tokens are all inline in the record (TC <= kTaskTokens)
    static_assert(TC <= kTaskTokens, "first chunk must fit the inline tokens");
    int t0[TC];
#pragma unroll
    for (int mm = 0; mm < TC; ++mm) t0[mm] = tk0[4 + mm];
    const int mc = min(TC, cur.M);
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      int m, c;
      slot_of<TC>(i, lane, mc, nchunk, m, c);
      int t = t0[0];
#pragma unroll
      for (int mm = 1; mm < TC; ++mm) t = (m == mm) ? t0[mm] : t;
      tok[i] = t;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kN; ++i) tok[i] = 0;
  }
  XSlots<TC, PK> xl;
  issue_x(cur, tok, xl);
  u32x4 ring[R][kD];
  {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int stride;
      const uint32_t* src = wsrc(cur, r, stride);
#pragma unroll
      for (int i = 0; i < kD; ++i)
        if (BPP || i < bpp) ring[r][i] = load_row_block_nt(src + static_cast<size_t>(i) * stride);
    }
  }
  if (static_cast<int>(threadIdx.x) < kMaxExperts)
    sm.hdr[threadIdx.x] = make_int2(hv.x < 0 ? -1 : (hv.x | (hv.z << 8)), hv.y);
  // A block of 64 x parts threads holds fewer threads than records when K
  // splits into one to three parts and more experts are active: the rest of
  // the records, here (their wait also covers the weight loads above).
  for (int i = static_cast<int>(threadIdx.x + blockDim.x); i < min(a.max_active, kMaxExperts);
       i += static_cast<int>(blockDim.x)) {
    const int4 h = reinterpret_cast<const int4*>(a.tasks)[static_cast<size_t>(i) * (kTaskInts / 4)];
    sm.hdr[i] = make_int2(h.x < 0 ? -1 : (h.x | (h.z << 8)), h.y);
  }
  if constexpr (kGated && kTok > 1)
    if (static_cast<int>(threadIdx.x) < a.slots) sm.tok[threadIdx.x] = tv;
  __syncthreads();

  store_x<TC, PK>(xl, sm.x[p], min(TC, cur.M), nchunk, lane);

  auto next_of = [&](const Step& s) -> Step {
    Step n;
    if ((s.c + 1) * TC < s.M) {
      n = s;
      n.c = s.c + 1;
      return n;
    }
    const int q = (s.j * ntp + s.tp) + G;
    n.j = q / ntp;
    n.tp = q - n.j * ntp;
    n.c = 0;
    n.valid = n.j < nact;
    const int2 h = sm.hdr[n.valid ? n.j : 0];
    n.valid = n.valid && h.x >= 0;
    n.e = h.x & 0xff;
    n.M = h.x >> 8;
    n.off = h.y;
    return n;
  };

  for (;;) {
    const Step nxt = next_of(cur);
    // token ids of the next step's activation slots (gate_up): small loads
    // that land long before the next step's activations are issued
    int ntok[kN];
    if constexpr (kGated) {
      const int mc = nxt.valid ? min(TC, nxt.M - nxt.c * TC) : 1;
#pragma unroll
      for (int i = 0; i < kN; ++i) {
        int m, c;
        slot_of<TC>(i, lane, mc, nchunk, m, c);
        const int mg = nxt.c * TC + m;
        if constexpr (kTok > 1) {
          ntok[i] = nxt.valid ? sm.tok[nxt.off + mg] : 0;
        } else {
          const int32_t* tp = !nxt.valid ? a.tasks
                              : mg < kTaskTokens ? a.tasks + static_cast<size_t>(nxt.j) * kTaskInts + 4 + mg
                                                 : a.perm_token + nxt.off + mg;
          ntok[i] = *tp;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kN; ++i) ntok[i] = 0;
    }
    const int mc = __builtin_amdgcn_readfirstlane(min(TC, cur.M - cur.c * TC));
    const float(*sx)[PK] = sm.x[p];
    int cstride[R], nstride[R];
    const uint32_t* csrc[R];
    const uint32_t* nsrc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      csrc[r] = wsrc(cur, r, cstride[r]);
      nsrc[r] = wsrc(nxt, r, nstride[r]);
    }
    uint32_t nsc[R][kMaxBpp / 4];
    uint16_t nbraw = 0;
    float acc[R][TC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < TC; ++m) acc[r][m] = 0.0f;
    // wave-uniform: does any live scale byte of this step hold code 0 or 255?
    // (Then the exact special-code decode runs; otherwise the conversion alone.)
    bool sp = false;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < (kLoop + 3) / 4; ++q) {
        const int live = min(max(bpp - 4 * q, 0), 4);
        const uint32_t mask = live >= 4 ? 0xffffffffu : ((1u << (8 * live)) - 1u);
        sp = sp || has_special_code(sc[r][q], mask);
      }
    const bool wave_sp = __ballot(sp) != 0ull;
#pragma unroll
    for (int i = 0; i < kLoop; ++i) {
      if (i == kLoop - kD) {
        // the next step's bias, scales and activations go ahead of its blocks
        nbraw = bias_raw(nxt, rt);
        load_sc(nxt, nsc);
        issue_x(nxt, ntok, xl);
      }
      if (BPP || i < bpp) {
        float cs[R], scf[R];
        bool spc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t code = (sc[r][i >> 2] >> (8 * (i & 3))) & 0xffu;
          scf[r] = e8m0_to_f32(code);
          spc[r] = (code - 1u) >= 254u;
          cs[r] = spc[r] ? 1.0f : scf[r];
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          float wf[R][8];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            decode8_regular(ring[r][i % kD][d], cs[r], wf[r]);
            if (wave_sp) {
              // codes 0 and 255: exact e2m1 values times the IEEE scale
#pragma unroll
              for (int j = 0; j < 8; ++j) wf[r][j] = spc[r] ? wf[r][j] * scf[r] : wf[r][j];
            }
          }
#pragma unroll
          for (int m = 0; m < TC; ++m) {
            if (m < mc) {
              const f32x4 xa = *reinterpret_cast<const f32x4*>(&sx[m][i * 32 + d * 8]);
              const f32x4 xb = *reinterpret_cast<const f32x4*>(&sx[m][i * 32 + d * 8 + 4]);
#pragma unroll
              for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) acc[r][m] = __builtin_fmaf(xa[cc], wf[r][cc], acc[r][m]);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) acc[r][m] = __builtin_fmaf(xb[cc], wf[r][4 + cc], acc[r][m]);
              }
            }
          }
        }
      }
      // refill the ring slot just consumed
      const int ni = i + kD;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (ni < kLoop) {
          if (BPP || ni < bpp)
            ring[r][i % kD] = load_row_block_nt(csrc[r] + static_cast<size_t>(ni) * cstride[r]);
        } else {
          if (BPP || ni - kLoop < bpp)
            ring[r][i % kD] = load_row_block_nt(nsrc[r] + static_cast<size_t>(ni - kLoop) * nstride[r]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // Part sums replace this wave's activations (only this wave read them).
    float* ps = &sm.x[p][0][0];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < TC; ++m)
        if (m < mc) ps[(m * R + r) * kTileRows + lane] = acc[r][m];
    __syncthreads();
    // Reduction over the parts, spread over the whole work-group: output q is
    // token q / (R*64), row rr = q % (R*64), and a wave's lanes hold 64
    // consecutive rows (gate/up pairs on adjacent lanes).  Where R*64
    // divides the block (64 * parts threads), rr is the thread's own row rt
    // on every pass and its prefetched bias serves; otherwise (an odd part
    // count with R = 2) a pass whose rows are not rt loads their bias itself.
    // rr - rt is the same on every lane of a wave, so the branch is uniform.
    const size_t row0 = static_cast<size_t>(cur.tp) * R * kTileRows;
    for (int q = threadIdx.x; q < mc * R * kTileRows; q += blockDim.x) {
      const int m = q / (R * kTileRows), rr = q - m * (R * kTileRows);
      const bool row_ok = cur.tp * R + rr / kTileRows < ntiles;
      const uint16_t bq = rr == rt ? braw : bias_raw(cur, rr);
      float v = (&sm.x[0][0][0])[q];
      for (int pp = 1; pp < g.parts; ++pp) v = v + (&sm.x[pp][0][0])[q];
      const size_t slot = static_cast<size_t>(cur.off + cur.c * TC + m);
      const uint16_t h = f32_to_bf16(v + bf16_to_f32(bq));
      if constexpr (kGated) {
        if (row_ok && a.gate_up != nullptr) a.gate_up[slot * N + row0 + rr] = h;
        const float gu = bf16_to_f32(h);
        const float up = __shfl_xor(gu, 1, kWave);
        if (row_ok && (rr & 1) == 0)
          a.out[slot * (N / 2) + (row0 + rr) / 2] = f32_to_bf16(gx_swiglu(gu, up, a.alpha, a.limit));
      } else {
        if (row_ok) a.out[slot * N + row0 + rr] = h;
      }
    }
    if (!nxt.valid) break;
    // the next step's activations (issued before its blocks, so this wait
    // leaves those in flight) overwrite the part sums once all are read
    __syncthreads();
    store_x<TC, PK>(xl, sm.x[p], min(TC, nxt.M - nxt.c * TC), nchunk, lane);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < kMaxBpp / 4; ++q) sc[r][q] = nsc[r][q];
    braw = nbraw;
    cur = nxt;
  }
}

// out[t] = bf16(sum_k fma(w[t,k], y[gather_map[t,k]]) + residual[t]) in the
// order of moe_combine.cu:69-115; one thread per 8 outputs (16-byte loads).
__global__ __launch_bounds__(256) void combine8_kernel(const uint16_t* __restrict__ y,
                                                       const int32_t* __restrict__ gather_map,
                                                       const float* __restrict__ w,
                                                       const uint16_t* __restrict__ residual,
                                                       uint16_t* __restrict__ out, int T, int H, int k) {
  const int per_row = H >> 3;
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= T * per_row) return;
  const int t = q / per_row, c = q - t * per_row;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  // every slot's map entry and weight and the residual piece, then every
  // expert row, in flight at once: two dependent round trips in all (the
  // residual read after the rows would make a third; measured on the decode
  // steps, the two forms time the same)
  int gm[kMaxTopK];
  float ws[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    gm[s] = s < k ? gather_map[t * k + s] : -1;
    ws[s] = s < k ? w[t * k + s] : 0.0f;
  }
  uint4 rv = make_uint4(0u, 0u, 0u, 0u);
  if (residual != nullptr) rv = *reinterpret_cast<const uint4*>(residual + static_cast<size_t>(t) * H + c * 8);
  uint4 v[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s)
    v[s] = gm[s] >= 0 ? *reinterpret_cast<const uint4*>(y + static_cast<size_t>(gm[s]) * H + c * 8)
                      : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    if (gm[s] < 0) continue;  // dropped slot (or s >= k): nothing added, as the reference skips it
    const uint32_t d[4] = {v[s].x, v[s].y, v[s].z, v[s].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __builtin_fmaf(ws[s], __uint_as_float(d[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = __builtin_fmaf(ws[s], __uint_as_float(d[i] & 0xffff0000u), acc[2 * i + 1]);
    }
  }
  if (residual != nullptr) {
    const uint32_t d[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = acc[2 * i] + __uint_as_float(d[i] << 16);
      acc[2 * i + 1] = acc[2 * i + 1] + __uint_as_float(d[i] & 0xffff0000u);
    }
  }
  uint4 o;
  o.x = f32_to_bf16(acc[0]) | (static_cast<uint32_t>(f32_to_bf16(acc[1])) << 16);
  o.y = f32_to_bf16(acc[2]) | (static_cast<uint32_t>(f32_to_bf16(acc[3])) << 16);
  o.z = f32_to_bf16(acc[4]) | (static_cast<uint32_t>(f32_to_bf16(acc[5])) << 16);
  o.w = f32_to_bf16(acc[6]) | (static_cast<uint32_t>(f32_to_bf16(acc[7])) << 16);
  *reinterpret_cast<uint4*>(out + static_cast<size_t>(t) * H + c * 8) = o;
}

// Row-major [N][K/2] nibbles -> tiled: one thread per (row, block), its 16
// bytes to the four dwords tiled_dword(row % 64, g).
__global__ void pack_nib_kernel(const uint4* __restrict__ src, int N, int nb, uint32_t* __restrict__ dst) {
  const size_t total = static_cast<size_t>(N) * nb;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t row = q / nb, b = q % nb;
    const size_t tile = row / kTileRows;
    const int r = static_cast<int>(row % kTileRows);
    uint32_t* blk = dst + (tile * nb + b) * 256;
    const uint4 v = src[q];
    blk[tiled_dword(r, 0)] = v.x;
    blk[tiled_dword(r, 1)] = v.y;
    blk[tiled_dword(r, 2)] = v.z;
    blk[tiled_dword(r, 3)] = v.w;
  }
}

__global__ void pack_scale_kernel(const uint8_t* __restrict__ src, int N, TiledGeom g, uint8_t* __restrict__ dst) {
  const size_t total = static_cast<size_t>(N / kTileRows) * g.parts * kTileRows;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t lane = q % kTileRows, tp = q / kTileRows;
    const size_t p = tp % g.parts, tile = tp / g.parts;
    const size_t row = tile * kTileRows + lane;
    for (int i = 0; i < g.spad; ++i)
      dst[q * g.spad + i] = (i < g.bpp) ? src[row * g.nb + p * g.bpp + i] : 0;
  }
}

// Scales in the slot order of the nibbles: per (tile, block) 64 bytes, byte
// 4 j + i = row 64 t + 16 i + j.  One thread per output byte.
__global__ void pack_mscale_kernel(const uint8_t* __restrict__ src, int N, int nb, uint8_t* __restrict__ dst) {
  const size_t total = static_cast<size_t>(N) * nb;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t tb = q >> 6;
    const int o = static_cast<int>(q & 63);
    const size_t tile = tb / nb, b = tb % nb;
    const size_t row = tile * kTileRows + 16 * (o & 3) + (o >> 2);
    dst[q] = src[row * nb + b];
  }
}

}  // namespace

// Launch shapes.  Decode batches of up to 64 routed slots (8 tokens at
// top-4) put one row on each lane (the most work-groups for a latency-bound
// step) and stage the slot -> token map in LDS; larger batches put two
// rows on each lane (half the LDS activation traffic per FMA) and stage 4
// tokens per step.  The grid never exceeds the items a launch can have
// (max_active x tile groups) nor what stays resident on the device.
template <int BPP, int R, int TC, int D, bool kGated, int kTok>
static void launch_stream_t(const ExpertArgs& a, const TiledGeom& g, bool gated, hipStream_t s) {
  StreamParams p{};
  p.x = gated ? a.x : a.act;
  p.wn = gated ? a.w1n : a.w2n;
  p.ws = gated ? a.w1s : a.w2s;
  p.bias = gated ? a.b1 : a.b2;
  p.tasks = a.plan.tasks;
  p.n_active = a.plan.n_active;
  p.perm_token = a.plan.perm_token;
  p.slots = a.T * a.k;
  p.out = gated ? a.act : a.y;
  p.gate_up = gated ? a.gate_up : nullptr;
  p.max_active = a.max_active;
  p.alpha = a.alpha;
  p.limit = a.limit;
  p.g = g;
  const int ntp = (g.N / kTileRows + R - 1) / R;
  const int items = a.max_active * ntp;
  const int resident = 256 * 2;
  const int grid = items < resident ? items : resident;
  gx_launch(expert_stream_kernel<BPP, R, TC, D, kGated, kTok>, dim3(grid), dim3(kTileRows * g.parts), 0, s, a.timer,
            p);
}

template <int BPP, bool kGated>
static void launch_stream_b(const ExpertArgs& a, const TiledGeom& g, hipStream_t s) {
  constexpr int kLoop = BPP ? BPP : kMaxBpp;
  if (a.T * a.k <= 16) launch_stream_t<BPP, 1, 2, kLoop, kGated, 64>(a, g, kGated, s);
  else if (a.T * a.k <= 64) launch_stream_t<BPP, 1, 2, (kLoop % 5 == 0 ? 5 : kLoop), kGated, 64>(a, g, kGated, s);
  else launch_stream_t<BPP, 2, 4, (kLoop % 3 == 0 ? 3 : kLoop), kGated, 1>(a, g, kGated, s);
}

// Blocks per K-part: 15 for K = 2880 (GPT-OSS), 1 for small K; any other
// value runs the generic loop.
hipError_t launch_w1(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g1 = tiled_geom(2 * a.I, a.H);
  if (g1.bpp == 15) launch_stream_b<15, true>(a, g1, s);
  else if (g1.bpp == 1) launch_stream_b<1, true>(a, g1, s);
  else launch_stream_b<0, true>(a, g1, s);
  return hipGetLastError();
}

hipError_t launch_w2(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g2 = tiled_geom(a.H, a.I);
  if (g2.bpp == 15) launch_stream_b<15, false>(a, g2, s);
  else if (g2.bpp == 1) launch_stream_b<1, false>(a, g2, s);
  else launch_stream_b<0, false>(a, g2, s);
  return hipGetLastError();
}

hipError_t launch_combine_slots(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0) return hipSuccess;
  const int n = a.T * (a.H / 8);
  gx_launch(combine8_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a.timer, static_cast<const uint16_t*>(a.y),
            static_cast<const int32_t*>(a.plan.gather_map), a.w, a.residual, a.out, a.T, a.H, a.k);
  return hipGetLastError();
}

hipError_t launch_experts(const ExpertArgs& a, hipStream_t s) {
  hipError_t err = launch_w1(a, s);
  if (err == hipSuccess) err = launch_w2(a, s);
  if (err == hipSuccess) err = launch_combine_slots(a, s);
  return err;
}

hipError_t launch_pack_tiled(const uint8_t* packed, const uint8_t* scales, int N, int K,
                             uint8_t* tiled_nib, uint8_t* tiled_scales, hipStream_t s) {
  const TiledGeom g = tiled_geom(N, K);
  hipLaunchKernelGGL(pack_nib_kernel, dim3(1024), dim3(256), 0, s, reinterpret_cast<const uint4*>(packed), N, g.nb,
                     reinterpret_cast<uint32_t*>(tiled_nib));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(pack_scale_kernel, dim3(256), dim3(256), 0, s, scales, N, g, tiled_scales);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(pack_mscale_kernel, dim3(512), dim3(256), 0, s, scales, N, g.nb, tiled_scales + g.mscale_off);
  return hipGetLastError();
}

}  // namespace gxmoe
