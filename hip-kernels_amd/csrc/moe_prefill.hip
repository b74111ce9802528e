// moe_prefill.hip -- prefill-path (grouped) MXFP4 expert products on the
// gfx950 matrix cores.
//
// Replaces the reference's prefill expert loop (moe_layer.cu:1316-1487): per
// batch of 8 active experts, mxfp4_dequant_batched (mxfp4_dequant.cu:263-375)
// to bf16 staging, CublasHandle::gemm_bf16_lt per expert (cuda_utils.h:
// 226-308), bias_add_rows (moe_layer.cu:171-194) and swiglu_forward
// (swiglu.cu:117-211), with host synchronisations between batches.  Here one
// launch covers every expert of the routing plan:
//
//   grouped_mfma_kernel<gated>   y = x W_e^T + b_e over each expert's rows;
//                                gated: bf16 gate/up, clamped SwiGLU, bf16
//                                activations (the gate_up never reaches HBM)
//
// Work decomposition: a work-group (gate_up: four waves, two work-groups per
// CU; down: eight waves, one per CU) computes a tile of kBM = 128 permuted
// rows (one expert's tokens) x 64 weight rows per wave; each wave owns one
// 64-row tile of the tiled MXFP4 layout (the layout the decode kernels
// stream, so one copy of the weights serves both paths).  The m-tiles are counted expert by expert from the plan's offsets
// on the device (no host synchronisation); the tile sequence runs kGroupM
// m-tiles x all n-tiles at a time (a weight tile is read by the group's
// m-tiles close together, from L2) and is cut into eight equal contiguous
// ranges, one per XCD, so every XCD gets the same number of real tiles.
//
// Data movement: every operand of a 32-element K block (the tile's tokens,
// each wave's 64 nibble slots and scale dwords) reaches an LDS ring stage
// through direct global -> LDS loads, so no register waits on memory and
// every wait is an explicit vmcnt count of whole blocks.  The work-group
// synchronises every second block; each wave runs a software pipeline in
// which block kb's products issue while block kb + 1's LDS reads land and
// its A operands decode, and the refill loads are issued behind the products.
//
// Matrix-core mapping (v_mfma_f32_16x16x32_bf16, fp32 accumulation): the A
// operand of sub-tile i (rows 16i..16i+15 of the wave's tile) is dword i of
// the lane's 16-byte slot of the tiled block, decoded from MXFP4 in
// registers with the gfx950 scaled fp4 -> bf16 conversion (exact: e2m1 x
// 2^(s-127) has at most two significant bits); lane l holds row l % 16,
// elements 8(l/16)..8(l/16)+7 of the 32-element block, exactly the
// operand's K order, so one 32-element block is one K step.  The B operand
// is 16 tokens of the LDS stage.  The accumulator gives each lane four
// consecutive weight rows of one token, so the interleaved gate/up pairs
// meet in one lane.  Partial m-tiles (an expert's last rows) load and
// multiply only the 16-token fragments that hold rows.  Scale codes 0 and
// 255 (decoded as the reference's register path does) send the wave through
// an exact unpipelined pass after the main loop.
//
// Numerics: products are exact, sums are fp32 in the matrix core's order, so
// results are not bit-identical to the canonical order of the decode path;
// they differ by fp32 rounding (relative ~1e-7 of the row's magnitude) before
// the bf16 rounding.
#include <type_traits>

#include "moe_device.h"
#include "moe_kernels.h"

namespace gxmoe {
namespace {

typedef gx_bf16x8 bf16x8_t;
typedef gx_u32x4 u32x4_t;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBM = 128;  // permuted rows per work-group tile

// Work-group shape: kW waves (a 64-row weight tile each), 8 / kW work-groups
// per CU (two waves per SIMD) and the LDS ring of each.  gate_up runs four
// waves, two work-groups per CU: one work-group's SwiGLU epilogue overlaps
// the other's products.  down runs eight, one work-group per CU: its light
// epilogue leaves little to overlap, and one token stage serves 512 weight
// rows, half the direct-to-LDS loads per product (measured at 4096 tokens:
// down 0.339 against 0.351 ms with Zipf routing, 0.253 against 0.273 with
// full tiles only; gate_up with eight waves 0.649 against 0.630).
template <int kW>
struct WgShape {
  static constexpr int kPerCU = 8 / kW;
  static constexpr int kRingBytes = (kPerCU == 1 ? 152 : 76) * 1024;  // with room to spare
};
constexpr int kGateUpWaves = 4;
constexpr int kDownWaves = 8;

// One LDS ring stage holds a 32-element block of kF 16-token fragments
// (tile rows 16t..16t+15 in KiB t), each wave's 64 nibble slots (16 bytes
// each, at kWOff + 1024 w) and its 16 scale dwords (at kSOff + 64 w).  Tiles
// with fewer rows use smaller stages and so a deeper ring.
template <int kW, int kFrags>
struct Ring {
  static constexpr int kF = kFrags;
  static constexpr int kXPW = kFrags >= kW ? kFrags / kW : 1;  // token KiBs per wave (waves past kF load none)
  static constexpr int kWOff = kFrags * 1024;
  static constexpr int kSOff = kWOff + kW * 1024;
  static constexpr int kBytes = kSOff + kW * 64;
  static constexpr int kStages = WgShape<kW>::kRingBytes / kBytes;
  static constexpr int kMaxLoads = kXPW + 2;  // direct loads per wave and block: token KiBs, nibbles, scales
  static_assert(kStages >= 5 && kMaxLoads * (kStages - 2) < 64, "ring depth and vmcnt range");
};
#ifndef GX_PREFILL_GROUP_M
#define GX_PREFILL_GROUP_M 4
#endif
constexpr int kGroupM = GX_PREFILL_GROUP_M;  // m-tiles per tile group
constexpr int kExpertsPerLane = kMaxExperts / kWave;

struct GroupedParams {
  const uint16_t* x;         // [*][K] bf16 rows
  const int32_t* row_index;  // [rows] permuted position -> row of x, or null (identity)
  const int32_t* offsets;    // [E+1] first permuted position of each expert
  int E;
  const uint8_t* wn;         // tiled nibbles, g.nib_bytes per expert
  const uint8_t* ws;         // tiled scales, g.scale_bytes per expert
  TiledGeom g;               // [N][K] geometry
  const uint16_t* bias;      // [E][N] or null
  uint16_t* out;             // gated: [rows][N/2] activations; else [rows][N]
  uint16_t* gate_up;         // gated and optional: [rows][N] bf16 gate/up values
  float alpha, limit;
  int nwt;                   // work-group n-tiles: ceil(N / (64 kW))
  int* queue;                // null: one tile per work-group; else per-XCD tile counters (persistent grid)
  // block-scaled variant (grouped_mx_kernel)
  const uint8_t* xq;         // [*][K/32][64] e4m3 hi | lo parts of x's rows
  const uint32_t* xqs;       // [*][K/32] their scale codes
  uint8_t* outq;             // gated, may be null: [rows][N/64][64] the activations' parts
  uint32_t* outqs;           // [rows][N/64] their scale codes
};

struct TileCoord {
  int e;    // expert
  int m0;   // first row within the expert
  int off;  // the expert's first permuted position
  int cnt;  // the expert's rows
  int nt;   // n-tile
};

// The tile list.  Expert e's rows form M_e / kBM full m-tiles and, if
// M_e % kBM != 0, one partial m-tile (its last rows); each m-tile pairs with
// nwt n-tiles.  The full tiles come first, group by group (kGroupM m-tiles
// x nwt n-tiles, m fastest: a weight tile is read by the group's m-tiles
// close together, from L2), cut into 8 contiguous chunks, chunk x heading
// XCD x's queue.  The partial m-tiles follow, longest first: ranked by
// class (more than 64 rows, more than 32, the rest; the loop's cost follows
// the 16-token fragments it loads), by expert within a class, and dealt
// round-robin, rank i to XCD i % 8, each with its nwt n-tiles in a row
// (they share its tokens).  The shortest tiles end every queue, so the last
// work-groups to finish wait least for each other.
__device__ __forceinline__ int partial_class(int rem) {  // 0: no partial m-tile, else 1..3
  return rem == 0 ? 0 : (rem > 64 ? 1 : (rem > 32 ? 2 : 3));
}

struct TileList {
  int f[kExpertsPerLane];  // full m-tiles of the lane's experts
  int q[kExpertsPerLane];  // class of their partial m-tile, 0 if none
  int ef;                  // lane's exclusive prefix of full m-tiles
  int ep1, ep2, ep3;       // and of partial m-tiles of class 1, 2, 3
  int F, P1, P2, P3;       // totals (every lane)
};

// The offsets a lane reads for make_tile_list, all in flight at once.
__device__ __forceinline__ void load_tile_offsets(const int32_t* __restrict__ offsets, int E, int lane,
                                                  int (&o)[kExpertsPerLane + 1]) {
  const int e0 = lane * kExpertsPerLane;
#pragma unroll
  for (int i = 0; i <= kExpertsPerLane; ++i) o[i] = offsets[min(e0 + i, E)];
}

__device__ __forceinline__ TileList make_tile_list(const int (&o)[kExpertsPerLane + 1], int E, int lane) {
  TileList L;
  const int e0 = lane * kExpertsPerLane;
  int lf = 0, l1 = 0, l2 = 0, l3 = 0;
#pragma unroll
  for (int i = 0; i < kExpertsPerLane; ++i) {
    const int m = e0 + i < E ? o[i + 1] - o[i] : 0;
    L.f[i] = m / kBM;
    L.q[i] = partial_class(m % kBM);
    lf += L.f[i];
    l1 += L.q[i] == 1;
    l2 += L.q[i] == 2;
    l3 += L.q[i] == 3;
  }
  // four prefix sums in two scans of 16-bit fields (full counts < 2^16,
  // the launcher checks; partial counts <= kMaxExperts)
  int ia = lf | (l1 << 16), ib = l2 | (l3 << 16);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int ta = __shfl_up(ia, d, kWave);
    const int tb = __shfl_up(ib, d, kWave);
    if (lane >= d) {
      ia += ta;
      ib += tb;
    }
  }
  const int ta = __builtin_amdgcn_readlane(ia, kWave - 1), tb = __builtin_amdgcn_readlane(ib, kWave - 1);
  L.ef = (ia & 0xffff) - lf;
  L.ep1 = (ia >> 16) - l1;
  L.ep2 = (ib & 0xffff) - l2;
  L.ep3 = (ib >> 16) - l3;
  L.F = ta & 0xffff;
  L.P1 = ta >> 16;
  L.P2 = tb & 0xffff;
  L.P3 = tb >> 16;
  return L;
}

// Tiles in XCD x's queue; `lenF` of them full.
__device__ __forceinline__ int queue_len(const TileList& L, int nwt, int x, int& lenF) {
  const int totF = L.F * nwt;
  const int cf = (totF + 7) >> 3;
  lenF = min(max(totF - x * cf, 0), cf);
  const int P = L.P1 + L.P2 + L.P3;
  return lenF + (P > x ? ((P - x + 7) >> 3) * nwt : 0);  // ranks x, x + 8, ... below P
}

// Coordinates of entry t < queue_len of XCD x's queue.  Every lane returns
// the same values, in scalar registers (buffer descriptors, branches).
__device__ __forceinline__ void tile_at(const TileList& L, const int32_t* __restrict__ offsets, int nwt, int x, int t,
                                        int lenF, int lane, TileCoord& tc) {
  const int e0 = lane * kExpertsPerLane;
  int key, nt;  // m-tile index within its part (full) or class (partial)
  int cls = 0;  // 0: full, else the partial class
  const bool full = t < lenF;
  if (full) {
    const int v = x * ((L.F * nwt + 7) >> 3) + t;
    const int gsz = kGroupM * nwt;
    const int grp = v / gsz;
    const int r = v - grp * gsz;
    const int gm = min(kGroupM, L.F - grp * kGroupM);  // m-tiles in this group
    key = grp * kGroupM + r % gm;
    nt = r / gm;
  } else {
    const int v = t - lenF;
    const int j = v / nwt;
    nt = v - j * nwt;
    key = x + 8 * j;  // rank among the partial m-tiles
    cls = 1;
    if (key >= L.P1) {
      key -= L.P1;
      cls = 2;
      if (key >= L.P2) {
        key -= L.P2;
        cls = 3;
      }
    }
  }
  // the lane's start in its part, as a sum (a select between the fields
  // becomes a load from a selected address, which puts the list on the stack)
  const int start = L.ef * (cls == 0) + L.ep1 * (cls == 1) + L.ep2 * (cls == 2) + L.ep3 * (cls == 3);
  // the lane holding m-tile `key` and its expert
  int ee = -1, base = 0, run = start;
#pragma unroll
  for (int k = 0; k < kExpertsPerLane; ++k) {
    const int c = full ? L.f[k] : L.q[k] == cls;
    if (ee < 0 && key < run + c) {
      ee = e0 + k;
      base = run;
    }
    run += c;
  }
  // ee >= 0: key below the lane's end; key >= the lane's start: the one owner
  const unsigned long long bal = __ballot(ee >= 0 && key >= start);
  const int src = __ffsll(static_cast<long long>(bal)) - 1;
  tc.e = __builtin_amdgcn_readfirstlane(__shfl(ee, src, kWave));
  tc.off = __builtin_amdgcn_readfirstlane(offsets[tc.e]);
  tc.cnt = __builtin_amdgcn_readfirstlane(offsets[tc.e + 1]) - tc.off;
  tc.m0 = full ? __builtin_amdgcn_readfirstlane((key - __shfl(base, src, kWave)) * kBM) : (tc.cnt / kBM) * kBM;
  tc.nt = __builtin_amdgcn_readfirstlane(nt);
}

// s_waitcnt vmcnt(N), other counters untouched.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// s_waitcnt vmcnt(NB * per) for a wave issuing `per` loads per block
// (wave-uniform, 2 .. kMax).
template <int NB, int kMax>
__device__ __forceinline__ void wait_blocks(int per) {
  static_assert(kMax >= 2 && kMax <= 4, "two to four loads per block");
  if (kMax >= 4 && per >= 4) wait_vm<NB * (kMax >= 4 ? 4 : 2)>();
  else if (kMax >= 3 && per == 3) wait_vm<NB * (kMax >= 3 ? 3 : 2)>();
  else wait_vm<NB * 2>();
}

// Scale codes 0 and 255 (none in a regular checkpoint): the wave's tile
// recomputed block by block with the reference's decode of those codes,
// tokens read from global memory (no LDS, no barriers: the other waves are
// not involved).
template <bool kFull, int kFrags>
__device__ __forceinline__ void tile_special_pass(const GroupedParams& a, const TileCoord& tc,
                                                  __amdgpu_buffer_rsrc_t wrs, __amdgpu_buffer_rsrc_t srs, int wvoff,
                                                  int svoff, int nfr, int mc, int lane, f32x4_t (&acc)[4][kFrags]) {
  const int K = a.g.K, nb = a.g.nb;
  const int bj = lane & 15;
  const uint16_t* trow[kFrags];
#pragma unroll
  for (int t = 0; t < kFrags; ++t) {
    const int j = min(16 * t + bj, mc - 1);
    const int prow = a.row_index ? a.row_index[tc.off + tc.m0 + j] : tc.off + tc.m0 + j;
    trow[t] = a.x + static_cast<size_t>(prow) * K + 8 * (lane >> 4);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < kFrags; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kb = 0; kb < nb; ++kb) {
    const u32x4_t wv = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, wvoff, kb * 1024, 0));
    const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b32(srs, svoff, kb * 64, 0);
    bf16x8_t av1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) av1[i] = decode8_bf16_special(wv[i], (sv >> (8 * i)) & 0xffu);
#pragma unroll
    for (int t = 0; t < kFrags; ++t)
      if (kFull || t < nfr) {
        const bf16x8_t b1 = *reinterpret_cast<const bf16x8_t*>(trow[t] + kb * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av1[i], b1, acc[i][t], 0, 0, 0);
      }
  }
}

// Epilogue of a wave's 64-row tile.  acc[i][t][r] is row 16i + 4(l/16) + r of
// the tile for token 16t + l % 16.  Token by token: one row check (none in
// full tiles) and one output address per token, the sub-tiles' stores at
// fixed offsets from it.
template <bool kGated, bool kFull, int kFrags>
__device__ __forceinline__ void tile_epilogue(const GroupedParams& a, const TileCoord& tc, int tile, int mc, int lane,
                                              const f32x4_t (&acc)[4][kFrags]) {
  const int N = a.g.N;
  const int bj = lane & 15;
  const int nrow0 = tile * kTileRows + 4 * (lane >> 4);
  // bias rows nrow0 + 16 i .. + 3, packed bf16 pairs
  uint2 bb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) bb[i] = make_uint2(0u, 0u);
  if (a.bias) {
    const uint16_t* brow = a.bias + static_cast<size_t>(tc.e) * N + nrow0;
#pragma unroll
    for (int i = 0; i < 4; ++i) bb[i] = *reinterpret_cast<const uint2*>(brow + 16 * i);
  }
#pragma unroll
  for (int t = 0; t < kFrags; ++t) {
    const int j = 16 * t + bj;
    if (kFull || j < mc) {
      const size_t p = static_cast<size_t>(tc.off + tc.m0 + j);
      uint16_t* const orow = a.out + p * (kGated ? N / 2 : N) + (kGated ? nrow0 / 2 : nrow0);
      uint16_t* const grow = kGated && a.gate_up ? a.gate_up + p * N + nrow0 : nullptr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t y01 = pack_bf16x2(acc[i][t][0] + __uint_as_float(bb[i].x << 16),
                                         acc[i][t][1] + __uint_as_float(bb[i].x & 0xffff0000u));
        const uint32_t y23 = pack_bf16x2(acc[i][t][2] + __uint_as_float(bb[i].y << 16),
                                         acc[i][t][3] + __uint_as_float(bb[i].y & 0xffff0000u));
        if constexpr (kGated) {
          // rows n, n+2 are gate (even), n+1, n+3 up (odd)
          const float a0 = gx_swiglu(__uint_as_float(y01 << 16), __uint_as_float(y01 & 0xffff0000u), a.alpha, a.limit);
          const float a1 = gx_swiglu(__uint_as_float(y23 << 16), __uint_as_float(y23 & 0xffff0000u), a.alpha, a.limit);
          *reinterpret_cast<uint32_t*>(orow + 8 * i) = pack_bf16x2(a0, a1);
          if (grow) *reinterpret_cast<uint2*>(grow + 16 * i) = make_uint2(y01, y23);
        } else {
          *reinterpret_cast<uint2*>(orow + 16 * i) = make_uint2(y01, y23);
        }
      }
    }
  }
}

template <int kW, bool kGated, bool kFull, int kCls>
__device__ __forceinline__ void grouped_tile(const GroupedParams& a, const TileCoord& tc, uint8_t* xs, int lane,
                                             int w) {
  const TiledGeom& g = a.g;
  const int K = g.K, N = g.N, nb = g.nb;
  const int mc = min(kBM, tc.cnt - tc.m0);
  using R = Ring<kW, kCls>;
  constexpr int kFrags = R::kF, kXPerWave = R::kXPW, kStages = R::kStages, kStageBytes = R::kBytes;
  constexpr int kWOff = R::kWOff, kSOff = R::kSOff;
  const int nfr = kFull ? kFrags : (mc + 15) >> 4;  // 16-token fragments holding rows (<= kFrags)
  const int tile = tc.nt * kW + w;
  const bool active = tile < N / kTileRows;  // wave-uniform: rows past N (last n-tile) only stage tokens

  // Everything a block needs reaches LDS by direct loads (no registers wait
  // on memory): per stage, the tokens (wave w fills KiBs kXPerWave w + c;
  // lane l writes bytes 16l..16l+15 of a KiB), wave w's nibble slots and its
  // scale dwords.  Token LDS unit u = 4j + (q ^ swz(j)) holds quarter q of
  // token j, swz(j) = (j/2) % 4, so the 16 tokens of a B fragment read at
  // one quarter hit distinct banks 8 at a time.
  const uint16_t* xsrc[kXPerWave];
#pragma unroll
  for (int c = 0; c < kXPerWave; ++c) {
    const int j = 16 * (kXPerWave * w + c) + (lane >> 2);
    const int q = (lane & 3) ^ ((j >> 1) & 3);
    const int jr = j < mc ? j : 0;  // rows past the expert's end stage a valid row (their outputs are not stored)
    const int prow = a.row_index ? a.row_index[tc.off + tc.m0 + jr] : tc.off + tc.m0 + jr;
    xsrc[c] = a.x + static_cast<size_t>(prow) * K + q * 8;
  }
  // Token KiBs of this wave holding rows (the others are not loaded).
  const int nxw = kFull ? kXPerWave : max(0, min(kXPerWave, nfr - kXPerWave * w));  // <= kFrags - kXPerWave w
  // B fragment t: token 16t + l % 16, quarter l / 16.
  const int bj = lane & 15;
  const int boff = bj * 64 + 16 * ((lane >> 4) ^ ((bj >> 1) & 3));

  // Nibbles: the lane's 16-byte slot of each block of the wave's tile;
  // scales: dword l % 16 of the (tile, block) scale group (rows 16i + l % 16,
  // byte i).  Inactive waves read past the buffer end (zeros, no memory
  // access) so every wave issues the same loads.
  const size_t eoff_n = static_cast<size_t>(tc.e) * g.nib_bytes;
  const size_t eoff_s = static_cast<size_t>(tc.e) * g.scale_bytes + g.mscale_off;
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.wn + eoff_n), 0, static_cast<int>(g.nib_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.ws + eoff_s), 0, static_cast<int>(static_cast<size_t>(N) * nb), 0x00020000);
  const int wvoff = active ? tile * nb * 1024 + 16 * lane : static_cast<int>(g.nib_bytes);
  const int svoff = active ? tile * nb * 64 + 4 * (lane & 15) : N * nb;

  // Block kb's loads into stage st (clamped to the last block past the end:
  // the stage is not read again).
  auto issue = [&](int kb, int st) __attribute__((always_inline)) {
    const int bb = kb < nb ? kb : nb - 1;
    uint8_t* sp = xs + st * kStageBytes;
#pragma unroll
    for (int c = 0; c < kXPerWave; ++c)
      if (c < nxw)
        __builtin_amdgcn_global_load_lds(xsrc[c] + static_cast<size_t>(bb) * 32,
                                         (lds_void_t*)(sp + 1024 * (kXPerWave * w + c)), 16, 0, 0);
    // A partial m-tile's weights are read once (its expert's full m-tiles ran
    // earlier): nontemporal, so they do not displace tokens and the group's
    // shared weight tiles in L2 (measured: gate_up 0.614 -> 0.601 ms, Zipf).
    constexpr int kWPol = kFull ? 0 : 2;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void_t*)(sp + kWOff + 1024 * w), 16, wvoff, bb * 1024, 0, kWPol);
    if (lane < 16)  // the 16 distinct scale dwords
      __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_void_t*)(sp + kSOff + 64 * w), 4, svoff, bb * 64, 0, kWPol);
  };
  // Software pipeline over blocks: step kb runs block kb's products from
  // registers while the LDS reads of block kb + 1 land and its A operands
  // are decoded.  The work-group synchronises every second step: at even kb
  // it waits for blocks kb + 1, kb + 2 and refills the stages of kb - 1 and
  // kb with blocks kb + kStages - 1, kb + kStages.  The ring then holds
  // blocks kb - 1 .. kb + kStages - 2 before the refill.
#pragma unroll
  for (int b = 0; b < kStages - 1; ++b) issue(b, b);

  f32x4_t acc[4][kFrags];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < kFrags; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Operands of one block: raw nibbles and scales, decoded A, B fragments.
  auto read_stage = [&](int st, u32x4_t& wv, uint32_t& sv, bf16x8_t (&bv)[kFrags]) __attribute__((always_inline)) {
    const uint8_t* sp = xs + st * kStageBytes;
    wv = *reinterpret_cast<const u32x4_t*>(sp + kWOff + 1024 * w + 16 * lane);
    sv = *reinterpret_cast<const uint32_t*>(sp + kSOff + 64 * w + 4 * (lane & 15));
#pragma unroll
    for (int t = 0; t < kFrags; ++t)
      if (kFull || t < nfr) bv[t] = *reinterpret_cast<const bf16x8_t*>(sp + boff + 1024 * t);
  };
  // Decoded as codes 1..254 (exact); a block holding code 0 or 255 marks
  // the wave, which then recomputes its tile on the exact path below.
  bool spec = false;
  auto decode = [&](const u32x4_t& wv, uint32_t sv, bf16x8_t (&av)[4]) __attribute__((always_inline)) {
    spec |= has_special_code(sv, 0xffffffffu);
#pragma unroll
    for (int i = 0; i < 4; ++i) av[i] = decode8_bf16(wv[i], __uint_as_float(((sv >> (8 * i)) & 0xffu) << 23));
  };
  bf16x8_t av[2][4], bv[2][kFrags];

  // Block 0: its loads were followed by those of blocks 1 .. kStages - 2.
  const int per = nxw + 2;  // this wave's loads per block
  wait_blocks<kStages - 2, R::kMaxLoads>(per);
  __builtin_amdgcn_s_barrier();
  if (active) {
    u32x4_t wv;
    uint32_t sv;
    read_stage(0, wv, sv, bv[0]);
    decode(wv, sv, av[0]);
  }

  int st = 0;  // stage of block kb
  auto step = [&](auto P, int kb) __attribute__((always_inline)) {
    constexpr int p = decltype(P)::value;  // register set of block kb = kb % 2
    const int st1 = st == kStages - 1 ? 0 : st + 1;
    if constexpr (p == 0) {
      // Blocks kb + 1, kb + 2 were followed by kb + 3 .. kb + kStages - 2.
      // This wave's reads of stages kb - 1 and kb are complete, so after the
      // barrier no wave reads them any more and kb + 1, kb + 2 are visible.
      wait_blocks<kStages - 4, R::kMaxLoads>(per);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    if (active) {
      // Block kb + 1's reads go out in two halves, each ahead of the
      // products of the half of block kb whose fragments it replaces.
      const uint8_t* sp = xs + st1 * kStageBytes;
      const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(sp + kWOff + 1024 * w + 16 * lane);
      const uint32_t sv = *reinterpret_cast<const uint32_t*>(sp + kSOff + 64 * w + 4 * (lane & 15));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = h * kFrags / 2; t < (h + 1) * kFrags / 2; ++t)
          if (kFull || t < nfr) bv[p ^ 1][t] = *reinterpret_cast<const bf16x8_t*>(sp + boff + 1024 * t);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = h * kFrags / 2; t < (h + 1) * kFrags / 2; ++t)
          if (kFull || t < nfr) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[p][i], bv[p][t], acc[i][t], 0, 0, 0);
          }
        __builtin_amdgcn_sched_barrier(0);
      }
      decode(wv, sv, av[p ^ 1]);
    }
    // The refill, issued behind the products so a stalled address queue
    // overlaps the matrix cores.
    if constexpr (p == 0) {
      __builtin_amdgcn_sched_barrier(0);
      issue(kb + kStages - 1, st == 0 ? kStages - 1 : st - 1);
      issue(kb + kStages, st);
      __builtin_amdgcn_sched_barrier(0);
    }
    st = st1;
  };
  int kb0 = 0;
  for (; kb0 + 2 <= nb; kb0 += 2) {
    step(std::integral_constant<int, 0>{}, kb0);
    step(std::integral_constant<int, 1>{}, kb0 + 1);
  }
  if (kb0 < nb) step(std::integral_constant<int, 0>{}, kb0);
  wait_vm<0>();  // the clamped loads past the last block land before the work-group ends
  if (!active) return;

  if (__builtin_expect(__ballot(spec) != 0ull, 0))
    tile_special_pass<kFull, kFrags>(a, tc, wrs, srs, wvoff, svoff, nfr, mc, lane, acc);
  tile_epilogue<kGated, kFull, kFrags>(a, tc, tile, mc, lane, acc);
}

template <int kW, bool kGated>
__device__ __forceinline__ void run_tile(const GroupedParams& a, const TileCoord& tc, uint8_t* xs, int lane, int w) {
  const int mc = min(kBM, tc.cnt - tc.m0);
  if (mc == kBM)
    grouped_tile<kW, kGated, true, 8>(a, tc, xs, lane, w);
  else if (mc > 64)
    grouped_tile<kW, kGated, false, 8>(a, tc, xs, lane, w);
  else if (mc > 32)
    grouped_tile<kW, kGated, false, 4>(a, tc, xs, lane, w);
  else
    grouped_tile<kW, kGated, false, 2>(a, tc, xs, lane, w);
}

// ---- block-scaled variant: v_mfma_scale_f32_16x16x128_f8f6f4 ----------------
//
// The same tiles (kBM tokens x 256 weight rows, four waves of one 64-row
// tiled MXFP4 tile each), with the products on the block-scaled matrix core:
// the fp4 weights and their e8m0 scales are its A operand and scale as they
// are stored, and the activations enter as two e4m3 parts with per-block
// scales (launch_quant_fp8x2), hi and lo, one product each.  No register
// decodes the weights.  One product covers 128 K (four blocks): lane l holds
// row l % 16 of a 16-row sub-tile and block l / 16 of the four (its 16 bytes
// of fp4), and for B token l % 16 at K 16(l/16)..+15 and 64 + 16(l/16)..+15;
// the scale of (row or token r, block kb) comes from lane r + 16 kb, its byte
// picked by op_sel (sub-tile i: byte i of the dword holding rows 16i + r;
// hi: byte 0, lo: byte 1 of the token's code pair).  Output layout as the
// bf16 product: lane l holds rows 4(l/16)..+3 of the sub-tile for token l % 16.
//
// One work-group per CU; the LDS ring holds kMxGroups groups of four blocks
// (stage = one block: the tokens' hi | lo rows, each wave's tiled KiB and its
// scale dwords, the tokens' scale codes), every operand reaching it by direct
// global -> LDS loads.  A group's products run while the next groups' loads
// are in flight; the work-group synchronises once per group.
constexpr int kMxW = 4;                       // waves per work-group (a 64-row weight tile each)
constexpr int kMxRingBytes = 160 * 1024 - 64;  // the LDS of a CU, less the queue words

template <int kFrags>
struct MxRing {
  static constexpr int kF = kFrags;                       // 16-token fragments per stage
  static constexpr int kAOff = kFrags * 1024;             // tokens: 16 kF rows x 64 B
  static constexpr int kASOff = kAOff + kMxW * 1024;      // each wave's tiled block
  static constexpr int kBSOff = kASOff + kMxW * 64;       // each wave's scale dwords
  static constexpr int kBytes = kBSOff + 64 * kFrags;     // the tokens' scale code pairs (4 B each)
  static constexpr int kFit = kMxRingBytes / (4 * kBytes);
  static constexpr int kGroups = kFit < 4 ? kFit : 4;     // 128-K groups in the ring
  static constexpr int kStages = 4 * kGroups;
  static constexpr int kKiBPerWave = kFrags >= kMxW ? kFrags / kMxW : 1;
  static_assert(kGroups >= 3, "the ring holds the computed group and two in flight");
};

// s_waitcnt vmcnt(G * 4 * per) for a wave issuing `per` loads per block
// (wave-uniform: 2, 4 or 6).
template <int G>
__device__ __forceinline__ void wait_mx_groups(int per) {
  if (per >= 6) wait_vm<(G * 24 < 63 ? G * 24 : 63)>();
  else if (per >= 4) wait_vm<(G * 16 < 63 ? G * 16 : 63)>();
  else wait_vm<(G * 8 < 63 ? G * 8 : 63)>();
}

typedef int mx_v8i __attribute__((ext_vector_type(8)));

template <bool kGated, bool kFull, int kCls, bool kLo>
__device__ __forceinline__ void mx_tile(const GroupedParams& a, const TileCoord& tc, uint8_t* xs, int lane, int w) {
  const TiledGeom& g = a.g;
  const int N = g.N, nb = g.nb;
  const int mc = min(kBM, tc.cnt - tc.m0);
  using R = MxRing<kCls>;
  constexpr int kFrags = R::kF, kStages = R::kStages, kStageBytes = R::kBytes, kGroups = R::kGroups;
  constexpr int kAOff = R::kAOff, kASOff = R::kASOff, kBSOff = R::kBSOff, kKW = R::kKiBPerWave;
  const int nfr = kFull ? kFrags : (mc + 15) >> 4;  // 16-token fragments holding rows
  const int tile = tc.nt * kMxW + w;
  const bool active = tile < N / kTileRows;  // wave-uniform
  const int ngroups = (nb + 3) >> 2;
  const size_t qrow = static_cast<size_t>(nb) * 64;

  // Token KiBs this wave loads: kk = w + kMxW c.  Lane L stages token
  // 16 kk + L / 4, 16-byte chunk L % 4 of its 64-byte block row, holding the
  // row's chunk (L % 4) ^ swz (swz = (token / 4) % 4: the 16 tokens of a B
  // read at one chunk hit distinct banks 8 lanes at a time).  Lanes < 16 also
  // stage the scale code pair of token 16 kk + L.
  const uint8_t* qsrc[kKW];
  const uint32_t* ssrc[kKW];
  int nkw = 0;
#pragma unroll
  for (int c = 0; c < kKW; ++c) {
    const int kk = w + kMxW * c;
    if (kk < kFrags) nkw = c + 1;
    const int j = 16 * (kk < kFrags ? kk : 0) + (lane >> 2);
    const int jr = j < mc ? j : 0;
    const int prow = a.row_index ? a.row_index[tc.off + tc.m0 + jr] : tc.off + tc.m0 + jr;
    qsrc[c] = a.xq + static_cast<size_t>(prow) * qrow + 16 * ((lane & 3) ^ ((j >> 2) & 3));
    const int js = 16 * (kk < kFrags ? kk : 0) + (lane & 15);
    const int jsr = js < mc ? js : 0;
    const int psrow = a.row_index ? a.row_index[tc.off + tc.m0 + jsr] : tc.off + tc.m0 + jsr;
    ssrc[c] = a.xqs + static_cast<size_t>(psrow) * nb;
  }
  const int per = 2 + 2 * nkw;  // this wave's loads per block

  const size_t eoff_n = static_cast<size_t>(tc.e) * g.nib_bytes;
  const size_t eoff_s = static_cast<size_t>(tc.e) * g.scale_bytes + g.mscale_off;
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.wn + eoff_n), 0, static_cast<int>(g.nib_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.ws + eoff_s), 0, static_cast<int>(static_cast<size_t>(N) * nb), 0x00020000);
  const int wvoff = active ? tile * nb * 1024 + 16 * lane : static_cast<int>(g.nib_bytes);
  const int svoff = active ? tile * nb * 64 + 4 * (lane & 15) : N * nb;

  // Block kb's loads into its stage (blocks past nb load block nb - 1: they
  // keep every wave's load count uniform and are never read as data).
  auto issue = [&](int kb) __attribute__((always_inline)) {
    const int bb = kb < nb ? kb : nb - 1;
    uint8_t* sp = xs + (kb % kStages) * kStageBytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void_t*)(sp + kAOff + 1024 * w), 16, wvoff, bb * 1024, 0, 0);
    if (lane < 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(srs, (lds_void_t*)(sp + kASOff + 64 * w), 4, svoff, bb * 64, 0, 0);
#pragma unroll
    for (int c = 0; c < kKW; ++c)
      if (c < nkw) {
        const int kk = w + kMxW * c;
        __builtin_amdgcn_global_load_lds(qsrc[c] + static_cast<size_t>(bb) * 64, (lds_void_t*)(sp + 1024 * kk), 16, 0, 0);
        if (lane < 16)
          __builtin_amdgcn_global_load_lds(ssrc[c] + bb, (lds_void_t*)(sp + kBSOff + 64 * kk), 4, 0, 0);
      }
  };
#pragma unroll
  for (int kb = 0; kb < 4 * kGroups; ++kb) issue(kb);

  f32x4_t acc[4][kFrags];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < kFrags; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  const int n = lane & 15, gq = lane >> 4;
  const int swz = (n >> 2) & 3;
  bool spec = false;
  for (int q = 0; q < ngroups; ++q) {
    // This wave's loads of group q have landed once at most the groups
    // issued after it are outstanding; after the barrier every wave's have,
    // and no wave reads group q - 1's stages any more.
    if (q == 0) wait_mx_groups<kGroups - 1>(per);
    else wait_mx_groups<kGroups - 2>(per);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (q > 0) {
#pragma unroll
      for (int b = 0; b < 4; ++b) issue(4 * (q + kGroups - 1) + b);
    }
    if (!active) continue;
    // A operands: the lane's block 4q + gq, the four 16-byte slots holding its
    // row of each sub-tile; dword i of slot 16 g' + n = bytes 4 g'..4 g' + 3
    // of row 16 i + n.  Blocks past nb contribute zeros.
    const int ba = 4 * q + gq;
    mx_v8i av[4];
    uint32_t sa = 0x7f7f7f7fu;
    if (ba < nb) {
      const uint8_t* sp = xs + (ba % kStages) * kStageBytes;
      u32x4_t r[4];
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) r[gg] = *reinterpret_cast<const u32x4_t*>(sp + kAOff + 1024 * w + 16 * (16 * gg + n));
      sa = *reinterpret_cast<const uint32_t*>(sp + kASOff + 64 * w + 4 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        av[i] = mx_v8i{static_cast<int>(r[0][i]), static_cast<int>(r[1][i]), static_cast<int>(r[2][i]),
                       static_cast<int>(r[3][i]), 0, 0, 0, 0};
      spec |= has_special_code(sa, 0xffffffffu);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = mx_v8i{0, 0, 0, 0, 0, 0, 0, 0};
    }
    // B operands: chunks g % 2 (hi) and 2 + g % 2 (lo) of block 4q + g/2 (K
    // 16 g..16 g + 15) and of block 4q + 2 + g/2 (K 64 + 16 g..); the scale
    // pair of block 4q + g.
    const int b0 = 4 * q + (gq >> 1), b1 = b0 + 2;
    const uint8_t* s0 = xs + (b0 % kStages) * kStageBytes;
    const uint8_t* s1 = xs + (b1 % kStages) * kStageBytes;
    const uint8_t* ss = xs + ((4 * q + gq) % kStages) * kStageBytes + kBSOff;
    const int ch = 16 * ((gq & 1) ^ swz), cl = 16 * ((2 + (gq & 1)) ^ swz);
    const bool h0 = b0 < nb, h1 = b1 < nb, hs = 4 * q + gq < nb;
#pragma unroll
    for (int t = 0; t < kFrags; ++t) {
      if (kFull || t < nfr) {
        const int ro = 1024 * t + 64 * n;
        u32x4_t z{0u, 0u, 0u, 0u};
        const u32x4_t hA = h0 ? *reinterpret_cast<const u32x4_t*>(s0 + ro + ch) : z;
        const u32x4_t hB = h1 ? *reinterpret_cast<const u32x4_t*>(s1 + ro + ch) : z;
        const u32x4_t lA = kLo && h0 ? *reinterpret_cast<const u32x4_t*>(s0 + ro + cl) : z;
        const u32x4_t lB = kLo && h1 ? *reinterpret_cast<const u32x4_t*>(s1 + ro + cl) : z;
        const uint32_t sb = hs ? *reinterpret_cast<const uint32_t*>(ss + 4 * (16 * t + n)) : 0x7f7fu;
        const mx_v8i bh{static_cast<int>(hA[0]), static_cast<int>(hA[1]), static_cast<int>(hA[2]), static_cast<int>(hA[3]),
                        static_cast<int>(hB[0]), static_cast<int>(hB[1]), static_cast<int>(hB[2]), static_cast<int>(hB[3])};
        const mx_v8i bl{static_cast<int>(lA[0]), static_cast<int>(lA[1]), static_cast<int>(lA[2]), static_cast<int>(lA[3]),
                        static_cast<int>(lB[0]), static_cast<int>(lB[1]), static_cast<int>(lB[2]), static_cast<int>(lB[3])};
        const int sai = static_cast<int>(sa), sbi = static_cast<int>(sb);
        acc[0][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[0], bh, acc[0][t], 4, 0, 0, sai, 0, sbi);
        acc[1][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[1], bh, acc[1][t], 4, 0, 1, sai, 0, sbi);
        acc[2][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[2], bh, acc[2][t], 4, 0, 2, sai, 0, sbi);
        acc[3][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[3], bh, acc[3][t], 4, 0, 3, sai, 0, sbi);
        if constexpr (kLo) {
          acc[0][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[0], bl, acc[0][t], 4, 0, 0, sai, 1, sbi);
          acc[1][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[1], bl, acc[1][t], 4, 0, 1, sai, 1, sbi);
          acc[2][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[2], bl, acc[2][t], 4, 0, 2, sai, 1, sbi);
          acc[3][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[3], bl, acc[3][t], 4, 0, 3, sai, 1, sbi);
        }
      }
    }
  }
  wait_vm<0>();  // the clamped loads past the last block land before the work-group ends
  if (!active) return;

  const int bj = n;
  // Scale codes 0 and 255 (none in a regular checkpoint; the block-scaled
  // product cannot express the reference's decode of them): redo the wave's
  // tile block by block with that decode on the bf16 product, tokens read
  // from the bf16 rows of x.
  if (__builtin_expect(__ballot(spec) != 0ull, 0)) {
    const uint16_t* trow[kFrags];
#pragma unroll
    for (int t = 0; t < kFrags; ++t) {
      const int j = min(16 * t + bj, mc - 1);
      const int prow = a.row_index ? a.row_index[tc.off + tc.m0 + j] : tc.off + tc.m0 + j;
      trow[t] = a.x + static_cast<size_t>(prow) * g.K + 8 * (lane >> 4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int t = 0; t < kFrags; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int kb = 0; kb < nb; ++kb) {
      const u32x4_t wv = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wrs, wvoff, kb * 1024, 0));
      const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b32(srs, svoff, kb * 64, 0);
      bf16x8_t av1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av1[i] = decode8_bf16_special(wv[i], (sv >> (8 * i)) & 0xffu);
#pragma unroll
      for (int t = 0; t < kFrags; ++t)
        if (kFull || t < nfr) {
          const bf16x8_t b1 = *reinterpret_cast<const bf16x8_t*>(trow[t] + kb * 32);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av1[i], b1, acc[i][t], 0, 0, 0);
        }
    }
  }

  // Epilogue.  acc[i][t][r] is row 16i + 4(l/16) + r of the tile for token
  // 16t + l % 16.  gated with outq: the tile's 32 activations of a token are
  // one block of the down product's input; its four lanes (l / 16 = 0..3)
  // hold positions 8i + 2(l/16) + {0, 1} and quantise them with a common scale.
  const int nrow0 = tile * kTileRows + 4 * (lane >> 4);
  const uint16_t* brow = a.bias ? a.bias + static_cast<size_t>(tc.e) * N : nullptr;
  float bias[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = nrow0 + 16 * i;
    bias[i][0] = bias[i][1] = bias[i][2] = bias[i][3] = 0.0f;
    if (brow) {
      const uint2 bb = *reinterpret_cast<const uint2*>(brow + nn);
      bias[i][0] = bf16_to_f32(static_cast<uint16_t>(bb.x));
      bias[i][1] = bf16_to_f32(static_cast<uint16_t>(bb.x >> 16));
      bias[i][2] = bf16_to_f32(static_cast<uint16_t>(bb.y));
      bias[i][3] = bf16_to_f32(static_cast<uint16_t>(bb.y >> 16));
    }
  }
  const int nbo = N / kTileRows;  // blocks of a quantised activation row (gated)
#pragma unroll
  for (int t = 0; t < kFrags; ++t) {
    const int j = 16 * t + bj;
    const bool live = j < mc;
    const size_t p = static_cast<size_t>(tc.off + tc.m0 + (live ? j : 0));
    if constexpr (kGated) {
      float act[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int nn = nrow0 + 16 * i;
        uint16_t y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = f32_to_bf16(acc[i][t][r] + bias[i][r]);
        // rows nn, nn+2 are gate (even), nn+1, nn+3 up (odd)
        const uint16_t a0 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[0]), bf16_to_f32(y[1]), a.alpha, a.limit));
        const uint16_t a1 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[2]), bf16_to_f32(y[3]), a.alpha, a.limit));
        act[i][0] = bf16_to_f32(a0);
        act[i][1] = bf16_to_f32(a1);
        if (live) {
          *reinterpret_cast<uint32_t*>(a.out + p * (N / 2) + nn / 2) = a0 | (static_cast<uint32_t>(a1) << 16);
          if (a.gate_up)
            *reinterpret_cast<uint2*>(a.gate_up + p * N + nn) =
                make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
        }
      }
      if (a.outq != nullptr) {
        float m = 0.0f;
        bool fin = true;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const float v = __builtin_fabsf(act[i][r]);
            m = __builtin_fmaxf(m, v);
            fin = fin && (__float_as_uint(v) < 0x7f800000u);
          }
        // the token's four lanes: l, l ^ 16, l ^ 32, l ^ 48
        m = __builtin_fmaxf(m, __shfl_xor(m, 16, kWave));
        m = __builtin_fmaxf(m, __shfl_xor(m, 32, kWave));
        int fi = fin ? 1 : 0;
        fi &= __shfl_xor(fi, 16, kWave);
        fi &= __shfl_xor(fi, 32, kWave);
        float inv_s;
        const uint32_t codes = fp8x2_codes(m, inv_s);
        uint32_t h01, l01, h23, l23;
        fp8x2_quant4(act[0][0], act[0][1], act[1][0], act[1][1], inv_s, fi != 0, h01, l01);
        fp8x2_quant4(act[2][0], act[2][1], act[3][0], act[3][1], inv_s, fi != 0, h23, l23);
        if (live) {
          uint8_t* qo = a.outq + (p * nbo + tile) * 64 + 2 * (lane >> 4);
          *reinterpret_cast<uint16_t*>(qo + 0) = static_cast<uint16_t>(h01);
          *reinterpret_cast<uint16_t*>(qo + 8) = static_cast<uint16_t>(h01 >> 16);
          *reinterpret_cast<uint16_t*>(qo + 16) = static_cast<uint16_t>(h23);
          *reinterpret_cast<uint16_t*>(qo + 24) = static_cast<uint16_t>(h23 >> 16);
          *reinterpret_cast<uint16_t*>(qo + 32) = static_cast<uint16_t>(l01);
          *reinterpret_cast<uint16_t*>(qo + 40) = static_cast<uint16_t>(l01 >> 16);
          *reinterpret_cast<uint16_t*>(qo + 48) = static_cast<uint16_t>(l23);
          *reinterpret_cast<uint16_t*>(qo + 56) = static_cast<uint16_t>(l23 >> 16);
          if ((lane >> 4) == 0) a.outqs[p * nbo + tile] = codes;
        }
      }
    } else {
      if (live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int nn = nrow0 + 16 * i;
          uint16_t y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = f32_to_bf16(acc[i][t][r] + bias[i][r]);
          *reinterpret_cast<uint2*>(a.out + p * N + nn) =
              make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
        }
      }
    }
  }
}

template <bool kGated, bool kLo>
__device__ __forceinline__ void run_mx_tile(const GroupedParams& a, const TileCoord& tc, uint8_t* xs, int lane,
                                            int w) {
  const int mc = min(kBM, tc.cnt - tc.m0);
  if (mc == kBM)
    mx_tile<kGated, true, 8, kLo>(a, tc, xs, lane, w);
  else if (mc > 64)
    mx_tile<kGated, false, 8, kLo>(a, tc, xs, lane, w);
  else if (mc > 32)
    mx_tile<kGated, false, 4, kLo>(a, tc, xs, lane, w);
  else
    mx_tile<kGated, false, 2, kLo>(a, tc, xs, lane, w);
}

__global__ __launch_bounds__(256) void quant_fp8x2_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                         uint8_t* __restrict__ q, uint32_t* __restrict__ qs) {
  const int nb = K >> 5;
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<long>(rows) * nb) return;
  const long r = i / nb;
  const int b = static_cast<int>(i - r * nb);
  const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(r) * K + 32 * b);
  float v[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 u = src[c];
    const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[8 * c + 2 * e] = bf16_to_f32(static_cast<uint16_t>(d[e]));
      v[8 * c + 2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(d[e] >> 16));
    }
  }
  float m = 0.0f;
  bool fin = true;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float av = __builtin_fabsf(v[e]);
    m = __builtin_fmaxf(m, av);
    fin = fin && (__float_as_uint(av) < 0x7f800000u);
  }
  float inv_s;
  const uint32_t codes = fp8x2_codes(m, inv_s);
  uint32_t hi[8], lo[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) fp8x2_quant4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3], inv_s, fin, hi[c], lo[c]);
  uint4* dst = reinterpret_cast<uint4*>(q + static_cast<size_t>(i) * 64);
  dst[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  dst[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
  dst[2] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  dst[3] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
  qs[i] = codes;
}

// Counters of the persistent grid: XCD x's queue at queue[kQueueStride x],
// the finished work-groups at queue[kQueueStride * 8].  All start at zero;
// the last work-group to finish zeroes them for the next launch.
constexpr int kQueueStride = 32;  // one 128-byte line per counter

// LDS words of the persistent loop, past every ring layout: word[0..1] the
// taken index (alternating rounds), word[2] the next queue to try.
constexpr int kWordNext = 2;

// Queue (x0 + k) & 7 was found empty: the next queue of the rotation that
// still holds entries, as the new k, or 8 for none.  Thread 0 reads every
// counter in one round trip; a counter at or past its queue's length marks
// the queue empty for good (counters only grow), so only queues with
// entries left are tried, where trying each in turn cost an atomic round
// trip and a tile-list rebuild apiece at the end of the launch.
__device__ __forceinline__ int next_queue(const int* queue, int* word, int x0, int k, const TileList& L, int nwt) {
  if (threadIdx.x == 0) {
    int c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = __hip_atomic_load(&queue[kQueueStride * j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int nk = 8;
#pragma unroll
    for (int j = 7; j > 0; --j) {
      const int x = (x0 + j) & 7;
      int lf;
      if (j > k && c[x] < queue_len(L, nwt, x, lf)) nk = j;
    }
    word[kWordNext] = nk;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(word[kWordNext]);
}

template <bool kGated, int kW>
__global__ __launch_bounds__(kW * kWave, WgShape<kW>::kPerCU) void grouped_mfma_kernel(GroupedParams a) {
  constexpr int kRingBytes = WgShape<kW>::kRingBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t xs[kRingBytes];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int vb = static_cast<int>(blockIdx.x);
  const int x0 = vb & 7;  // work-group vb runs on XCD vb % 8
  // Without a queue: entry vb / 8 of XCD x0's queue, one tile.  With one
  // (persistent grid): entries of this XCD's queue, then of the others'; the
  // taken index is passed through two alternating LDS words past every ring
  // layout (a wave is at most one round behind: each round has a barrier).
  int* word = reinterpret_cast<int*>(xs + kRingBytes - 64);
  const bool persistent = a.queue != nullptr;
  int k = 0;  // queues found empty
  for (int round = 0;; ++round) {
    const int x = (x0 + k) & 7;
    // The tile list's loads go out ahead of the take, so the tile switch
    // waits for the longer of the two round trips rather than their sum.
    int toff[kExpertsPerLane + 1];
    load_tile_offsets(a.offsets, a.E, lane, toff);
    int t;
    if (persistent) {
      if (threadIdx.x == 0) word[round & 1] = atomicAdd(&a.queue[kQueueStride * x], 1);
      __syncthreads();
      t = __builtin_amdgcn_readfirstlane(word[round & 1]);
    } else {
      if (round > 0) break;
      t = vb >> 3;
    }
    const TileList L = make_tile_list(toff, a.E, lane);
    int lenF;
    if (t >= queue_len(L, a.nwt, x, lenF)) {
      if (!persistent) break;
      k = next_queue(a.queue, word, x0, k, L, a.nwt);
      if (k == 8) break;
      continue;
    }
    TileCoord tc;
    tile_at(L, a.offsets, a.nwt, x, t, lenF, lane, tc);
    // Recomputed per tile rather than hoisted out of the loop: values kept
    // live across tiles would push the tile's registers into scratch.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    run_tile<kW, kGated>(a, tc, xs, ln, w);
  }
  if (!persistent) return;
  if (threadIdx.x == 0 && atomicAdd(&a.queue[kQueueStride * 8], 1) == static_cast<int>(gridDim.x) - 1) {
#pragma unroll
    for (int x = 0; x <= 8; ++x) atomicExch(&a.queue[kQueueStride * x], 0);
  }
}

// The block-scaled grouped product: the persistent loop of
// grouped_mfma_kernel over the same tile queues, one work-group per CU.
template <bool kGated, bool kLo>
__global__ __launch_bounds__(kMxW * kWave, 1) void grouped_mx_kernel(GroupedParams a) {
  __shared__ __attribute__((aligned(1024))) uint8_t xs[kMxRingBytes + 64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int x0 = static_cast<int>(blockIdx.x) & 7;  // work-group vb runs on XCD vb % 8
  int* word = reinterpret_cast<int*>(xs + kMxRingBytes);
  int k = 0;  // queues found empty
  for (int round = 0;; ++round) {
    const int x = (x0 + k) & 7;
    int toff[kExpertsPerLane + 1];
    load_tile_offsets(a.offsets, a.E, lane, toff);  // ahead of the take, as in grouped_mfma_kernel
    if (threadIdx.x == 0) word[round & 1] = atomicAdd(&a.queue[kQueueStride * x], 1);
    __syncthreads();
    const int t = __builtin_amdgcn_readfirstlane(word[round & 1]);
    const TileList L = make_tile_list(toff, a.E, lane);
    int lenF;
    if (t >= queue_len(L, a.nwt, x, lenF)) {
      k = next_queue(a.queue, word, x0, k, L, a.nwt);
      if (k == 8) break;
      continue;
    }
    TileCoord tc;
    tile_at(L, a.offsets, a.nwt, x, t, lenF, lane, tc);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    run_mx_tile<kGated, kLo>(a, tc, xs, ln, w);
  }
  if (threadIdx.x == 0 && atomicAdd(&a.queue[kQueueStride * 8], 1) == static_cast<int>(gridDim.x) - 1) {
#pragma unroll
    for (int x = 0; x <= 8; ++x) atomicExch(&a.queue[kQueueStride * x], 0);
  }
}

}  // namespace

hipError_t launch_quant_fp8x2(const uint16_t* x, int rows, int K, uint8_t* q, uint32_t* qs, hipStream_t s,
                              const KernelTimer& t) {
  if (rows <= 0) return hipSuccess;
  if (K <= 0 || K % 32 != 0) return hipErrorInvalidValue;
  const long n = static_cast<long>(rows) * (K / 32);
  gx_launch(quant_fp8x2_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, t, x, rows, K, q, qs);
  return hipGetLastError();
}

bool grouped_supported(int N, int K, int E) {
  return N > 0 && K > 0 && N % kTileRows == 0 && K % 32 == 0 && E > 0 && E <= kMaxExperts;
}

hipError_t launch_grouped_mxfp4(const GroupedArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (!grouped_supported(a.N, a.K, a.E)) return hipErrorInvalidValue;
  GroupedParams p{};
  p.x = a.x;
  p.row_index = a.row_index;
  p.offsets = a.offsets;
  p.E = a.E;
  p.wn = a.wn;
  p.ws = a.ws;
  p.g = tiled_geom(a.N, a.K);
  p.bias = a.bias;
  p.out = a.out;
  p.gate_up = a.gate_up;
  p.alpha = a.alpha;
  p.limit = a.limit;
  const int kw = a.gated ? kGateUpWaves : kDownWaves;
  p.nwt = (a.N / kTileRows + kw - 1) / kw;
  p.queue = a.queue;
  p.xq = a.xq;
  p.xqs = a.xqs;
  p.outq = a.gated ? a.outq : nullptr;
  p.outqs = a.gated ? a.outqs : nullptr;
  const bool mx = a.xq != nullptr;
  if (mx) {  // the block-scaled kernel: persistent grid, a queue and four-wave tiles
    if (a.queue == nullptr || a.xqs == nullptr || a.num_cus <= 0 || (a.outq != nullptr) != (a.outqs != nullptr))
      return hipErrorInvalidValue;
    p.nwt = (a.N / kTileRows + kMxW - 1) / kMxW;
  }
  // full m-tiles <= rows / kBM, partial ones <= experts with rows; the
  // kernel counts the real tiles
  const long fb = static_cast<long>(a.rows / kBM) * p.nwt, pm = a.E < a.rows ? a.E : a.rows;
  const long per_xcd = (fb + 7) / 8 + (pm + 7) / 8 * p.nwt;
  if (per_xcd > (1L << 27) || fb >= (1L << 16) * p.nwt || static_cast<size_t>(a.N) * (a.K / 32) > (1u << 30) ||
      p.g.nib_bytes >= (static_cast<size_t>(1) << 31))
    return hipErrorInvalidValue;  // tile counts (16-bit scan fields) and buffer offsets (32-bit)
  int grid = static_cast<int>(8 * per_xcd);
  if (mx) {
    const int slots = 8 * ((a.num_cus + 7) / 8);  // one work-group per CU, a multiple of 8
    grid = grid < slots ? grid : slots;
    if (a.mx_single) {
      if (a.gated)
        gx_launch(grouped_mx_kernel<true, false>, dim3(grid), dim3(kMxW * kWave), 0, s, a.timer, p);
      else
        gx_launch(grouped_mx_kernel<false, false>, dim3(grid), dim3(kMxW * kWave), 0, s, a.timer, p);
    } else if (a.gated) {
      gx_launch(grouped_mx_kernel<true, true>, dim3(grid), dim3(kMxW * kWave), 0, s, a.timer, p);
    } else {
      gx_launch(grouped_mx_kernel<false, true>, dim3(grid), dim3(kMxW * kWave), 0, s, a.timer, p);
    }
    return hipGetLastError();
  }
  if (a.queue) {
    const int slots = 8 * ((8 / kw * a.num_cus + 7) / 8);  // every work-group slot, a multiple of 8
    if (a.num_cus <= 0) return hipErrorInvalidValue;
    grid = grid < slots ? grid : slots;
  }
  if (a.gated)
    gx_launch(grouped_mfma_kernel<true, kGateUpWaves>, dim3(grid), dim3(kGateUpWaves * kWave), 0, s, a.timer, p);
  else
    gx_launch(grouped_mfma_kernel<false, kDownWaves>, dim3(grid), dim3(kDownWaves * kWave), 0, s, a.timer, p);
  return hipGetLastError();
}

}  // namespace gxmoe
