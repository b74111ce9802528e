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
// Work decomposition: a work-group computes a tile of kBM permuted rows (one
// expert's tokens) x 256 weight rows; its four waves own one 64-row tile of
// the tiled MXFP4 layout each (the layout the decode kernels stream, so one
// copy of the weights serves both paths).  The (m-tile, n-tile) pairs are
// counted expert by expert from the plan's offsets on the device, so no host
// synchronisation is needed; consecutive tiles share their token rows and
// land on the same XCD (one L2).
//
// Matrix-core mapping (v_mfma_f32_32x32x16_bf16, fp32 accumulation): the A
// operand is 32 weight rows, decoded from MXFP4 in registers with the gfx950
// scaled fp4 -> bf16 conversion (exact: e2m1 x 2^(s-127) has at most two
// significant bits); the B operand is 32 tokens read from an LDS tile.  The
// accumulator layout gives each lane four consecutive weight rows of one
// token, so the interleaved gate/up pairs meet in one lane.  The K order
// inside an MFMA is a permutation shared by both operands: lane half h takes
// elements 16h..16h+15 of each 32-element block (dwords 2h, 2h+1 of the
// tiled row block), elements 16h+8s..16h+8s+7 in k16 step s.
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
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGW = 4;                    // waves per work-group (a 64-row weight tile each)
constexpr int kBM = 64;                   // permuted rows per work-group tile (2 x 32 tokens)
constexpr int kGD = 4;                    // blocks in flight ahead of the one computed
constexpr int kStageBytes = kBM * 64;     // one 32-element bf16 block of kBM rows
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
  int nwt;                   // work-group n-tiles: ceil(N / (64 kGW))
  int total;                 // virtual tiles (bound on m-tiles x nwt)
};

// Expert, first row (within the expert), offset and row count of m-tile
// `mt`, counting ceil(M_e / kBM) m-tiles per expert in expert order; e = -1
// past the last.  Every lane returns the same values.
__device__ __forceinline__ void find_mtile(const int32_t* __restrict__ offsets, int E, int mt, int lane, int& e,
                                           int& m0, int& off, int& cnt) {
  int c[kExpertsPerLane], o[kExpertsPerLane + 1];
  const int e0 = lane * kExpertsPerLane;
#pragma unroll
  for (int i = 0; i <= kExpertsPerLane; ++i) o[i] = offsets[min(e0 + i, E)];  // all in flight at once
  int local = 0;
#pragma unroll
  for (int i = 0; i < kExpertsPerLane; ++i) {
    c[i] = e0 + i < E ? (o[i + 1] - o[i] + kBM - 1) / kBM : 0;
    local += c[i];
  }
  int incl = local;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int t = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += t;
  }
  const int excl = incl - local;
  const bool mine = mt >= excl && mt < incl;
  const unsigned long long bal = __ballot(mine);
  if (bal == 0ull) {
    e = -1;
    return;
  }
  const int src = __ffsll(static_cast<long long>(bal)) - 1;
  int ee = -1, base = excl;
#pragma unroll
  for (int i = 0; i < kExpertsPerLane; ++i) {
    if (ee < 0) {
      if (mt < base + c[i]) ee = e0 + i;
      else base += c[i];
    }
  }
  e = __shfl(ee, src, kWave);
  m0 = (mt - __shfl(base, src, kWave)) * kBM;
  off = offsets[e];
  cnt = offsets[e + 1] - off;
}

template <bool kGated>
__global__ __launch_bounds__(kGW * kWave) void grouped_mfma_kernel(GroupedParams a) {
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][kStageBytes];
  const int G = gridDim.x;  // a multiple of 8: block b runs on XCD b % 8
  const int vb = static_cast<int>(blockIdx.x);
  const int v = (vb & 7) * (G >> 3) + (vb >> 3);
  if (v >= a.total) return;
  const int nt = v % a.nwt, mt = v / a.nwt;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  int e, m0, off, cnt;
  find_mtile(a.offsets, a.E, mt, lane, e, m0, off, cnt);
  if (e < 0) return;  // the whole work-group: no barrier has been passed
  const int mc = min(kBM, cnt - m0);
  const TiledGeom& g = a.g;
  const int K = g.K, N = g.N, nb = g.nb;
  const int tile = nt * kGW + w;
  const bool active = tile < N / kTileRows;  // wave-uniform: rows past N (last n-tile) only stage tokens

  // Token staging: lane -> row pm = 16w + lane/4 of the tile, LDS quarter
  // lane%4 holding global quarter (lane%4) ^ swz(pm), swz(m) = (m/2)%4, so
  // that 8 consecutive rows read at one quarter hit distinct banks.
  const int pm = 16 * w + (lane >> 2);
  const int pq = (lane & 3) ^ ((pm >> 1) & 3);
  const int pmr = pm < mc ? pm : 0;  // rows past the expert's end stage a valid row (their outputs are not stored)
  const int prow = a.row_index ? a.row_index[off + m0 + pmr] : off + m0 + pmr;
  const uint16_t* xsrc = a.x + static_cast<size_t>(prow) * K + pq * 8;
  uint8_t* xdst0 = &xs[0][0] + 1024 * w + 16 * lane;

  // Weights: frag f = rows 32f + lane%32 of the wave's tile, dwords 2h and
  // 2h + 1 (h = lane/32) of each 16-byte row block: tiled_dword(row, 2h) and
  // the dword 64 after it; row 32 + r sits 2 dwords after row r.  Scales:
  // one byte per (row, block).
  const int tl = active ? tile : 0;
  const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(a.wn + static_cast<size_t>(e) * g.nib_bytes +
                                                           static_cast<size_t>(tl) * nb * 1024) +
                         tiled_dword(lane & 31, 2 * (lane >> 5));
  const uint8_t* ssrc = a.ws + static_cast<size_t>(e) * g.scale_bytes +
                        (static_cast<size_t>(tl) * g.parts * kTileRows + (lane & 31)) * g.spad;
  const size_t spart = static_cast<size_t>(kTileRows) * g.spad;  // scale bytes per part
  const size_t sfrag = static_cast<size_t>(32) * g.spad;

  u32x4_t xr[kGD];
  u32x2_t wr[kGD][2];
  uint32_t sr[kGD][2];
  int ssh[kGD];  // bit offset of the scale byte in sr
  // Prefetch cursor (block index of the next loads, clamped to the last block).
  int lb = 0, lp = 0, lq = 0;
  auto issue = [&](u32x4_t& xv, u32x2_t (&wv)[2], uint32_t (&sv)[2], int& sh) __attribute__((always_inline)) {
    const int bb = lb < nb ? lb : nb - 1;
    const int bp = lb < nb ? lp : (nb - 1) / g.bpp;
    const int bq = lb < nb ? lq : (nb - 1) % g.bpp;
    xv = *reinterpret_cast<const u32x4_t*>(xsrc + static_cast<size_t>(bb) * 32);
    // Every wave issues the same loads (an inactive one reads tile 0), so the
    // wait counts are the same on every path.
    const uint32_t* wp = wsrc + static_cast<size_t>(bb) * 256;
    wv[0] = u32x2_t{wp[0], wp[64]};  // cached: every m-tile of the expert reads them
    wv[1] = u32x2_t{wp[2], wp[66]};
    // The aligned dword holding the scale byte (extracted at its use: a
    // loop-carried byte load is re-masked where the loop wraps, which waits
    // for the loads in flight).
    const uint8_t* sp = ssrc + bp * spart + (bq & ~3);
    sv[0] = *reinterpret_cast<const uint32_t*>(sp);
    sv[1] = *reinterpret_cast<const uint32_t*>(sp + sfrag);
    sh = 8 * (bq & 3);
    ++lb;
    if (++lq == g.bpp) {
      lq = 0;
      ++lp;
    }
  };

  issue(xr[0], wr[0], sr[0], ssh[0]);
  issue(xr[1], wr[1], sr[1], ssh[1]);
  issue(xr[2], wr[2], sr[2], ssh[2]);
  issue(xr[3], wr[3], sr[3], ssh[3]);
  *reinterpret_cast<u32x4_t*>(xdst0) = xr[0];
  __syncthreads();

  f32x16_t acc[2][2];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[f][t][r] = 0.0f;

  // B operand: token j = 32t + lane%32, quarter 2h + s of the 32-element block.
  const int h = lane >> 5;
  int boff[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = 32 * t + (lane & 31);
#pragma unroll
    for (int s = 0; s < 2; ++s) boff[t][s] = j * 64 + 16 * ((2 * h + s) ^ ((j >> 1) & 3));
  }

  // One block of the main loop; the ring slot u is a compile-time constant
  // so the ring stays in registers.
  auto step = [&](auto U, int kb) __attribute__((always_inline)) {
    constexpr int u = decltype(U)::value;
    const uint8_t* stage = &xs[kb & 1][0];
    bf16x8_t av[2][2];
    if (active) {
      const uint32_t c0 = __builtin_amdgcn_ubfe(sr[u][0], ssh[u], 8), c1 = __builtin_amdgcn_ubfe(sr[u][1], ssh[u], 8);
      const bool special = ((c0 - 1u) >= 254u) || ((c1 - 1u) >= 254u);
      if (__builtin_expect(__ballot(special) != 0ull, 0)) {
        av[0][0] = decode8_bf16_special(wr[u][0].x, c0);
        av[0][1] = decode8_bf16_special(wr[u][0].y, c0);
        av[1][0] = decode8_bf16_special(wr[u][1].x, c1);
        av[1][1] = decode8_bf16_special(wr[u][1].y, c1);
      } else {
        // c0, c1 are zero-extended bytes: code << 23 is the e8m0 scale
        const float s0 = __uint_as_float(c0 << 23), s1 = __uint_as_float(c1 << 23);
        av[0][0] = decode8_bf16(wr[u][0].x, s0);
        av[0][1] = decode8_bf16(wr[u][0].y, s0);
        av[1][0] = decode8_bf16(wr[u][1].x, s1);
        av[1][1] = decode8_bf16(wr[u][1].y, s1);
      }
    }
    // The ring slot is free: fetch block kb + kGD into it.
    issue(xr[u], wr[u], sr[u], ssh[u]);
    if (active) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8_t bv[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) bv[t] = *reinterpret_cast<const bf16x8_t*>(stage + boff[t][s]);
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int t = 0; t < 2; ++t)
            acc[f][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[f][s], bv[t], acc[f][t], 0, 0, 0);
      }
    }
    // Stage block kb + 1 (fetched kGD - 1 steps ago) into the other buffer.
    *reinterpret_cast<u32x4_t*>(&xs[(kb + 1) & 1][0] + 1024 * w + 16 * lane) = xr[(u + 1) % kGD];
    __syncthreads();
  };
  static_assert(kGD == 4, "the main loop is unrolled by hand for a ring of 4");
  int kb0 = 0;
  for (; kb0 + kGD <= nb; kb0 += kGD) {
    step(std::integral_constant<int, 0>{}, kb0);
    step(std::integral_constant<int, 1>{}, kb0 + 1);
    step(std::integral_constant<int, 2>{}, kb0 + 2);
    step(std::integral_constant<int, 3>{}, kb0 + 3);
  }
  if (kb0 < nb) {
    step(std::integral_constant<int, 0>{}, kb0);
    if (kb0 + 1 < nb) {
      step(std::integral_constant<int, 1>{}, kb0 + 1);
      if (kb0 + 2 < nb) step(std::integral_constant<int, 2>{}, kb0 + 2);
    }
  }
  if (!active) return;

  // Epilogue.  acc[f][t][4q + r] is row 32f + 8q + 4h + r of the tile for
  // token 32t + lane%32.
  const int nrow0 = tile * kTileRows + 4 * h;
  const uint16_t* brow = a.bias ? a.bias + static_cast<size_t>(e) * N : nullptr;
#pragma unroll
  for (int f = 0; f < 2; ++f) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nrow0 + 32 * f + 8 * q;  // four consecutive rows n..n+3
      float bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (brow) {
        const uint2 bb = *reinterpret_cast<const uint2*>(brow + n);
        bias[0] = bf16_to_f32(static_cast<uint16_t>(bb.x));
        bias[1] = bf16_to_f32(static_cast<uint16_t>(bb.x >> 16));
        bias[2] = bf16_to_f32(static_cast<uint16_t>(bb.y));
        bias[3] = bf16_to_f32(static_cast<uint16_t>(bb.y >> 16));
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int j = 32 * t + (lane & 31);
        if (j < mc) {
          const size_t p = static_cast<size_t>(off + m0 + j);
          uint16_t y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = f32_to_bf16(acc[f][t][4 * q + r] + bias[r]);
          if constexpr (kGated) {
            // rows n, n+2 are gate (even), n+1, n+3 up (odd)
            const uint16_t a0 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[0]), bf16_to_f32(y[1]), a.alpha, a.limit));
            const uint16_t a1 = f32_to_bf16(gx_swiglu(bf16_to_f32(y[2]), bf16_to_f32(y[3]), a.alpha, a.limit));
            *reinterpret_cast<uint32_t*>(a.out + p * (N / 2) + n / 2) = a0 | (static_cast<uint32_t>(a1) << 16);
            if (a.gate_up)
              *reinterpret_cast<uint2*>(a.gate_up + p * N + n) =
                  make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
          } else {
            *reinterpret_cast<uint2*>(a.out + p * N + n) =
                make_uint2(y[0] | (static_cast<uint32_t>(y[1]) << 16), y[2] | (static_cast<uint32_t>(y[3]) << 16));
          }
        }
      }
    }
  }
}

}  // namespace

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
  p.nwt = (a.N / kTileRows + kGW - 1) / kGW;
  // sum_e ceil(M_e / kBM) <= rows / kBM + (experts with rows)
  const long mt_bound = (a.rows + kBM - 1) / kBM + (a.E < a.rows ? a.E : a.rows);
  const long total = mt_bound * p.nwt;
  if (total > (1L << 30)) return hipErrorInvalidValue;
  p.total = static_cast<int>(total);
  const int grid = (p.total + 7) & ~7;
  if (a.gated)
    gx_launch(grouped_mfma_kernel<true>, dim3(grid), dim3(kGW * kWave), 0, s, a.timer, p);
  else
    gx_launch(grouped_mfma_kernel<false>, dim3(grid), dim3(kGW * kWave), 0, s, a.timer, p);
  return hipGetLastError();
}

}  // namespace gxmoe
