// moe_experts.hip -- decode-path MXFP4 expert products on gfx950.
//
// Replaces fused_mxfp4_gemv_forward / _multi_forward (fused_mxfp4_gemv.cu:
// 76-310), the bias kernels (moe_layer.cu:171-194, 442-473), swiglu_forward
// (swiglu.cu:117-211), moe_combine_forward (moe_combine.cu:31-117) and the
// per-batch host loop of moe_layer.cu:1316-1487 with two launches:
//
//   w1_kernel  grid (2I/64 tiles, max_active), P waves per work-group.
//              Work-group (tile, j) streams the 64 gate/up rows of tile
//              `tile` of the j-th active expert once and applies them to all
//              tokens routed to that expert; epilogue: + bias, bf16 gate_up,
//              clamped SwiGLU, bf16 activation.
//   w2_kernel  grid (H/64 tiles, max_active): down rows, + bias, bf16 expert
//              output; the last expert to finish a tile (atomic ticket)
//              forms out = bf16(sum_k w_k*y_k + residual) for that tile.
//
// Memory layout (tiled MXFP4, built once by pack_tiled_kernel): for each
// expert, each 64-row tile holds nb = K/32 blocks of [64 lanes][16 bytes]
// (one 32-element MXFP4 block of row tile*64+lane per lane), so one wave's
// 16-byte loads of block b are one contiguous 1 KiB.  Scales of each
// (tile, part, lane) are one contiguous group of `spad` bytes (bpp used).
//
// Arithmetic (the canonical expert dot): lane = row, wave = K-part; each
// lane runs one ascending fmaf chain over its part; the P part sums are added
// in part order; + bias; bf16.  The token activations are wave-uniform and
// are read through the scalar cache.
#include <float.h>

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
  g.scale_bytes = static_cast<size_t>(N / kTileRows) * g.parts * kTileRows * g.spad;
  return g;
}

namespace {

constexpr int kMaxBpp = 16;                 // blocks per K-part kept resident in VGPRs
constexpr int kTokChunk = 2;                // tokens per pass over the resident weights
constexpr int kPartK = kMaxBpp * 32;        // LDS row length of one staged K-part
constexpr int kXLoads = (kTokChunk * kPartK / 8 + kWave - 1) / kWave;  // 16-byte x loads per lane

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per work-group LDS (about 27 KB, so two work-groups share a CU): each wave's
// staged activations (fp32), the part sums and the bf16-rounded gate/up values.
struct ExpertSmem {
  float x[kMaxParts][kTokChunk][kPartK];
  float part[kMaxParts][kTokChunk][kTileRows];
  float gu[kTokChunk][kTileRows];
};

// Activations of one token chunk for one wave's K-part, in flight in VGPRs.
struct XLoad {
  uint4 v[kXLoads];
};

// Issue the 16-byte loads of the bf16 activations [k0, k0 + plen) of the
// token rows r0 (m = 0) and r1 (m = 1).  Lane l takes chunks l, l + 64, ...;
// chunks past the end re-read the last valid one, so every lane issues the
// same number of loads (the wait counts stay static).
__device__ __forceinline__ void issue_x(XLoad& xl, const uint16_t* r0, const uint16_t* r1, int mc, int k0, int plen,
                                        int lane) {
  const int nchunk = plen >> 3;
  const int last = mc * nchunk - 1;
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    int q = lane + i * kWave;
    q = q > last ? last : q;
    const int m = q >= nchunk ? 1 : 0;
    const int c = q - m * nchunk;
    xl.v[i] = *reinterpret_cast<const uint4*>((m ? r1 : r0) + k0 + c * 8);
  }
}

// Widen the loaded activations to fp32 into this wave's LDS rows, then make
// them visible to the whole wave (LDS writes complete before any lane reads).
// Lanes past the end wrote the clamped last chunk again (same data, same
// place), so the stores need no branch.
__device__ __forceinline__ void store_x(const XLoad& xl, float (*sx)[kPartK], int mc, int plen, int lane) {
  const int nchunk = plen >> 3;
  const int last = mc * nchunk - 1;
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    int q = lane + i * kWave;
    q = q > last ? last : q;
    const int m = q >= nchunk ? 1 : 0;
    const int c = q - m * nchunk;
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

// One lane's part of the canonical dot for up to kTokChunk tokens: an
// ascending fmaf chain over the lane's blocks (BPP of them; BPP == 0 means
// g_bpp, a runtime count), activations read from LDS as broadcasts.
template <int BPP>
__device__ __forceinline__ void part_dot(const u32x4 (&nib)[kMaxBpp], const uint32_t (&sc)[kMaxBpp / 4], int g_bpp,
                                         const float (*sx)[kPartK], int mc, float (&acc)[kTokChunk]) {
  constexpr int kLoop = BPP ? BPP : kMaxBpp;
#pragma unroll
  for (int m = 0; m < kTokChunk; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int i = 0; i < kLoop; ++i) {
    if (BPP || i < g_bpp) {
      const uint32_t code = (sc[i >> 2] >> (8 * (i & 3))) & 0xffu;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float wf[8];
        decode8(nib[i][d], code, wf);
#pragma unroll
        for (int m = 0; m < kTokChunk; ++m) {
          if (m < mc) {
            const f32x4 xa = *reinterpret_cast<const f32x4*>(&sx[m][i * 32 + d * 8]);
            const f32x4 xb = *reinterpret_cast<const f32x4*>(&sx[m][i * 32 + d * 8 + 4]);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[m] = __builtin_fmaf(xa[c], wf[c], acc[m]);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[m] = __builtin_fmaf(xb[c], wf[4 + c], acc[m]);
          }
        }
      }
    }
    // keep the scheduler from hoisting the LDS reads of later blocks (they
    // would all be held in registers at once)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Issue the loads of a lane's scales and blocks of tile `tile`, part `p`.
template <int BPP>
__device__ __forceinline__ void load_part(const uint8_t* __restrict__ nib_base, const uint8_t* __restrict__ sc_base,
                                          const TiledGeom& g, int tile, int p, int lane,
                                          u32x4 (&nib)[kMaxBpp], uint32_t (&sc)[kMaxBpp / 4]) {
  constexpr int kLoop = BPP ? BPP : kMaxBpp;
  const int bpp = BPP ? BPP : g.bpp;
  const uint32_t* s32 = reinterpret_cast<const uint32_t*>(
      sc_base + (static_cast<size_t>(tile) * g.parts + p) * kTileRows * g.spad + static_cast<size_t>(lane) * g.spad);
#pragma unroll
  for (int q = 0; q < (kLoop + 3) / 4; ++q)
    if (BPP || q * 4 < bpp) sc[q] = s32[q];
  __builtin_amdgcn_sched_barrier(0);  // scales before blocks: block 0's wait then covers them
  const u32x4* src = reinterpret_cast<const u32x4*>(nib_base + static_cast<size_t>(tile) * g.nb * 1024) +
                     static_cast<size_t>(p) * bpp * kTileRows + lane;
#pragma unroll
  for (int i = 0; i < kLoop; ++i)
    if (BPP || i < bpp) nib[i] = src[static_cast<size_t>(i) * kTileRows];
}

// Shared body of the two expert kernels: stream the tile's weights once and
// apply them to the expert's tokens, kTokChunk at a time.  row(m) is the bf16
// activation row of the expert's m-th token; emit(mg, m, r, v) receives the
// fp32 sum over all parts of row r for token mg (chunk position m);
// chunk_end(m0, mc) runs after the emits of a chunk (block-wide).
template <int BPP, typename RowFn, typename EmitFn, typename ChunkEndFn>
__device__ __forceinline__ void expert_tile(ExpertSmem& sm, const uint8_t* __restrict__ wn,
                                            const uint8_t* __restrict__ ws, const TiledGeom& g, int e, int tile,
                                            int M, RowFn row, EmitFn emit, ChunkEndFn chunk_end) {
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bpp = BPP ? BPP : g.bpp;
  const int plen = bpp * 32, k0 = p * plen;
  for (int m0 = 0; m0 < M; m0 += kTokChunk) {
    const int mc = min(kTokChunk, M - m0);
    // The activations are issued first, so waiting for them leaves the
    // weight loads in flight; the weights then arrive block by block while
    // the dot proceeds.  Chunks after the first re-read the tile (from L2):
    // an opaque zero offset keeps the loads and the decode inside the loop,
    // where they cost far fewer registers than 480 decoded weights would.
    XLoad xl;
    issue_x(xl, row(m0), row(mc > 1 ? m0 + 1 : m0), mc, k0, plen, lane);
    __builtin_amdgcn_sched_barrier(0);
    int opaque = 0;
    asm volatile("" : "+s"(opaque));
    u32x4 nib[kMaxBpp];
    uint32_t sc[kMaxBpp / 4];
    load_part<BPP>(wn + static_cast<size_t>(e) * g.nib_bytes + opaque, ws + static_cast<size_t>(e) * g.scale_bytes, g,
                   tile, p, lane, nib, sc);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait
    store_x(xl, sm.x[p], mc, plen, lane);
    float acc[kTokChunk];
    part_dot<BPP>(nib, sc, bpp, sm.x[p], mc, acc);
#pragma unroll
    for (int m = 0; m < kTokChunk; ++m)
      if (m < mc) sm.part[p][m][lane] = acc[m];
    __syncthreads();
    for (int q = threadIdx.x; q < mc * kTileRows; q += blockDim.x) {
      const int m = q >> 6, r = q & 63;
      float v = sm.part[0][m][r];
      for (int pp = 1; pp < g.parts; ++pp) v = v + sm.part[pp][m][r];
      emit(m0 + m, m, r, v);
    }
    chunk_end(m0, mc);
  }
}

template <int BPP>
__global__ __launch_bounds__(kTileRows * kMaxParts) __attribute__((amdgpu_waves_per_eu(3))) void w1_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w1n, const uint8_t* __restrict__ w1s,
    const uint16_t* __restrict__ b1, const int32_t* __restrict__ n_active_p, const int32_t* __restrict__ active,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_token, uint16_t* __restrict__ act,
    uint16_t* __restrict__ gate_up, int H, int I, float alpha, float limit, TiledGeom g) {
  __shared__ __attribute__((aligned(16))) ExpertSmem sm;
  const int tile = blockIdx.x;
  const int j = blockIdx.y;
  if (j >= *n_active_p) return;
  const int e = active[j];
  const int off = offsets[e];
  const int M = offsets[e + 1] - off;
  const int N1 = 2 * I;
  expert_tile<BPP>(
      sm, w1n, w1s, g, e, tile, M,
      [&](int m) { return x + static_cast<size_t>(perm_token[off + m]) * H; },
      [&](int mg, int m, int r, float v) {
        const int n = tile * kTileRows + r;
        if (b1 != nullptr) v = v + bf16_to_f32(b1[static_cast<size_t>(e) * N1 + n]);
        const uint16_t h = f32_to_bf16(v);
        sm.gu[m][r] = bf16_to_f32(h);
        if (gate_up != nullptr) gate_up[static_cast<size_t>(off + mg) * N1 + n] = h;
      },
      [&](int m0, int mc) {
        __syncthreads();
        for (int q = threadIdx.x; q < mc * (kTileRows / 2); q += blockDim.x) {
          const int m = q >> 5, jj = q & 31;
          const float r = gx_swiglu(sm.gu[m][2 * jj], sm.gu[m][2 * jj + 1], alpha, limit);
          act[static_cast<size_t>(off + m0 + m) * I + tile * (kTileRows / 2) + jj] = f32_to_bf16(r);
        }
        __syncthreads();
      });
}

template <int BPP>
__global__ __launch_bounds__(kTileRows * kMaxParts) __attribute__((amdgpu_waves_per_eu(3))) void w2_kernel(
    const uint16_t* __restrict__ act, const uint8_t* __restrict__ w2n, const uint8_t* __restrict__ w2s,
    const uint16_t* __restrict__ b2, const int32_t* __restrict__ n_active_p, const int32_t* __restrict__ active,
    const int32_t* __restrict__ offsets, uint16_t* __restrict__ y, int H, int I, TiledGeom g) {
  __shared__ __attribute__((aligned(16))) ExpertSmem sm;
  const int tile = blockIdx.x;
  const int j = blockIdx.y;
  if (j >= *n_active_p) return;
  const int e = active[j];
  const int off = offsets[e];
  const int M = offsets[e + 1] - off;
  expert_tile<BPP>(
      sm, w2n, w2s, g, e, tile, M, [&](int m) { return act + static_cast<size_t>(off + m) * I; },
      [&](int mg, int m, int r, float v) {
        const int n = tile * kTileRows + r;
        if (b2 != nullptr) v = v + bf16_to_f32(b2[static_cast<size_t>(e) * H + n]);
        y[static_cast<size_t>(off + mg) * H + n] = f32_to_bf16(v);
      },
      [&](int, int) { __syncthreads(); });
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
  for (int s = 0; s < k; ++s) {
    const int gm = gather_map[t * k + s];
    if (gm < 0) continue;
    const float ws = w[t * k + s];
    const uint4 v = *reinterpret_cast<const uint4*>(y + static_cast<size_t>(gm) * H + c * 8);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __builtin_fmaf(ws, __uint_as_float(d[i] << 16), acc[2 * i]);
      acc[2 * i + 1] = __builtin_fmaf(ws, __uint_as_float(d[i] & 0xffff0000u), acc[2 * i + 1]);
    }
  }
  if (residual != nullptr) {
    const uint4 v = *reinterpret_cast<const uint4*>(residual + static_cast<size_t>(t) * H + c * 8);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
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

__global__ void pack_nib_kernel(const uint4* __restrict__ src, int N, int nb, uint4* __restrict__ dst) {
  const size_t total = static_cast<size_t>(N) * nb;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t row = q / nb, b = q % nb;
    const size_t tile = row / kTileRows, lane = row % kTileRows;
    dst[(tile * nb + b) * kTileRows + lane] = src[q];
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

}  // namespace

template <int BPP>
static void launch_w1_t(const ExpertArgs& a, const TiledGeom& g1, hipStream_t s) {
  hipLaunchKernelGGL(w1_kernel<BPP>, dim3(g1.N / kTileRows, a.max_active), dim3(kTileRows * g1.parts), 0, s, a.x,
                     a.w1n, a.w1s, a.b1, a.plan.n_active, a.plan.active, a.plan.offsets, a.plan.perm_token, a.act,
                     a.gate_up, a.H, a.I, a.alpha, a.limit, g1);
}

template <int BPP>
static void launch_w2_t(const ExpertArgs& a, const TiledGeom& g2, hipStream_t s) {
  hipLaunchKernelGGL(w2_kernel<BPP>, dim3(g2.N / kTileRows, a.max_active), dim3(kTileRows * g2.parts), 0, s, a.act,
                     a.w2n, a.w2s, a.b2, a.plan.n_active, a.plan.active, a.plan.offsets, a.y, a.H, a.I, g2);
}

// Blocks per K-part: 15 for K = 2880 (GPT-OSS), 1 for small K; any other
// value runs the generic loop.
hipError_t launch_w1(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g1 = tiled_geom(2 * a.I, a.H);
  if (g1.bpp == 15) launch_w1_t<15>(a, g1, s);
  else if (g1.bpp == 1) launch_w1_t<1>(a, g1, s);
  else launch_w1_t<0>(a, g1, s);
  return hipGetLastError();
}

hipError_t launch_w2(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g2 = tiled_geom(a.H, a.I);
  if (g2.bpp == 15) launch_w2_t<15>(a, g2, s);
  else if (g2.bpp == 1) launch_w2_t<1>(a, g2, s);
  else launch_w2_t<0>(a, g2, s);
  return hipGetLastError();
}

hipError_t launch_combine_slots(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0) return hipSuccess;
  const int n = a.T * (a.H / 8);
  hipLaunchKernelGGL(combine8_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a.y, a.plan.gather_map, a.w, a.residual,
                     a.out, a.T, a.H, a.k);
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
                     reinterpret_cast<uint4*>(tiled_nib));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(pack_scale_kernel, dim3(256), dim3(256), 0, s, scales, N, g, tiled_scales);
  return hipGetLastError();
}

}  // namespace gxmoe
