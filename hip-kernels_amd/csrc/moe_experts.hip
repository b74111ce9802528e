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

constexpr int kMaxBpp = 16;       // blocks per part kept resident in VGPRs
constexpr int kTokChunk = 8;      // tokens per pass over the resident weights

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Accumulate one lane's part of the canonical dot for up to kTokChunk token
// rows.  `nib` holds the lane's bpp 16-byte blocks, `sc` its scale bytes.
// xrow[m] points at the fp32 activations of token m, already offset to the
// first k of this part.
__device__ __forceinline__ void part_dot(const u32x4 (&nib)[kMaxBpp], const uint32_t (&sc)[kMaxBpp / 4],
                                         int bpp, const float* const (&xrow)[kTokChunk], int mc,
                                         float (&acc)[kTokChunk]) {
#pragma unroll
  for (int m = 0; m < kTokChunk; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxBpp; ++i) {
    if (i < bpp) {
      const uint32_t code = (sc[i >> 2] >> (8 * (i & 3))) & 0xffu;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float wf[8];
        decode8(nib[i][d], code, wf);
#pragma unroll
        for (int m = 0; m < kTokChunk; ++m) {
          if (m < mc) {
            const float* __restrict__ xr = xrow[m] + i * 32 + d * 8;
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[m] = __builtin_fmaf(xr[c], wf[c], acc[m]);
          }
        }
      }
    }
  }
}

// Load a lane's resident blocks and scales of tile `tile`, part `p`.
__device__ __forceinline__ void load_part(const uint8_t* __restrict__ nib_base, const uint8_t* __restrict__ sc_base,
                                          const TiledGeom& g, int tile, int p, int lane,
                                          u32x4 (&nib)[kMaxBpp], uint32_t (&sc)[kMaxBpp / 4]) {
  const u32x4* src = reinterpret_cast<const u32x4*>(nib_base + static_cast<size_t>(tile) * g.nb * 1024) +
                     static_cast<size_t>(p) * g.bpp * kTileRows + lane;
#pragma unroll
  for (int i = 0; i < kMaxBpp; ++i)
    if (i < g.bpp) nib[i] = __builtin_nontemporal_load(src + static_cast<size_t>(i) * kTileRows);
  const uint32_t* s32 = reinterpret_cast<const uint32_t*>(
      sc_base + (static_cast<size_t>(tile) * g.parts + p) * kTileRows * g.spad + static_cast<size_t>(lane) * g.spad);
#pragma unroll
  for (int q = 0; q < kMaxBpp / 4; ++q)
    if (q * 4 < g.bpp) sc[q] = s32[q];
}

__global__ __launch_bounds__(kTileRows * kMaxParts) __attribute__((amdgpu_waves_per_eu(3))) void w1_kernel(
    const float* __restrict__ xf, const uint8_t* __restrict__ w1n, const uint8_t* __restrict__ w1s,
    const uint16_t* __restrict__ b1, const int32_t* __restrict__ n_active_p, const int32_t* __restrict__ active,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm_token, float* __restrict__ act,
    uint16_t* __restrict__ gate_up, int H, int I, float alpha, float limit, TiledGeom g) {
  const int tile = blockIdx.x;
  const int j = blockIdx.y;
  const int n_active = *n_active_p;
  if (j >= n_active) return;
  const int e = active[j];
  const int off = offsets[e];
  const int M = offsets[e + 1] - off;
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int P = g.parts, N1 = 2 * I;

  __shared__ float s_part[kMaxParts][kTokChunk][kTileRows];
  __shared__ float s_gu[kTokChunk][kTileRows];

  u32x4 nib[kMaxBpp];
  uint32_t sc[kMaxBpp / 4];
  load_part(w1n + static_cast<size_t>(e) * g.nib_bytes, w1s + static_cast<size_t>(e) * g.scale_bytes, g,
            tile, p, lane, nib, sc);
  const int k0 = p * g.bpp * 32;

  for (int m0 = 0; m0 < M; m0 += kTokChunk) {
    const int mc = min(kTokChunk, M - m0);
    const float* xrow[kTokChunk];
#pragma unroll
    for (int m = 0; m < kTokChunk; ++m) {
      const int tok = (m < mc) ? perm_token[off + m0 + m] : 0;
      xrow[m] = xf + static_cast<size_t>(tok) * H + k0;
    }
    float acc[kTokChunk];
    part_dot(nib, sc, g.bpp, xrow, mc, acc);
#pragma unroll
    for (int m = 0; m < kTokChunk; ++m)
      if (m < mc) s_part[p][m][lane] = acc[m];
    __syncthreads();
    for (int q = threadIdx.x; q < mc * kTileRows; q += blockDim.x) {
      const int m = q >> 6, r = q & 63;
      float v = s_part[0][m][r];
      for (int pp = 1; pp < P; ++pp) v = v + s_part[pp][m][r];
      const int n = tile * kTileRows + r;
      if (b1 != nullptr) v = v + bf16_to_f32(b1[static_cast<size_t>(e) * N1 + n]);
      const uint16_t h = f32_to_bf16(v);
      s_gu[m][r] = bf16_to_f32(h);
      if (gate_up != nullptr) gate_up[static_cast<size_t>(off + m0 + m) * N1 + n] = h;
    }
    __syncthreads();
    for (int q = threadIdx.x; q < mc * (kTileRows / 2); q += blockDim.x) {
      const int m = q >> 5, jj = q & 31;
      const float r = gx_swiglu(s_gu[m][2 * jj], s_gu[m][2 * jj + 1], alpha, limit);
      act[static_cast<size_t>(off + m0 + m) * I + tile * (kTileRows / 2) + jj] = round_bf16(r);
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kTileRows * kMaxParts) __attribute__((amdgpu_waves_per_eu(3))) void w2_kernel(
    const float* __restrict__ act, const uint8_t* __restrict__ w2n, const uint8_t* __restrict__ w2s,
    const uint16_t* __restrict__ b2, const int32_t* __restrict__ n_active_p, const int32_t* __restrict__ active,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ gather_map, const float* __restrict__ w,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ y, uint16_t* __restrict__ out,
    uint32_t* __restrict__ tile_counter, int T, int H, int I, int k, TiledGeom g) {
  const int tile = blockIdx.x;
  const int j = blockIdx.y;
  const int n_active = *n_active_p;
  if (j >= n_active) return;
  const int e = active[j];
  const int off = offsets[e];
  const int M = offsets[e + 1] - off;
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int P = g.parts;

  __shared__ float s_part[kMaxParts][kTokChunk][kTileRows];
  __shared__ uint32_t s_ticket;

  u32x4 nib[kMaxBpp];
  uint32_t sc[kMaxBpp / 4];
  load_part(w2n + static_cast<size_t>(e) * g.nib_bytes, w2s + static_cast<size_t>(e) * g.scale_bytes, g,
            tile, p, lane, nib, sc);
  const int k0 = p * g.bpp * 32;

  for (int m0 = 0; m0 < M; m0 += kTokChunk) {
    const int mc = min(kTokChunk, M - m0);
    const float* xrow[kTokChunk];
#pragma unroll
    for (int m = 0; m < kTokChunk; ++m)
      xrow[m] = act + static_cast<size_t>(off + m0 + (m < mc ? m : 0)) * I + k0;
    float acc[kTokChunk];
    part_dot(nib, sc, g.bpp, xrow, mc, acc);
#pragma unroll
    for (int m = 0; m < kTokChunk; ++m)
      if (m < mc) s_part[p][m][lane] = acc[m];
    __syncthreads();
    for (int q = threadIdx.x; q < mc * kTileRows; q += blockDim.x) {
      const int m = q >> 6, r = q & 63;
      float v = s_part[0][m][r];
      for (int pp = 1; pp < P; ++pp) v = v + s_part[pp][m][r];
      const int n = tile * kTileRows + r;
      if (b2 != nullptr) v = v + bf16_to_f32(b2[static_cast<size_t>(e) * H + n]);
      y[static_cast<size_t>(off + m0 + m) * H + n] = f32_to_bf16(v);
    }
    __syncthreads();
  }

  // The last active expert to finish this tile combines it for every token
  // (moe_combine.cu:69-115 order: accum = sum_k fma(w_k, y_k), then + residual).
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) s_ticket = atomicAdd(&tile_counter[tile], 1u);
  __syncthreads();
  if (s_ticket != static_cast<uint32_t>(n_active - 1)) return;
  __threadfence();
  if (threadIdx.x == 0) tile_counter[tile] = 0u;
  const uint16_t* ycomb = y;  // written by other work-groups: plain (vector) loads after the fence
  for (int q = threadIdx.x; q < T * kTileRows; q += blockDim.x) {
    const int t = q >> 6, n = tile * kTileRows + (q & 63);
    float acc = 0.0f;
    for (int s = 0; s < k; ++s) {
      const int gm = gather_map[t * k + s];
      if (gm < 0) continue;
      acc = __builtin_fmaf(w[t * k + s], bf16_to_f32(ycomb[static_cast<size_t>(gm) * H + n]), acc);
    }
    if (residual != nullptr) acc = acc + bf16_to_f32(residual[static_cast<size_t>(t) * H + n]);
    out[static_cast<size_t>(t) * H + n] = f32_to_bf16(acc);
  }
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

hipError_t launch_w1(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g1 = tiled_geom(2 * a.I, a.H);
  hipLaunchKernelGGL(w1_kernel, dim3(g1.N / kTileRows, a.max_active), dim3(kTileRows * g1.parts), 0, s, a.xf, a.w1n,
                     a.w1s, a.b1, a.plan.n_active, a.plan.active, a.plan.offsets, a.plan.perm_token, a.act,
                     a.gate_up, a.H, a.I, a.alpha, a.limit, g1);
  return hipGetLastError();
}

hipError_t launch_w2(const ExpertArgs& a, hipStream_t s) {
  if (a.T <= 0 || a.max_active <= 0) return hipSuccess;
  const TiledGeom g2 = tiled_geom(a.H, a.I);
  hipLaunchKernelGGL(w2_kernel, dim3(g2.N / kTileRows, a.max_active), dim3(kTileRows * g2.parts), 0, s, a.act, a.w2n,
                     a.w2s, a.b2, a.plan.n_active, a.plan.active, a.plan.offsets, a.plan.gather_map, a.w,
                     a.residual, a.y, a.out, a.tile_counter, a.T, a.H, a.I, a.k, g2);
  return hipGetLastError();
}

hipError_t launch_experts(const ExpertArgs& a, hipStream_t s) {
  hipError_t err = launch_w1(a, s);
  if (err != hipSuccess) return err;
  return launch_w2(a, s);
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
