// moe_stages.hip -- single-stage kernels of the MoE block (gfx950).
//
// The fused decode path (moe_route.hip, moe_experts.hip) does not need these;
// they are the C-ABI replacements of the reference's individual launchers,
// with the same arithmetic as the fused kernels so every stage can be checked
// on its own:
//   dense MXFP4 GEMV   fused_mxfp4_gemv_forward   (fused_mxfp4_gemv.cu:452-464)
//   SwiGLU             swiglu_forward             (swiglu.cu:178-211)
//   combine            moe_combine_forward        (moe_combine.cu:175-204)
//   scatter            moe_scatter_tokens         (moe_permute.cu:241-259)
//   dequant            mxfp4_dequant_batched      (mxfp4_dequant.cu:353-375)
//   RMSNorm            rmsnorm_forward            (rmsnorm.cu:47-83), used by
//                      the layer's forward() entry.
#include "moe_device.h"
#include "moe_kernels.h"
#include "moe_stages.h"

namespace gxmoe {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kRows = 8;  // token rows per work-group of the dense GEMV

// Dense MXFP4 GEMV: grid (N/64 tiles, ceil(M/8)), 64*P threads.  Lane = row
// of the tile, wave = K-part; same canonical dot as the fused expert kernels.
__global__ __launch_bounds__(kTileRows * kMaxParts) void dense_gemv_kernel(
    const uint16_t* __restrict__ x, int M, const uint8_t* __restrict__ wn, const uint8_t* __restrict__ ws,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, TiledGeom g) {
  __shared__ float s_part[kMaxParts][kRows][kTileRows];
  const int tile = blockIdx.x;
  const int m0 = blockIdx.y * kRows;
  const int mc = min(kRows, M - m0);
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int K = g.K;
  const uint32_t* src = reinterpret_cast<const uint32_t*>(wn + static_cast<size_t>(tile) * g.nb * 1024) +
                        static_cast<size_t>(p) * g.bpp * 256 + tiled_dword(lane, 0);
  const uint8_t* sc = ws + (static_cast<size_t>(tile) * g.parts + p) * kTileRows * g.spad +
                      static_cast<size_t>(lane) * g.spad;
  float acc[kRows];
#pragma unroll
  for (int m = 0; m < kRows; ++m) acc[m] = 0.0f;
  for (int i = 0; i < g.bpp; ++i) {
    const u32x4 blk = load_row_block(src + static_cast<size_t>(i) * 256);
    const uint32_t code = sc[i];
    const int kb = (p * g.bpp + i) * 32;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float wf[8];
      decode8(blk[d], code, wf);
#pragma unroll
      for (int m = 0; m < kRows; ++m) {
        if (m < mc) {
          const uint16_t* xr = x + static_cast<size_t>(m0 + m) * K + kb + d * 8;
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[m] = __builtin_fmaf(bf16_to_f32(xr[c]), wf[c], acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kRows; ++m)
    if (m < mc) s_part[p][m][lane] = acc[m];
  __syncthreads();
  for (int q = threadIdx.x; q < mc * kTileRows; q += blockDim.x) {
    const int m = q >> 6, r = q & 63;
    float v = s_part[0][m][r];
    for (int pp = 1; pp < g.parts; ++pp) v = v + s_part[pp][m][r];
    const int n = tile * kTileRows + r;
    if (bias != nullptr) v = v + bf16_to_f32(bias[n]);
    y[static_cast<size_t>(m0 + m) * g.N + n] = f32_to_bf16(v);
  }
}

__global__ void swiglu_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out, int T, int I,
                              float alpha, float limit) {
  const size_t total = static_cast<size_t>(T) * I;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t t = q / I, j = q % I;
    const float g = bf16_to_f32(in[t * 2 * I + 2 * j]);
    const float u = bf16_to_f32(in[t * 2 * I + 2 * j + 1]);
    out[q] = f32_to_bf16(gx_swiglu(g, u, alpha, limit));
  }
}

__global__ void combine_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ y,
                               const int32_t* __restrict__ gather_map, const float* __restrict__ w,
                               const uint16_t* __restrict__ residual, int T, int H, int k) {
  const size_t total = static_cast<size_t>(T) * H;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int t = static_cast<int>(q / H), n = static_cast<int>(q % H);
    float acc = 0.0f;
    for (int s = 0; s < k; ++s) {
      const int gm = gather_map[t * k + s];
      if (gm < 0) continue;
      acc = __builtin_fmaf(w[t * k + s], bf16_to_f32(y[static_cast<size_t>(gm) * H + n]), acc);
    }
    if (residual != nullptr) acc = acc + bf16_to_f32(residual[q]);
    out[q] = f32_to_bf16(acc);
  }
}

__global__ void scatter_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ gather_map,
                               uint16_t* __restrict__ permuted, int T, int H, int k) {
  const int S = T * k;
  const int chunks = H / 8;
  const size_t total = static_cast<size_t>(S) * chunks;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int s = static_cast<int>(q / chunks), c = static_cast<int>(q % chunks);
    const int gm = gather_map[s];
    if (gm < 0) continue;
    reinterpret_cast<uint4*>(permuted + static_cast<size_t>(gm) * H)[c] =
        reinterpret_cast<const uint4*>(x + static_cast<size_t>(s / k) * H)[c];
  }
}

__global__ void dequant_kernel(const uint8_t* __restrict__ wn, const uint8_t* __restrict__ ws, TiledGeom g,
                               uint16_t* __restrict__ out) {
  // one thread per (row, block): 32 outputs
  const size_t total = static_cast<size_t>(g.N) * g.nb;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < total;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t row = q / g.nb, b = q % g.nb;
    const size_t tile = row / kTileRows, lane = row % kTileRows;
    const u32x4 blk = load_row_block(reinterpret_cast<const uint32_t*>(wn) + (tile * g.nb + b) * 256 +
                                     tiled_dword(static_cast<int>(lane), 0));
    const size_t p = b / g.bpp, i = b % g.bpp;
    const uint32_t code = ws[((tile * g.parts + p) * kTileRows + lane) * g.spad + i];
    uint16_t* o = out + row * g.K + b * 32;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      float wf[8];
      decode8(blk[d], code, wf);
#pragma unroll
      for (int c = 0; c < 8; ++c) o[d * 8 + c] = f32_to_bf16(wf[c]);
    }
  }
}

// RMSNorm: sum of squares with the gemv_bf16 tree (256 strided chains of
// 8-element chunks, xor butterfly, 4 waves in order), inv = 1/sqrt(mean+eps),
// out = bf16((x * inv) * w).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                     uint16_t* __restrict__ out, int H, float eps) {
  __shared__ float s_w[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  const uint16_t* xr = x + static_cast<size_t>(t) * H;
  float acc = 0.0f;
  const int KV = H >> 3;
  for (int kv = tid; kv < KV; kv += 256) {
    const uint4 v = reinterpret_cast<const uint4*>(xr)[kv];
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __uint_as_float(d[i] << 16), b = __uint_as_float(d[i] & 0xffff0000u);
      acc = __builtin_fmaf(a, a, acc);
      acc = __builtin_fmaf(b, b, acc);
    }
  }
  for (int kk = KV * 8 + tid; kk < H; kk += 256) {
    const float a = bf16_to_f32(xr[kk]);
    acc = __builtin_fmaf(a, a, acc);
  }
  acc = wave_butterfly_sum(acc);
  if (lane == 0) s_w[warp] = acc;
  __syncthreads();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = ss + s_w[i];
  const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(H) + eps);
  for (int h = tid; h < H; h += 256)
    out[static_cast<size_t>(t) * H + h] = f32_to_bf16((bf16_to_f32(xr[h]) * inv) * bf16_to_f32(w[h]));
}

// Fused residual + RMSNorm (rmsnorm.cu:224-337): s = r + d in fp32 (kept
// per chunk: a thread's chunks are kv = tid, tid + 256), sum_out = bf16(s),
// the sum of squares of s with the same tree as rmsnorm_kernel, then
// normed = bf16((s * inv) * w).
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(const uint16_t* __restrict__ r,
                                                               const uint16_t* __restrict__ d,
                                                               const uint16_t* __restrict__ w,
                                                               uint16_t* __restrict__ normed,
                                                               uint16_t* __restrict__ sum_out, int H, float eps) {
  __shared__ float s_w[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, warp = tid >> 6;
  const size_t row = static_cast<size_t>(t) * H;
  const int KV = H >> 3;
  auto sum8 = [&](int kv, float (&s8)[8]) __attribute__((always_inline)) {
    const uint4 a = reinterpret_cast<const uint4*>(r + row)[kv];
    const uint4 b = reinterpret_cast<const uint4*>(d + row)[kv];
    const uint32_t da[4] = {a.x, a.y, a.z, a.w}, db[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s8[2 * i] = __uint_as_float(da[i] << 16) + __uint_as_float(db[i] << 16);
      s8[2 * i + 1] = __uint_as_float(da[i] & 0xffff0000u) + __uint_as_float(db[i] & 0xffff0000u);
    }
  };
  float acc = 0.0f;
  for (int kv = tid; kv < KV; kv += 256) {
    float s8[8];
    sum8(kv, s8);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(s8[i], s8[i], acc);
    if (sum_out) {
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = f32_to_bf16(s8[2 * i]) | (static_cast<uint32_t>(f32_to_bf16(s8[2 * i + 1])) << 16);
      reinterpret_cast<uint4*>(sum_out + row)[kv] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  for (int kk = KV * 8 + tid; kk < H; kk += 256) {
    const float v = bf16_to_f32(r[row + kk]) + bf16_to_f32(d[row + kk]);
    acc = __builtin_fmaf(v, v, acc);
    if (sum_out) sum_out[row + kk] = f32_to_bf16(v);
  }
  acc = wave_butterfly_sum(acc);
  if (lane == 0) s_w[warp] = acc;
  __syncthreads();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = ss + s_w[i];
  const float inv = 1.0f / __builtin_sqrtf(ss / static_cast<float>(H) + eps);
  for (int h = tid; h < H; h += 256) {
    const float v = bf16_to_f32(r[row + h]) + bf16_to_f32(d[row + h]);
    normed[row + h] = f32_to_bf16((v * inv) * bf16_to_f32(w[h]));
  }
}

int grid_for(size_t total, int threads) {
  size_t b = (total + threads - 1) / threads;
  if (b > 4096) b = 4096;
  if (b < 1) b = 1;
  return static_cast<int>(b);
}

}  // namespace

hipError_t launch_dense_gemv(const uint16_t* x, int M, const uint8_t* wn, const uint8_t* ws, const uint16_t* bias,
                             uint16_t* y, int N, int K, hipStream_t s) {
  if (M <= 0) return hipSuccess;
  const TiledGeom g = tiled_geom(N, K);
  hipLaunchKernelGGL(dense_gemv_kernel, dim3(N / kTileRows, (M + kRows - 1) / kRows), dim3(kTileRows * g.parts), 0,
                     s, x, M, wn, ws, bias, y, g);
  return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* in, uint16_t* out, int T, int I, float alpha, float limit, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(static_cast<size_t>(T) * I, 256)), dim3(256), 0, s, in, out, T, I,
                     alpha, limit);
  return hipGetLastError();
}

hipError_t launch_combine(uint16_t* out, const uint16_t* y, const int32_t* gather_map, const float* w,
                          const uint16_t* residual, int T, int H, int k, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3(grid_for(static_cast<size_t>(T) * H, 256)), dim3(256), 0, s, out, y,
                     gather_map, w, residual, T, H, k);
  return hipGetLastError();
}

hipError_t launch_scatter(const uint16_t* x, const int32_t* gather_map, uint16_t* permuted, int T, int H, int k,
                          hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(scatter_kernel, dim3(grid_for(static_cast<size_t>(T) * k * (H / 8), 256)), dim3(256), 0, s, x,
                     gather_map, permuted, T, H, k);
  return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* wn, const uint8_t* ws, int N, int K, uint16_t* out, hipStream_t s) {
  const TiledGeom g = tiled_geom(N, K);
  hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(static_cast<size_t>(N) * g.nb, 256)), dim3(256), 0, s, wn, ws, g,
                     out);
  return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(const uint16_t* r, const uint16_t* d, const uint16_t* w, uint16_t* normed,
                                   uint16_t* sum_out, int T, int H, float eps, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(T), dim3(256), 0, s, r, d, w, normed, sum_out, H, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int T, int H, float eps,
                          hipStream_t s) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, s, x, w, out, H, eps);
  return hipGetLastError();
}

}  // namespace gxmoe
