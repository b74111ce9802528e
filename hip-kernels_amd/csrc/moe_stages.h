// moe_stages.h -- host launchers of the single-stage kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gxmoe {

hipError_t launch_dense_gemv(const uint16_t* x, int M, const uint8_t* wn, const uint8_t* ws, const uint16_t* bias,
                             uint16_t* y, int N, int K, hipStream_t s);
hipError_t launch_swiglu(const uint16_t* in, uint16_t* out, int T, int I, float alpha, float limit, hipStream_t s);
hipError_t launch_combine(uint16_t* out, const uint16_t* y, const int32_t* gather_map, const float* w,
                          const uint16_t* residual, int T, int H, int k, hipStream_t s);
hipError_t launch_scatter(const uint16_t* x, const int32_t* gather_map, uint16_t* permuted, int T, int H, int k,
                          hipStream_t s);
hipError_t launch_dequant(const uint8_t* wn, const uint8_t* ws, int N, int K, uint16_t* out, hipStream_t s);
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint16_t* out, int T, int H, float eps,
                          hipStream_t s);
// fused_residual_rmsnorm_forward: s = r + d (fp32), sum_out = bf16(s) (may be
// null), normed = bf16((s * inv) * w), inv from the gemv-tree sum of s^2.
hipError_t launch_residual_rmsnorm(const uint16_t* r, const uint16_t* d, const uint16_t* w, uint16_t* normed,
                                   uint16_t* sum_out, int T, int H, float eps, hipStream_t s);

}  // namespace gxmoe
