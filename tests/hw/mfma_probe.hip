// mfma_probe.hip -- test infrastructure, not part of the library: one wave
// runs one matrix-core instruction on operands the test gives, so the
// tests can pin how the instruction sums its products.
//
//   mfma_probe_bf16     v_mfma_f32_16x16x32_bf16          a, b: [64 lanes][4] dwords
//   mfma_probe_f8f6f4   v_mfma_scale_f32_16x16x128_f8f6f4 a, b: [64 lanes][8] dwords,
//                       A as e4m3 (a_fp4 = 0) or e2m1 (a_fp4 = 1, dwords 0..3), B as e4m3,
//                       scale dwords sa, sb per lane (e8m0 bytes, byte 0 used)
//
// d: [64 lanes][4] fp32, the lane's accumulator registers after one
// instruction from zero.  Pointers are device pointers; the calls are
// synchronous and return a hipError_t.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(64) void bf16_kernel(const uint32_t* a, const uint32_t* b, float* d) {
  const int l = threadIdx.x;
  const u32x4_t av{a[4 * l], a[4 * l + 1], a[4 * l + 2], a[4 * l + 3]};
  const u32x4_t bv{b[4 * l], b[4 * l + 1], b[4 * l + 2], b[4 * l + 3]};
  const f32x4_t r = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                             __builtin_bit_cast(bf16x8_t, bv),
                                                             f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
  for (int i = 0; i < 4; ++i) d[4 * l + i] = r[i];
}

template <int kAFmt>
__global__ __launch_bounds__(64) void f8f6f4_kernel(const uint32_t* a, const uint32_t* b, const uint32_t* sa,
                                                     const uint32_t* sb, float* d) {
  const int l = threadIdx.x;
  i32x8_t av, bv;
  for (int i = 0; i < 8; ++i) {
    av[i] = static_cast<int>(a[8 * l + i]);
    bv[i] = static_cast<int>(b[8 * l + i]);
  }
  const f32x4_t r = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
      av, bv, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, kAFmt, 0, 0, static_cast<int>(sa[l]), 0, static_cast<int>(sb[l]));
  for (int i = 0; i < 4; ++i) d[4 * l + i] = r[i];
}

extern "C" {

int mfma_probe_bf16(const uint32_t* a, const uint32_t* b, float* d) {
  hipLaunchKernelGGL(bf16_kernel, dim3(1), dim3(64), 0, nullptr, a, b, d);
  hipError_t e = hipGetLastError();
  return e != hipSuccess ? e : hipDeviceSynchronize();
}

int mfma_probe_f8f6f4(const uint32_t* a, const uint32_t* b, const uint32_t* sa, const uint32_t* sb, int a_fp4,
                      float* d) {
  if (a_fp4)
    hipLaunchKernelGGL(f8f6f4_kernel<4>, dim3(1), dim3(64), 0, nullptr, a, b, sa, sb, d);
  else
    hipLaunchKernelGGL(f8f6f4_kernel<0>, dim3(1), dim3(64), 0, nullptr, a, b, sa, sb, d);
  hipError_t e = hipGetLastError();
  return e != hipSuccess ? e : hipDeviceSynchronize();
}

}  // extern "C"
