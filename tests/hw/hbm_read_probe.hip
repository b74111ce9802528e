// hbm_read_probe.hip -- measurement infrastructure: the HBM read rate a plain
// streaming kernel reaches on this device, the practical ceiling against
// which the decode streams' rate is compared (the 8 TB/s figure is the
// published peak, not what a read reaches).
//
// One pass over a buffer with 16-byte nontemporal loads: work-group b of G
// (256 threads) reads the 256 x U pieces of its stripe, stripes G apart;
// every lane issues U loads before it uses any.  Lanes past the end read the
// last piece (in bounds).  The loaded words are folded into one value that
// is stored only if it equals a constant, so the loads stay live and nothing
// is written in practice.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink) {
  uint32_t acc = 0;
  const size_t stride = static_cast<size_t>(gridDim.x) * 256 * U;
  for (size_t base = static_cast<size_t>(blockIdx.x) * 256 * U + threadIdx.x; base < n16; base += stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + 256 * u;
      v[u] = __builtin_nontemporal_load(p + (i < n16 ? i : n16 - 1));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// One read pass over `bytes` bytes at `p` (16-byte aligned, a multiple of 16,
// at least 16) with `grid` work-groups of 256 threads and `unroll` loads in
// flight per lane (2, 4 or 8), on `stream`.  `sink` holds 256 words.
// Returns 0, or -1 for invalid arguments, or the HIP error of the launch.
int hbm_read_probe(const void* p, size_t bytes, int grid, int unroll, uint32_t* sink, hipStream_t stream) {
  if (p == nullptr || sink == nullptr || bytes < 16 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(p) & 15) ||
      grid < 1 || grid > (1 << 20))
    return -1;
  const u32x4* q = static_cast<const u32x4*>(p);
  const size_t n16 = bytes / 16;
  switch (unroll) {
    case 2: hipLaunchKernelGGL(read_kernel<2>, dim3(grid), dim3(256), 0, stream, q, n16, sink); break;
    case 4: hipLaunchKernelGGL(read_kernel<4>, dim3(grid), dim3(256), 0, stream, q, n16, sink); break;
    case 8: hipLaunchKernelGGL(read_kernel<8>, dim3(grid), dim3(256), 0, stream, q, n16, sink); break;
    default: return -1;
  }
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
