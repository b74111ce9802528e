// moe_kernels.h -- host-side launchers of the gfx950 MoE kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gxmoe {

constexpr int kMaxExperts = 256;  // LDS tables of the routing plan
constexpr int kMaxTopK = 8;       // topk_softmax.cu:34
constexpr int kRouteTokensPerGroup = 8;
constexpr int kRouteExpertsPerGroup = 4;
constexpr int kTileRows = 64;     // rows of an MXFP4 tile (one per lane)
constexpr int kMaxParts = 6;      // K-parts of the canonical dot (waves per tile)
constexpr int kTaskInts = 16;     // ints per expert task record
constexpr int kTaskTokens = 12;   // token ids held inline in a task record

// Number of contiguous K-parts of the canonical expert dot for K inputs:
// the largest p <= 6 dividing K/32.
inline int dot_parts(int K) {
  int nb = K / 32;
  for (int p = kMaxParts; p > 1; --p)
    if (nb % p == 0) return p;
  return 1;
}

// Tiled MXFP4 geometry of one [N, K] matrix.
struct TiledGeom {
  int N, K;
  int nb;      // K / 32 blocks per row
  int parts;   // dot_parts(K)
  int bpp;     // blocks per part
  int spad;    // scale bytes per (tile, part, lane), multiple of 4
  size_t nib_bytes;    // N * K / 2
  size_t scale_bytes;  // (N/64) * parts * 64 * spad
};
TiledGeom tiled_geom(int N, int K);

// Routing plan produced on the device.
struct PlanBufs {
  int32_t* counts;      // [E]
  int32_t* offsets;     // [E+1]
  int32_t* gather_map;  // [T*k]
  int32_t* perm_token;  // [T*k]
  int32_t* active;      // [E]
  int32_t* n_active;    // [1]
  // [E][kTaskInts] or null: record j describes the j-th active expert as
  // {expert, offset, count, 0, token ids of its first kTaskTokens slots};
  // records j >= n_active hold expert -1.  One load gives an expert kernel
  // everything it needs to start streaming weights and activations.
  int32_t* tasks;
};

struct RouteArgs {
  const uint16_t* x;       // [T][H] bf16
  const uint16_t* W;       // [E][H] bf16
  const uint16_t* b;       // [E] bf16 or null
  int T, E, H, k;
  int logits_fp32;         // 1: fp32 logits, 0: bf16 logits
  void* logits;            // [T][E]
  float* xf;               // [T][H] fp32 copy of x, or null
  int32_t* idx;            // [T][k]
  float* w;                // [T][k]
  PlanBufs plan;           // plan outputs (all may be null to skip the plan)
  uint32_t* group_counter; // [ceil(T/8)] zero at rest
  uint32_t* done_counter;  // [1] zero at rest
  float* xchg_logits;      // [T][E] fp32 exchange (the logits as rounded)
  int32_t* xchg_idx;       // [T][k] exchange of the selections (T > 8)
};

// Bytes of route scratch: counters, then the exchange buffers (256-aligned).
size_t route_scratch_bytes(int T, int E, int k);
void route_scratch_carve(void* scratch, int T, int E, int k, RouteArgs& a);
hipError_t launch_route(const RouteArgs& a, hipStream_t s);

// Standalone top-k softmax over given logits (bf16 or fp32).
hipError_t launch_topk(const void* logits, int logits_fp32, int T, int E, int k,
                       int32_t* idx, float* w, int32_t* tokens_per_expert, hipStream_t s);

// Standalone plan (histogram, scan, stable gather map) from expert indices.
hipError_t launch_plan(const int32_t* idx, int T, int k, int E, PlanBufs plan, hipStream_t s);

struct ExpertArgs {
  const uint16_t* x;          // [T][H] bf16 expert input (the normed activations)
  const uint8_t* w1n;         // tiled W1 nibbles, [E] x geom1.nib_bytes
  const uint8_t* w1s;         // tiled W1 scales,  [E] x geom1.scale_bytes
  const uint16_t* b1;         // [E][2I] or null
  const uint8_t* w2n;         // tiled W2 nibbles
  const uint8_t* w2s;         // tiled W2 scales
  const uint16_t* b2;         // [E][H] or null
  int T, E, H, I, k;
  float alpha, limit;
  PlanBufs plan;
  const float* w;             // [T][k] routing weights
  uint16_t* act;              // [T*k][I] bf16 SwiGLU output (permuted order)
  uint16_t* gate_up;          // [T*k][2I] bf16 or null (debug output)
  uint16_t* y;                // [T*k][H] bf16 expert outputs
  const uint16_t* residual;   // [T][H] or null
  uint16_t* out;              // [T][H]
  int max_active;             // grid bound on active experts: min(E, T*k)
};
hipError_t launch_experts(const ExpertArgs& a, hipStream_t s);
// The two launches of launch_experts, for callers that time them separately.
hipError_t launch_w1(const ExpertArgs& a, hipStream_t s);
hipError_t launch_w2(const ExpertArgs& a, hipStream_t s);
hipError_t launch_combine_slots(const ExpertArgs& a, hipStream_t s);

// Grouped MXFP4 product on the matrix cores (prefill): for each expert e and
// permuted position p in [offsets[e], offsets[e+1]),
//   y[p][n] = bf16(sum_k x[row(p)][k] * W_e[n][k] + bias[e][n]),
// row(p) = row_index[p] (or p when row_index is null).  gated: out[p][n/2] =
// bf16(SwiGLU(y[p][n], y[p][n+1])) for even n (gate_up optionally gets y);
// else out[p][n] = y[p][n].  rows bounds offsets[E] (the grid is sized by it).
struct GroupedArgs {
  const uint16_t* x;
  const int32_t* row_index;
  const int32_t* offsets;
  int E, rows;
  const uint8_t* wn;   // tiled nibbles, [E] x tiled_geom(N, K).nib_bytes
  const uint8_t* ws;   // tiled scales
  int N, K;
  const uint16_t* bias;
  uint16_t* out;
  uint16_t* gate_up;
  int gated;
  float alpha, limit;
};
bool grouped_supported(int N, int K, int E);
hipError_t launch_grouped_mxfp4(const GroupedArgs& a, hipStream_t s);

// Row-major MXFP4 [N][K/2] + [N][K/32] -> tiled layout.
hipError_t launch_pack_tiled(const uint8_t* packed, const uint8_t* scales, int N, int K,
                             uint8_t* tiled_nib, uint8_t* tiled_scales, hipStream_t s);

}  // namespace gxmoe
