// moe_kernels.h -- host-side launchers of the gfx950 MoE kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <hip/hip_ext.h>

namespace gxmoe {

// Optional per-launch timing: with start set, the kernel is launched through
// hipExtLaunchKernelGGL, which stamps start/stop with the dispatch's own
// begin and end (no marker packets between launches).
struct KernelTimer {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Either event may be null (a sequence of launches timed from the first
// one's start to the last one's stop).
template <typename F, typename... Args>
inline void gx_launch(F kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t s, const KernelTimer& t,
                      Args... args) {
  if (t.start || t.stop)
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(shmem), s, t.start, t.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}

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
//
// Nibbles: per 64-row tile t and 32-element block b, one KiB at
// (t * nb + b) * 1024 of [64 slots][4 dwords].  Slot s = 16 g + j holds, in
// dword i, bytes 4g..4g+3 (elements 8g..8g+7, low nibble first) of row
// 64 t + 16 i + j's block b.  A wave's 16-byte load of slot `lane` is then
// the A operand of four 16x16x32 matrix-core products (sub-tiles i = 0..3)
// for one block, and row r's 16 bytes are the dwords (16 g + r % 16, r / 16).
//
// Scales, two regions per matrix:
//   [0, mscale_off): per (tile, K-part, row) one group of spad e8m0 bytes
//     (the part's blocks, zero-padded), the order the exact kernels read;
//   [mscale_off, scale_bytes): per (tile, block) 64 bytes, byte 4 j + i =
//     the scale of row 64 t + 16 i + j, the order of the nibble slots.
struct TiledGeom {
  int N, K;
  int nb;      // K / 32 blocks per row
  int parts;   // dot_parts(K)
  int bpp;     // blocks per part
  int spad;    // scale bytes per (tile, part, lane), multiple of 4
  size_t nib_bytes;    // N * K / 2
  size_t mscale_off;   // (N/64) * parts * 64 * spad
  size_t scale_bytes;  // mscale_off + N * nb
};
TiledGeom tiled_geom(int N, int K);

// Dword index (within one 64-row tile's block KiB) of dword g of row r's
// 16-byte block: slot 16 g + r % 16, dword r / 16.
__host__ __device__ constexpr int tiled_dword(int r, int g) { return (16 * g + (r & 15)) * 4 + (r >> 4); }

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
  // Scratch of the multi-launch plan for many slots (plan_chunk_ints(S, E)
  // ints), or null: one work-group builds the plan.
  int32_t* chunk;
};

// Ints of PlanBufs::chunk for S slots and E experts: per 1024-slot chunk
// and expert a count (then a base), and each expert's active index.
constexpr int kPlanChunkSlots = 1024;
inline size_t plan_chunk_ints(int S, int E) {
  return (static_cast<size_t>((S + kPlanChunkSlots - 1) / kPlanChunkSlots) + 1) * static_cast<size_t>(E);
}

struct RouteArgs {
  const uint16_t* x;       // [T][H] bf16
  const uint16_t* W;       // [E][H] bf16
  const uint16_t* b;       // [E] bf16 or null
  int T, E, H, k;
  int logits_fp32;         // 1: fp32 logits, 0: bf16 logits
  void* logits;            // [T][E]
  int32_t* idx;            // [T][k]
  float* w;                // [T][k]
  PlanBufs plan;           // plan outputs (all may be null to skip the plan)
  // Fused residual RMSNorm (norm_w != null): x is the residual stream, the
  // router reads s = x + delta (fp32), normalises it with norm_w / eps, and
  // writes normed (bf16, the experts' input) and sum_out (bf16(s), the new
  // residual); the logits are those of normed.
  const uint16_t* delta;
  const uint16_t* norm_w;
  float eps;
  uint16_t* normed;
  uint16_t* sum_out;
  KernelTimer timer;       // from the first launch's start to the last one's stop
  int logits_only;         // 1: the logits (and norm) only; top-k and plan are the caller's
};

// Bytes of route scratch (reserved: the launches need none).
size_t route_scratch_bytes(int T, int E, int k);
hipError_t launch_route(const RouteArgs& a, hipStream_t s);

// Standalone top-k softmax over given logits (bf16 or fp32).
hipError_t launch_topk(const void* logits, int logits_fp32, int T, int E, int k,
                       int32_t* idx, float* w, int32_t* tokens_per_expert, hipStream_t s);

// Standalone plan (histogram, scan, stable gather map) from expert indices.
hipError_t launch_plan(const int32_t* idx, int T, int k, int E, PlanBufs plan, hipStream_t s,
                       const KernelTimer& timer = KernelTimer{});

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
  // matrix-core decode (launch_w1_mc / launch_w2_mc)
  const int32_t* special1;    // [E] W1 scales hold code 0 or 255 (launch_special_scan), or null
  const int32_t* special2;    // [E] same for W2
  int special_any1, special_any2;  // any flag set (read back at layer init)
  int distinct_slots;         // 1: each token's k experts are distinct (this library's top-k), so an
                              // expert holds at most T slots; 0: caller-given indices, unchecked
  int num_cus;                // compute units of the device (persistent grid size)
  int mc_shape[6];            // {P, D, NC} launch shape overrides of gate_up, then down; 0 = automatic
  KernelTimer timer;          // of the next launch_w1* / launch_w2* / launch_combine_slots
  // launch_w1_mc with the routing in its prologue (decode_route_in_w1): the
  // router's logits; idx, w and plan are written by the launch.
  const void* route_logits;   // [T][E] bf16 or fp32, or null (plan from a plan launch)
  int route_fp32, route_variant;
  int32_t* route_idx;
  float* route_w;
};
hipError_t launch_experts(const ExpertArgs& a, hipStream_t s);
// The two launches of launch_experts, for callers that time them separately.
hipError_t launch_w1(const ExpertArgs& a, hipStream_t s);
hipError_t launch_w2(const ExpertArgs& a, hipStream_t s);
hipError_t launch_combine_slots(const ExpertArgs& a, hipStream_t s);
// The decode expert products on the matrix cores (moe_decode.hip): same
// outputs as launch_w1 / launch_w2 up to fp32 summation order.
hipError_t launch_w1_mc(const ExpertArgs& a, hipStream_t s);
hipError_t launch_w2_mc(const ExpertArgs& a, hipStream_t s);
// Can the matrix-core decode kernels run T tokens of this layer shape?
// (At most 1024 routed slots, so the slot -> token map fits LDS, and every
// weight and activation buffer below 4 GiB for 32-bit buffer offsets.)
bool decode_mc_supported(int T, int k, int E, int H, int I);
// Is {P, D, NC} a compiled matrix-core decode shape that fits nb blocks?
bool decode_shape_valid(int nb, int P, int D, int NC);
// Does the matrix-core gate_up launch for T tokens (shape override mc_shape,
// may be null) route in its prologue, so the router's top-k launch can be
// left out?  (T <= 8 tokens, regular scale codes checked by the caller.)
bool decode_route_in_w1(int T, int k, int E, int H, int I, const int* mc_shape);
// flags[e] = 1 if expert e's slot-order scales (tiled_geom(N, K)) hold an
// e8m0 code 0 or 255, else 0.
hipError_t launch_special_scan(const uint8_t* ws, int N, int K, int E, int32_t* flags, hipStream_t s);

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
  int32_t* queue;  // null, or grouped_queue_ints() zeroed ints (persistent grid; left zeroed)
  int num_cus;     // with a queue: compute units of the device
  KernelTimer timer;
  // Block-scaled variant (v_mfma_scale_f32_16x16x128_f8f6f4, fp4 weights x
  // fp8 activations): xq / xqs non-null select it.  xq, xqs: the rows of x
  // quantised by launch_quant_fp8x2 (read through row_index like x; x itself
  // is then read only for weights with e8m0 codes 0 or 255).  gated: outq /
  // outqs (may be null) receive the activations quantised the same way, the
  // down product's input.
  const uint8_t* xq;
  const uint32_t* xqs;
  uint8_t* outq;
  uint32_t* outqs;
  int mx_single;  // block-scaled: the hi part alone (one product per block)
};
// Ints of the persistent grouped kernel's tile queue.
constexpr int grouped_queue_ints() { return 9 * 32; }
bool grouped_supported(int N, int K, int E);
hipError_t launch_grouped_mxfp4(const GroupedArgs& a, hipStream_t s);

// Activations for the block-scaled products: every 32-element block of a bf16
// row becomes two e4m3 parts with one power-of-two scale s = 2^(e - 7), e the
// exponent of the block's largest magnitude:
//   hi = RNE(v / s),  lo = RNE((v / s - hi) * 32),  v = (hi + lo / 32) * s,
// exact for every |v| >= max * 2^-13 and within max * 2^-17 below.  Row r,
// block b: q[r][64 b .. 64 b + 31] = hi, [+32 .. +63] = lo;
// qs[r][b] = e8m0 code of s | (code of s / 32) << 8.  A block holding inf or
// NaN gets NaN parts.
hipError_t launch_quant_fp8x2(const uint16_t* x, int rows, int K, uint8_t* q, uint32_t* qs, hipStream_t s,
                              const KernelTimer& t = KernelTimer{});

// Row-major MXFP4 [N][K/2] + [N][K/32] -> tiled layout.
hipError_t launch_pack_tiled(const uint8_t* packed, const uint8_t* scales, int N, int K,
                             uint8_t* tiled_nib, uint8_t* tiled_scales, hipStream_t s);

}  // namespace gxmoe
