// moe_capi.hip -- C ABI of the gfx950 MoE block (include/gptoss_moe.h).
//
// The layer object mirrors gptoss::MoELayer (moe_layer.cu:607-1549): it
// borrows the router/bias weights, owns (or borrows) the tiled MXFP4 experts
// and owns its scratch.  A forward is two launches on the caller's stream
// (route, experts) plus an RMSNorm launch for forward(); nothing synchronises
// the host, so a forward can be captured in a hipGraph.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gptoss_moe.h"
#include "moe_kernels.h"
#include "moe_stages.h"
#include "moe_status.h"
#include "moe_checkpoint.h"

using namespace gxmoe;

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace gxmoe {

// Messages quote names and paths read from files: keep well-formed UTF-8
// (the bindings decode it as such) and write every other byte, including
// a sequence cut by the buffer's end, as '?'.
static void assign_utf8(std::string& dst, const char* s) {
  dst.clear();
  const auto* u = reinterpret_cast<const unsigned char*>(s);
  size_t left = strlen(s);
  while (left > 0) {
    const int n = utf8_seq_len(u, left);
    if (n == 0) {
      dst.push_back('?');
      ++u;
      --left;
    } else {
      dst.append(reinterpret_cast<const char*>(u), static_cast<size_t>(n));
      u += n;
      left -= static_cast<size_t>(n);
    }
  }
}

int vset_error(int code, const char* fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  assign_utf8(g_last_error, buf);
  return code;
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset_error(code, fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace gxmoe

namespace {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset_error(code, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  clear_error();
  return GPTOSS_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(GPTOSS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                     \
  do {                                          \
    hipError_t _e = (expr);                     \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// [a, a + bytes) and [b, b + bytes) share at least one byte.
bool overlaps(const void* a, const void* b, size_t bytes) {
  if (a == nullptr || b == nullptr || bytes == 0) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bytes && y < x + bytes;
}

bool valid_topk(int k) { return k == 1 || k == 2 || k == 4 || k == 8; }

// Shape limits of the tiled expert kernels: K a multiple of 32 with at most 16
// blocks per K-part, N a multiple of 64.
int check_mxfp4_shape(int N, int K) {
  if (N <= 0 || K <= 0) return fail(GPTOSS_ERR_INVALID, "MXFP4 matrix shape %dx%d must be positive", N, K);
  if (K % 32 != 0) return fail(GPTOSS_ERR_INVALID, "MXFP4 K=%d is not a multiple of the 32-element block", K);
  if (N % kTileRows != 0) return fail(GPTOSS_ERR_UNSUPPORTED, "MXFP4 N=%d is not a multiple of 64 rows", N);
  const TiledGeom g = tiled_geom(N, K);
  if (g.bpp > 16)
    return fail(GPTOSS_ERR_UNSUPPORTED, "MXFP4 K=%d splits into %d parts of %d blocks (> 16 per part)", K, g.parts, g.bpp);
  return GPTOSS_OK;
}

struct ScopedDevice {
  int prev = -1;
  bool changed = false;
  hipError_t err = hipSuccess;
  explicit ScopedDevice(int dev) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != dev) {
      err = hipSetDevice(dev);
      changed = (err == hipSuccess);
    }
  }
  ~ScopedDevice() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// The layer's per-forward scratch, carved from one workspace.  The grouped
// kernel's tile queue sits first at a fixed offset, so layers of any shape
// that share a workspace share one queue; it must read zero when a grouped
// launch starts, and every launch leaves it zero.
struct WsLayout {
  size_t queue, logits, idx, w, counts, offsets, gmap, ptok, active, n_active, tasks, act, y, pchunk, normed,
      sumres, xq, xqs, aq, aqs, total;
};

WsLayout ws_layout(const gptoss_moe_config& c) {
  const size_t T = static_cast<size_t>(c.max_tokens), S = T * c.top_k, E = c.num_experts;
  const size_t H = c.hidden_size, I = c.intermediate_size;
  WsLayout l{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~static_cast<size_t>(255);
    return at;
  };
  l.queue = take(grouped_queue_ints() * 4);
  l.logits = take(T * E * 4);
  l.idx = take(S * 4);
  l.w = take(S * 4);
  l.counts = take(E * 4);
  l.offsets = take((E + 1) * 4);
  l.gmap = take(S * 4);
  l.ptok = take(S * 4);
  l.active = take(E * 4);
  l.n_active = take(4);
  l.tasks = take(E * kTaskInts * 4);
  l.act = take(S * I * 2);
  l.y = take(S * H * 2);
  l.pchunk = take(plan_chunk_ints(static_cast<int>(S), static_cast<int>(E)) * 4);
  l.normed = take(T * H * 2);
  l.sumres = take(T * H * 2);
  // the block-scaled prefill's quantised inputs: e4m3 hi | lo per 32-element
  // block (64 bytes) and a scale dword, for the tokens and for the activations
  const bool mx = c.prefill_block_scaled && c.prefill_min_tokens > 0 && c.max_tokens >= c.prefill_min_tokens;
  l.xq = take(mx ? T * H * 2 : 0);
  l.xqs = take(mx ? T * (H / 32) * 4 : 0);
  l.aq = take(mx ? S * I * 2 : 0);
  l.aqs = take(mx ? S * (I / 32) * 4 : 0);
  l.total = off;
  return l;
}

// Device pointers of one forward's scratch, carved from a workspace laid out
// by ws_layout.
struct Scratch {
  void* logits = nullptr;
  int32_t* idx = nullptr;
  float* w = nullptr;
  int32_t* counts = nullptr;
  int32_t* offsets = nullptr;
  int32_t* gmap = nullptr;
  int32_t* ptok = nullptr;
  int32_t* active = nullptr;
  int32_t* n_active = nullptr;
  int32_t* tasks = nullptr;
  uint16_t* act = nullptr;
  uint16_t* y = nullptr;
  uint16_t* normed = nullptr;
  uint16_t* sumres = nullptr;  // residual + delta of forward_residual when the caller keeps no copy
  int32_t* gqueue = nullptr;   // tile queue of the persistent grouped kernel (zeroed; left zeroed)
  int32_t* pchunk = nullptr;   // scratch of the multi-launch plan (many tokens)
  uint16_t* gate_up = nullptr; // bf16 gate_up trace (layer-owned), or null
  uint8_t* xq = nullptr;       // block-scaled prefill: quantised tokens and activations
  uint32_t* xqs = nullptr;
  uint8_t* aq = nullptr;
  uint32_t* aqs = nullptr;
  PlanBufs plan() const { return PlanBufs{counts, offsets, gmap, ptok, active, n_active, tasks, pchunk}; }
};

Scratch carve(void* base, const WsLayout& l) {
  char* ws = static_cast<char*>(base);
  Scratch c;
  c.gqueue = reinterpret_cast<int32_t*>(ws + l.queue);
  c.logits = ws + l.logits;
  c.idx = reinterpret_cast<int32_t*>(ws + l.idx);
  c.w = reinterpret_cast<float*>(ws + l.w);
  c.counts = reinterpret_cast<int32_t*>(ws + l.counts);
  c.offsets = reinterpret_cast<int32_t*>(ws + l.offsets);
  c.gmap = reinterpret_cast<int32_t*>(ws + l.gmap);
  c.ptok = reinterpret_cast<int32_t*>(ws + l.ptok);
  c.active = reinterpret_cast<int32_t*>(ws + l.active);
  c.n_active = reinterpret_cast<int32_t*>(ws + l.n_active);
  c.tasks = reinterpret_cast<int32_t*>(ws + l.tasks);
  c.act = reinterpret_cast<uint16_t*>(ws + l.act);
  c.y = reinterpret_cast<uint16_t*>(ws + l.y);
  c.pchunk = reinterpret_cast<int32_t*>(ws + l.pchunk);
  c.normed = reinterpret_cast<uint16_t*>(ws + l.normed);
  c.sumres = reinterpret_cast<uint16_t*>(ws + l.sumres);
  c.xq = reinterpret_cast<uint8_t*>(ws + l.xq);
  c.xqs = reinterpret_cast<uint32_t*>(ws + l.xqs);
  c.aq = reinterpret_cast<uint8_t*>(ws + l.aq);
  c.aqs = reinterpret_cast<uint32_t*>(ws + l.aqs);
  return c;
}

// Forward scratch of gptoss_moe_layer_forward_prenormed_noalloc, for callers
// that cannot allocate (graph capture, serving loops).  Every GPU that runs
// the library holds its own copy of this array until the process ends; host
// code reaches a GPU's copy only through the address hipGetSymbolAddress
// returns with that GPU current (the array's name is a host-side stand-in).
constexpr int kNoAllocMaxTokens = 64;
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(8) << 20;
constexpr int kNoAllocMaxDevices = 64;

__global__ void zero_ints_kernel(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_dev[kNoAllocMaxDevices] = {};  // per device: its copy of `scratch`, once resolved

// The current device's copy of `scratch` (device is current).
int noalloc_scratch(int device, void** out) {
  if (device < 0 || device >= kNoAllocMaxDevices)
    return fail(GPTOSS_ERR_UNSUPPORTED, "device %d outside the %d the static scratch covers", device,
                kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[device] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_dev[device] = p;
  }
  *out = g_scratch_dev[device];
  return GPTOSS_OK;
}

}  // namespace

struct gptoss_moe_layer {
  bool initialized = false;
  gptoss_moe_config cfg{};
  int device = 0;
  const uint16_t* norm_w = nullptr;
  const uint16_t* router_w = nullptr;
  const uint16_t* router_b = nullptr;
  const uint16_t* b1 = nullptr;
  const uint16_t* b2 = nullptr;
  const uint8_t* w1n = nullptr;
  const uint8_t* w1s = nullptr;
  const uint8_t* w2n = nullptr;
  const uint8_t* w2s = nullptr;
  std::vector<void*> owned;
  Scratch sc;                   // this layer's forward scratch (in its workspace)
  uint16_t* gate_up = nullptr;  // bf16 gate_up trace buffer (gptoss_moe_layer_set_trace_gate_up)
  void* workspace = nullptr;    // per-forward scratch (owned, or borrowed and shared)
  int32_t* special1 = nullptr;  // [E] W1 / W2 scales hold e8m0 code 0 or 255
  int32_t* special2 = nullptr;
  int special_any1 = 0, special_any2 = 0;
  int num_cus = 0;
  int mc_shape[6] = {0, 0, 0, 0, 0, 0};  // matrix-core decode launch shape overrides (gate_up, down)
  bool trace_gu = false;
  // per-launch timing (gptoss_moe_layer_set_profiling): 4 events per recorded forward
  std::vector<hipEvent_t> prof_events;
  std::vector<double> prof_host_us;  // host steady-clock time at which each recorded forward was enqueued
  std::vector<int> prof_tokens;      // and its token count
  int prof_capacity = 0;
  int prof_count = 0;

  void release() {
    for (void* p : owned) (void)hipFree(p);
    owned.clear();
    for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
    prof_events.clear();
    prof_capacity = prof_count = 0;
  }
  int alloc(void** p, size_t bytes, const char* what) {
    hipError_t e = hipMalloc(p, bytes < 256 ? 256 : bytes);
    if (e != hipSuccess) return fail(GPTOSS_ERR_OOM, "hipMalloc(%zu) for %s: %s", bytes, what, hipGetErrorString(e));
    owned.push_back(*p);
    return GPTOSS_OK;
  }
};

extern "C" {

const char* gptoss_last_error(void) { return g_last_error.c_str(); }
int gptoss_abi_version(void) { return GPTOSS_MOE_ABI_VERSION; }

int gptoss_moe_config_default(gptoss_moe_config* cfg, int num_experts, int max_tokens) {
  if (cfg == nullptr) return fail(GPTOSS_ERR_INVALID, "cfg is NULL");
  cfg->hidden_size = 2880;        // config.h:12
  cfg->num_experts = num_experts; // config.h:20 (128) or 32 for the 20B shape
  cfg->top_k = 4;                 // config.h:21
  cfg->intermediate_size = 2880;  // config.h:22
  cfg->swiglu_alpha = 1.702f;     // config.h:43
  cfg->swiglu_limit = 7.0f;       // config.h:42
  cfg->rms_norm_eps = 1e-5f;      // config.h:39
  cfg->logits_fp32 = 0;
  cfg->max_tokens = max_tokens;
  cfg->prefill_min_tokens = 128;
  cfg->decode_exact = 0;
  cfg->prefill_block_scaled = 0;
  return ok();
}

int gptoss_mxfp4_tiled_size(int N, int K, size_t* nibble_bytes, size_t* scale_bytes) {
  int rc = check_mxfp4_shape(N, K);
  if (rc != GPTOSS_OK) return rc;
  const TiledGeom g = tiled_geom(N, K);
  if (nibble_bytes) *nibble_bytes = g.nib_bytes;
  if (scale_bytes) *scale_bytes = g.scale_bytes;
  return ok();
}

int gptoss_mxfp4_pack_tiled(const uint8_t* packed, const uint8_t* scales, int N, int K, uint8_t* tiled_nibbles,
                            uint8_t* tiled_scales, void* stream) {
  int rc = check_mxfp4_shape(N, K);
  if (rc != GPTOSS_OK) return rc;
  if (!packed || !scales || !tiled_nibbles || !tiled_scales) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(packed) || !aligned16(tiled_nibbles))
    return fail(GPTOSS_ERR_INVALID, "MXFP4 nibble buffers must be 16-byte aligned");
  HIP_TRY(launch_pack_tiled(packed, scales, N, K, tiled_nibbles, tiled_scales, static_cast<hipStream_t>(stream)),
          "pack_tiled launch");
  return ok();
}

gptoss_moe_layer* gptoss_moe_layer_create(void) {
  g_last_error.clear();
  return new (std::nothrow) gptoss_moe_layer();
}

void gptoss_moe_layer_destroy(gptoss_moe_layer* layer) {
  if (layer == nullptr) return;
  {
    ScopedDevice sd(layer->device);
    layer->release();
  }
  delete layer;
}

static int layer_init(gptoss_moe_layer* L, const gptoss_moe_config* cfg, int device_id,
                      const gptoss_moe_weights* wt, void* workspace, size_t workspace_bytes) {
  if (L == nullptr || cfg == nullptr || wt == nullptr) return fail(GPTOSS_ERR_INVALID, "null argument");
  if (L->initialized) return fail(GPTOSS_ERR_STATE, "layer already initialised");
  const int H = cfg->hidden_size, E = cfg->num_experts, k = cfg->top_k, I = cfg->intermediate_size;
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  if (!valid_topk(k) || k > E) return fail(GPTOSS_ERR_INVALID, "top_k=%d must be 1, 2, 4 or 8 and <= num_experts", k);
  if (cfg->max_tokens < 1) return fail(GPTOSS_ERR_INVALID, "max_tokens=%d must be >= 1", cfg->max_tokens);
  if (cfg->prefill_min_tokens < 0)
    return fail(GPTOSS_ERR_INVALID, "prefill_min_tokens=%d must be >= 0", cfg->prefill_min_tokens);
  if (cfg->decode_exact != 0 && cfg->decode_exact != 1)
    return fail(GPTOSS_ERR_INVALID, "decode_exact=%d must be 0 or 1", cfg->decode_exact);
  if (cfg->prefill_block_scaled < 0 || cfg->prefill_block_scaled > 2)
    return fail(GPTOSS_ERR_INVALID, "prefill_block_scaled=%d must be 0, 1 or 2", cfg->prefill_block_scaled);
  if (H % kTileRows != 0) return fail(GPTOSS_ERR_UNSUPPORTED, "hidden_size=%d must be a multiple of 64", H);
  int rc = check_mxfp4_shape(2 * I, H);
  if (rc != GPTOSS_OK) return rc;
  rc = check_mxfp4_shape(H, I);
  if (rc != GPTOSS_OK) return rc;
  if (!wt->router_weight) return fail(GPTOSS_ERR_INVALID, "router_weight is NULL");
  if (!aligned16(wt->router_weight)) return fail(GPTOSS_ERR_INVALID, "router_weight must be 16-byte aligned");
  const bool tiled = wt->mlp1_tiled_nibbles != nullptr;
  if (tiled) {
    if (!wt->mlp1_tiled_scales || !wt->mlp2_tiled_nibbles || !wt->mlp2_tiled_scales)
      return fail(GPTOSS_ERR_INVALID, "tiled weights: all four tiled buffers are required");
  } else if (!wt->mlp1_packed || !wt->mlp1_scales || !wt->mlp2_packed || !wt->mlp2_scales) {
    return fail(GPTOSS_ERR_INVALID, "expert weights missing (neither reference-layout tables nor tiled buffers)");
  }

  const WsLayout lay = ws_layout(*cfg);
  if (workspace != nullptr) {
    if (workspace_bytes < lay.total)
      return fail(GPTOSS_ERR_INVALID, "workspace of %zu bytes, this config needs %zu", workspace_bytes, lay.total);
    if (reinterpret_cast<uintptr_t>(workspace) & 255u)
      return fail(GPTOSS_ERR_INVALID, "workspace must be 256-byte aligned");
  }

  ScopedDevice sd(device_id);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  L->cfg = *cfg;
  L->device = device_id;
  L->norm_w = wt->moe_norm_weight;
  L->router_w = wt->router_weight;
  L->router_b = wt->router_bias;
  L->b1 = wt->gate_up_bias;
  L->b2 = wt->down_bias;

  const TiledGeom g1 = tiled_geom(2 * I, H);
  const TiledGeom g2 = tiled_geom(H, I);
  if (tiled) {
    L->w1n = wt->mlp1_tiled_nibbles;
    L->w1s = wt->mlp1_tiled_scales;
    L->w2n = wt->mlp2_tiled_nibbles;
    L->w2s = wt->mlp2_tiled_scales;
  } else {
    void *a, *b, *c, *d;
    if ((rc = L->alloc(&a, g1.nib_bytes * E, "W1 tiled nibbles")) ||
        (rc = L->alloc(&b, g1.scale_bytes * E, "W1 tiled scales")) ||
        (rc = L->alloc(&c, g2.nib_bytes * E, "W2 tiled nibbles")) ||
        (rc = L->alloc(&d, g2.scale_bytes * E, "W2 tiled scales"))) {
      L->release();
      return rc;
    }
    L->w1n = static_cast<uint8_t*>(a);
    L->w1s = static_cast<uint8_t*>(b);
    L->w2n = static_cast<uint8_t*>(c);
    L->w2s = static_cast<uint8_t*>(d);
    for (int e = 0; e < E; ++e) {
      if (!wt->mlp1_packed[e] || !wt->mlp1_scales[e] || !wt->mlp2_packed[e] || !wt->mlp2_scales[e] ||
          !aligned16(wt->mlp1_packed[e]) || !aligned16(wt->mlp2_packed[e])) {
        L->release();
        return fail(GPTOSS_ERR_INVALID, "expert %d: null or misaligned MXFP4 pointer", e);
      }
      hipError_t err = launch_pack_tiled(wt->mlp1_packed[e], wt->mlp1_scales[e], 2 * I, H,
                                         static_cast<uint8_t*>(a) + g1.nib_bytes * e,
                                         static_cast<uint8_t*>(b) + g1.scale_bytes * e, nullptr);
      if (err == hipSuccess)
        err = launch_pack_tiled(wt->mlp2_packed[e], wt->mlp2_scales[e], H, I,
                                static_cast<uint8_t*>(c) + g2.nib_bytes * e,
                                static_cast<uint8_t*>(d) + g2.scale_bytes * e, nullptr);
      if (err != hipSuccess) {
        L->release();
        return hip_fail(err, "pack_tiled");
      }
    }
  }

  if (workspace != nullptr) {
    L->workspace = workspace;
  } else if ((rc = L->alloc(&L->workspace, lay.total, "forward scratch")) != GPTOSS_OK) {
    L->release();
    return rc;
  }
  L->sc = carve(L->workspace, lay);
  void* p;
  if ((rc = L->alloc(&p, E * 4, "special1")) != GPTOSS_OK) return (L->release(), rc);
  L->special1 = static_cast<int32_t*>(p);
  if ((rc = L->alloc(&p, E * 4, "special2")) != GPTOSS_OK) return (L->release(), rc);
  L->special2 = static_cast<int32_t*>(p);
  // The work queue at the workspace's start reads zero between forwards.  A
  // shared workspace may have another layer's forward in flight on any stream
  // of the device: wait for all of it before zeroing, so the zeroing never
  // lands inside a running grouped launch.
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemset(L->sc.gqueue, 0, grouped_queue_ints() * 4);
  if (err == hipSuccess) err = launch_special_scan(L->w1s, 2 * I, H, E, L->special1, nullptr);
  if (err == hipSuccess) err = launch_special_scan(L->w2s, H, I, E, L->special2, nullptr);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&L->num_cus, hipDeviceAttributeMultiprocessorCount, device_id);
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    std::vector<int32_t> f1(E), f2(E);
    err = hipMemcpy(f1.data(), L->special1, sizeof(int32_t) * E, hipMemcpyDeviceToHost);
    if (err == hipSuccess) err = hipMemcpy(f2.data(), L->special2, sizeof(int32_t) * E, hipMemcpyDeviceToHost);
    for (int e = 0; e < E; ++e) {
      L->special_any1 |= f1[e] != 0;
      L->special_any2 |= f2[e] != 0;
    }
  }
  // Tuning override of the matrix-core decode launch shapes: "P,D,NC" for
  // both expert products or "P,D,NC/P,D,NC" for gate_up, then down (waves
  // per work-group, ring depth, 16-token chunks); a shape that is not
  // compiled for its matrix is ignored.
  if (const char* ov = getenv("GPTOSS_MOE_DECODE_SHAPE")) {
    int v[6] = {0, 0, 0, 0, 0, 0};
    const int n = sscanf(ov, "%d,%d,%d/%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4], &v[5]);
    if (n == 3)
      for (int i = 0; i < 3; ++i) v[3 + i] = v[i];
    if (n == 3 || n == 6) {
      if (decode_shape_valid(H / 32, v[0], v[1], v[2]))
        for (int i = 0; i < 3; ++i) L->mc_shape[i] = v[i];
      if (decode_shape_valid(I / 32, v[3], v[4], v[5]))
        for (int i = 3; i < 6; ++i) L->mc_shape[i] = v[i];
    }
  }
  if (err != hipSuccess) {
    L->release();
    return hip_fail(err, "layer init");
  }
  L->initialized = true;
  return ok();
}

int gptoss_moe_layer_init(gptoss_moe_layer* L, const gptoss_moe_config* cfg, int device_id,
                          const gptoss_moe_weights* wt) {
  return layer_init(L, cfg, device_id, wt, nullptr, 0);
}

size_t gptoss_moe_layer_workspace_bytes(const gptoss_moe_config* cfg) {
  if (cfg == nullptr || cfg->max_tokens < 1 || cfg->num_experts < 1 || cfg->top_k < 1 || cfg->hidden_size < 1 ||
      cfg->intermediate_size < 1)
    return 0;
  return ws_layout(*cfg).total;
}

int gptoss_moe_layer_init_with_workspace(gptoss_moe_layer* L, const gptoss_moe_config* cfg, int device_id,
                                         const gptoss_moe_weights* wt, void* workspace, size_t workspace_bytes) {
  if (workspace == nullptr) return fail(GPTOSS_ERR_INVALID, "workspace is NULL");
  return layer_init(L, cfg, device_id, wt, workspace, workspace_bytes);
}

// One allocation with every weight of the layer (the checkpoint reader
// fills it and tiles the experts), then the borrowed-tiled init over it; the
// layer takes the allocation over.
static int gptoss_moe_layer_init_from_checkpoint_impl(gptoss_moe_layer* L, const gptoss_moe_config* cfg, int device_id,
                                          const gptoss_checkpoint* ckpt, int layer_index) {
  if (L == nullptr || cfg == nullptr || ckpt == nullptr) return fail(GPTOSS_ERR_INVALID, "null argument");
  if (L->initialized) return fail(GPTOSS_ERR_STATE, "layer already initialised");
  const int H = cfg->hidden_size, E = cfg->num_experts, I = cfg->intermediate_size;
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  int rc = check_mxfp4_shape(2 * I, H);
  if (rc != GPTOSS_OK) return rc;
  if ((rc = check_mxfp4_shape(H, I)) != GPTOSS_OK) return rc;
  // names, shapes and dtypes first, on the host
  LayerSource* src = nullptr;
  if ((rc = ckpt_resolve_layer(ckpt, *cfg, layer_index, &src)) != GPTOSS_OK) return rc;
  ScopedDevice sd(device_id);
  if (sd.err != hipSuccess) {
    ckpt_free_source(src);
    return hip_fail(sd.err, "hipSetDevice");
  }
  void* blob = nullptr;
  gptoss_moe_weights wt{};
  rc = ckpt_upload_layer(src, &blob, &wt);
  ckpt_free_source(src);
  if (rc != GPTOSS_OK) return rc;
  if ((rc = gptoss_moe_layer_init(L, cfg, device_id, &wt)) != GPTOSS_OK) {
    (void)hipFree(blob);
    return rc;
  }
  L->owned.push_back(blob);
  return ok();
}

int gptoss_moe_layer_init_from_checkpoint(gptoss_moe_layer* L, const gptoss_moe_config* cfg, int device_id,
                                          const gptoss_checkpoint* ckpt, int layer_index) {
  return guarded([&] { return gptoss_moe_layer_init_from_checkpoint_impl(L, cfg, device_id, ckpt, layer_index); });
}

// Timing of one profiled forward (gptoss_moe_layer_set_profiling): launch i
// (0 route or plan, 1 gate_up, 2 down, 3 combine) between events 2i and
// 2i + 1, stamped by the dispatch itself (hipExtLaunchKernelGGL).
struct ProfForward {
  hipEvent_t* ev = nullptr;
  KernelTimer timer(int i) const { return ev ? KernelTimer{ev[2 * i], ev[2 * i + 1]} : KernelTimer{}; }
};
constexpr int kProfEvents = 8;

// The layer's own scratch for a forward, with its gate_up trace buffer when
// tracing is on.
static Scratch layer_scratch(const gptoss_moe_layer* L) {
  Scratch S = L->sc;
  S.gate_up = L->trace_gu ? L->gate_up : nullptr;
  return S;
}

// Expert products and combine after the plan (decode: weight-streaming
// kernels, on the matrix cores or exact; prefill: grouped matrix-core GEMMs).
// w: routing weights [T][k].
static int layer_experts(gptoss_moe_layer* L, const Scratch& S, const uint16_t* normed, const uint16_t* residual,
                         const float* w, uint16_t* out, int T, hipStream_t s, const ProfForward& pf,
                         bool own_routing, bool route_in_w1 = false) {
  const gptoss_moe_config& c = L->cfg;
  ExpertArgs ea{};
  ea.x = normed;
  ea.w1n = L->w1n;
  ea.w1s = L->w1s;
  ea.b1 = L->b1;
  ea.w2n = L->w2n;
  ea.w2s = L->w2s;
  ea.b2 = L->b2;
  ea.T = T;
  ea.E = c.num_experts;
  ea.H = c.hidden_size;
  ea.I = c.intermediate_size;
  ea.k = c.top_k;
  ea.alpha = c.swiglu_alpha;
  ea.limit = c.swiglu_limit;
  ea.plan = PlanBufs{S.counts, S.offsets, S.gmap, S.ptok, S.active, S.n_active, S.tasks};
  ea.w = w;
  ea.act = S.act;
  ea.gate_up = S.gate_up;
  ea.y = S.y;
  ea.residual = residual;
  ea.out = out;
  ea.max_active = T * c.top_k < c.num_experts ? T * c.top_k : c.num_experts;
  ea.special1 = L->special1;
  ea.special2 = L->special2;
  ea.special_any1 = L->special_any1;
  ea.special_any2 = L->special_any2;
  ea.distinct_slots = own_routing ? 1 : 0;
  ea.num_cus = L->num_cus;
  for (int i = 0; i < 6; ++i) ea.mc_shape[i] = L->mc_shape[i];
  if (route_in_w1) {  // the gate_up launch selects the experts from the router's logits
    ea.route_logits = S.logits;
    ea.route_fp32 = c.logits_fp32;
    ea.route_variant = 1;  // T <= 8 (topk_softmax.cu:399)
    ea.route_idx = S.idx;
    ea.route_w = S.w;
  }
  if (c.prefill_min_tokens > 0 && T >= c.prefill_min_tokens) {
    GroupedArgs g{};
    g.x = normed;
    g.row_index = S.ptok;
    g.offsets = S.offsets;
    g.E = c.num_experts;
    g.rows = T * c.top_k;
    g.wn = L->w1n;
    g.ws = L->w1s;
    g.N = 2 * c.intermediate_size;
    g.K = c.hidden_size;
    g.bias = L->b1;
    g.out = S.act;
    g.gate_up = ea.gate_up;
    g.gated = 1;
    g.alpha = c.swiglu_alpha;
    g.limit = c.swiglu_limit;
    g.queue = S.gqueue;
    g.num_cus = L->num_cus;
    g.timer = pf.timer(1);
    if (c.prefill_block_scaled) {  // the tokens as e4m3 parts, then block-scaled products
      const KernelTimer t1 = pf.timer(1);
      HIP_TRY(launch_quant_fp8x2(normed, T, c.hidden_size, S.xq, S.xqs, s, KernelTimer{t1.start, nullptr}),
              "quantise launch");
      g.timer = KernelTimer{nullptr, t1.stop};
      g.xq = S.xq;
      g.xqs = S.xqs;
      g.outq = S.aq;
      g.outqs = S.aqs;
      g.mx_single = c.prefill_block_scaled == 2;
    }
    HIP_TRY(launch_grouped_mxfp4(g, s), "grouped gate_up launch");
    g.x = S.act;
    g.row_index = nullptr;
    if (c.prefill_block_scaled) {
      g.xq = S.aq;
      g.xqs = S.aqs;
      g.outq = nullptr;
      g.outqs = nullptr;
    }
    g.wn = L->w2n;
    g.ws = L->w2s;
    g.N = c.hidden_size;
    g.K = c.intermediate_size;
    g.bias = L->b2;
    g.out = S.y;
    g.gate_up = nullptr;
    g.gated = 0;
    g.timer = pf.timer(2);
    HIP_TRY(launch_grouped_mxfp4(g, s), "grouped down launch");
  } else {
    const bool exact =
        c.decode_exact || !decode_mc_supported(T, c.top_k, c.num_experts, c.hidden_size, c.intermediate_size);
    ea.timer = pf.timer(1);
    HIP_TRY(exact ? launch_w1(ea, s) : launch_w1_mc(ea, s), "w1 launch");
    ea.timer = pf.timer(2);
    HIP_TRY(exact ? launch_w2(ea, s) : launch_w2_mc(ea, s), "w2 launch");
  }
  ea.timer = pf.timer(3);
  HIP_TRY(launch_combine_slots(ea, s), "combine launch");
  return ok();
}

// Forwards being captured into a graph are not timed (events inside a graph
// cannot be timed on this runtime) and leave the profiling slots unused.
static ProfForward next_prof(gptoss_moe_layer* L, hipStream_t s, int T) {
  ProfForward pf;
  if (L->prof_count < L->prof_capacity) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
    if (!capturing) {
      const int i = L->prof_count++;
      pf.ev = &L->prof_events[kProfEvents * static_cast<size_t>(i)];
      L->prof_host_us[i] = std::chrono::duration<double, std::micro>(
                               std::chrono::steady_clock::now().time_since_epoch()).count();
      L->prof_tokens[i] = T;
    }
  }
  return pf;
}

// The router (optionally with the residual RMSNorm in front: delta != null)
// then the experts and the combine.
static int layer_forward_core(gptoss_moe_layer* L, const Scratch& S, const uint16_t* normed, const uint16_t* residual,
                              uint16_t* out, int T, hipStream_t s, const uint16_t* delta = nullptr,
                              uint16_t* sum_out = nullptr) {
  const gptoss_moe_config& c = L->cfg;
  RouteArgs ra{};
  ra.x = normed;
  if (delta != nullptr) {  // normed is the residual stream here
    ra.delta = delta;
    ra.norm_w = L->norm_w;
    ra.eps = c.rms_norm_eps;
    ra.normed = S.normed;
    ra.sum_out = sum_out;
  }
  ra.W = L->router_w;
  ra.b = L->router_b;
  ra.T = T;
  ra.E = c.num_experts;
  ra.H = c.hidden_size;
  ra.k = c.top_k;
  ra.logits_fp32 = c.logits_fp32;
  ra.logits = S.logits;
  ra.idx = S.idx;
  ra.w = S.w;
  ra.plan = S.plan();
  // Up to 8 tokens on the matrix-core decode path, the gate_up launch makes
  // the top-k and plan itself: the router launch computes the logits only.
  const bool prefill = c.prefill_min_tokens > 0 && T >= c.prefill_min_tokens;
  const bool route_in_w1 = !prefill && !c.decode_exact && !L->special_any1 &&
                           decode_mc_supported(T, c.top_k, c.num_experts, c.hidden_size, c.intermediate_size) &&
                           decode_route_in_w1(T, c.top_k, c.num_experts, c.hidden_size, c.intermediate_size,
                                              L->mc_shape);
  ra.logits_only = route_in_w1 ? 1 : 0;
  const ProfForward pf = next_prof(L, s, T);
  ra.timer = pf.timer(0);
  HIP_TRY(launch_route(ra, s), "route launch");
  if (delta != nullptr) return layer_experts(L, S, S.normed, sum_out, S.w, out, T, s, pf, true, route_in_w1);
  return layer_experts(L, S, normed, residual, S.w, out, T, s, pf, true, route_in_w1);
}

static int check_forward_args(gptoss_moe_layer* L, const void* in, const void* out, int T) {
  if (L == nullptr) return fail(GPTOSS_ERR_INVALID, "layer is NULL");
  if (!L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (T < 0 || T > L->cfg.max_tokens)
    return fail(GPTOSS_ERR_INVALID, "num_tokens=%d outside [0, max_tokens=%d]", T, L->cfg.max_tokens);
  if (T > 0 && (in == nullptr || out == nullptr)) return fail(GPTOSS_ERR_INVALID, "null input/output");
  if (T > 0 && !aligned16(in)) return fail(GPTOSS_ERR_INVALID, "input must be 16-byte aligned");
  return GPTOSS_OK;
}

int gptoss_moe_layer_forward_prenormed(gptoss_moe_layer* L, const uint16_t* normed, const uint16_t* residual,
                                       uint16_t* out, int T, void* stream) {
  int rc = check_forward_args(L, normed, out, T);
  if (rc != GPTOSS_OK) return rc;
  if (T == 0) return ok();
  ScopedDevice sd(L->device);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  return layer_forward_core(L, layer_scratch(L), normed, residual, out, T, static_cast<hipStream_t>(stream));
}

int gptoss_moe_layer_forward(gptoss_moe_layer* L, const uint16_t* input, uint16_t* out, int T, void* stream) {
  int rc = check_forward_args(L, input, out, T);
  if (rc != GPTOSS_OK) return rc;
  if (L->norm_w == nullptr) return fail(GPTOSS_ERR_STATE, "forward() needs moe_norm_weight (init passed NULL)");
  if (T == 0) return ok();
  ScopedDevice sd(L->device);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Scratch S = layer_scratch(L);
  HIP_TRY(launch_rmsnorm(input, L->norm_w, S.normed, T, L->cfg.hidden_size, L->cfg.rms_norm_eps, s),
          "rmsnorm launch");
  return layer_forward_core(L, S, S.normed, input, out, T, s);
}

int gptoss_moe_layer_forward_residual(gptoss_moe_layer* L, const uint16_t* residual, const uint16_t* delta,
                                      uint16_t* residual_out, uint16_t* out, int T, void* stream) {
  int rc = check_forward_args(L, residual, out, T);
  if (rc != GPTOSS_OK) return rc;
  if (L->norm_w == nullptr) return fail(GPTOSS_ERR_STATE, "forward_residual() needs moe_norm_weight (init passed NULL)");
  if (T == 0) return ok();
  if (delta == nullptr) return fail(GPTOSS_ERR_INVALID, "null delta");
  if (!aligned16(delta) || (residual_out && !aligned16(residual_out)))
    return fail(GPTOSS_ERR_INVALID, "delta and residual_out must be 16-byte aligned");
  // Every work-group of the router launch reads residual and delta while one
  // of them writes residual_out, and the combine reads residual_out while it
  // writes out: residual_out must not share memory with residual or delta,
  // and out is either residual_out itself or apart from it.
  const size_t rows = static_cast<size_t>(T) * L->cfg.hidden_size * sizeof(uint16_t);
  if (overlaps(residual_out, residual, rows) || overlaps(residual_out, delta, rows))
    return fail(GPTOSS_ERR_INVALID, "residual_out overlaps residual or delta (the sum needs its own buffer)");
  if (out != residual_out && overlaps(out, residual_out, rows))
    return fail(GPTOSS_ERR_INVALID, "out partially overlaps residual_out");
  ScopedDevice sd(L->device);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  const Scratch S = layer_scratch(L);
  return layer_forward_core(L, S, residual, nullptr, out, T, static_cast<hipStream_t>(stream), delta,
                            residual_out ? residual_out : S.sumres);
}

int gptoss_moe_layer_forward_routed(gptoss_moe_layer* L, const uint16_t* normed, const uint16_t* residual,
                                    const int32_t* idx, const float* w, uint16_t* out, int T, void* stream) {
  int rc = check_forward_args(L, normed, out, T);
  if (rc != GPTOSS_OK) return rc;
  if (T == 0) return ok();
  if (idx == nullptr || w == nullptr) return fail(GPTOSS_ERR_INVALID, "null expert indices / weights");
  ScopedDevice sd(L->device);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const gptoss_moe_config& c = L->cfg;
  const ProfForward pf = next_prof(L, s, T);
  const Scratch S = layer_scratch(L);
  HIP_TRY(launch_plan(idx, T, c.top_k, c.num_experts, S.plan(), s, pf.timer(0)), "plan launch");
  return layer_experts(L, S, normed, residual, w, out, T, s, pf, false);
}

int gptoss_moe_layer_forward_prenormed_noalloc(gptoss_moe_layer* L, const uint16_t* normed, const uint16_t* residual,
                                               uint16_t* out, int T, void* stream) {
  if (L == nullptr) return fail(GPTOSS_ERR_INVALID, "layer is NULL");
  if (!L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (T < 0 || T > kNoAllocMaxTokens)
    return fail(GPTOSS_ERR_INVALID, "num_tokens=%d outside [0, %d] (the static forward scratch)", T,
                kNoAllocMaxTokens);
  if (T > 0 && (normed == nullptr || out == nullptr)) return fail(GPTOSS_ERR_INVALID, "null input/output");
  if (T > 0 && !aligned16(normed)) return fail(GPTOSS_ERR_INVALID, "input must be 16-byte aligned");
  if (T == 0) return ok();
  gptoss_moe_config c = L->cfg;
  c.max_tokens = T;
  const WsLayout lay = ws_layout(c);
  if (lay.total > kNoAllocScratchBytes)
    return fail(GPTOSS_ERR_INVALID, "this layer needs %zu bytes of forward scratch at %d tokens, the static array "
                "holds %zu", lay.total, T, kNoAllocScratchBytes);
  ScopedDevice sd(L->device);
  if (sd.err != hipSuccess) return hip_fail(sd.err, "hipSetDevice");
  void* base = nullptr;
  const int rc = noalloc_scratch(L->device, &base);
  if (rc != GPTOSS_OK) return rc;
  const Scratch S = carve(base, lay);  // no gate_up trace: the layer's trace buffer is sized for its own tokens
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (c.prefill_min_tokens > 0 && T >= c.prefill_min_tokens) {
    // the grouped kernels' tile queue must read zero: a fill kernel, since a
    // caller may be capturing this stream
    hipLaunchKernelGGL(zero_ints_kernel, dim3(1), dim3(256), 0, s, S.gqueue, grouped_queue_ints());
    HIP_TRY(hipGetLastError(), "zero_ints launch");
  }
  return layer_forward_core(L, S, normed, residual, out, T, s);
}

const uint16_t* gptoss_moe_layer_get_ffn_norm_weight(const gptoss_moe_layer* L) {
  return L ? L->norm_w : nullptr;
}

int gptoss_moe_layer_get_config(const gptoss_moe_layer* L, gptoss_moe_config* cfg, int* device_id) {
  if (L == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (cfg) *cfg = L->cfg;
  if (device_id) *device_id = L->device;
  return ok();
}

int gptoss_moe_layer_set_trace_gate_up(gptoss_moe_layer* L, int enable) {
  if (L == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (enable && L->gate_up == nullptr) {
    ScopedDevice sd(L->device);
    void* p;
    const size_t bytes = static_cast<size_t>(L->cfg.max_tokens) * L->cfg.top_k * 2 * L->cfg.intermediate_size * 2;
    int rc = L->alloc(&p, bytes, "gate_up trace");
    if (rc != GPTOSS_OK) return rc;
    L->gate_up = static_cast<uint16_t*>(p);
  }
  L->trace_gu = enable != 0;
  return ok();
}

int gptoss_moe_layer_trace(const gptoss_moe_layer* L, gptoss_moe_trace* t) {
  if (L == nullptr || t == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  const Scratch& S = L->sc;
  t->logits = S.logits;
  t->expert_indices = S.idx;
  t->expert_weights = S.w;
  t->expert_counts = S.counts;
  t->expert_offsets = S.offsets;
  t->gather_map = S.gmap;
  t->perm_token = S.ptok;
  t->active_experts = S.active;
  t->n_active = S.n_active;
  t->gate_up = L->trace_gu ? L->gate_up : nullptr;
  t->act = S.act;
  t->expert_out = S.y;
  return ok();
}

int gptoss_moe_layer_set_profiling(gptoss_moe_layer* L, int max_forwards) {
  if (L == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (max_forwards < 0) return fail(GPTOSS_ERR_INVALID, "max_forwards=%d < 0", max_forwards);
  ScopedDevice sd(L->device);
  for (hipEvent_t e : L->prof_events) (void)hipEventDestroy(e);
  L->prof_events.assign(kProfEvents * static_cast<size_t>(max_forwards), nullptr);
  L->prof_host_us.assign(static_cast<size_t>(max_forwards), 0.0);
  L->prof_tokens.assign(static_cast<size_t>(max_forwards), 0);
  L->prof_capacity = 0;
  L->prof_count = 0;
  for (auto& e : L->prof_events) HIP_TRY(hipEventCreate(&e), "hipEventCreate");
  L->prof_capacity = max_forwards;
  L->prof_count = 0;
  return ok();
}

int gptoss_moe_layer_profile_read(gptoss_moe_layer* L, float* route_ms, float* w1_ms, float* w2_ms, float* combine_ms,
                                  int* n_forwards) {
  if (L == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  ScopedDevice sd(L->device);
  double sum[4] = {0, 0, 0, 0};
  for (int i = 0; i < L->prof_count; ++i) {
    hipEvent_t* ev = &L->prof_events[kProfEvents * static_cast<size_t>(i)];
    HIP_TRY(hipEventSynchronize(ev[kProfEvents - 1]), "hipEventSynchronize");
    for (int j = 0; j < 4; ++j) {
      float t;
      HIP_TRY(hipEventElapsedTime(&t, ev[2 * j], ev[2 * j + 1]), "hipEventElapsedTime");
      sum[j] += t;
    }
  }
  if (route_ms) *route_ms = static_cast<float>(sum[0]);
  if (w1_ms) *w1_ms = static_cast<float>(sum[1]);
  if (w2_ms) *w2_ms = static_cast<float>(sum[2]);
  if (combine_ms) *combine_ms = static_cast<float>(sum[3]);
  if (n_forwards) *n_forwards = L->prof_count;
  return ok();
}

int gptoss_moe_layer_profile_records(gptoss_moe_layer* L, gptoss_moe_prof_record* records, int capacity,
                                     int* n_records) {
  if (L == nullptr || !L->initialized) return fail(GPTOSS_ERR_STATE, "layer not initialised");
  if (capacity < 0 || (capacity > 0 && records == nullptr))
    return fail(GPTOSS_ERR_INVALID, "records: capacity=%d with %s buffer", capacity, records ? "a" : "no");
  ScopedDevice sd(L->device);
  const int n = L->prof_count < capacity ? L->prof_count : capacity;
  const gptoss_moe_config& c = L->cfg;
  for (int i = 0; i < n; ++i) {
    hipEvent_t* ev = &L->prof_events[kProfEvents * static_cast<size_t>(i)];
    HIP_TRY(hipEventSynchronize(ev[kProfEvents - 1]), "hipEventSynchronize");
    gptoss_moe_prof_record& r = records[i];
    r.host_us = L->prof_host_us[i];
    r.num_tokens = L->prof_tokens[i];
    r.prefill = c.prefill_min_tokens > 0 && r.num_tokens >= c.prefill_min_tokens ? 1 : 0;
    for (int j = 0; j < 4; ++j) {
      HIP_TRY(hipEventElapsedTime(&r.start_ms[j], ev[0], ev[2 * j]), "hipEventElapsedTime");
      HIP_TRY(hipEventElapsedTime(&r.dur_ms[j], ev[2 * j], ev[2 * j + 1]), "hipEventElapsedTime");
    }
  }
  if (n_records) *n_records = L->prof_count;
  return ok();
}

size_t gptoss_moe_route_scratch_bytes(int T, int E, int k) {
  if (T < 0 || E < 1 || k < 1) return 0;
  return route_scratch_bytes(T, E, k);
}

int gptoss_moe_route(const uint16_t* x, const uint16_t* router_w, const uint16_t* router_b, int T, int E, int H,
                     int k, int logits_fp32, void* logits, int32_t* idx, float* w, void* scratch, void* stream) {
  if (T < 0) return fail(GPTOSS_ERR_INVALID, "num_tokens=%d < 0", T);
  if (T == 0) return ok();
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  if (!valid_topk(k) || k > E) return fail(GPTOSS_ERR_INVALID, "top_k=%d must be 1, 2, 4 or 8 and <= E", k);
  if (H <= 0 || H % 8 != 0) return fail(GPTOSS_ERR_INVALID, "hidden=%d must be a positive multiple of 8", H);
  if (!x || !router_w || !logits || !idx || !w || !scratch) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(x) || !aligned16(router_w)) return fail(GPTOSS_ERR_INVALID, "x and router_w must be 16-byte aligned");
  RouteArgs ra{};
  ra.x = x;
  ra.W = router_w;
  ra.b = router_b;
  ra.T = T;
  ra.E = E;
  ra.H = H;
  ra.k = k;
  ra.logits_fp32 = logits_fp32 ? 1 : 0;
  ra.logits = logits;
  ra.idx = idx;
  ra.w = w;
  ra.plan = PlanBufs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  HIP_TRY(launch_route(ra, static_cast<hipStream_t>(stream)), "route launch");
  return ok();
}

int gptoss_topk_softmax_forward(const void* logits, int logits_fp32, int32_t* idx, float* w, int32_t* tpe, int T,
                                int E, int k, void* stream) {
  if (T < 0) return fail(GPTOSS_ERR_INVALID, "num_tokens=%d < 0", T);
  if (T == 0) return ok();
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  if (!valid_topk(k) || k > E) return fail(GPTOSS_ERR_INVALID, "top_k=%d must be 1, 2, 4 or 8 and <= E", k);
  if (!logits || !idx || !w) return fail(GPTOSS_ERR_INVALID, "null pointer");
  HIP_TRY(launch_topk(logits, logits_fp32, T, E, k, idx, w, tpe, static_cast<hipStream_t>(stream)), "topk launch");
  return ok();
}

int gptoss_moe_permute_plan(const int32_t* idx, int T, int k, int E, int32_t* counts, int32_t* offsets,
                            int32_t* gather_map, int32_t* perm_token, int32_t* active, int32_t* n_active,
                            void* stream) {
  if (T < 0) return fail(GPTOSS_ERR_INVALID, "num_tokens=%d < 0", T);
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  if (k < 1 || k > kMaxTopK) return fail(GPTOSS_ERR_INVALID, "top_k=%d outside [1, 8]", k);
  if (T == 0) return ok();
  if (!idx || !counts || !offsets || !gather_map || !perm_token || !active || !n_active)
    return fail(GPTOSS_ERR_INVALID, "null pointer");
  HIP_TRY(launch_plan(idx, T, k, E, PlanBufs{counts, offsets, gather_map, perm_token, active, n_active, nullptr},
                      static_cast<hipStream_t>(stream)),
          "plan launch");
  return ok();
}

int gptoss_moe_scatter_tokens(const uint16_t* x, const int32_t* gather_map, uint16_t* permuted, int T, int H, int k,
                              void* stream) {
  if (T < 0 || k < 1 || H <= 0 || H % 8 != 0) return fail(GPTOSS_ERR_INVALID, "bad shape T=%d H=%d k=%d", T, H, k);
  if (T == 0) return ok();
  if (!x || !gather_map || !permuted) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(x) || !aligned16(permuted)) return fail(GPTOSS_ERR_INVALID, "x/permuted must be 16-byte aligned");
  HIP_TRY(launch_scatter(x, gather_map, permuted, T, H, k, static_cast<hipStream_t>(stream)), "scatter launch");
  return ok();
}

int gptoss_mxfp4_gemv_forward(const uint16_t* x, int M, const uint8_t* wn, const uint8_t* ws, const uint16_t* bias,
                              uint16_t* y, int N, int K, void* stream) {
  int rc = check_mxfp4_shape(N, K);
  if (rc != GPTOSS_OK) return rc;
  if (M < 0) return fail(GPTOSS_ERR_INVALID, "M=%d < 0", M);
  if (M == 0) return ok();
  if (!x || !wn || !ws || !y) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(wn)) return fail(GPTOSS_ERR_INVALID, "tiled nibbles must be 16-byte aligned");
  HIP_TRY(launch_dense_gemv(x, M, wn, ws, bias, y, N, K, static_cast<hipStream_t>(stream)), "gemv launch");
  return ok();
}

int gptoss_swiglu_forward(const uint16_t* in, uint16_t* out, int T, int I, float alpha, float limit, void* stream) {
  if (T < 0 || I <= 0) return fail(GPTOSS_ERR_INVALID, "bad shape T=%d I=%d", T, I);
  if (T == 0) return ok();
  if (!in || !out) return fail(GPTOSS_ERR_INVALID, "null pointer");
  HIP_TRY(launch_swiglu(in, out, T, I, alpha, limit, static_cast<hipStream_t>(stream)), "swiglu launch");
  return ok();
}

int gptoss_fused_residual_rmsnorm_forward(const uint16_t* residual, const uint16_t* delta, const uint16_t* weight,
                                          uint16_t* normed, uint16_t* sum_out, int T, int H, float eps,
                                          void* stream) {
  if (T < 0 || H <= 0 || H % 8 != 0)
    return fail(GPTOSS_ERR_INVALID, "bad shape T=%d H=%d (H a positive multiple of 8)", T, H);
  if (T == 0) return ok();
  if (!residual || !delta || !weight || !normed) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(residual) || !aligned16(delta) || (sum_out && !aligned16(sum_out)))
    return fail(GPTOSS_ERR_INVALID, "residual, delta and sum_out must be 16-byte aligned");
  HIP_TRY(launch_residual_rmsnorm(residual, delta, weight, normed, sum_out, T, H, eps,
                                  static_cast<hipStream_t>(stream)),
          "residual rmsnorm launch");
  return ok();
}

int gptoss_moe_combine_forward(uint16_t* out, const uint16_t* y, const int32_t* gather_map, const float* w,
                               const uint16_t* residual, int T, int H, int k, void* stream) {
  if (T < 0 || H <= 0 || k < 1 || k > kMaxTopK) return fail(GPTOSS_ERR_INVALID, "bad shape T=%d H=%d k=%d", T, H, k);
  if (T == 0) return ok();
  if (!out || !y || !gather_map || !w) return fail(GPTOSS_ERR_INVALID, "null pointer");
  HIP_TRY(launch_combine(out, y, gather_map, w, residual, T, H, k, static_cast<hipStream_t>(stream)),
          "combine launch");
  return ok();
}

int gptoss_moe_grouped_mxfp4_gemm(const uint16_t* x, const int32_t* row_index, const int32_t* offsets, int E,
                                  int rows, const uint8_t* nib, const uint8_t* sc, const uint16_t* bias, int N, int K,
                                  int swiglu, float alpha, float limit, uint16_t* out, uint16_t* gate_up,
                                  void* stream) {
  int rc = check_mxfp4_shape(N, K);
  if (rc != GPTOSS_OK) return rc;
  if (E < 1 || E > kMaxExperts) return fail(GPTOSS_ERR_UNSUPPORTED, "num_experts=%d outside [1, %d]", E, kMaxExperts);
  if (rows < 0) return fail(GPTOSS_ERR_INVALID, "rows=%d < 0", rows);
  if (rows == 0) return ok();
  if (!x || !offsets || !nib || !sc || !out) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(x) || !aligned16(out) || (gate_up && !aligned16(gate_up)) || !aligned16(nib))
    return fail(GPTOSS_ERR_INVALID, "x, out, gate_up and the nibbles must be 16-byte aligned");
  if (bias && (reinterpret_cast<uintptr_t>(bias) & 7u))
    return fail(GPTOSS_ERR_INVALID, "bias must be 8-byte aligned");
  if (swiglu && N % 2 != 0) return fail(GPTOSS_ERR_INVALID, "swiglu needs an even N");
  GroupedArgs g{};
  g.x = x;
  g.row_index = row_index;
  g.offsets = offsets;
  g.E = E;
  g.rows = rows;
  g.wn = nib;
  g.ws = sc;
  g.N = N;
  g.K = K;
  g.bias = bias;
  g.out = out;
  g.gate_up = swiglu ? gate_up : nullptr;
  g.gated = swiglu != 0;
  g.alpha = alpha;
  g.limit = limit;
  HIP_TRY(launch_grouped_mxfp4(g, static_cast<hipStream_t>(stream)), "grouped gemm launch");
  return ok();
}

int gptoss_mxfp4_dequant(const uint8_t* wn, const uint8_t* ws, int N, int K, uint16_t* out, void* stream) {
  int rc = check_mxfp4_shape(N, K);
  if (rc != GPTOSS_OK) return rc;
  if (!wn || !ws || !out) return fail(GPTOSS_ERR_INVALID, "null pointer");
  if (!aligned16(wn)) return fail(GPTOSS_ERR_INVALID, "tiled nibbles must be 16-byte aligned");
  HIP_TRY(launch_dequant(wn, ws, N, K, out, static_cast<hipStream_t>(stream)), "dequant launch");
  return ok();
}

}  // extern "C"
