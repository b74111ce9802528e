// gptoss_moe_compat.cpp -- the reference's C++ MoE operator (namespace
// gptoss, moe_layer.cu:1556-1615) forwarding to the C ABI of gptoss_moe.h.
// Error behaviour follows the reference: print the message and abort.
#include "gptoss_moe_compat.hpp"

#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <mutex>
#include <vector>

#include "gptoss_moe.h"

namespace gptoss {

class MoELayer {
 public:
  gptoss_moe_layer* impl = nullptr;
  int device = -1;  // device whose shared workspace this layer holds a reference on
};

namespace {

constexpr int kExperts = 128;  // ModelConfig::experts_per_gpu with ep_size 1 (config.h:20,63)
// The engine's MoE scratch capacity (MAX_TOKENS, engine.cu:860): its prefill
// passes up to this many tokens to moe_layer_forward (transformer.cu:494-499).
constexpr int kDefaultMaxTokens = 8192;

// One forward workspace per device, shared by every layer on it, as the
// engine hands all its layers one set of scratch buffers (engine.cu:975-1000);
// the engine runs a device's layers one after another on one stream.  Freed
// with the last layer on the device.
struct SharedWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  int users = 0;
};
std::mutex g_ws_mu;
std::map<int, SharedWorkspace> g_ws;

[[noreturn]] void die(const char* what) {
  fprintf(stderr, "gptoss MoE: %s failed: %s\n", what, gptoss_last_error());
  abort();
}

void check(int rc, const char* what) {
  if (rc != GPTOSS_OK) die(what);
}

const uint16_t* u16(const __hip_bfloat16* p) { return reinterpret_cast<const uint16_t*>(p); }

}  // namespace

int moe_layer_max_tokens() {
  const char* env = getenv("GPTOSS_MOE_MAX_TOKENS");
  if (env != nullptr) {
    const int v = atoi(env);
    if (v > 0) return v;
  }
  return kDefaultMaxTokens;
}

MoELayer* moe_layer_create() {
  MoELayer* l = new MoELayer();
  l->impl = gptoss_moe_layer_create();
  if (l->impl == nullptr) die("moe_layer_create");
  return l;
}

void moe_layer_destroy(MoELayer* l) {
  if (l == nullptr) return;
  gptoss_moe_layer_destroy(l->impl);
  if (l->device >= 0) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    SharedWorkspace& ws = g_ws[l->device];
    if (--ws.users == 0) {
      int prev = -1;
      const bool have_prev = hipGetDevice(&prev) == hipSuccess;
      if (hipSetDevice(l->device) == hipSuccess) {
        (void)hipDeviceSynchronize();  // no forward on any stream may still use it
        (void)hipFree(ws.ptr);
      }
      if (have_prev) (void)hipSetDevice(prev);
      g_ws.erase(l->device);
    }
  }
  delete l;
}

void moe_layer_init(MoELayer* layer, int, int device_id, int, EPComm*, const CublasHandle*, const CublasHandle*,
                    hipStream_t, hipStream_t, const __hip_bfloat16* moe_norm_weight,
                    const __hip_bfloat16* router_weight, const __hip_bfloat16* router_bias,
                    const __hip_bfloat16* gate_up_proj_bias, const __hip_bfloat16* down_proj_bias,
                    MXFP4Weight* expert_mlp1, MXFP4Weight* expert_mlp2, __hip_bfloat16*, __hip_bfloat16*, int32_t*,
                    float*, int32_t*, __hip_bfloat16*, int32_t*, int32_t*, int32_t*, int32_t*, __hip_bfloat16*,
                    __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*,
                    __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*, ncclComm_t) {
  if (layer == nullptr || expert_mlp1 == nullptr || expert_mlp2 == nullptr) {
    fprintf(stderr, "gptoss MoE: moe_layer_init: null layer or expert table\n");
    abort();
  }
  gptoss_moe_config cfg;
  check(gptoss_moe_config_default(&cfg, kExperts, moe_layer_max_tokens()), "moe_layer_init (config)");
  std::vector<const uint8_t*> p1(kExperts), s1(kExperts), p2(kExperts), s2(kExperts);
  for (int e = 0; e < kExperts; ++e) {
    p1[e] = expert_mlp1[e].packed;
    s1[e] = expert_mlp1[e].scales;
    p2[e] = expert_mlp2[e].packed;
    s2[e] = expert_mlp2[e].scales;
  }
  gptoss_moe_weights w{};
  w.moe_norm_weight = u16(moe_norm_weight);
  w.router_weight = u16(router_weight);
  w.router_bias = u16(router_bias);
  w.gate_up_bias = u16(gate_up_proj_bias);
  w.down_bias = u16(down_proj_bias);
  w.mlp1_packed = p1.data();
  w.mlp1_scales = s1.data();
  w.mlp2_packed = p2.data();
  w.mlp2_scales = s2.data();
  // the device's shared workspace, grown when this config needs more
  void* ws_ptr = nullptr;
  size_t ws_bytes = 0;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    SharedWorkspace& ws = g_ws[device_id];
    const size_t need = gptoss_moe_layer_workspace_bytes(&cfg);
    if (need == 0) {
      fprintf(stderr, "gptoss MoE: moe_layer_init: invalid configuration\n");
      abort();
    }
    if (ws.bytes < need) {
      if (ws.users > 0) {
        fprintf(stderr, "gptoss MoE: moe_layer_init: layers on device %d need %zu workspace bytes, the shared "
                        "workspace holds %zu\n", device_id, need, ws.bytes);
        abort();
      }
      int prev = -1;
      if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(device_id) != hipSuccess ||
          hipMalloc(&ws.ptr, need) != hipSuccess) {
        fprintf(stderr, "gptoss MoE: moe_layer_init: hipMalloc(%zu) of the shared workspace failed\n", need);
        abort();
      }
      (void)hipSetDevice(prev);
      ws.bytes = need;
    }
    ws.users++;
    layer->device = device_id;
    ws_ptr = ws.ptr;
    ws_bytes = ws.bytes;
  }
  check(gptoss_moe_layer_init_with_workspace(layer->impl, &cfg, device_id, &w, ws_ptr, ws_bytes), "moe_layer_init");
}

void moe_layer_forward(MoELayer* layer, const __hip_bfloat16* input, __hip_bfloat16* output, int num_tokens,
                       hipStream_t stream) {
  check(gptoss_moe_layer_forward(layer->impl, u16(input), reinterpret_cast<uint16_t*>(output), num_tokens, stream),
        "moe_layer_forward");
}

void moe_layer_forward_prenormed(MoELayer* layer, const __hip_bfloat16* normed_input,
                                 const __hip_bfloat16* residual_input, __hip_bfloat16* output, int num_tokens,
                                 hipStream_t stream) {
  check(gptoss_moe_layer_forward_prenormed(layer->impl, u16(normed_input), u16(residual_input),
                                           reinterpret_cast<uint16_t*>(output), num_tokens, stream),
        "moe_layer_forward_prenormed");
}

const __hip_bfloat16* moe_layer_get_ffn_norm_weight(MoELayer* layer) {
  return reinterpret_cast<const __hip_bfloat16*>(gptoss_moe_layer_get_ffn_norm_weight(layer->impl));
}

}  // namespace gptoss
