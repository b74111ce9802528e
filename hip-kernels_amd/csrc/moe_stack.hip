// moe_stack.hip -- a stack of MoE layers stepped as the engine's decode step
// does, optionally as one cached hipGraph per token count.
//
// The reference engine's decode step (transformer.cu:653-753) is, per layer:
// attention -> delta; fused_residual_rmsnorm_forward(residual, delta) ->
// (normed, sum); moe_layer_forward_prenormed(normed, sum) -> residual.  Its
// MoE synchronises the host for expert offsets, so the step is launched
// eagerly every time (engine.cu:309-320).  Here each layer is one
// gptoss_moe_layer_forward_residual call, in place on the stack's residual
// buffer, and no call synchronises the host: the whole step, hook launches
// included, is captured once per token count on the stack's own stream and
// replayed on the caller's.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <new>
#include <vector>

#include "../../include/gptoss_moe.h"
#include "moe_status.h"

using namespace gxmoe;

namespace {

struct DeviceScope {
  int prev = -1;
  bool changed = false;
  hipError_t err = hipSuccess;
  explicit DeviceScope(int dev) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != dev) {
      err = hipSetDevice(dev);
      changed = err == hipSuccess;
    }
  }
  ~DeviceScope() {
    if (changed) (void)hipSetDevice(prev);
  }
};

struct StepGraph {
  gptoss_layer_hook hook = nullptr;
  void* user = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

}  // namespace

struct gptoss_moe_stack {
  std::vector<gptoss_moe_layer*> layers;
  bool owns_layers = false;
  int device = 0;
  int H = 0;
  int max_tokens = 0;
  uint16_t* residual = nullptr;  // [max_tokens][H], the stack's own or bound
  uint16_t* deltas = nullptr;    // [layers][max_tokens][H], likewise
  uint16_t* own_residual = nullptr;
  uint16_t* own_deltas = nullptr;
  hipStream_t capture = nullptr;
  std::map<int, StepGraph> graphs;  // by token count

  static void drop(StepGraph& g) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
    g = StepGraph{};
  }
  ~gptoss_moe_stack() {
    DeviceScope ds(device);
    (void)hipDeviceSynchronize();  // replays still running on the callers' streams end first
    for (auto& kv : graphs) drop(kv.second);
    if (capture) (void)hipStreamDestroy(capture);
    if (own_residual) (void)hipFree(own_residual);
    if (own_deltas) (void)hipFree(own_deltas);
    if (owns_layers)
      for (gptoss_moe_layer* L : layers) gptoss_moe_layer_destroy(L);
  }

  // The eager step: every layer's hook and forward_residual on `s`.
  int run(int T, gptoss_layer_hook hook, void* user, hipStream_t s) {
    const size_t stride = static_cast<size_t>(max_tokens) * H;
    for (size_t l = 0; l < layers.size(); ++l) {
      uint16_t* d = deltas + stride * l;
      if (hook) hook(user, static_cast<int>(l), residual, d, T, s);
      const int rc = gptoss_moe_layer_forward_residual(layers[l], residual, d, nullptr, residual, T, s);
      if (rc != GPTOSS_OK) return rc;
    }
    return GPTOSS_OK;
  }
};

namespace {

// Buffers and the capture stream, once the layers are in place.
int finish_create(gptoss_moe_stack* st) {
  gptoss_moe_config c0{};
  int dev0 = 0;
  int rc = gptoss_moe_layer_get_config(st->layers[0], &c0, &dev0);
  if (rc != GPTOSS_OK) return rc;
  st->device = dev0;
  st->H = c0.hidden_size;
  st->max_tokens = c0.max_tokens;
  for (size_t l = 0; l < st->layers.size(); ++l) {
    gptoss_moe_config c{};
    int dev = 0;
    if ((rc = gptoss_moe_layer_get_config(st->layers[l], &c, &dev)) != GPTOSS_OK) return rc;
    if (dev != dev0 || c.hidden_size != c0.hidden_size)
      return set_error(GPTOSS_ERR_INVALID, "layer %zu: device %d / hidden %d differ from layer 0 (%d / %d)", l, dev,
                       c.hidden_size, dev0, c0.hidden_size);
    if (gptoss_moe_layer_get_ffn_norm_weight(st->layers[l]) == nullptr)
      return set_error(GPTOSS_ERR_INVALID, "layer %zu has no moe_norm_weight", l);
    if (c.max_tokens < st->max_tokens) st->max_tokens = c.max_tokens;
  }
  DeviceScope ds(st->device);
  if (ds.err != hipSuccess) return set_error(GPTOSS_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(ds.err));
  const size_t tok = static_cast<size_t>(st->max_tokens) * st->H * 2;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&st->own_residual), tok);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&st->own_deltas), tok * st->layers.size());
  if (e != hipSuccess) return set_error(GPTOSS_ERR_OOM, "stack buffers: %s", hipGetErrorString(e));
  st->residual = st->own_residual;
  st->deltas = st->own_deltas;
  e = hipMemset(st->residual, 0, tok);
  if (e == hipSuccess) e = hipMemset(st->deltas, 0, tok * st->layers.size());
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&st->capture, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "stack init: %s", hipGetErrorString(e));
  return GPTOSS_OK;
}

}  // namespace

extern "C" {

static int gptoss_moe_stack_create_impl(const gptoss_moe_config* cfg, int device_id, const gptoss_checkpoint* ckpt,
                                        int first_layer, int num_layers, gptoss_moe_stack** out) {
  if (!cfg || !ckpt || !out) return set_error(GPTOSS_ERR_INVALID, "null argument");
  *out = nullptr;
  if (num_layers < 1 || first_layer < 0)
    return set_error(GPTOSS_ERR_INVALID, "layers [%d, %d + %d) is empty or negative", first_layer, first_layer,
                     num_layers);
  std::unique_ptr<gptoss_moe_stack> st(new gptoss_moe_stack());
  st->owns_layers = true;
  for (int l = 0; l < num_layers; ++l) {
    gptoss_moe_layer* L = gptoss_moe_layer_create();
    if (!L) return set_error(GPTOSS_ERR_OOM, "out of host memory");
    st->layers.push_back(L);
    const int rc = gptoss_moe_layer_init_from_checkpoint(L, cfg, device_id, ckpt, first_layer + l);
    if (rc != GPTOSS_OK) return rc;  // the message names the layer's tensor
  }
  const int rc = finish_create(st.get());
  if (rc != GPTOSS_OK) return rc;
  *out = st.release();
  clear_error();
  return GPTOSS_OK;
}

int gptoss_moe_stack_create(const gptoss_moe_config* cfg, int device_id, const gptoss_checkpoint* ckpt,
                            int first_layer, int num_layers, gptoss_moe_stack** out) {
  return guarded([&] { return gptoss_moe_stack_create_impl(cfg, device_id, ckpt, first_layer, num_layers, out); });
}

static int gptoss_moe_stack_create_from_layers_impl(gptoss_moe_layer* const* layers, int num_layers,
                                                    gptoss_moe_stack** out) {
  if (!layers || !out) return set_error(GPTOSS_ERR_INVALID, "null argument");
  *out = nullptr;
  if (num_layers < 1) return set_error(GPTOSS_ERR_INVALID, "num_layers=%d must be >= 1", num_layers);
  std::unique_ptr<gptoss_moe_stack> st(new gptoss_moe_stack());
  for (int l = 0; l < num_layers; ++l) {
    if (!layers[l]) return set_error(GPTOSS_ERR_INVALID, "layer %d is NULL", l);
    st->layers.push_back(layers[l]);
  }
  const int rc = finish_create(st.get());
  if (rc != GPTOSS_OK) return rc;
  *out = st.release();
  clear_error();
  return GPTOSS_OK;
}

int gptoss_moe_stack_create_from_layers(gptoss_moe_layer* const* layers, int num_layers, gptoss_moe_stack** out) {
  return guarded([&] { return gptoss_moe_stack_create_from_layers_impl(layers, num_layers, out); });
}

int gptoss_moe_stack_io(gptoss_moe_stack* st, uint16_t** residual, uint16_t** deltas, int* max_tokens,
                        int* num_layers) {
  if (!st) return set_error(GPTOSS_ERR_INVALID, "stack is NULL");
  if (residual) *residual = st->residual;
  if (deltas) *deltas = st->deltas;
  if (max_tokens) *max_tokens = st->max_tokens;
  if (num_layers) *num_layers = static_cast<int>(st->layers.size());
  clear_error();
  return GPTOSS_OK;
}

int gptoss_moe_stack_bind(gptoss_moe_stack* st, uint16_t* residual, uint16_t* deltas) {
  if (!st) return set_error(GPTOSS_ERR_INVALID, "stack is NULL");
  if ((reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(deltas)) & 15u)
    return set_error(GPTOSS_ERR_INVALID, "residual and deltas must be 16-byte aligned");
  {
    DeviceScope ds(st->device);
    (void)hipDeviceSynchronize();  // replays still running end before their graphs go
    for (auto& kv : st->graphs) gptoss_moe_stack::drop(kv.second);  // they hold the old pointers
    st->graphs.clear();
  }
  st->residual = residual ? residual : st->own_residual;
  st->deltas = deltas ? deltas : st->own_deltas;
  clear_error();
  return GPTOSS_OK;
}

int gptoss_moe_stack_layer(gptoss_moe_stack* st, int index, gptoss_moe_layer** layer) {
  if (!st || !layer) return set_error(GPTOSS_ERR_INVALID, "null argument");
  if (index < 0 || index >= static_cast<int>(st->layers.size()))
    return set_error(GPTOSS_ERR_INVALID, "layer %d outside [0, %zu)", index, st->layers.size());
  *layer = st->layers[index];
  clear_error();
  return GPTOSS_OK;
}

static int gptoss_moe_stack_decode_step_impl(gptoss_moe_stack* st, int T, gptoss_layer_hook hook, void* user,
                                             int use_graph, void* stream) {
  if (!st) return set_error(GPTOSS_ERR_INVALID, "stack is NULL");
  if (T < 0 || T > st->max_tokens)
    return set_error(GPTOSS_ERR_INVALID, "num_tokens=%d outside [0, max_tokens=%d]", T, st->max_tokens);
  if (T == 0) {
    clear_error();
    return GPTOSS_OK;
  }
  DeviceScope ds(st->device);
  if (ds.err != hipSuccess) return set_error(GPTOSS_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(ds.err));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!use_graph) {
    const int rc = st->run(T, hook, user, s);
    if (rc == GPTOSS_OK) clear_error();
    return rc;
  }
  StepGraph& g = st->graphs[T];
  if (g.exec && (g.hook != hook || g.user != user)) gptoss_moe_stack::drop(g);
  if (!g.exec) {
    // capture on the stack's stream, which nothing else uses: the caller's
    // stream may be the null stream, which cannot be captured
    hipError_t e = hipStreamBeginCapture(st->capture, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    const int rc = st->run(T, hook, user, st->capture);
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(st->capture, &graph);
    if (rc != GPTOSS_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return rc;
    }
    if (e != hipSuccess) {
      if (graph) (void)hipGraphDestroy(graph);
      return set_error(GPTOSS_ERR_HIP, "hipStreamEndCapture (did the hook synchronise?): %s", hipGetErrorString(e));
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGraphDestroy(graph);
      return set_error(GPTOSS_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    g.graph = graph;
    g.exec = exec;
    g.hook = hook;
    g.user = user;
  }
  const hipError_t e = hipGraphLaunch(g.exec, s);
  if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "hipGraphLaunch: %s", hipGetErrorString(e));
  clear_error();
  return GPTOSS_OK;
}

int gptoss_moe_stack_decode_step(gptoss_moe_stack* st, int T, gptoss_layer_hook hook, void* user, int use_graph,
                                 void* stream) {
  return guarded([&] { return gptoss_moe_stack_decode_step_impl(st, T, hook, user, use_graph, stream); });
}

void gptoss_moe_stack_destroy(gptoss_moe_stack* st) { delete st; }

}  // extern "C"
