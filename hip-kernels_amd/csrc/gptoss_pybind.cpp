// gptoss_pybind.cpp -- the reference's `gptoss` Python module
// (src/python/bindings.cpp:215-446) over the C ABI of gptoss_moe.h.
//
// Surface kept from the reference: InferenceEngine (init / shutdown /
// is_initialized / generate / generate_batch), ModelConfig's read-only
// static properties and methods, profiler_enabled(), __version__ and
// MODEL_NAME; argument errors raise ValueError and engine failures
// RuntimeError (bindings.cpp:105-141), and the GIL is released around every
// call into the library (bindings.cpp:236,253,279,299).  This build covers the
// MoE half of the model, so the engine loads and runs the MoE layers of a
// checkpoint (decode_step), generate() validates its arguments as the
// reference does and then raises RuntimeError, and MoELayer exposes one
// layer's operator (moe_layer_forward / _prenormed, bindings-level).
//
// Tensors are taken by duck typing (data_ptr, shape, dtype, is_contiguous,
// device), so the module needs no torch headers; torch is imported first when
// it is installed, so that libgptoss_moe.so, opened here with dlopen, binds to
// the HIP runtime torch already loaded.
#include <dlfcn.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "gptoss_moe.h"

namespace py = pybind11;

namespace {

// ---- the C ABI, resolved at import -----------------------------------------
struct Api {
  const char* (*last_error)();
  int (*abi_version)();
  int (*config_default)(gptoss_moe_config*, int, int);
  gptoss_moe_layer* (*layer_create)();
  void (*layer_destroy)(gptoss_moe_layer*);
  int (*layer_init_from_checkpoint)(gptoss_moe_layer*, const gptoss_moe_config*, int, const gptoss_checkpoint*, int);
  int (*layer_forward)(gptoss_moe_layer*, const uint16_t*, uint16_t*, int, void*);
  int (*layer_forward_prenormed)(gptoss_moe_layer*, const uint16_t*, const uint16_t*, uint16_t*, int, void*);
  int (*layer_forward_residual)(gptoss_moe_layer*, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*, int,
                                void*);
  int (*layer_forward_routed)(gptoss_moe_layer*, const uint16_t*, const uint16_t*, const int32_t*, const float*,
                              uint16_t*, int, void*);
  int (*layer_set_profiling)(gptoss_moe_layer*, int);
  int (*layer_profile_read)(gptoss_moe_layer*, float*, float*, float*, float*, int*);
  int (*layer_profile_records)(gptoss_moe_layer*, gptoss_moe_prof_record*, int, int*);
  int (*checkpoint_open)(const char*, gptoss_checkpoint**);
  void (*checkpoint_close)(gptoss_checkpoint*);
  int (*checkpoint_find)(const gptoss_checkpoint*, const char*, gptoss_tensor_info*);
  int (*stack_create)(const gptoss_moe_config*, int, const gptoss_checkpoint*, int, int, gptoss_moe_stack**);
  int (*stack_io)(gptoss_moe_stack*, uint16_t**, uint16_t**, int*, int*);
  int (*stack_bind)(gptoss_moe_stack*, uint16_t*, uint16_t*);
  int (*stack_layer)(gptoss_moe_stack*, int, gptoss_moe_layer**);
  int (*stack_decode_step)(gptoss_moe_stack*, int, gptoss_layer_hook, void*, int, void*);
  void (*stack_destroy)(gptoss_moe_stack*);
};
Api api{};

template <typename F>
void resolve(void* h, F& fn, const char* name) {
  fn = reinterpret_cast<F>(dlsym(h, name));
  if (fn == nullptr) throw std::runtime_error(std::string("libgptoss_moe.so lacks ") + name);
}

void load_library(const std::string& path) {
  void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (h == nullptr) throw py::import_error(std::string("cannot load ") + path + ": " + dlerror());
  resolve(h, api.last_error, "gptoss_last_error");
  resolve(h, api.abi_version, "gptoss_abi_version");
  resolve(h, api.config_default, "gptoss_moe_config_default");
  resolve(h, api.layer_create, "gptoss_moe_layer_create");
  resolve(h, api.layer_destroy, "gptoss_moe_layer_destroy");
  resolve(h, api.layer_init_from_checkpoint, "gptoss_moe_layer_init_from_checkpoint");
  resolve(h, api.layer_forward, "gptoss_moe_layer_forward");
  resolve(h, api.layer_forward_prenormed, "gptoss_moe_layer_forward_prenormed");
  resolve(h, api.layer_forward_residual, "gptoss_moe_layer_forward_residual");
  resolve(h, api.layer_forward_routed, "gptoss_moe_layer_forward_routed");
  resolve(h, api.layer_set_profiling, "gptoss_moe_layer_set_profiling");
  resolve(h, api.layer_profile_read, "gptoss_moe_layer_profile_read");
  resolve(h, api.layer_profile_records, "gptoss_moe_layer_profile_records");
  resolve(h, api.checkpoint_open, "gptoss_checkpoint_open");
  resolve(h, api.checkpoint_close, "gptoss_checkpoint_close");
  resolve(h, api.checkpoint_find, "gptoss_checkpoint_find");
  resolve(h, api.stack_create, "gptoss_moe_stack_create");
  resolve(h, api.stack_io, "gptoss_moe_stack_io");
  resolve(h, api.stack_bind, "gptoss_moe_stack_bind");
  resolve(h, api.stack_layer, "gptoss_moe_stack_layer");
  resolve(h, api.stack_decode_step, "gptoss_moe_stack_decode_step");
  resolve(h, api.stack_destroy, "gptoss_moe_stack_destroy");
  if (api.abi_version() != GPTOSS_MOE_ABI_VERSION)
    throw py::import_error("libgptoss_moe.so ABI " + std::to_string(api.abi_version()) + ", this module expects " +
                           std::to_string(GPTOSS_MOE_ABI_VERSION));
}

// A status code from the library as the reference bindings map errors:
// argument errors to ValueError, everything else to RuntimeError.
struct Status {
  int rc = GPTOSS_OK;
  std::string msg;
};

Status status(int rc) {
  Status s;
  s.rc = rc;
  if (rc != GPTOSS_OK) s.msg = api.last_error();
  return s;
}

void raise(const Status& s, const char* what) {
  if (s.rc == GPTOSS_OK) return;
  const std::string m = std::string(what) + ": " + s.msg;
  if (s.rc == GPTOSS_ERR_INVALID) throw py::value_error(m);
  throw std::runtime_error(m);
}

// ---- tensors by duck typing ------------------------------------------------
struct Tensor {
  uintptr_t ptr = 0;
  std::vector<int64_t> shape;
};

// A contiguous tensor on cuda:`device` with the given trailing shape (a -1
// leading entry accepts any row count) whose dtype's name is one of `dtypes`.
Tensor tensor_arg(py::handle t, const char* name, const std::vector<int64_t>& want, int device,
                  const std::vector<std::string>& dtypes) {
  if (t.is_none() || !py::hasattr(t, "data_ptr")) throw py::value_error(std::string(name) + " must be a tensor");
  Tensor v;
  for (py::handle d : t.attr("shape")) v.shape.push_back(d.cast<int64_t>());
  bool ok = v.shape.size() == want.size();
  for (size_t i = 0; ok && i < want.size(); ++i) ok = want[i] < 0 || want[i] == v.shape[i];
  if (!ok) {
    std::string ws = "[", gs = "[";
    for (size_t i = 0; i < want.size(); ++i) ws += (i ? ", " : "") + (want[i] < 0 ? std::string("T") : std::to_string(want[i]));
    for (size_t i = 0; i < v.shape.size(); ++i) gs += (i ? ", " : "") + std::to_string(v.shape[i]);
    throw py::value_error(std::string(name) + " has shape " + gs + "], expected " + ws + "]");
  }
  const std::string dt = py::str(t.attr("dtype"));
  bool dt_ok = false;
  for (const auto& d : dtypes) dt_ok = dt_ok || dt == d;
  if (!dt_ok) throw py::value_error(std::string(name) + " has dtype " + dt + ", expected " + dtypes[0]);
  if (!t.attr("is_contiguous")().cast<bool>()) throw py::value_error(std::string(name) + " must be contiguous");
  py::object dev = t.attr("device");
  const std::string type = py::str(dev.attr("type"));
  py::object idx = dev.attr("index");
  if (type != "cuda" || idx.is_none() || idx.cast<int>() != device)
    throw py::value_error(std::string(name) + " is on " + std::string(py::str(dev)) + ", expected cuda:" +
                          std::to_string(device));
  v.ptr = t.attr("data_ptr")().cast<uintptr_t>();
  return v;
}

const std::vector<std::string> kBf16 = {"torch.bfloat16", "torch.int16", "torch.uint16"};

void* stream_arg(py::handle stream) {
  if (!stream.is_none()) return reinterpret_cast<void*>(stream.cast<uintptr_t>());
  try {  // the caller's current torch stream, as torch code would expect
    py::object torch = py::module_::import("torch");
    return reinterpret_cast<void*>(torch.attr("cuda").attr("current_stream")().attr("cuda_stream").cast<uintptr_t>());
  } catch (const py::error_already_set&) {
    return nullptr;
  }
}

py::object empty_like(py::handle t) { return t.attr("new_empty")(t.attr("shape")); }

// ---- checkpoint helpers ----------------------------------------------------
struct Checkpoint {
  gptoss_checkpoint* h = nullptr;
  explicit Checkpoint(const std::string& path) {
    Status s;
    {
      py::gil_scoped_release nogil;
      s = status(api.checkpoint_open(path.c_str(), &h));
    }
    if (s.rc != GPTOSS_OK) throw std::runtime_error("Engine init failed: " + s.msg);
  }
  ~Checkpoint() {
    if (h) api.checkpoint_close(h);
  }
  bool find(const std::string& name, gptoss_tensor_info* info) const {
    return api.checkpoint_find(h, name.c_str(), info) == GPTOSS_OK;
  }
  // (E, H, I) of layer `l` from its router weight [E][H] and gate_up tensors.
  bool moe_shape(int l, int* E, int* H, int* I) const {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    gptoss_tensor_info t{};
    if (!find(p + "mlp.gate.weight", &t) && !find(p + "mlp.router.weight", &t)) return false;
    *E = static_cast<int>(t.shape[0]);
    *H = static_cast<int>(t.shape[1]);
    for (const char* n : {"mlp.experts.gate_up_proj_blocks", "mlp.experts.gate_up_proj_bias"})
      if (find(p + n, &t)) return (*I = static_cast<int>(t.shape[1] / 2)), true;
    for (const char* n : {"mlp.experts.0.mlp1.weight", "mlp.experts.0.gate_up_proj.weight", "mlp.experts.0.w1.weight"})
      if (find(p + n, &t)) return (*I = static_cast<int>(t.shape[0] / 2)), true;
    return false;
  }
};

gptoss_moe_config make_config(int E, int H, int I, int max_tokens, int top_k, int prefill_min_tokens,
                              bool decode_exact) {
  gptoss_moe_config c{};
  raise(status(api.config_default(&c, E, max_tokens)), "config");
  c.hidden_size = H;
  c.intermediate_size = I;
  c.top_k = top_k;
  c.prefill_min_tokens = prefill_min_tokens;
  c.decode_exact = decode_exact ? 1 : 0;
  return c;
}

// ---- the module-level profiler (bindings.cpp:421-439, profiler.cu) -------
// The reference records a HIP event pair per PROF region of the engine and
// writes them as a Chrome trace or a summary per (category, name).  Here the
// regions are the MoE launches of every live MoELayer and engine layer: each
// registers its layer handles, profiler_reset(max_forwards) arms per-launch
// timing on all of them (and on layers created later) and clears what was
// recorded, and the save functions read the records back through the C ABI.
// Launch i of a forward is "moe_route" (the plan for forward_routed),
// "moe_gate_up", "moe_down" or "moe_combine", in category "moe_decode" or
// "moe_prefill" (grouped kernels).
struct ProfSource {
  gptoss_moe_layer* h;
  int layer;
  int device;
};
std::mutex g_prof_mu;
std::map<const void*, std::vector<ProfSource>> g_prof_sources;  // owner -> its layers
int g_prof_forwards = 0;                                         // armed capacity per layer; 0: off

void prof_register(const void* owner, std::vector<ProfSource> layers) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (g_prof_forwards > 0)
    for (const ProfSource& p : layers) (void)api.layer_set_profiling(p.h, g_prof_forwards);
  g_prof_sources[owner] = std::move(layers);
}

void prof_unregister(const void* owner) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_sources.erase(owner);
}

struct ProfEvent {
  const char* name;
  const char* category;
  int device, layer;
  double ts_us;  // host-clock start
  float dur_ms;
};

constexpr const char* kLaunchNames[4] = {"moe_route", "moe_gate_up", "moe_down", "moe_combine"};

// Every recorded launch of every registered layer (waits for their events).
std::vector<ProfEvent> prof_collect() {
  std::vector<ProfEvent> ev;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (const auto& kv : g_prof_sources)
    for (const ProfSource& p : kv.second) {
      int n = 0;
      if (api.layer_profile_records(p.h, nullptr, 0, &n) != GPTOSS_OK || n <= 0) continue;
      std::vector<gptoss_moe_prof_record> r(static_cast<size_t>(n));
      if (api.layer_profile_records(p.h, r.data(), n, &n) != GPTOSS_OK) continue;
      for (const gptoss_moe_prof_record& f : r)
        for (int i = 0; i < 4; ++i)
          ev.push_back({kLaunchNames[i], f.prefill ? "moe_prefill" : "moe_decode", p.device, p.layer,
                        f.host_us + 1000.0 * f.start_ms[i], f.dur_ms[i]});
    }
  std::sort(ev.begin(), ev.end(), [](const ProfEvent& a, const ProfEvent& b) { return a.ts_us < b.ts_us; });
  return ev;
}

void profiler_reset(int max_forwards) {
  if (max_forwards < 0) throw py::value_error("max_forwards must be non-negative");
  py::gil_scoped_release nogil;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_forwards = max_forwards;
  for (const auto& kv : g_prof_sources)
    for (const ProfSource& p : kv.second) (void)api.layer_set_profiling(p.h, max_forwards);
}

// profiler_save_chrome_trace (profiler.cu:215-270): one "X" event per launch,
// named L<layer>/<launch>, on thread <device>, with ts relative to the first.
void profiler_save_trace(const std::string& path) {
  std::vector<ProfEvent> ev;
  {
    py::gil_scoped_release nogil;
    ev = prof_collect();
  }
  FILE* f = std::fopen(path.c_str(), "w");
  if (f == nullptr) {
    std::fprintf(stderr, "profiler: cannot open %s for writing\n", path.c_str());
    return;
  }
  const double base = ev.empty() ? 0.0 : ev.front().ts_us;
  std::fprintf(f, "{\"traceEvents\":[\n");
  std::vector<int> devs;
  for (const ProfEvent& e : ev)
    if (std::find(devs.begin(), devs.end(), e.device) == devs.end()) devs.push_back(e.device);
  std::sort(devs.begin(), devs.end());
  for (int d : devs)
    std::fprintf(f, "{\"name\":\"thread_name\",\"ph\":\"M\",\"pid\":0,\"tid\":%d,\"args\":{\"name\":\"GPU %d\"}},\n", d,
                 d);
  for (size_t i = 0; i < ev.size(); ++i) {
    const ProfEvent& e = ev[i];
    long long dur = static_cast<long long>(e.dur_ms * 1000.0f);
    if (dur < 1) dur = 1;
    std::fprintf(f,
                 "{\"name\":\"L%d/%s\",\"cat\":\"%s\",\"ph\":\"X\",\"ts\":%lld,\"dur\":%lld,\"pid\":0,\"tid\":%d,"
                 "\"args\":{\"layer\":%d,\"dur_ms\":%.4f}}%s\n",
                 e.layer, e.name, e.category, static_cast<long long>(e.ts_us - base), dur, e.device, e.layer,
                 e.dur_ms, i + 1 < ev.size() ? "," : "");
  }
  std::fprintf(f, "]}\n");
  std::fclose(f);
  std::fprintf(stderr, "profiler: wrote %zu events to %s\n", ev.size(), path.c_str());
}

// profiler_save_summary_json (profiler.cu:276-360): per (category, name) the
// count, total, average, minimum and maximum milliseconds and the share of
// the total, sorted by total descending.
void profiler_save_summary(const std::string& path) {
  std::vector<ProfEvent> ev;
  {
    py::gil_scoped_release nogil;
    ev = prof_collect();
  }
  struct Agg {
    std::string name, category;
    int count = 0;
    double total = 0, mn = 1e30, mx = 0;
  };
  std::vector<Agg> agg;
  double all = 0;
  for (const ProfEvent& e : ev) {
    auto it = std::find_if(agg.begin(), agg.end(),
                           [&](const Agg& a) { return a.name == e.name && a.category == e.category; });
    if (it == agg.end()) {
      agg.push_back(Agg{e.name, e.category});
      it = agg.end() - 1;
    }
    it->count += 1;
    it->total += e.dur_ms;
    it->mn = std::min(it->mn, static_cast<double>(e.dur_ms));
    it->mx = std::max(it->mx, static_cast<double>(e.dur_ms));
    all += e.dur_ms;
  }
  std::sort(agg.begin(), agg.end(), [](const Agg& a, const Agg& b) { return a.total > b.total; });
  FILE* f = std::fopen(path.c_str(), "w");
  if (f == nullptr) {
    std::fprintf(stderr, "profiler: cannot open %s for writing\n", path.c_str());
    return;
  }
  std::fprintf(f, "{\n  \"total_events\": %zu,\n  \"total_ms\": %.4f,\n  \"kernels\": [\n", ev.size(), all);
  for (size_t i = 0; i < agg.size(); ++i) {
    const Agg& a = agg[i];
    std::fprintf(f,
                 "    {\"name\":\"%s\",\"category\":\"%s\",\"count\":%d,\"total_ms\":%.4f,\"avg_ms\":%.4f,"
                 "\"min_ms\":%.4f,\"max_ms\":%.4f,\"pct\":%.2f}%s\n",
                 a.name.c_str(), a.category.c_str(), a.count, a.total, a.total / a.count, a.mn, a.mx,
                 all > 0 ? 100.0 * a.total / all : 0.0, i + 1 < agg.size() ? "," : "");
  }
  std::fprintf(f, "  ]\n}\n");
  std::fclose(f);
  std::fprintf(stderr, "profiler: wrote summary (%zu kernels) to %s\n", agg.size(), path.c_str());
}

// ---- MoELayer: the operator of one layer -----------------------------------
class PyMoELayer {
 public:
  PyMoELayer(const std::string& weights_dir, int layer, int max_tokens, int device, int top_k,
             int prefill_min_tokens, bool decode_exact) : device_(device) {
    if (max_tokens < 1) throw py::value_error("max_tokens must be positive");
    Checkpoint ck(weights_dir);
    int E = 0, H = 0, I = 0;
    if (!ck.moe_shape(layer, &E, &H, &I))
      throw std::runtime_error("no MoE layer " + std::to_string(layer) + " in " + weights_dir);
    cfg_ = make_config(E, H, I, max_tokens, top_k, prefill_min_tokens, decode_exact);
    h_ = api.layer_create();
    if (h_ == nullptr) throw std::runtime_error("gptoss_moe_layer_create failed");
    Status s;
    {
      py::gil_scoped_release nogil;
      s = status(api.layer_init_from_checkpoint(h_, &cfg_, device, ck.h, layer));
    }
    if (s.rc != GPTOSS_OK) {
      api.layer_destroy(h_);
      h_ = nullptr;
      raise(s, "MoELayer init");
    }
    prof_register(this, {ProfSource{h_, layer, device}});
  }
  ~PyMoELayer() { close(); }
  PyMoELayer(const PyMoELayer&) = delete;
  PyMoELayer& operator=(const PyMoELayer&) = delete;

  void close() {
    if (h_) {
      py::gil_scoped_release nogil;
      prof_unregister(this);
      api.layer_destroy(h_);
      h_ = nullptr;
    }
  }

  gptoss_moe_layer* handle() const {
    if (h_ == nullptr) throw std::runtime_error("MoELayer is closed");
    return h_;
  }

  py::object forward(py::object x, py::object out, py::object stream) {
    const Tensor tx = rows(x, "x", -1);
    if (out.is_none()) out = empty_like(x);
    const Tensor to = rows(out, "out", tx.shape[0]);
    void* s = stream_arg(stream);
    gptoss_moe_layer* h = handle();
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.layer_forward(h, u16(tx), u16(to), static_cast<int>(tx.shape[0]), s));
    }
    raise(st, "moe_layer_forward");
    return out;
  }

  py::object forward_prenormed(py::object normed, py::object residual, py::object out, py::object stream) {
    const Tensor tn = rows(normed, "normed", -1);
    const int T = static_cast<int>(tn.shape[0]);
    const Tensor tr = residual.is_none() ? Tensor{} : rows(residual, "residual", T);
    if (out.is_none()) out = empty_like(normed);
    const Tensor to = rows(out, "out", T);
    void* s = stream_arg(stream);
    gptoss_moe_layer* h = handle();
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.layer_forward_prenormed(h, u16(tn), u16(tr), u16(to), T, s));
    }
    raise(st, "moe_layer_forward_prenormed");
    return out;
  }

  py::object forward_residual(py::object residual, py::object delta, py::object residual_out, py::object out,
                              py::object stream) {
    const Tensor tr = rows(residual, "residual", -1);
    const int T = static_cast<int>(tr.shape[0]);
    const Tensor td = rows(delta, "delta", T);
    const Tensor ts = residual_out.is_none() ? Tensor{} : rows(residual_out, "residual_out", T);
    if (out.is_none()) out = empty_like(residual);
    const Tensor to = rows(out, "out", T);
    void* s = stream_arg(stream);
    gptoss_moe_layer* h = handle();
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.layer_forward_residual(h, u16(tr), u16(td), u16(ts), u16(to), T, s));
    }
    raise(st, "forward_residual");
    return out;
  }

  py::object forward_routed(py::object normed, py::object idx, py::object w, py::object residual, py::object out,
                            py::object stream) {
    const Tensor tn = rows(normed, "normed", -1);
    const int T = static_cast<int>(tn.shape[0]);
    const Tensor ti = tensor_arg(idx, "expert_indices", {T, cfg_.top_k}, device_, {"torch.int32"});
    const Tensor tw = tensor_arg(w, "expert_weights", {T, cfg_.top_k}, device_, {"torch.float32"});
    const Tensor tr = residual.is_none() ? Tensor{} : rows(residual, "residual", T);
    if (out.is_none()) out = empty_like(normed);
    const Tensor to = rows(out, "out", T);
    void* s = stream_arg(stream);
    gptoss_moe_layer* h = handle();
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.layer_forward_routed(h, u16(tn), u16(tr), reinterpret_cast<const int32_t*>(ti.ptr),
                                           reinterpret_cast<const float*>(tw.ptr), u16(to), T, s));
    }
    raise(st, "forward_routed");
    return out;
  }

  void set_profiling(int n) { raise(status(api.layer_set_profiling(handle(), n)), "set_profiling"); }

  py::tuple profile_read() {
    float r = 0, a = 0, b = 0, c = 0;
    int n = 0;
    gptoss_moe_layer* h = handle();
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.layer_profile_read(h, &r, &a, &b, &c, &n));
    }
    raise(st, "profile_read");
    return py::make_tuple(r, a, b, c, n);
  }

  const gptoss_moe_config& cfg() const { return cfg_; }
  int device() const { return device_; }

 private:
  Tensor rows(py::handle t, const char* name, int64_t T) const {
    return tensor_arg(t, name, {T, cfg_.hidden_size}, device_, kBf16);
  }
  static uint16_t* u16(const Tensor& t) { return reinterpret_cast<uint16_t*>(t.ptr); }

  gptoss_moe_layer* h_ = nullptr;
  gptoss_moe_config cfg_{};
  int device_ = 0;
};

// ---- InferenceEngine --------------------------------------------------------
class PyInferenceEngine {
 public:
  PyInferenceEngine() = default;
  ~PyInferenceEngine() { shutdown_impl(); }
  PyInferenceEngine(const PyInferenceEngine&) = delete;
  PyInferenceEngine& operator=(const PyInferenceEngine&) = delete;

  // InferenceEngine::init (bindings.cpp:225-240): here the MoE layers of the
  // checkpoint, in one layer stack on `device`.
  void init(const std::string& weights_dir, int max_tokens, int device, int top_k) {
    if (stack_ != nullptr) throw std::runtime_error("Engine init failed: [InferenceEngine] Already initialized");
    if (max_tokens < 1) throw py::value_error("max_tokens must be positive");
    Checkpoint ck(weights_dir);
    int E = 0, H = 0, I = 0;
    if (!ck.moe_shape(0, &E, &H, &I)) throw std::runtime_error("Engine init failed: no MoE layer 0 in " + weights_dir);
    int n = 0;
    for (int E2, H2, I2; ck.moe_shape(n, &E2, &H2, &I2);) ++n;
    gptoss_moe_config cfg = make_config(E, H, I, max_tokens, top_k, 128, false);
    Status st;
    {
      py::gil_scoped_release nogil;
      st = status(api.stack_create(&cfg, device, ck.h, 0, n, &stack_));
    }
    if (st.rc != GPTOSS_OK) {
      stack_ = nullptr;
      throw std::runtime_error("Engine init failed: " + st.msg);
    }
    cfg_ = cfg;
    device_ = device;
    num_layers_ = n;
    std::vector<ProfSource> layers;
    for (int l = 0; l < n; ++l) {
      gptoss_moe_layer* h = nullptr;
      if (api.stack_layer(stack_, l, &h) == GPTOSS_OK && h != nullptr) layers.push_back(ProfSource{h, l, device});
    }
    prof_register(this, std::move(layers));
  }

  bool is_initialized() const { return stack_ != nullptr; }

  void shutdown() {
    py::gil_scoped_release nogil;
    shutdown_impl();
  }

  // The MoE half of the decode step for all layers, in place on residual[:T]:
  // per layer residual = bf16(residual + delta[l]) + MoE_l(RMSNorm(...))
  // (transformer.cu:653-753).  residual [max_tokens][H] and deltas
  // [num_layers][max_tokens][H] are the caller's buffers, bound to the stack
  // (a new binding drops the captured graphs); use_graph replays one hipGraph
  // per token count.
  void decode_step(py::object residual, py::object deltas, int num_tokens, bool use_graph, py::object stream) {
    if (stack_ == nullptr) throw std::runtime_error("[InferenceEngine] Not initialized");
    if (num_tokens < 1 || num_tokens > cfg_.max_tokens)
      throw py::value_error("num_tokens must be in [1, " + std::to_string(cfg_.max_tokens) + "]");
    const Tensor tr = tensor_arg(residual, "residual", {cfg_.max_tokens, cfg_.hidden_size}, device_, kBf16);
    const Tensor td =
        tensor_arg(deltas, "deltas", {num_layers_, cfg_.max_tokens, cfg_.hidden_size}, device_, kBf16);
    void* s = stream_arg(stream);
    Status st;
    {
      py::gil_scoped_release nogil;
      if (tr.ptr != bound_r_ || td.ptr != bound_d_) {
        st = status(api.stack_bind(stack_, reinterpret_cast<uint16_t*>(tr.ptr), reinterpret_cast<uint16_t*>(td.ptr)));
        if (st.rc == GPTOSS_OK) {
          bound_r_ = tr.ptr;
          bound_d_ = td.ptr;
        }
      }
      if (st.rc == GPTOSS_OK) st = status(api.stack_decode_step(stack_, num_tokens, nullptr, nullptr, use_graph ? 1 : 0, s));
    }
    raise(st, "decode_step");
  }

  // generate / generate_batch (bindings.cpp:100-185): the same argument
  // checks, then RuntimeError -- attention, sampling and the tokenizer are not
  // part of this build.
  std::vector<int32_t> generate(const std::vector<int32_t>& prompt, int max_tokens, float temperature, float top_p) {
    if (prompt.empty()) throw py::value_error("prompt_tokens must not be empty");
    if (max_tokens <= 0) throw py::value_error("max_tokens must be positive");
    if (temperature < 0.0f) throw py::value_error("temperature must be non-negative");
    if (top_p <= 0.0f || top_p > 1.0f) throw py::value_error("top_p must be in (0, 1]");
    throw std::runtime_error(not_built());
  }

  std::vector<std::vector<int32_t>> generate_batch(const std::vector<std::vector<int32_t>>& prompts, int, float,
                                                   float) {
    if (prompts.empty()) throw py::value_error("prompts must not be empty");
    for (const auto& p : prompts)
      if (p.size() != prompts[0].size()) throw py::value_error("All prompts must have the same length");
    throw std::runtime_error(not_built());
  }

  int num_layers() const { return num_layers_; }
  int max_tokens() const { return stack_ ? cfg_.max_tokens : 0; }

 private:
  std::string not_built() const {
    return std::string("Generation failed: this gptoss build runs the MoE block only (attention, sampling and the "
                       "tokenizer are not part of it); use decode_step() for the MoE half of a decode step") +
           (stack_ ? "" : " [InferenceEngine] Not initialized");
  }
  void shutdown_impl() {
    if (stack_ != nullptr) {
      prof_unregister(this);
      api.stack_destroy(stack_);
      stack_ = nullptr;
    }
    bound_r_ = bound_d_ = 0;
    num_layers_ = 0;
  }

  gptoss_moe_stack* stack_ = nullptr;
  gptoss_moe_config cfg_{};
  int device_ = 0;
  int num_layers_ = 0;
  uintptr_t bound_r_ = 0, bound_d_ = 0;
};

// ModelConfig (include/config.h): the constants the reference exposes.
struct ModelConfig {
  static constexpr int num_layers = 36;
  static constexpr int hidden_size = 2880;
  static constexpr int num_q_heads = 64;
  static constexpr int num_kv_heads = 8;
  static constexpr int head_dim = 64;
  static constexpr int qkv_size = (num_q_heads + 2 * num_kv_heads) * head_dim;
  static constexpr int attn_out_size = num_q_heads * head_dim;
  static constexpr int num_experts = 128;
  static constexpr int num_active_experts = 4;
  static constexpr int expert_intermediate_size = 2880;
  static constexpr int vocab_size = 201088;
  static constexpr float rope_theta = 150000.0f;
  static constexpr int rope_max_pos = 131072;
  static constexpr int sliding_window_size = 128;
  static constexpr int full_attention_interval = 2;
  static constexpr int gqa_ratio = num_q_heads / num_kv_heads;
  static constexpr int kv_block_size = 16;
  static constexpr int world_size = 1;
  static constexpr int experts_per_gpu = num_experts / world_size;
  static constexpr float rms_norm_eps = 1e-5f;
  static constexpr float swiglu_limit = 7.0f;
  static constexpr float activation_alpha = 1.702f;
  static bool is_full_attention(int layer) { return layer % full_attention_interval == full_attention_interval - 1; }
  static int get_window_size(int layer) { return is_full_attention(layer) ? 0 : sliding_window_size; }
};

}  // namespace

PYBIND11_MODULE(gptoss, m) {
  m.doc() = "GPT-OSS MoE block on one MI355X (gfx950) -- the reference's gptoss module surface";
  try {  // torch first, so the library shares torch's HIP runtime
    py::module_::import("torch");
  } catch (const py::error_already_set&) {
  }
  {
    py::object here = py::module_::import("os").attr("path").attr("dirname")(m.attr("__file__"));
    load_library(py::str(here).cast<std::string>() + "/libgptoss_moe.so");
  }

  py::class_<PyInferenceEngine>(m, "InferenceEngine",
                                "GPT-OSS engine lifecycle over the MoE layers of a checkpoint on one GPU.\n\n"
                                "  engine = gptoss.InferenceEngine()\n"
                                "  engine.init('/weights/gpt-oss-120b')\n"
                                "  engine.decode_step(residual, deltas, num_tokens)\n"
                                "  engine.shutdown()")
      .def(py::init<>(), "Create an InferenceEngine instance (does not touch the GPU).")
      .def("init", &PyInferenceEngine::init, py::arg("weights_dir"), py::arg("max_tokens") = 64,
           py::arg("device") = 0, py::arg("top_k") = 4,
           "Load every MoE layer of the checkpoint into one layer stack.\n\n"
           "Raises:\n    RuntimeError: if the weights cannot be loaded.")
      .def("generate", &PyInferenceEngine::generate, py::arg("prompt_tokens"), py::arg("max_tokens") = 512,
           py::arg("temperature") = 0.8f, py::arg("top_p") = 0.95f,
           "Checks its arguments (ValueError), then raises RuntimeError: generation needs attention and sampling, "
           "which this build does not contain.")
      .def("generate_batch", &PyInferenceEngine::generate_batch, py::arg("prompts"), py::arg("max_tokens") = 512,
           py::arg("temperature") = 0.0f, py::arg("top_p") = 1.0f,
           "Checks its arguments (ValueError), then raises RuntimeError (see generate).")
      .def("decode_step", &PyInferenceEngine::decode_step, py::arg("residual"), py::arg("deltas"),
           py::arg("num_tokens"), py::arg("use_graph") = true, py::arg("stream") = py::none(),
           "The MoE half of one decode step over all layers, in place on residual[:num_tokens].")
      .def("shutdown", &PyInferenceEngine::shutdown, "Release the layers and their GPU memory.")
      .def_property_readonly("is_initialized", &PyInferenceEngine::is_initialized,
                             "True if the engine has been initialized.")
      .def_property_readonly("num_layers", &PyInferenceEngine::num_layers)
      .def_property_readonly("max_tokens", &PyInferenceEngine::max_tokens)
      .def("__repr__", [](const PyInferenceEngine& e) {
        return std::string("<gptoss.InferenceEngine initialized=") + (e.is_initialized() ? "True" : "False") + ">";
      });

  py::class_<PyMoELayer>(m, "MoELayer", "One MoE layer of a checkpoint (the moe_layer_* operator).")
      .def(py::init<const std::string&, int, int, int, int, int, bool>(), py::arg("weights_dir"), py::arg("layer"),
           py::arg("max_tokens") = 64, py::arg("device") = 0, py::arg("top_k") = 4,
           py::arg("prefill_min_tokens") = 128, py::arg("decode_exact") = false)
      .def("forward", &PyMoELayer::forward, py::arg("x"), py::arg("out") = py::none(), py::arg("stream") = py::none(),
           "out = x + MoE(RMSNorm(x))  (moe_layer_forward)")
      .def("forward_prenormed", &PyMoELayer::forward_prenormed, py::arg("normed"), py::arg("residual") = py::none(),
           py::arg("out") = py::none(), py::arg("stream") = py::none(),
           "out = residual + MoE(normed)  (moe_layer_forward_prenormed)")
      .def("forward_residual", &PyMoELayer::forward_residual, py::arg("residual"), py::arg("delta"),
           py::arg("residual_out") = py::none(), py::arg("out") = py::none(), py::arg("stream") = py::none(),
           "s = residual + delta; out = bf16(s) + MoE(RMSNorm(s))")
      .def("forward_routed", &PyMoELayer::forward_routed, py::arg("normed"), py::arg("expert_indices"),
           py::arg("expert_weights"), py::arg("residual") = py::none(), py::arg("out") = py::none(),
           py::arg("stream") = py::none(), "The expert half with the routing given.")
      .def("set_profiling", &PyMoELayer::set_profiling, py::arg("max_forwards"))
      .def("profile_read", &PyMoELayer::profile_read,
           "(route_ms, gate_up_ms, down_ms, combine_ms, forwards) summed over the recorded forwards")
      .def("close", &PyMoELayer::close)
      .def_property_readonly("hidden_size", [](const PyMoELayer& l) { return l.cfg().hidden_size; })
      .def_property_readonly("num_experts", [](const PyMoELayer& l) { return l.cfg().num_experts; })
      .def_property_readonly("top_k", [](const PyMoELayer& l) { return l.cfg().top_k; })
      .def_property_readonly("intermediate_size", [](const PyMoELayer& l) { return l.cfg().intermediate_size; })
      .def_property_readonly("max_tokens", [](const PyMoELayer& l) { return l.cfg().max_tokens; })
      .def_property_readonly("device", &PyMoELayer::device);

  py::class_<ModelConfig>(m, "ModelConfig", "Read-only model architecture constants for GPT-OSS-120B.")
      .def(py::init<>())
      .def_property_readonly_static("num_layers", [](py::object) { return ModelConfig::num_layers; })
      .def_property_readonly_static("hidden_size", [](py::object) { return ModelConfig::hidden_size; })
      .def_property_readonly_static("num_q_heads", [](py::object) { return ModelConfig::num_q_heads; })
      .def_property_readonly_static("num_kv_heads", [](py::object) { return ModelConfig::num_kv_heads; })
      .def_property_readonly_static("head_dim", [](py::object) { return ModelConfig::head_dim; })
      .def_property_readonly_static("qkv_size", [](py::object) { return ModelConfig::qkv_size; })
      .def_property_readonly_static("attn_out_size", [](py::object) { return ModelConfig::attn_out_size; })
      .def_property_readonly_static("num_experts", [](py::object) { return ModelConfig::num_experts; })
      .def_property_readonly_static("num_active_experts", [](py::object) { return ModelConfig::num_active_experts; })
      .def_property_readonly_static("expert_intermediate_size",
                                    [](py::object) { return ModelConfig::expert_intermediate_size; })
      .def_property_readonly_static("experts_per_gpu", [](py::object) { return ModelConfig::experts_per_gpu; })
      .def_property_readonly_static("vocab_size", [](py::object) { return ModelConfig::vocab_size; })
      .def_property_readonly_static("rope_theta", [](py::object) { return ModelConfig::rope_theta; })
      .def_property_readonly_static("rope_max_pos", [](py::object) { return ModelConfig::rope_max_pos; })
      .def_property_readonly_static("sliding_window_size", [](py::object) { return ModelConfig::sliding_window_size; })
      .def_property_readonly_static("full_attention_interval",
                                    [](py::object) { return ModelConfig::full_attention_interval; })
      .def_property_readonly_static("gqa_ratio", [](py::object) { return ModelConfig::gqa_ratio; })
      .def_property_readonly_static("kv_block_size", [](py::object) { return ModelConfig::kv_block_size; })
      .def_property_readonly_static("world_size", [](py::object) { return ModelConfig::world_size; })
      .def_property_readonly_static("rms_norm_eps", [](py::object) { return ModelConfig::rms_norm_eps; })
      .def_property_readonly_static("swiglu_limit", [](py::object) { return ModelConfig::swiglu_limit; })
      .def_property_readonly_static("activation_alpha", [](py::object) { return ModelConfig::activation_alpha; })
      .def_static("is_full_attention", &ModelConfig::is_full_attention, py::arg("layer"))
      .def_static("get_window_size", &ModelConfig::get_window_size, py::arg("layer"))
      .def("__repr__", [](const ModelConfig&) {
        return "<gptoss.ModelConfig layers=36 hidden=2880 q_heads=64 kv_heads=8 experts=128 active=4 vocab=201088>";
      });

  // Per-launch timing is always compiled in: the reference's profiler functions
  // (bindings.cpp:421-439) exist whenever profiler_enabled() returns True.
  m.def("profiler_enabled", []() { return true; }, "Returns True: per-launch timing is built in.");
  m.def("profiler_reset", &profiler_reset, py::arg("max_forwards") = 1024,
        "Clear all profiler records and time the MoE launches of the next max_forwards forwards of every layer "
        "(0 stops recording). Recording starts here; forwards replayed from a hipGraph are not timed.");
  m.def("profiler_save_trace", &profiler_save_trace, py::arg("path"),
        "Save the recorded MoE launches to Chrome Trace Format JSON.");
  m.def("profiler_save_summary", &profiler_save_summary, py::arg("path"),
        "Save aggregated launch timing (per category and name) to JSON.");
  m.attr("__version__") = "0.1.0";
  m.attr("MODEL_NAME") = "gpt-oss-120b";
  m.attr("ABI_VERSION") = GPTOSS_MOE_ABI_VERSION;
}
