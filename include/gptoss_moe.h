/*
 * gptoss_moe.h -- C ABI of the MI355X (gfx950) GPT-OSS MoE block.
 *
 * Drop-in boundary for the MoE hot path of the reference engine
 * (Jayluci4/hip-kernels).  Every entry point takes plain pointers and sizes;
 * device pointers are HIP device memory of the current device, `stream` is
 * a hipStream_t (NULL = the null stream).  Every call returns a status code
 * (GPTOSS_OK = 0) and records a message readable with gptoss_last_error() on
 * the calling thread; nothing aborts the process (the reference aborts on
 * every HIP error, include/cuda_utils.h:17-35).
 *
 * Numerics: fp32 accumulation; bf16 rounding at the reference's points
 * (logits, gate_up, SwiGLU output, expert output, layer output); expert
 * indices chosen by (logit desc, index asc) as topk_softmax.cu:60-72.
 *
 * bf16 values are passed as uint16_t bit patterns.
 */
#ifndef GPTOSS_MOE_H
#define GPTOSS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPTOSS_MOE_ABI_VERSION 7

enum {
  GPTOSS_OK = 0,
  GPTOSS_ERR_INVALID = 1,      /* bad argument (shape, null pointer, k > 8, ...) */
  GPTOSS_ERR_UNSUPPORTED = 2,  /* valid but not supported by this build (shape limits) */
  GPTOSS_ERR_HIP = 3,          /* a HIP runtime call failed */
  GPTOSS_ERR_STATE = 4,        /* object not initialised / already initialised */
  GPTOSS_ERR_OOM = 5,          /* device allocation failed */
  GPTOSS_ERR_NOT_FOUND = 6,    /* checkpoint tensor or shard file not found */
  GPTOSS_ERR_IO = 7            /* checkpoint file unreadable or not valid safetensors */
};

/* Message of the last failing call on this thread ("" if none); UTF-8, with
 * any byte of a quoted name or path that is not well-formed UTF-8 as '?'. */
const char* gptoss_last_error(void);
int gptoss_abi_version(void);

/* MoE shape and constants.  Replaces the compile-time ModelConfig MoE fields
 * (include/config.h:20-23, 40-43, 53, 57): E and k are runtime values here, so
 * the 20B (E=32) and 120B (E=128) shapes run from one library. */
typedef struct gptoss_moe_config {
  int hidden_size;        /* H (2880) */
  int num_experts;        /* E (128 for 120B, 32 for 20B) */
  int top_k;              /* k (4); 1, 2, 4 or 8 */
  int intermediate_size;  /* I (2880); gate_up rows = 2I, interleaved gate/up */
  float swiglu_alpha;     /* 1.702 (config.h:43) */
  float swiglu_limit;     /* 7.0   (config.h:42) */
  float rms_norm_eps;     /* 1e-5  (config.h:39), used by forward() only */
  int logits_fp32;        /* 0: bf16 router logits (reference), 1: fp32 logits */
  int max_tokens;         /* largest T a forward call may pass (scratch sizing) */
  /* Forwards of at least this many tokens run the expert products as grouped
   * GEMMs on the matrix cores (fp32 accumulation in the matrix core's order:
   * within one bf16 rounding step of the canonical result, not bit-identical).
   * 0 = never.  Default 128. */
  int prefill_min_tokens;
  /* Smaller forwards (decode) stream the expert weights once per step.
   * 0 (default): on the matrix cores, fp32 accumulation in the matrix core's
   * order (like prefill).  1: through the exact VALU kernels, whose results
   * are bit-identical to the canonical order (one ascending fma chain per
   * K-part, parts added in order), at a lower streaming rate.  The
   * matrix-core decode kernels take at most 1024 slots (T * top_k); larger
   * forwards below prefill_min_tokens (only when it is 0 or above 256 at
   * top-4) run the exact kernels, about 14 ms for 1024 GPT-OSS-120B tokens
   * against 0.49 ms on the prefill path. */
  int decode_exact;
  /* Prefill expert products (T >= prefill_min_tokens).  0 (default): the
   * bf16 matrix core with the weights decoded in registers; fp32 accumulation.
   * 1: the block-scaled matrix core (v_mfma_scale_f32_16x16x128_f8f6f4): the
   * fp4 weights with their e8m0 scales as stored, times the activations split
   * into two e4m3 parts per 32-element block (hi + lo/32, exact for every
   * value above 2^-13 of its block's largest), two products each.  2: the
   * same with the hi part alone (each activation rounded to four significant
   * bits).  The block-scaled product sums inside each instruction at less
   * than fp32 precision, so 1 and 2 fall outside the north-star tolerance at
   * GPT-OSS-120B's K = 2880, and on gfx950 neither is faster than 0: they
   * are kept as measured alternatives, not as the default. */
  int prefill_block_scaled;
} gptoss_moe_config;

/* Fill `cfg` with the GPT-OSS constants for `num_experts` experts. */
int gptoss_moe_config_default(gptoss_moe_config* cfg, int num_experts, int max_tokens);

/* ---- MXFP4 weight layout (src/memory) ----------------------------------
 * Reference layout of one expert matrix [N rows, K inputs]
 * (weight_loader.cu:782-842, fused_mxfp4_gemv.cu:13-15): packed [N][K/2]
 * bytes, low nibble = even k; scales [N][K/32] e8m0 bytes.
 * The kernels read a tiled layout: per 64-row tile, K/32 blocks of one KiB
 * holding the 64 rows' 16-byte blocks as dwords ordered for the matrix
 * cores (slot 16g + r%16, dword r/16 = bytes 4g..4g+3 of row r); scales
 * twice, per (tile, K-part, row) and per (tile, block) in slot order. */
int gptoss_mxfp4_tiled_size(int N, int K, size_t* nibble_bytes, size_t* scale_bytes);
int gptoss_mxfp4_pack_tiled(const uint8_t* packed, const uint8_t* scales, int N, int K,
                            uint8_t* tiled_nibbles, uint8_t* tiled_scales, void* stream);

/* ---- Layer object: replaces gptoss::MoELayer and moe_layer_* -------------
 * (src/model/moe_layer.cu:1556-1615). */
typedef struct gptoss_moe_layer gptoss_moe_layer;

typedef struct gptoss_moe_weights {
  const uint16_t* moe_norm_weight;  /* [H] bf16, used by forward() (may be NULL otherwise) */
  const uint16_t* router_weight;    /* [E][H] bf16 (mlp.router.weight) */
  const uint16_t* router_bias;      /* [E] bf16 or NULL */
  const uint16_t* gate_up_bias;     /* [E][2I] bf16 or NULL */
  const uint16_t* down_bias;        /* [E][H] bf16 or NULL */
  /* Either: reference-layout experts, host arrays of E device pointers
   * (MXFP4Weight tables of moe_layer.cu:585-589); the layer packs them into
   * its own tiled copy at init. */
  const uint8_t* const* mlp1_packed;  /* [E] -> [2I][H/2] */
  const uint8_t* const* mlp1_scales;  /* [E] -> [2I][H/32] */
  const uint8_t* const* mlp2_packed;  /* [E] -> [H][I/2] */
  const uint8_t* const* mlp2_scales;  /* [E] -> [H][I/32] */
  /* Or: already tiled, expert-major contiguous buffers (borrowed, not copied):
   * E x gptoss_mxfp4_tiled_size(2I, H) and E x gptoss_mxfp4_tiled_size(H, I). */
  const uint8_t* mlp1_tiled_nibbles;
  const uint8_t* mlp1_tiled_scales;
  const uint8_t* mlp2_tiled_nibbles;
  const uint8_t* mlp2_tiled_scales;
} gptoss_moe_weights;

gptoss_moe_layer* gptoss_moe_layer_create(void);                    /* moe_layer_create */
/* moe_layer_init: the layer allocates its per-forward scratch for
 * cfg->max_tokens tokens (gptoss_moe_layer_workspace_bytes bytes). */
int gptoss_moe_layer_init(gptoss_moe_layer* layer, const gptoss_moe_config* cfg, int device_id,
                          const gptoss_moe_weights* weights);       /* moe_layer_init */
/* Bytes of per-forward scratch (routing plan, SwiGLU activations, expert
 * outputs, norm output) of a layer of this config, sized for
 * cfg->max_tokens; 0 for an invalid config. */
size_t gptoss_moe_layer_workspace_bytes(const gptoss_moe_config* cfg);
/* moe_layer_init with the per-forward scratch in a caller-owned device buffer
 * of device_id (at least gptoss_moe_layer_workspace_bytes(cfg) bytes,
 * 256-byte aligned), as the reference engine hands every layer the same
 * scratch buffers (engine.cu:975-1000, moe_layer.cu:1585-1600).  Layers whose
 * forwards are ordered on one stream may share one workspace, whatever their
 * configs (each needs the bytes of its own); forwards that can overlap in time
 * need separate workspaces.  The first 1152 bytes hold a work queue that must
 * read zero whenever no forward is running: init zeroes it (after waiting for
 * all work already queued on the device, so a forward in flight on another
 * stream is not disturbed) and every forward leaves it zero, so nothing else
 * may write there; a forward enqueued on it by another host thread while an
 * init runs races with that zeroing.  The workspace must
 * outlive the layer; a trace (gptoss_moe_layer_trace) then shows the last
 * forward of any layer on it. */
int gptoss_moe_layer_init_with_workspace(gptoss_moe_layer* layer, const gptoss_moe_config* cfg, int device_id,
                                         const gptoss_moe_weights* weights, void* workspace,
                                         size_t workspace_bytes);
/* out = input + MoE(RMSNorm(input))  (moe_layer_forward, moe_layer.cu:982-1005) */
int gptoss_moe_layer_forward(gptoss_moe_layer* layer, const uint16_t* input, uint16_t* output,
                             int num_tokens, void* stream);
/* The decode step's residual add + RMSNorm and the MoE in one call: it
 * replaces fused_residual_rmsnorm_forward(residual, delta, moe_norm_weight,
 * normed, sum) followed by moe_layer_forward_prenormed(normed, sum, out)
 * (transformer.cu:696-715, rmsnorm.cu:224-337).  sum = residual + delta is
 * formed in fp32; residual_out (may be NULL) receives bf16(sum); out =
 * bf16(sum) + MoE(RMSNorm(sum)).  Up to 4 tokens the norm runs inside the
 * router's launch (one launch fewer), above in a launch of its own.  Needs
 * moe_norm_weight.  residual_out must not overlap residual or delta (the
 * reference double-buffers the residual stream, transformer.cu:697-701;
 * GPTOSS_ERR_INVALID otherwise); out may equal residual, residual_out or
 * neither, but must not partially overlap residual_out. */
int gptoss_moe_layer_forward_residual(gptoss_moe_layer* layer, const uint16_t* residual,
                                      const uint16_t* delta, uint16_t* residual_out, uint16_t* output,
                                      int num_tokens, void* stream);
/* out = residual + MoE(normed)  (moe_layer_forward_prenormed, moe_layer.cu:960-980);
 * residual may be NULL (out = MoE(normed)). */
int gptoss_moe_layer_forward_prenormed(gptoss_moe_layer* layer, const uint16_t* normed,
                                       const uint16_t* residual, uint16_t* output,
                                       int num_tokens, void* stream);
/* The layer's expert half with the routing given: out = residual +
 * sum_k w[t,k] * FFN_{idx[t,k]}(normed[t]).  This is forward_core's
 * permute / experts / combine (moe_layer.cu:1196-1549) entered after its
 * single-GPU top-k (moe_layer.cu:1188), for callers that route elsewhere (or inject a routing, as prefill
 * benchmarks with skewed expert popularity do).  Indices must lie in
 * [0, num_experts) and be distinct per token; weights are used as given. */
int gptoss_moe_layer_forward_routed(gptoss_moe_layer* layer, const uint16_t* normed,
                                    const uint16_t* residual, const int32_t* expert_indices,
                                    const float* expert_weights, uint16_t* output, int num_tokens,
                                    void* stream);
/* forward_prenormed with no allocation and no use of the layer's own scratch:
 * no counterpart in the reference.  For callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the forward scratch is a static device array of 8 MiB
 * that the library holds on every GPU it runs on until the process ends, so
 * num_tokens is limited to 64 and to configs whose scratch fits (the
 * GPT-OSS-120B layer at 64 tokens takes about 3.7 MiB); larger calls return
 * GPTOSS_ERR_INVALID.  The layer's max_tokens does not bound it.  Calls on one
 * GPU share that array: calls that overlap in time on one GPU (other streams,
 * other threads) race, and the layer's trace does not show these calls.
 * Results are those of gptoss_moe_layer_forward_prenormed. */
int gptoss_moe_layer_forward_prenormed_noalloc(gptoss_moe_layer* layer, const uint16_t* normed,
                                               const uint16_t* residual, uint16_t* output, int num_tokens,
                                               void* stream);
const uint16_t* gptoss_moe_layer_get_ffn_norm_weight(const gptoss_moe_layer* layer);
/* The config and device the layer was initialised with. */
int gptoss_moe_layer_get_config(const gptoss_moe_layer* layer, gptoss_moe_config* cfg, int* device_id);
void gptoss_moe_layer_destroy(gptoss_moe_layer* layer);           /* moe_layer_destroy */

/* ---- Checkpoints (src/memory/weight_loader.cu) ---------------------------
 * A safetensors checkpoint: every `*.safetensors` file of a directory in
 * name order (weight_loader.cu:456-482), or one file, mapped read-only
 * (:488-537).  The index maps names to tensors; a name present in several
 * shards resolves to the last shard in name order (:546-555). */
typedef struct gptoss_checkpoint gptoss_checkpoint;

typedef struct gptoss_tensor_info {
  const char* name;   /* valid while the checkpoint is open */
  const char* dtype;  /* as in the header: "BF16", "F32", "U8", ... */
  int ndim;           /* at most 8 */
  int64_t shape[8];
  uint64_t nbytes;    /* data_offsets end - begin */
  const void* data;   /* host address inside the read-only mapping */
  int shard;          /* shard index in name order */
} gptoss_tensor_info;

/* WeightLoader::init's shard scan, mmap and header parse
 * (weight_loader.cu:297-345, 456-540).  Malformed files return
 * GPTOSS_ERR_IO instead of aborting. */
int gptoss_checkpoint_open(const char* path, gptoss_checkpoint** out);
void gptoss_checkpoint_close(gptoss_checkpoint* ckpt);              /* WeightLoader::destroy */
int gptoss_checkpoint_num_tensors(const gptoss_checkpoint* ckpt);
int gptoss_checkpoint_tensor_at(const gptoss_checkpoint* ckpt, int i, gptoss_tensor_info* info);
/* has_tensor / get_tensor_data (weight_loader.cu:556-575): GPTOSS_ERR_NOT_FOUND
 * when absent. */
int gptoss_checkpoint_find(const gptoss_checkpoint* ckpt, const char* name, gptoss_tensor_info* info);
/* Size of each of the two pinned host and two device staging slots that
 * gptoss_moe_layer_init_from_checkpoint streams experts through (default
 * 32 MiB; a slot always holds at least one expert matrix).  The checkpoint
 * keeps the staging of each device it has loaded a layer onto until it is
 * closed, so the layers of a model reuse one pinned allocation. */
int gptoss_checkpoint_set_staging_bytes(gptoss_checkpoint* ckpt, size_t bytes);

/* One MoE layer from a checkpoint: WeightLoader::load_layer_weights' MoE part
 * (weight_loader.cu:1083-1165) with load_packed_experts (:818-842) or
 * load_per_expert_weights (:847-895), then moe_layer_init.  Names under
 * "model.layers.<layer_index>.": mlp.gate|router.{weight,bias},
 * post_attention_layernorm.weight, mlp.experts.{gate_up,down}_proj_{blocks,
 * scales,bias} or mlp.experts.<e>.{mlp1|gate_up_proj|w1, mlp2|down_proj|w2}
 * .weight[_scale].  bf16 tensors stored as F32 or F16 are rounded to bf16
 * (nearest even).  The layer owns one device allocation holding every
 * weight, the experts already tiled; names, shapes and dtypes are checked
 * against cfg before any device work.  Loads from one checkpoint run one at
 * a time (they share its staging). */
int gptoss_moe_layer_init_from_checkpoint(gptoss_moe_layer* layer, const gptoss_moe_config* cfg,
                                          int device_id, const gptoss_checkpoint* ckpt, int layer_index);

/* ---- Layer stack: the MoE half of the engine's decode step ----------------
 * The engine's decode step (transformer.cu:653-753) runs, per layer,
 * attention (a delta), fused_residual_rmsnorm_forward and
 * moe_layer_forward_prenormed, and is never graph-captured because the
 * reference MoE synchronises the host (engine.cu:309-320).  A stack runs the
 * same per-layer sequence over its layers, in place on a residual buffer it
 * owns:
 *     hook(layer, residual, delta[layer])            (optional: attention)
 *     residual = bf16(residual + delta[layer]) + MoE_layer(RMSNorm(...))
 * and, since nothing in it synchronises the host, can capture the whole step
 * in one hipGraph per token count, kept and replayed by later steps. */
typedef struct gptoss_moe_stack gptoss_moe_stack;

/* Writes layer `layer`'s delta [T][H] from the current residual [T][H] with
 * launches on `stream` (the engine's attention).  With graph replay the hook
 * runs once, while its step is captured: its launches are replayed as
 * captured, so they must not synchronise the host or change pointers. */
typedef void (*gptoss_layer_hook)(void* user, int layer, const uint16_t* residual, uint16_t* delta,
                                  int num_tokens, void* stream);

/* num_layers layers from first_layer on, each loaded as
 * gptoss_moe_layer_init_from_checkpoint does (needs
 * post_attention_layernorm.weight). */
int gptoss_moe_stack_create(const gptoss_moe_config* cfg, int device_id, const gptoss_checkpoint* ckpt,
                            int first_layer, int num_layers, gptoss_moe_stack** out);
/* Over initialised layers (borrowed; one device, one shape, each with
 * moe_norm_weight). */
int gptoss_moe_stack_create_from_layers(gptoss_moe_layer* const* layers, int num_layers,
                                        gptoss_moe_stack** out);
/* The stack's device buffers: residual [max_tokens][H] and deltas
 * [num_layers][max_tokens][H], bf16.  Any output may be NULL. */
int gptoss_moe_stack_io(gptoss_moe_stack* stack, uint16_t** residual, uint16_t** deltas, int* max_tokens,
                        int* num_layers);
/* Step on caller-owned buffers of the same shapes instead (NULL: back to the
 * stack's own); waits for the device, then drops the captured graphs, which
 * hold the old pointers. */
int gptoss_moe_stack_bind(gptoss_moe_stack* stack, uint16_t* residual, uint16_t* deltas);
int gptoss_moe_stack_layer(gptoss_moe_stack* stack, int index, gptoss_moe_layer** layer);
/* One step over every layer, ordered on `stream`.  use_graph = 1: replay
 * the step's graph for num_tokens (captured on first use, and again when
 * hook or user change). */
int gptoss_moe_stack_decode_step(gptoss_moe_stack* stack, int num_tokens, gptoss_layer_hook hook, void* user,
                                 int use_graph, void* stream);
void gptoss_moe_stack_destroy(gptoss_moe_stack* stack);

/* Device views of the layer's scratch after the last forward on `stream`
 * (valid until the next forward): routing and per-slot intermediates in the
 * permuted (expert-sorted) order.  Any output pointer may be NULL. */
typedef struct gptoss_moe_trace {
  const void* logits;         /* [T][E] bf16 or fp32 (cfg.logits_fp32) */
  const int32_t* expert_indices;  /* [T][k] */
  const float* expert_weights;    /* [T][k] */
  const int32_t* expert_counts;   /* [E] */
  const int32_t* expert_offsets;  /* [E+1] */
  const int32_t* gather_map;      /* [T*k] slot -> permuted row, -1 if dropped */
  const int32_t* perm_token;      /* [T*k] permuted row -> token */
  const int32_t* active_experts;  /* [E] ascending, first n_active valid */
  const int32_t* n_active;        /* [1] */
  const uint16_t* gate_up;        /* [T*k][2I] bf16 (only if trace_gate_up was enabled) */
  const uint16_t* act;            /* [T*k][I] bf16 SwiGLU output */
  const uint16_t* expert_out;     /* [T*k][H] bf16 */
} gptoss_moe_trace;
int gptoss_moe_layer_trace(const gptoss_moe_layer* layer, gptoss_moe_trace* trace);
/* Also write the bf16 gate_up intermediate on the next forwards (debug). */
int gptoss_moe_layer_set_trace_gate_up(gptoss_moe_layer* layer, int enable);

/* Per-launch timing, the role of the reference's PROF regions
 * (include/profiler.h:20-30, src/engine/profiler.cu:106-360): with
 * max_forwards > 0 the next max_forwards forwards time their route (or plan,
 * for forward_routed), gate_up (W1), down (W2) and combine launches with HIP
 * events stamped by each dispatch itself (hipExtLaunchKernelGGL: the
 * kernel's execution alone).  Forwards captured into a hipGraph are not
 * timed and use no slot.  profile_read waits for the events and returns the
 * summed milliseconds per launch and the count of recorded forwards (any
 * output pointer may be NULL).  Calling set_profiling again re-arms;
 * max_forwards = 0 turns recording off. */
int gptoss_moe_layer_set_profiling(gptoss_moe_layer* layer, int max_forwards);
int gptoss_moe_layer_profile_read(gptoss_moe_layer* layer, float* route_ms, float* w1_ms,
                                  float* w2_ms, float* combine_ms, int* n_forwards);
/* One recorded forward, for per-launch traces and summaries (the records
 * behind the reference's profiler_save_chrome_trace / _summary_json,
 * src/engine/profiler.cu:215-360): host_us is the host steady-clock time
 * (microseconds) at which the forward was enqueued; launch i (0 route, or the
 * plan for forward_routed; 1 gate_up; 2 down; 3 combine) started start_ms[i]
 * after launch 0 and ran dur_ms[i]. */
typedef struct gptoss_moe_prof_record {
  double host_us;
  int num_tokens;
  int prefill;       /* 1: the grouped prefill kernels ran (num_tokens >= prefill_min_tokens) */
  float start_ms[4];
  float dur_ms[4];
} gptoss_moe_prof_record;
/* Waits for the events of the first min(capacity, recorded) forwards since the
 * last set_profiling and writes their records; *n_records (may be NULL) gets
 * the number recorded. */
int gptoss_moe_layer_profile_records(gptoss_moe_layer* layer, gptoss_moe_prof_record* records,
                                     int capacity, int* n_records);

/* ---- Stage entry points (the reference's kernel launchers) --------------- */

/* Router + top-k softmax: replaces gemv_bf16_forward (T == 1,
 * gemv_bf16.cu:236-247) / gemm_bf16_lt (T > 1, cuda_utils.h:226-308) plus
 * topk_softmax_forward (topk_softmax.cu:380).  logits: [T][E] bf16 if
 * logits_fp32 == 0 else fp32 (the router output, rounded as the reference's
 * bf16 logits or kept in fp32).  `scratch` is reserved: it must be non-NULL
 * (gptoss_moe_route_scratch_bytes bytes of device memory, 256 today) and is
 * neither read nor written; routing exchanges no values between
 * work-groups, so no workspace is needed.
 * Up to 64 tokens every logit follows the reference's gemv_bf16 tree (its
 * T = 1 path, gemv_bf16.cu:57-129), bit-exact against the oracle.  Above 64
 * (when hidden % 32 == 0) the logits come from the matrix cores: fp32 sums of
 * exact bf16 products, four chains per logit (32-element blocks j, j + 4, ...
 * in block order), added pairwise, then the bias, as the reference's
 * hipBLASLt path for T > 1 sums in its own order; within the fp32 error bound
 * of the exact sum, deterministic, and independent of the other tokens in the
 * call.  router_b may be NULL (zero bias).  Logits need no alignment beyond
 * their element size. */
size_t gptoss_moe_route_scratch_bytes(int num_tokens, int num_experts, int top_k);
int gptoss_moe_route(const uint16_t* x, const uint16_t* router_w, const uint16_t* router_b,
                     int num_tokens, int num_experts, int hidden, int top_k, int logits_fp32,
                     void* logits, int32_t* expert_indices, float* expert_weights,
                     void* scratch, void* stream);

/* topk_softmax_forward (topk_softmax.cu:380-432) on given logits; bf16 logits
 * unless logits_fp32.  tokens_per_expert may be NULL (atomic histogram). */
int gptoss_topk_softmax_forward(const void* logits, int logits_fp32, int32_t* expert_indices,
                                float* expert_weights, int32_t* tokens_per_expert,
                                int num_tokens, int num_experts, int top_k, void* stream);

/* moe_permute_classify + moe_compute_gather_map_cpu (moe_permute.cu:129-236)
 * on the device: per-expert counts, offsets[E+1], stable gather map,
 * permuted token list, active expert list and its length. */
int gptoss_moe_permute_plan(const int32_t* expert_indices, int num_tokens, int top_k,
                            int num_experts, int32_t* counts, int32_t* offsets,
                            int32_t* gather_map, int32_t* perm_token, int32_t* active_experts,
                            int32_t* n_active, void* stream);

/* moe_scatter_tokens (moe_permute.cu:241-259): permuted[gather_map[s]] = x[s/k]. */
int gptoss_moe_scatter_tokens(const uint16_t* x, const int32_t* gather_map, uint16_t* permuted,
                              int num_tokens, int hidden, int top_k, void* stream);

/* fused_mxfp4_gemv_forward (fused_mxfp4_gemv.cu:452-464) generalised to M rows:
 * y[m][n] = bf16(sum_k x[m][k] * W[n][k] + bias[n]) with W in the tiled layout. */
int gptoss_mxfp4_gemv_forward(const uint16_t* x, int M, const uint8_t* tiled_nibbles,
                              const uint8_t* tiled_scales, const uint16_t* bias, uint16_t* y,
                              int N, int K, void* stream);

/* fused_residual_rmsnorm_forward (rmsnorm.cu:224-337): s = residual + delta
 * (fp32), sum_out = bf16(s) (may be NULL), normed = bf16((s * inv) * weight)
 * with inv = 1/sqrt(mean(s^2) + eps); the sum of squares follows the
 * router's gemv_bf16 tree and sqrt / divide are IEEE (the reference uses
 * rsqrtf). */
int gptoss_fused_residual_rmsnorm_forward(const uint16_t* residual, const uint16_t* delta,
                                          const uint16_t* weight, uint16_t* normed, uint16_t* sum_out,
                                          int num_tokens, int hidden, float eps, void* stream);

/* swiglu_forward (swiglu.cu:178-211): interleaved [T][2I] -> [T][I]. */
int gptoss_swiglu_forward(const uint16_t* gate_up, uint16_t* out, int num_tokens,
                          int intermediate, float alpha, float limit, void* stream);

/* moe_combine_forward (moe_combine.cu:175-204), single GPU (no remote rows):
 * out[t] = bf16(sum_k w[t,k] * expert_out[gather_map[t,k]] + residual[t]). */
int gptoss_moe_combine_forward(uint16_t* out, const uint16_t* expert_out,
                               const int32_t* gather_map, const float* expert_weights,
                               const uint16_t* residual, int num_tokens, int hidden,
                               int top_k, void* stream);

/* The prefill expert products: per active expert, mxfp4_dequant_batched
 * (mxfp4_dequant.cu:353-375) + CublasHandle::gemm_bf16_lt (cuda_utils.h:
 * 226-308) + bias_add_rows (moe_layer.cu:171-194) [+ swiglu_forward] as issued
 * by moe_layer.cu:1389-1487, in one grouped launch on the matrix cores:
 *   y[p][n] = bf16(sum_k x[row(p)][k] * W_e[n][k] + bias[e][n])
 * for every expert e and permuted row p in [offsets[e], offsets[e+1]), with
 * row(p) = row_index[p] (a gather from token rows, e.g. the plan's
 * perm_token) or p when row_index is NULL.  W_e is expert e of an
 * expert-major tiled array (E x gptoss_mxfp4_tiled_size(N, K)).
 * swiglu == 0: out[p][n] = y[p][n] ([rows][N]).  swiglu != 0: out[p][i] =
 * bf16(SwiGLU(y[p][2i], y[p][2i+1])) ([rows][N/2], interleaved gate/up rows),
 * and gate_up (may be NULL) receives y.  offsets (device, [E+1]) must be
 * nondecreasing from 0 with offsets[E] <= rows.  fp32 accumulation in the
 * matrix core's order (see prefill_min_tokens). */
int gptoss_moe_grouped_mxfp4_gemm(const uint16_t* x, const int32_t* row_index,
                                  const int32_t* expert_offsets, int num_experts, int rows,
                                  const uint8_t* tiled_nibbles, const uint8_t* tiled_scales,
                                  const uint16_t* bias, int N, int K, int swiglu, float alpha,
                                  float limit, uint16_t* out, uint16_t* gate_up, void* stream);

/* mxfp4_dequant_batched (mxfp4_dequant.cu:353-375) for one tiled matrix:
 * out[n][k] = bf16(e2m1 * 2^(scale-127)), row-major [N][K]. */
int gptoss_mxfp4_dequant(const uint8_t* tiled_nibbles, const uint8_t* tiled_scales, int N, int K,
                         uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* GPTOSS_MOE_H */
