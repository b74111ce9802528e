// gptoss_moe_compat.hpp -- the reference's C++ MoE operator interface
// (namespace gptoss, moe_layer.cu:1556-1615; declared by its callers at
// engine.cu:168-196 and transformer.cu:106-121), implemented on top of the
// C ABI of gptoss_moe.h by libgptoss_moe_compat.so.
//
// The signatures (and so the mangled symbol names) are the reference's, so
// its engine links against this library in place of moe_layer.cu.  As in the
// reference, failures abort the process after printing the library's error
// message (cuda_utils.h:17-35); there are no status codes at this level.
//
// Arguments the single-GPU path does not use are accepted and ignored:
// layer/gpu ids, the expert-parallel communicator, the BLAS handles, the
// second stream, the NCCL communicator and the 19 caller-owned scratch
// buffers.  In their place every layer of a device shares one forward
// workspace (gptoss_moe_layer_init_with_workspace), sized for
// moe_layer_max_tokens() tokens and freed with the device's last layer, so
// as in the reference a device's layers must run one after another (the
// engine runs them in order on one stream).
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

struct ncclComm;
typedef struct ncclComm* ncclComm_t;

namespace gptoss {

class MoELayer;
class EPComm;
struct CublasHandle;

// moe_layer.cu:585-589: one MXFP4 matrix of one expert, row-major packed
// nibbles [N][K/2] and e8m0 scales [N][K/32] in device memory.
struct MXFP4Weight {
  const uint8_t* packed;
  const uint8_t* scales;
  int num_elements;
};

MoELayer* moe_layer_create();
void moe_layer_destroy(MoELayer* l);

// moe_layer.cu:1585-1615.  expert_mlp1 / expert_mlp2 are host arrays of
// ModelConfig::experts_per_gpu (128) descriptors; gate_up rows interleave
// gate (even) and up (odd).  Tokens per forward: at most
// moe_layer_max_tokens() (default 8192, the engine's MAX_TOKENS, engine.cu:
// 860; the environment variable GPTOSS_MOE_MAX_TOKENS overrides it before
// the first init on a device).
void moe_layer_init(
    MoELayer* layer, int layer_id, int device_id, int gpu_id, EPComm* ep_comm,
    const CublasHandle* cublas_compute, const CublasHandle* cublas_comm, hipStream_t compute_stream,
    hipStream_t comm_stream, const __hip_bfloat16* moe_norm_weight, const __hip_bfloat16* router_weight,
    const __hip_bfloat16* router_bias, const __hip_bfloat16* gate_up_proj_bias,
    const __hip_bfloat16* down_proj_bias, MXFP4Weight* expert_mlp1, MXFP4Weight* expert_mlp2,
    __hip_bfloat16* norm_buf, __hip_bfloat16* router_logits_buf, int32_t* expert_indices_buf,
    float* expert_weights_buf, int32_t* tokens_per_expert, __hip_bfloat16* permuted_tokens,
    int32_t* expert_offsets, int32_t* gather_map, int32_t* per_peer_counts, int32_t* peer_recv_offsets,
    __hip_bfloat16* recv_buffer, __hip_bfloat16* dequant_mlp1_buf_0, __hip_bfloat16* dequant_mlp1_buf_1,
    __hip_bfloat16* dequant_mlp2_buf_0, __hip_bfloat16* dequant_mlp2_buf_1, __hip_bfloat16* gate_up_buf,
    __hip_bfloat16* swiglu_buf, __hip_bfloat16* expert_out_buf, __hip_bfloat16* moe_output_buf,
    ncclComm_t nccl_comm);

// moe_layer.cu:1561-1578 (forward: out = in + MoE(RMSNorm(in)); prenormed:
// out = residual + MoE(normed)).  Stream-ordered, no host synchronisation.
void moe_layer_forward(MoELayer* layer, const __hip_bfloat16* input, __hip_bfloat16* output, int num_tokens,
                       hipStream_t stream);
void moe_layer_forward_prenormed(MoELayer* layer, const __hip_bfloat16* normed_input,
                                 const __hip_bfloat16* residual_input, __hip_bfloat16* output, int num_tokens,
                                 hipStream_t stream);
const __hip_bfloat16* moe_layer_get_ffn_norm_weight(MoELayer* layer);

// Not in the reference: the token capacity a layer is initialised with.
int moe_layer_max_tokens();

}  // namespace gptoss
