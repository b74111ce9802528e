// moe_checkpoint.h -- internal interface between the checkpoint reader
// (moe_checkpoint.hip) and the layer object (moe_capi.hip).
#pragma once

#include "../../include/gptoss_moe.h"

namespace gxmoe {

// The tensors of one layer's MoE block, found and checked on the host:
// names resolved, shapes checked against cfg, bf16 tensors converted.
struct LayerSource;
int ckpt_resolve_layer(const gptoss_checkpoint* ck, const gptoss_moe_config& cfg, int layer, LayerSource** out);
void ckpt_free_source(LayerSource* src);

// Upload a resolved layer onto the current device.  On success *blob is one
// device allocation holding every weight (the caller owns it) and *wt
// points into it, experts in the tiled expert-major form.  Shape limits of
// the kernels are the caller's to check first.
int ckpt_upload_layer(const LayerSource* src, void** blob, gptoss_moe_weights* wt);

}  // namespace gxmoe
