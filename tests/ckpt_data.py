"""Synthetic GPT-OSS safetensors checkpoints for the checkpoint-loading tests.

Tensors are written by the `safetensors` package itself (an independent
writer of the format), under the names of the Hugging Face GPT-OSS export
that the reference loader reads (src/memory/weight_loader.cu:818-895,
1083-1165): model.layers.<L>.mlp.router.{weight,bias},
post_attention_layernorm.weight and mlp.experts.{gate_up,down}_proj_{blocks,
scales,bias}, or the per-expert form mlp.experts.<e>.<name>.weight[_scale].
The layer dicts come from moe_data.make_layer (reference layout, bf16 as
uint16)."""
from __future__ import annotations

import os

import numpy as np
import torch
from safetensors.torch import save_file


def bf16_tensor(u16) -> torch.Tensor:
    return torch.from_numpy(np.array(u16, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def layer_tensors(layer: int, w: dict, E: int, H: int, I: int, fmt: str = "packed", norm_w=None,
                  router_name: str = "router", expert_names=("mlp1", "mlp2"), floats: dict | None = None) -> dict:
    """The tensors of one MoE layer.  floats: name suffix -> torch tensor that
    replaces the bf16 array for that tensor (to store F32 or F16)."""
    P = f"model.layers.{layer}."
    floats = floats or {}
    t = {}

    def put(suffix, u16):
        t[P + suffix] = floats.get(suffix, bf16_tensor(u16) if u16 is not None else None)

    put(f"mlp.{router_name}.weight", w["router_w"])
    if w.get("router_b") is not None:
        put(f"mlp.{router_name}.bias", w["router_b"])
    if norm_w is not None:
        put("post_attention_layernorm.weight", norm_w)
    if w.get("w1_bias") is not None:
        put("mlp.experts.gate_up_proj_bias", w["w1_bias"])
    if w.get("w2_bias") is not None:
        put("mlp.experts.down_proj_bias", w["w2_bias"])
    if fmt == "packed":
        t[P + "mlp.experts.gate_up_proj_blocks"] = torch.from_numpy(w["w1_packed"].reshape(E, 2 * I, H // 32, 16).copy())
        t[P + "mlp.experts.gate_up_proj_scales"] = torch.from_numpy(w["w1_scales"].copy())
        t[P + "mlp.experts.down_proj_blocks"] = torch.from_numpy(w["w2_packed"].reshape(E, H, I // 32, 16).copy())
        t[P + "mlp.experts.down_proj_scales"] = torch.from_numpy(w["w2_scales"].copy())
    else:
        n1, n2 = expert_names
        for e in range(E):
            b = P + f"mlp.experts.{e}."
            t[b + f"{n1}.weight"] = torch.from_numpy(w["w1_packed"][e].reshape(2 * I, H // 32, 16).copy())
            t[b + f"{n1}.weight_scale"] = torch.from_numpy(w["w1_scales"][e].copy())
            t[b + f"{n2}.weight"] = torch.from_numpy(w["w2_packed"][e].reshape(H, I // 32, 16).copy())
            t[b + f"{n2}.weight_scale"] = torch.from_numpy(w["w2_scales"][e].copy())
    return {k: v.contiguous() for k, v in t.items() if v is not None}


def write_shards(directory: str, tensors: dict, n_shards: int = 2, metadata: dict | None = None) -> list:
    """Split tensors over n_shards files (round robin by sorted name) named
    model-0000i-of-0000n.safetensors; returns the paths."""
    os.makedirs(directory, exist_ok=True)
    names = sorted(tensors)
    paths = []
    for i in range(n_shards):
        part = {n: tensors[n] for n in names[i::n_shards]}
        path = os.path.join(directory, f"model-{i + 1:05d}-of-{n_shards:05d}.safetensors")
        save_file(part, path, metadata=metadata or {"format": "pt"})
        paths.append(path)
    return paths
