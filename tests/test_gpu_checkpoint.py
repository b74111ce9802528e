"""GPU tests of gptoss_moe_layer_init_from_checkpoint: a layer loaded from a
safetensors checkpoint (written by the `safetensors` package under the GPT-OSS
names the reference loader reads, weight_loader.cu:818-895, 1083-1165) runs
bit-identically to a layer initialised from the same arrays through the
per-expert pointer tables, and, on the exact decode kernels, to the CPU
oracle.  Covers the packed and per-expert expert formats, the alternative
names, the staging pipeline with one and several experts per chunk, F32 and
F16 tensors rounded to bf16 (against torch's own rounding), and the full
GPT-OSS expert shape with the default staging size."""
import time

import numpy as np
import pytest

import ckpt_data
import moe_data
from test_gpu_parity import DeviceLayer, assert_bf16_parity, dev, host, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _load(gpu, path, E, k, H, I, layer, max_tokens, exact, staging=None):
    cfg = gpu.default_config(E, max_tokens, decode_exact=exact)
    cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, k
    with gpu.Checkpoint(path) as ck:
        if staging is not None:
            ck.set_staging_bytes(staging)
        t0 = time.perf_counter()
        L = gpu.MoELayer().init_from_checkpoint(cfg, 0, ck, layer)
        dt = time.perf_counter() - t0
    return L, dt


def _expert_bytes(N, K):
    a = lambda x: (x + 255) // 256 * 256  # noqa: E731
    return a(N * K // 2) + a(N * K // 32)


CASES = [
    # fmt, names, staging (None = default), n_shards
    ("packed", {}, None, 2),
    ("per_expert", {}, 1, 3),                                              # one expert per chunk
    ("per_expert", {"expert_names": ("gate_up_proj", "down_proj")}, 3 * _expert_bytes(256, 256), 1),
    ("packed", {"router_name": "gate"}, 3 * _expert_bytes(256, 256), 2),   # chunks of 3, 3, 2
]


@pytest.mark.parametrize("fmt,kw,staging,n_shards", CASES)
def test_checkpoint_layer_matches_tables_and_oracle(gpu, orc, torch_mod, tmp_path, fmt, kw, staging, n_shards):
    torch = torch_mod
    E, k, H, I, T = 8, 4, 256, 128, 16
    w0 = moe_data.make_layer(70, E, H, I, bias="random")
    w1 = moe_data.make_layer(71, E, H, I, bias="random")
    t = ckpt_data.layer_tensors(0, w0, E, H, I, fmt=fmt, **kw)
    t.update(ckpt_data.layer_tensors(1, w1, E, H, I, fmt=fmt, **kw))
    ckpt_data.write_shards(str(tmp_path), t, n_shards=n_shards)
    say("checkpoint layer", fmt, kw, staging)
    L, _ = _load(gpu, str(tmp_path), E, k, H, I, 1, T, exact=True, staging=staging)
    ref_layer = DeviceLayer(gpu, torch, w1, E, k, H, I, max_tokens=T)
    x, res = moe_data.make_tokens(72, T, H)
    out = host(L.forward_prenormed(dev(x, torch), dev(res, torch)))
    out_ref = host(ref_layer.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    torch.cuda.synchronize()
    assert np.array_equal(out, out_ref)
    assert_bf16_parity(out, orc.moe_forward(w1, x, res, E, k, H, I), f"checkpoint {fmt}")
    L.destroy()


def test_checkpoint_float_tensors_round_to_bf16(gpu, orc, torch_mod, tmp_path):
    """Router weight and norm stored as F32, expert biases as F16 (subnormals
    included): the loader rounds them to bf16 (nearest even) as torch does."""
    torch = torch_mod
    E, k, H, I, T = 8, 4, 128, 128, 8
    rng = np.random.default_rng(80)
    w = moe_data.make_layer(80, E, H, I, bias="random")
    rw = torch.from_numpy(rng.normal(0.0, 0.02, (E, H)).astype(np.float32))
    nw = torch.from_numpy(rng.normal(1.0, 0.1, H).astype(np.float32))
    b1 = rng.normal(0.0, 0.5, (E, 2 * I)).astype(np.float16)
    b1[0, :8] = np.array([6e-8, -6e-8, 3e-6, 1e-5, -2e-7, 0.0, -0.0, 65504], np.float16)  # subnormals, max
    b1 = torch.from_numpy(b1)
    floats = {"mlp.router.weight": rw, "post_attention_layernorm.weight": nw, "mlp.experts.gate_up_proj_bias": b1}
    t = ckpt_data.layer_tensors(0, w, E, H, I, norm_w=np.zeros(H, np.uint16), floats=floats)
    ckpt_data.write_shards(str(tmp_path), t, n_shards=1)
    to_u16 = lambda x: x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    w["router_w"], w["w1_bias"] = to_u16(rw), to_u16(b1)
    norm = to_u16(nw)
    L, _ = _load(gpu, str(tmp_path), E, k, H, I, 0, T, exact=True)
    ref_layer = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T, norm_w=norm)
    x, _ = moe_data.make_tokens(81, T, H)
    out = host(L.forward(dev(x, torch)))
    out_ref = host(ref_layer.layer.forward(dev(x, torch)))
    torch.cuda.synchronize()
    assert np.array_equal(out, out_ref)
    L.destroy()


def test_checkpoint_full_gptoss_shape(gpu, torch_mod, tmp_path):
    """E=16 experts of the GPT-OSS shape (H = I = 2880) with the default
    staging (several experts per chunk, both slots in turn): the matrix-core
    decode (T=4) and prefill (T=256) paths give the same bits as a layer
    built through the pointer tables."""
    torch = torch_mod
    E, k, H, I = 16, 4, 2880, 2880
    w = moe_data.make_layer(90, E, H, I, bias="random")
    t = ckpt_data.layer_tensors(3, w, E, H, I, norm_w=moe_data.bf16(np.ones(H)))
    ckpt_data.write_shards(str(tmp_path), t, n_shards=2)
    say("full-shape checkpoint written", E, H, I)
    L, dt = _load(gpu, str(tmp_path), E, k, H, I, 3, 256, exact=False)
    nbytes = sum(v.numel() * v.element_size() for v in t.values())
    say(f"init_from_checkpoint: {nbytes / 1e6:.1f} MB in {dt * 1e3:.1f} ms ({nbytes / dt / 1e9:.2f} GB/s, page cache warm)")
    ref_layer = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=256, exact=False)
    for T in (4, 256):
        x, res = moe_data.make_tokens(91 + T, T, H)
        out = host(L.forward_prenormed(dev(x, torch), dev(res, torch)))
        out_ref = host(ref_layer.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
        torch.cuda.synchronize()
        assert np.array_equal(out, out_ref), T
    L.destroy()


def test_checkpoint_layers_share_staging(gpu, torch_mod, tmp_path):
    """Several layers from one open checkpoint: the staging is kept between
    loads, and remade when the staging size changes; every layer matches its
    pointer-table twin."""
    torch = torch_mod
    E, k, H, I, T = 8, 4, 256, 128, 8
    ws = [moe_data.make_layer(100 + l, E, H, I, bias="random") for l in range(3)]
    t = {}
    for l, w in enumerate(ws):
        t.update(ckpt_data.layer_tensors(l, w, E, H, I))
    ckpt_data.write_shards(str(tmp_path), t, n_shards=2)
    cfg = gpu.default_config(E, T, decode_exact=True)
    cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, k
    x, res = moe_data.make_tokens(105, T, H)
    with gpu.Checkpoint(str(tmp_path)) as ck:
        for l, staging in ((0, None), (1, None), (2, 1), (0, 1)):
            if staging is not None:
                ck.set_staging_bytes(staging)
            L = gpu.MoELayer().init_from_checkpoint(cfg, 0, ck, l)
            ref = DeviceLayer(gpu, torch, ws[l], E, k, H, I, max_tokens=T)
            out = host(L.forward_prenormed(dev(x, torch), dev(res, torch)))
            out_ref = host(ref.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
            torch.cuda.synchronize()
            assert np.array_equal(out, out_ref), (l, staging)
            L.destroy()
