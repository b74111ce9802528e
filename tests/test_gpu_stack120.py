"""GPU: BASELINE config 4 at its own shape -- the engine's decode-step MoE
sequence (transformer.cu:653-753: residual += delta, RMSNorm, MoE, per layer)
over a 36-layer GPT-OSS-120B stack resident on one GPU (36 x 128 experts,
~61 GB of MXFP4), batch 32, captured as one hipGraph.

Weights are generated on the GPU in the reference layout (uniform nibble
bytes, e8m0 scales 119..123, router ~N(0, 0.02)) and packed into the tiled
layout layer by layer; only the two spot-checked layers are copied to the
host for the oracle.  Checked:
  * the graph-replayed step is bit-identical to the eager step;
  * each layer's routing inside the step (indices and weights) equals a
    single-layer forward_residual on that layer's own input, run layer by
    layer, and the layer-by-layer result equals the step's;
  * layer 0 and the last layer, all 32 tokens, against the oracle: the
    residual add + RMSNorm bit-exact, the routing bit-exact, the layer output
    within the matrix-core tolerance (test_gpu_prefill.check_layer_out).
"""
import numpy as np
import pytest

import moe_data
from test_gpu_parity import dev, host, say
from test_gpu_prefill import check_layer_out

pytestmark = pytest.mark.gpu

NL, E, K, H, I, T = 36, 128, 4, 2880, 2880, 32
SPOT = (0, NL - 1)


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _layer_weights(gpu, torch, l, gen):
    """One layer: reference-layout MXFP4 drawn on the GPU, packed into the
    tiled layout; returns (tiled buffers, router w/b, norm, zero biases,
    reference-layout tensors)."""
    n1, s1 = gpu.tiled_size(2 * I, H)
    n2, s2 = gpu.tiled_size(H, I)
    p1 = torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device="cuda", generator=gen)
    c1 = torch.randint(119, 124, (E, 2 * I, H // 32), dtype=torch.uint8, device="cuda", generator=gen)
    p2 = torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device="cuda", generator=gen)
    c2 = torch.randint(119, 124, (E, H, I // 32), dtype=torch.uint8, device="cuda", generator=gen)
    tiled = [torch.empty(E * n, dtype=torch.uint8, device="cuda") for n in (n1, s1, n2, s2)]
    for e in range(E):
        gpu.pack_tiled(p1[e], c1[e], 2 * I, H, tiled[0][e * n1:(e + 1) * n1], tiled[1][e * s1:(e + 1) * s1])
        gpu.pack_tiled(p2[e], c2[e], H, I, tiled[2][e * n2:(e + 1) * n2], tiled[3][e * s2:(e + 1) * s2])
    rw = (torch.randn((E, H), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    rb = (torch.randn((E,), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    norm = (1.0 + 0.1 * torch.randn((H,), device="cuda", generator=gen)).to(torch.bfloat16)
    ref = (p1, c1, p2, c2) if l in SPOT else None
    return dict(tiled=tiled, rw=rw, rb=rb, norm=norm, b1=torch.zeros((E, 2 * I), dtype=torch.bfloat16, device="cuda"),
                b2=torch.zeros((E, H), dtype=torch.bfloat16, device="cuda"), ref=ref)


def _routing(gpu, torch, layer):
    tr = layer.trace()
    idx = gpu.copy_device_to_tensor(tr.expert_indices, T * K * 4, torch.int32).cpu().numpy().reshape(T, K)
    w = gpu.copy_device_to_tensor(tr.expert_weights, T * K * 4, torch.float32).cpu().numpy().reshape(T, K)
    return idx, w


def test_gptoss120b_36_layer_stack_b32(gpu, orc, torch_mod):
    torch = torch_mod
    gen = torch.Generator(device="cuda")
    gen.manual_seed(36032)
    say(f"building {NL} GPT-OSS-120B layers on the GPU (~61 GB)")
    lw, layers = [], []
    for l in range(NL):
        wl = _layer_weights(gpu, torch, l, gen)
        cfg = gpu.default_config(E, T)
        layers.append(gpu.MoELayer().init(cfg, 0, wl["rw"], wl["rb"], wl["b1"], wl["b2"], moe_norm_weight=wl["norm"],
                                          tiled=wl["tiled"]))
        lw.append(wl)
    torch.cuda.synchronize()
    say("layers ready; stack step")
    st = gpu.MoEStack.from_layers(layers)
    r0 = torch.randn((T, H), device="cuda", generator=gen).to(torch.bfloat16)
    deltas = torch.randn((NL, T, H), device="cuda", generator=gen).to(torch.bfloat16)

    def step(use_graph):
        st.residual[:T].copy_(r0)
        st.deltas[:, :T].copy_(deltas)
        return host(st.decode_step(T, use_graph=use_graph))

    eager = step(False)
    torch.cuda.synchronize()
    routes = [_routing(gpu, torch, L) for L in layers]
    for rep in range(3):  # capture, then replays with eager work between them
        assert np.array_equal(step(True), eager), rep
        torch.cuda.synchronize()
        say("graph replay", rep, "bit-identical to the eager step")

    # layer by layer: each layer's routing in the step is that of a
    # single-layer forward on its own input
    r = r0.clone()
    inputs = {}
    for l, L in enumerate(layers):
        if l in SPOT:
            inputs[l] = host(r)
        s = torch.empty_like(r)
        r = L.forward_residual(r, deltas[l], residual_out=s)
        idx, w = _routing(gpu, torch, L)
        assert np.array_equal(idx, routes[l][0]), l
        assert np.array_equal(w.view(np.uint32), routes[l][1].view(np.uint32)), l
    assert np.array_equal(host(r), eager)
    say("layer-by-layer forwards reproduce the step and its routing")

    for l in SPOT:
        p1, c1, p2, c2 = (t.cpu().numpy() for t in lw[l]["ref"])
        w = dict(router_w=host(lw[l]["rw"]), router_b=host(lw[l]["rb"]), w1_packed=p1, w1_scales=c1,
                 w1_bias=np.zeros((E, 2 * I), np.uint16), w2_packed=p2, w2_scales=c2,
                 w2_bias=np.zeros((E, H), np.uint16))
        res_l = inputs[l]
        d_l = host(deltas[l])
        normed, ssum = orc.residual_rmsnorm(res_l, d_l, host(lw[l]["norm"]))
        ref, tr = orc.moe_forward(w, normed, ssum, E, K, H, I, trace=True)
        assert np.array_equal(tr["idx"], routes[l][0]), l
        assert np.array_equal(tr["w"].view(np.uint32), routes[l][1].view(np.uint32)), l
        # the layer's own forward on its input from the layer-by-layer pass
        st.residual[:T].copy_(dev(res_l, torch))
        s = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        out = host(layers[l].forward_residual(st.residual[:T], deltas[l], residual_out=s))
        assert np.array_equal(host(s), ssum), l
        check_layer_out(out, ref, f"36-layer stack, layer {l}, {T} tokens")
    st.destroy()
    for L in layers:
        L.destroy()
