"""GPU tests of the layer stack (gptoss_moe_stack_*): the MoE half of the
engine's decode step (transformer.cu:653-753) over several layers, eager and
as a captured hipGraph, against the CPU oracle's per-layer sequence
residual_rmsnorm -> moe_forward, bit for bit on the exact decode kernels.
Graph replays read the buffers' current contents, so each replay gets new
inputs and is checked against a fresh oracle run, with eager work between
replays.  A hook (the engine's attention) that derives each layer's delta
from the current residual is captured into the graph and replayed."""
import ctypes

import numpy as np
import pytest

import ckpt_data
import moe_data
from test_gpu_parity import DeviceLayer, dev, host, say

pytestmark = pytest.mark.gpu

E, K, H, I, NL = 8, 4, 256, 128, 3


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """NL layers with random norms, written as one checkpoint."""
    ws = [moe_data.make_layer(200 + l, E, H, I, bias="random") for l in range(NL)]
    norms = [moe_data.bf16(np.random.default_rng(210 + l).normal(1.0, 0.1, H)) for l in range(NL)]
    t = {}
    for l in range(NL):
        t.update(ckpt_data.layer_tensors(l, ws[l], E, H, I, norm_w=norms[l]))
    d = tmp_path_factory.mktemp("stack_ckpt")
    ckpt_data.write_shards(str(d), t, n_shards=2)
    return dict(path=str(d), ws=ws, norms=norms)


def _oracle_step(orc, model, res, deltas):
    for l in range(NL):
        normed, s = orc.residual_rmsnorm(res, deltas[l], model["norms"][l])
        res = orc.moe_forward(model["ws"][l], normed, s, E, K, H, I)
    return res


def _stack(gpu, model, max_tokens=16, exact=True):
    cfg = gpu.default_config(E, max_tokens, decode_exact=exact)
    cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, K
    with gpu.Checkpoint(model["path"]) as ck:
        return gpu.MoEStack.from_checkpoint(cfg, 0, ck)


def _inputs(seed, T):
    res, _ = moe_data.make_tokens(seed, T, H)
    deltas = [moe_data.make_tokens(seed * 10 + l, T, H)[1] for l in range(NL)]
    return res, deltas


@pytest.mark.parametrize("T", [2, 5])
def test_stack_eager_and_graph_match_oracle(gpu, orc, torch_mod, model, T):
    """T=2: the norm inside the router's launch; T=5: its own launch."""
    torch = torch_mod
    st = _stack(gpu, model)
    assert st.num_layers == NL and st.max_tokens == 16
    for i, use_graph in enumerate([False, True, True, False, True]):
        res, deltas = _inputs(300 + 7 * i + T, T)
        st.residual[:T].copy_(dev(res, torch))
        for l in range(NL):
            st.deltas[l, :T].copy_(dev(deltas[l], torch))
        say("stack step", T, "graph" if use_graph else "eager", i)
        got = host(st.decode_step(T, use_graph=use_graph))
        torch.cuda.synchronize()
        assert np.array_equal(got, _oracle_step(orc, model, res, deltas)), (T, i, use_graph)
    st.destroy()


def test_stack_hook_is_captured(gpu, orc, torch_mod, model):
    """delta_l = RMSNorm(residual; w_l) written by a hook through the library's
    standalone residual-RMSNorm launcher on the stream it is given: the graph
    replays the hook's launch with the residual of that moment."""
    torch = torch_mod
    T = 3
    st = _stack(gpu, model)
    hw = [moe_data.bf16(np.random.default_rng(400 + l).normal(0.0, 0.3, H)) for l in range(NL)]
    hw_dev = [dev(w, torch) for w in hw]
    zeros = torch.zeros((st.max_tokens, H), dtype=torch.bfloat16, device="cuda")
    calls = []

    def hook(layer, residual, delta, n, stream):
        calls.append(layer)
        rc = gpu.lib.gptoss_fused_residual_rmsnorm_forward(residual, zeros.data_ptr(), hw_dev[layer].data_ptr(),
                                                           delta, None, n, H, ctypes.c_float(1e-5), stream)
        assert rc == 0

    def oracle(res):
        for l in range(NL):
            d, _ = orc.residual_rmsnorm(res, np.zeros_like(res), hw[l])
            normed, s = orc.residual_rmsnorm(res, d, model["norms"][l])
            res = orc.moe_forward(model["ws"][l], normed, s, E, K, H, I)
        return res

    for i, use_graph in enumerate([False, True, True, True]):
        res, _ = _inputs(500 + i, T)
        st.residual[:T].copy_(dev(res, torch))
        got = host(st.decode_step(T, hook=hook, use_graph=use_graph))
        torch.cuda.synchronize()
        assert np.array_equal(got, oracle(res)), (i, use_graph)
    # eager: 3 calls; the first graph step captures (3 more); replays call nothing
    assert calls == list(range(NL)) * 2
    st.destroy()


def test_stack_from_layers_bind_and_engine(gpu, orc, torch_mod, model):
    torch = torch_mod
    T = 4
    layers = [DeviceLayer(gpu, torch, model["ws"][l], E, K, H, I, max_tokens=8, norm_w=model["norms"][l])
              for l in range(NL)]
    st = gpu.MoEStack.from_layers([L.layer for L in layers])
    assert st.max_tokens == 8
    res, deltas = _inputs(600, T)
    ref = _oracle_step(orc, model, res, deltas)
    st.residual[:T].copy_(dev(res, torch))
    for l in range(NL):
        st.deltas[l, :T].copy_(dev(deltas[l], torch))
    assert np.array_equal(host(st.decode_step(T)), ref)
    # a token count above max_tokens is rejected
    with pytest.raises(ValueError):
        st.decode_step(9)
    # trace of a stack layer: its last forward's routing
    idx = gpu.copy_device_to_tensor(st.layer(NL - 1).trace().expert_indices, T * K * 4, torch.int32).cpu().numpy()
    assert idx.shape == (T * K,) and idx.min() >= 0 and idx.max() < E
    st.destroy()
    # a layer without a norm weight cannot join a stack
    bare = DeviceLayer(gpu, torch, model["ws"][0], E, K, H, I, max_tokens=8)
    with pytest.raises(ValueError):
        gpu.MoEStack.from_layers([bare.layer])

    # the engine surface: shapes from the checkpoint, same numbers
    eng = gpu.MoEEngine()
    assert not eng.is_initialized
    eng.init(model["path"], max_tokens=8)
    assert eng.is_initialized and "layers=3" in repr(eng)
    out = eng.decode_step(dev(res, torch), deltas=torch.stack([dev(d, torch) for d in deltas]))
    torch.cuda.synchronize()
    # the engine's layers run the default matrix-core decode: within tolerance of the oracle
    c = moe_data.compare_bf16(host(out), ref)
    assert c["max_abs"] <= 2e-2 and c["mean_rel"] <= 1e-3, c
    eng.shutdown()
    assert not eng.is_initialized


def test_stack_graph_prefill_path(gpu, torch_mod, model):
    """A step above prefill_min_tokens runs the grouped matrix-core kernels
    (persistent, with a tile queue reset by its last work-group): graph
    replays equal eager steps."""
    torch = torch_mod
    T = 160
    st = _stack(gpu, model, max_tokens=T, exact=False)
    for i in range(3):
        res, deltas = _inputs(700 + i, T)
        outs = []
        for use_graph in (False, True):
            st.residual[:T].copy_(dev(res, torch))
            for l in range(NL):
                st.deltas[l, :T].copy_(dev(deltas[l], torch))
            outs.append(host(st.decode_step(T, use_graph=use_graph)))
            torch.cuda.synchronize()
        assert np.array_equal(outs[0], outs[1]), i
    st.destroy()


def test_engine_one_token_graph(gpu, orc, torch_mod, model):
    """A one-token engine step on matrix-core layers (norm inside the
    router's launch, routing inside gate_up) replayed from its graph: bit
    for bit the eager step, and within the tolerance of the oracle."""
    torch = torch_mod
    eng = gpu.MoEEngine().init(model["path"], max_tokens=4)
    res, deltas = _inputs(1200, 1)
    dr = dev(res, torch)
    dd = torch.stack([dev(d, torch) for d in deltas])
    eager = host(eng.decode_step(dr, deltas=dd, use_graph=False))
    for rep in range(3):
        got = host(eng.decode_step(dr, deltas=dd, use_graph=True))
        torch.cuda.synchronize()
        assert np.array_equal(got, eager), rep
    c = moe_data.compare_bf16(eager, _oracle_step(orc, model, res, deltas))
    assert c["max_abs"] <= 2e-2 and c["mean_rel"] <= 1e-3, c
    eng.shutdown()
