"""GPU: gptoss_moe_layer_forward_prenormed_noalloc, the forward whose scratch
is the library's static device array, against gptoss_moe_layer_forward_prenormed
of the same weights, bit for bit (same kernels, same order).  Each case makes
two calls in a row, the second with fewer tokens, so the second call runs on
the array as the first left it.  The layer given to the no-allocation call is
initialised for one token: its own scratch is too small for the calls, which
therefore cannot be using it."""
import ctypes

import numpy as np
import pytest

import moe_data
from test_gpu_parity import DeviceLayer, dev, host, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _noalloc(gpu, layer, x, r, out, T, torch):
    return gpu.lib.gptoss_moe_layer_forward_prenormed_noalloc(
        layer._h, x.data_ptr(), None if r is None else r.data_ptr(), out.data_ptr(), T,
        torch.cuda.current_stream().cuda_stream)


def _pair(gpu, torch, w, E, k, H, I, prefill_min=None):
    ref = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=64, exact=False, via_tables=False)
    cfg = gpu.default_config(E, 1, prefill_min_tokens=prefill_min)
    cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, k
    one = gpu.MoELayer().init(cfg, 0, ref.t["router_w"], ref.t.get("router_b"), ref.t.get("w1_bias"),
                              ref.t.get("w2_bias"), tiled=ref.tiled)
    if prefill_min is not None:
        cfg2 = gpu.default_config(E, 64, prefill_min_tokens=prefill_min)
        cfg2.hidden_size, cfg2.intermediate_size, cfg2.top_k = H, I, k
        ref.layer.destroy()
        ref.layer = gpu.MoELayer().init(cfg2, 0, ref.t["router_w"], ref.t.get("router_b"), ref.t.get("w1_bias"),
                                        ref.t.get("w2_bias"), tiled=ref.tiled)
    return ref, one


@pytest.mark.parametrize("E,k,H,I,Ts,prefill_min", [
    (128, 4, 2880, 2880, (64, 8), None),   # GPT-OSS-120B decode on the matrix cores
    (32, 4, 2880, 2880, (1, 1), None),     # GPT-OSS-20B, one token (routing inside the gate_up launch)
    (16, 4, 256, 128, (40, 20), 16),       # grouped prefill kernels (tile queue in the array)
])
def test_noalloc_matches_forward_prenormed(gpu, torch_mod, E, k, H, I, Ts, prefill_min):
    torch = torch_mod
    w = moe_data.make_layer(900 + E + H, E, H, I, bias="random")
    ref, one = _pair(gpu, torch, w, E, k, H, I, prefill_min)
    for T in Ts:
        say("noalloc forward E", E, "H", H, "T", T)
        x, res = moe_data.make_tokens(910 + T + E, T, H)
        dx, dr = dev(x, torch), dev(res, torch)
        out = torch.empty_like(dx)
        gpu.check(_noalloc(gpu, one, dx, dr, out, T, torch))
        torch.cuda.synchronize()
        want = host(ref.layer.forward_prenormed(dx, dr))
        assert np.array_equal(host(out), want), (E, T)
    one.destroy()
    ref.layer.destroy()


def test_noalloc_limits_and_capture(gpu, torch_mod):
    """More than 64 tokens is refused before any launch; a call captured in a
    hipGraph replays to the eager result on every replay, with eager work on
    the same array between replays."""
    torch = torch_mod
    E, k, H, I = 16, 4, 256, 128
    w = moe_data.make_layer(930, E, H, I, bias="random")
    ref, one = _pair(gpu, torch, w, E, k, H, I)
    x65 = torch.zeros((65, H), dtype=torch.bfloat16, device="cuda")
    assert _noalloc(gpu, one, x65, None, torch.empty_like(x65), 65, torch) == gpu.GPTOSS_ERR_INVALID
    assert b"static" in gpu.lib.gptoss_last_error()
    with pytest.raises(ValueError, match="output"):
        one.forward_prenormed_noalloc(x65[:8])
    T = 8
    xs = [moe_data.make_tokens(940 + i, T, H) for i in range(3)]
    eager = [host(ref.layer.forward_prenormed(dev(x, torch), dev(r, torch))) for x, r in xs]
    sx, sr = dev(xs[0][0], torch), dev(xs[0][1], torch)
    so = torch.empty_like(sx)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        one.forward_prenormed_noalloc(sx, sr, out=so)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        one.forward_prenormed_noalloc(sx, sr, out=so)
    for rep in range(3):
        for i, (x, r) in enumerate(xs):
            sx.copy_(dev(x, torch))
            sr.copy_(dev(r, torch))
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(host(so), eager[i]), (rep, i)
            # eager use of the same array between replays, with another token count
            tmp = torch.empty((3, H), dtype=torch.bfloat16, device="cuda")
            one.forward_prenormed_noalloc(sx[:3], sr[:3], out=tmp)
    del g
    one.destroy()
    ref.layer.destroy()
