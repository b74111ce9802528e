"""GPU parity of the matrix-core decode path (the layer's default for
T < prefill_min_tokens): mc_stream_kernel gate_up (+ bias + SwiGLU) and down
(+ bias), against the CPU oracle and against the exact decode kernels on the
same weights.

Tolerance, as for the prefill path (test_gpu_prefill.py): the matrix core
adds the exact products (bf16 activations times exactly decoded MXFP4
weights) in its own fp32 order and the K-parts are added in part order, so
each value differs from the canonical fp32 sum by reordering alone, carried
through one bf16 rounding.  Each stage is checked against the canonical
computation of that stage on the GPU's own inputs:
  * gate_up and expert outputs (single rounding): within one bf16 step plus
    2^-9, differing on a small fraction of values, mean-rel <= 1e-3;
  * SwiGLU activations: bit-identical to the oracle's SwiGLU of the GPU's own
    gate_up values;
  * layer output: bit-identical to the combine of the GPU's own expert
    outputs, and end to end within mean-rel 1e-3 of the exact path / oracle,
    with the fraction of outputs past 2e-2 (whole bf16 steps at |out| > 4)
    bounded.
Routing (indices, weights, plan) is the same launch as the exact path and is
compared bit for bit.
"""
import os

import numpy as np
import pytest

import moe_data
from test_gpu_parity import DeviceLayer, _trace_arrays, dev, host, say
from test_gpu_prefill import check_layer_out, check_single_rounding

pytestmark = pytest.mark.gpu

E120, K120, H120, I120 = 128, 4, 2880, 2880


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _y_given(gpu, torch, act_dev, tiled, bias_t, offs, H, I):
    """Expert outputs from the given activations with the exact dense kernel
    (bit-identical to the oracle's canonical order)."""
    n2, s2 = gpu.tiled_size(H, I)
    y = np.zeros((act_dev.shape[0], H), np.uint16)
    for e in range(len(offs) - 1):
        a, b = int(offs[e]), int(offs[e + 1])
        if b > a:
            y[a:b] = host(gpu.mxfp4_gemv(act_dev[a:b], tiled[2][e * n2:(e + 1) * n2], tiled[3][e * s2:(e + 1) * s2],
                                         bias_t[e] if bias_t is not None else None, H, I))
    return y


@pytest.mark.parametrize("T", [1, 5, 8, 9, 40])
@pytest.mark.parametrize("bias", ["random", "none"])
def test_mc_layer_small_stagewise(gpu, orc, torch_mod, T, bias):
    """E=8, k=2, H=I=128 (4 blocks per row: the generic block loop), every
    stage against the oracle on the GPU's own inputs."""
    torch = torch_mod
    E, k, H, I = 8, 2, 128, 128
    w = moe_data.make_layer(20 + T, E, H, I, bias=bias)
    x, res = moe_data.make_tokens(20 + T, T, H)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=64, exact=False)
    L.layer.set_trace_gate_up(True)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    torch.cuda.synchronize()
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    got = _trace_arrays(gpu, L.layer, T, k, E, H, I, torch, True)
    assert np.array_equal(got["idx"], tr["idx"])
    assert np.array_equal(got["w"].view(np.uint32), tr["w"].view(np.uint32))
    assert np.array_equal(got["gather_map"], tr["gather_map"])
    check_single_rounding(got["gate_up"], tr["gate_up"], f"mc small T={T} gate_up")
    assert np.array_equal(got["act"], orc.swiglu_rows(got["gate_up"], I))
    offs = np.concatenate([[0], np.cumsum(np.bincount(tr["idx"].ravel(), minlength=E))])
    ylocal = np.zeros_like(got["y"])
    for e in range(E):
        a, b = int(offs[e]), int(offs[e + 1])
        if b > a:
            ylocal[a:b] = orc.mxfp4_gemv(got["act"][a:b], w["w2_packed"][e], w["w2_scales"][e],
                                         w["w2_bias"][e] if w["w2_bias"] is not None else None, H, I)
    check_single_rounding(got["y"], ylocal, f"mc small T={T} y (same activations)")
    assert np.array_equal(out, orc.combine(got["y"], tr["gather_map"], tr["w"], res, T, k, H))
    check_layer_out(out, ref, f"mc small T={T} bias={bias} out vs oracle")


@pytest.mark.parametrize("T,E,H,I", [(40, 8, 320, 96), (20, 8, 640, 160), (64, 8, 128, 224), (3, 8, 320, 96),
                                     (1, 30, 128, 128), (2, 30, 128, 128), (1, 6, 192, 128), (9, 6, 128, 128),
                                     (40, 30, 192, 128)])
def test_mc_layer_odd_block_counts(gpu, orc, torch_mod, T, E, H, I):
    """k=4 with K/32 = 10, 3, 20, 5, 4, 6 and 7 blocks per row (the generic
    one-part shapes take the ring depth that divides it), output tiles
    N / 64 = 3, 5 and 7, and E = 6 and 30 (not a multiple of the 64 experts
    a routing wave covers) at one, two and more tokens; every stage against
    the oracle on the GPU's inputs."""
    torch = torch_mod
    k = 4
    w = moe_data.make_layer(80 + T + H, E, H, I, bias="random")
    x, res = moe_data.make_tokens(80 + T + H, T, H)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=64, exact=False)
    L.layer.set_trace_gate_up(True)
    say("mc odd block counts", T, E, H, I)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    torch.cuda.synchronize()
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    got = _trace_arrays(gpu, L.layer, T, k, E, H, I, torch, True)
    assert np.array_equal(got["idx"], tr["idx"])
    check_single_rounding(got["gate_up"], tr["gate_up"], f"mc odd T={T} H={H} gate_up")
    assert np.array_equal(got["act"], orc.swiglu_rows(got["gate_up"], I))
    offs = np.concatenate([[0], np.cumsum(np.bincount(tr["idx"].ravel(), minlength=E))])
    ylocal = np.zeros_like(got["y"])
    for e in range(E):
        a, b = int(offs[e]), int(offs[e + 1])
        if b > a:
            ylocal[a:b] = orc.mxfp4_gemv(got["act"][a:b], w["w2_packed"][e], w["w2_scales"][e], w["w2_bias"][e], H, I)
    check_single_rounding(got["y"], ylocal, f"mc odd T={T} H={H} y (same activations)")
    check_layer_out(out, ref, f"mc odd T={T} H={H} I={I} out vs oracle")


@pytest.fixture(scope="module")
def pair120(gpu, torch_mod):
    """One tiled copy of GPT-OSS-120B-shaped weights (E=128, H=I=2880) under
    two layers: the matrix-core decode path and the exact decode path."""
    torch = torch_mod
    say("building GPT-OSS-120B-shaped layer pair (matrix-core / exact decode)")
    w = moe_data.make_layer(4321, E120, H120, I120, bias="random")
    ex = DeviceLayer(gpu, torch, w, E120, K120, H120, I120, max_tokens=64, via_tables=False, exact=True)
    mc = DeviceLayer(gpu, torch, w, E120, K120, H120, I120, max_tokens=64, exact=False, tiled=ex.tiled, t=ex.t)
    torch.cuda.synchronize()
    return w, ex, mc


def _stagewise_vs_exact(gpu, orc, torch, ex, mc, x, res, T, what, idx=None, wt=None):
    k, H, I = K120, H120, I120
    S = T * k
    dx, dr = dev(x, torch), dev(res, torch)
    mc.layer.set_trace_gate_up(True)
    ex.layer.set_trace_gate_up(True)
    if idx is None:
        out_mc = host(mc.layer.forward_prenormed(dx, dr))
    else:
        out_mc = host(mc.layer.forward_routed(dx, dev(idx, torch), dev(wt, torch), residual=dr))
    tr = mc.layer.trace()
    rd = lambda p, n, dt: gpu.copy_device_to_tensor(p, n * np.dtype(dt).itemsize).cpu().numpy().view(dt)  # noqa
    gu_mc = rd(tr.gate_up, S * 2 * I, np.uint16).reshape(S, 2 * I)
    act_dev = gpu.copy_device_to_tensor(tr.act, S * I * 2).view(torch.bfloat16).reshape(S, I)
    act_mc = host(act_dev)
    y_mc = rd(tr.expert_out, S * H, np.uint16).reshape(S, H)
    gm = rd(tr.gather_map, S, np.int32)
    wts = rd(tr.expert_weights, S, np.float32).reshape(T, k) if idx is None else wt
    offs = rd(tr.expert_offsets, E120 + 1, np.int32)
    if idx is None:
        out_ex = host(ex.layer.forward_prenormed(dx, dr))
    else:
        out_ex = host(ex.layer.forward_routed(dx, dev(idx, torch), dev(wt, torch), residual=dr))
    tr_ex = ex.layer.trace()
    gu_ex = rd(tr_ex.gate_up, S * 2 * I, np.uint16).reshape(S, 2 * I)
    assert np.array_equal(rd(tr_ex.gather_map, S, np.int32), gm)
    check_single_rounding(gu_mc, gu_ex, f"{what} gate_up")
    assert np.array_equal(act_mc, orc.swiglu_rows(gu_mc, I))
    y_given = _y_given(gpu, torch, act_dev, ex.tiled, ex.t["w2_bias"], offs, H, I)
    check_single_rounding(y_mc, y_given, f"{what} y (same activations)")
    assert np.array_equal(out_mc, orc.combine(y_mc, gm, wts, res, T, k, H))
    check_layer_out(out_mc, out_ex, f"{what} out vs exact")
    return out_mc, out_ex


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_mc_gptoss120b_decode(gpu, orc, torch_mod, pair120, T):
    """BASELINE config 2 (decode at batch 1/8/32/64): stage by stage against
    the exact kernels, end to end against the exact path and the oracle."""
    torch = torch_mod
    w, ex, mc = pair120
    x, res = moe_data.make_tokens(700 + T, T, H120)
    say("120B matrix-core decode T", T)
    out_mc, out_ex = _stagewise_vs_exact(gpu, orc, torch, ex, mc, x, res, T, f"120B mc T={T}")
    ref = orc.moe_forward(w, x, res, E120, K120, H120, I120)  # every token
    assert np.array_equal(out_ex, ref)
    check_layer_out(out_mc, ref, f"120B mc T={T} all tokens vs oracle")
    out2 = host(mc.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    assert np.array_equal(out_mc, out2)  # run-to-run deterministic


def test_mc_many_tokens_per_expert(gpu, orc, torch_mod, pair120):
    """Injected routing that sends all 64 tokens to experts 0..3 (64 slots per
    expert: several 16-token steps per weight tile) and 40 tokens to a skewed
    mix (a work-group's next step often the same tile's next chunk)."""
    torch = torch_mod
    w, ex, mc = pair120
    T = 64
    x, res = moe_data.make_tokens(811, T, H120)
    idx = np.tile(np.array([[0, 1, 2, 3]], np.int32), (T, 1))
    rng = np.random.default_rng(5)
    wt = rng.dirichlet(np.ones(K120), T).astype(np.float32)
    _stagewise_vs_exact(gpu, orc, torch, ex, mc, x, res, T, "mc 64 slots/expert", idx=idx, wt=wt)
    idx2, wt2 = moe_data.zipf_routing(812, T, E120, K120, s=2.0)
    _stagewise_vs_exact(gpu, orc, torch, ex, mc, x, res, T, "mc zipf(2.0) T=64", idx=idx2, wt=wt2)


# every compiled launch shape for the GPT-OSS K (90 blocks per row): waves
# per work-group P, ring depth D, 16-token chunks NC
MC_SHAPES = ["6,15,1", "6,5,1", "3,10,1", "3,15,1", "3,5,1", "2,9,1", "2,15,1", "1,9,1", "5,9,1", "5,18,1",
             "9,10,1", "2,9,2", "3,15,1/6,5,1"]


@pytest.mark.parametrize("shape", MC_SHAPES)
def test_mc_launch_shapes(gpu, orc, torch_mod, pair120, shape, monkeypatch):
    """Each compiled launch shape (selected by GPTOSS_MOE_DECODE_SHAPE at
    layer init) at T = 64, 3, 2 and 1 (up to two tokens: the gate_up launch
    with the routing in its prologue, for the shapes compiled with it),
    against the exact path."""
    torch = torch_mod
    w, ex, _ = pair120
    monkeypatch.setenv("GPTOSS_MOE_DECODE_SHAPE", shape)
    mc = DeviceLayer(gpu, torch, w, E120, K120, H120, I120, max_tokens=64, exact=False, tiled=ex.tiled, t=ex.t)
    try:
        for T in (64, 3, 2, 1):
            x, res = moe_data.make_tokens(900 + T, T, H120)
            say("mc shape", shape, "T", T)
            _stagewise_vs_exact(gpu, orc, torch, ex, mc, x, res, T, f"mc shape {shape} T={T}")
    finally:
        mc.layer.destroy()


def test_mc_special_scales(gpu, orc, torch_mod):
    """Experts whose scales hold e8m0 codes 0 (+0) and 255 (+inf): the
    checking variant runs; NaN / inf positions match the exact path and the
    finite values agree to the tolerance above."""
    torch = torch_mod
    E, k, H, I, T = 8, 2, 256, 128, 6
    w = moe_data.make_layer(61, E, H, I, bias="random")
    rng = np.random.default_rng(61)
    for e in (1, 5):
        s1 = w["w1_scales"][e]
        s1[rng.integers(0, s1.shape[0], 3), rng.integers(0, s1.shape[1], 3)] = 0
        s1[rng.integers(0, s1.shape[0], 1), rng.integers(0, s1.shape[1], 1)] = 255
        s2 = w["w2_scales"][e]
        s2[rng.integers(0, s2.shape[0], 3), rng.integers(0, s2.shape[1], 3)] = 0
    x, res = moe_data.make_tokens(61, T, H)
    idx = np.array([[1, 5], [5, 0], [2, 1], [3, 4], [6, 7], [1, 2]], np.int32)
    wt = np.full((T, k), 0.5, np.float32)
    ex = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=8, via_tables=False, exact=True)
    mc = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=8, exact=False, tiled=ex.tiled, t=ex.t)
    ex.layer.set_trace_gate_up(True)
    mc.layer.set_trace_gate_up(True)
    dx, dr, di, dw = dev(x, torch), dev(res, torch), dev(idx, torch), dev(wt, torch)
    out_mc = host(mc.layer.forward_routed(dx, di, dw, residual=dr))
    g_mc = _trace_arrays(gpu, mc.layer, T, k, E, H, I, torch, True)
    out_ex = host(ex.layer.forward_routed(dx, di, dw, residual=dr))
    g_ex = _trace_arrays(gpu, ex.layer, T, k, E, H, I, torch, True)
    c = moe_data.mfma_stats(g_mc["gate_up"], g_ex["gate_up"])
    say("mc special gate_up", c)
    assert c["nan_ok"] and c["inf_ok"] and c["max_excess"] <= 2.0 ** -9
    c = moe_data.mfma_stats(out_mc, out_ex)
    say("mc special out", c)
    assert c["nan_ok"] and c["inf_ok"]


@pytest.mark.parametrize("T", [1, 2])
def test_mc_repeated_expert_in_token(gpu, orc, torch_mod, pair120, T):
    """forward_routed with an expert repeated within a token (three slots of
    one expert at one token, four over two tokens): the one- and two-token
    down launch stages the input rows of two slots per expert only, so such
    a routing takes the per-lane loads and every slot's output is its own.
    Checked against the exact path and the oracle."""
    torch = torch_mod
    w, ex, mc = pair120
    idx = np.array([[3, 3, 3, 9], [3, 9, 9, 3]], np.int32)[:T]
    wt = np.array([[0.4, 0.3, 0.2, 0.1], [0.1, 0.2, 0.3, 0.4]], np.float32)[:T]
    x, res = moe_data.make_tokens(880 + T, T, H120)
    dx, dr, di, dw = dev(x, torch), dev(res, torch), dev(idx, torch), dev(wt, torch)
    out_mc = host(mc.layer.forward_routed(dx, di, dw, residual=dr))
    out_ex = host(ex.layer.forward_routed(dx, di, dw, residual=dr))
    ref = orc.moe_forward_routed(w, x, res, idx, wt, E120, K120, H120, I120)
    assert np.array_equal(out_ex, ref)
    check_layer_out(out_mc, ref, f"mc repeated expert T={T} vs oracle")


@pytest.mark.parametrize("T", [1, 8])
def test_mc_graph_replay(gpu, orc, torch_mod, T):
    """Matrix-core decode captured in a HIP graph: every replay matches the
    eager forward bit for bit (the path is deterministic).  One token: the
    gate_up launch routes and rewrites the plan on every replay."""
    torch = torch_mod
    E, k, H, I = 16, 4, 128, 128
    w = moe_data.make_layer(51, E, H, I)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T, exact=False)
    xs = [moe_data.make_tokens(60 + i, T, H) for i in range(4)]
    eager = [host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch))) for x, res in xs]
    sx, sr = dev(xs[0][0], torch), dev(xs[0][1], torch)
    so = torch.empty_like(sx)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        L.layer.forward_prenormed(sx, sr, out=so)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        L.layer.forward_prenormed(sx, sr, out=so)
    for rep in range(3):
        for i, (x, res) in enumerate(xs):
            sx.copy_(dev(x, torch))
            sr.copy_(dev(res, torch))
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(host(so), eager[i]), (rep, i)
    check_layer_out(eager[1], orc.moe_forward(w, xs[1][0], xs[1][1], E, k, H, I), "mc graph eager vs oracle")


def test_layer_profiling_events(gpu, torch_mod):
    """gptoss_moe_layer_set_profiling / profile_read: four timed launches per
    forward (route, gate_up, down, combine), positive and summing to at most
    the forwards' wall interval; a forward captured into a graph is not timed
    and leaves its slot to the next eager forward."""
    torch = torch_mod
    E, k, H, I, T = 16, 4, 128, 128, 8
    w = moe_data.make_layer(71, E, H, I)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T, exact=False)
    x, res = moe_data.make_tokens(71, T, H)
    dx, dr = dev(x, torch), dev(res, torch)
    out = torch.empty_like(dx)
    L.layer.forward_prenormed(dx, dr, out=out)
    torch.cuda.synchronize()
    L.layer.set_profiling(3)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(3):
        L.layer.forward_prenormed(dx, dr, out=out)
    t1.record()
    torch.cuda.synchronize()
    r, a, b, c, n = L.layer.profile_read()
    say("profiling eager ms", r, a, b, c, n, "wall", t0.elapsed_time(t1))
    assert n == 3 and min(r, a, b, c) > 0.0
    assert r + a + b + c <= t0.elapsed_time(t1) * 1.05
    # graph capture: not timed; the replays match the eager result
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    L.layer.set_profiling(1)
    with torch.cuda.graph(g, stream=s):
        L.layer.forward_prenormed(dx, dr, out=out)
    want = host(out)
    for _ in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), want)
    assert L.layer.profile_read()[4] == 0
    L.layer.forward_prenormed(dx, dr, out=out)
    r, a, b, c, n = L.layer.profile_read()
    assert n == 1 and min(r, a, b, c) > 0.0
    L.layer.set_profiling(0)


def test_mc_one_token_dropped_slots(gpu, orc, torch_mod):
    """One token on the matrix-core path with routed slots dropped (-1,
    >= E), every slot dropped (output = the residual, bit for bit) and a null
    residual."""
    torch = torch_mod
    E, k, H, I = 8, 4, 128, 128
    w = moe_data.make_layer(31, E, H, I, bias="random")
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=4, exact=False)
    x, res = moe_data.make_tokens(31, 1, H)
    wt = np.array([[0.4, 0.3, 0.2, 0.1]], np.float32)
    for case in ([[3, -1, 5, 1]], [[-1, -1, -1, -1]], [[2, 9, 0, 7]]):
        idx = np.array(case, np.int32)
        for r in (res, None):
            out = host(L.layer.forward_routed(dev(x, torch), dev(idx, torch), dev(wt, torch),
                                              residual=dev(r, torch) if r is not None else None))
            torch.cuda.synchronize()
            ref = orc.moe_forward_routed(w, x, r, idx, wt, E, k, H, I)
            if (idx < 0).all():
                assert np.array_equal(out, r if r is not None else np.zeros_like(out)), case
            else:
                check_layer_out(out, ref, f"one token {case} residual={r is not None}")


def _one_token_router(case, E, H, seed):
    """Router weights and bias (bf16) whose logits on an all-ones token hit
    the top-k's edge cases: exact ties, NaN / +inf / -inf logits, fewer
    visible experts than k, all NaN (degenerate: experts 0..k-1, weight
    1/k), all zero (+-0 ties)."""
    rng = np.random.default_rng(seed)
    W = rng.normal(0.0, 0.02, (E, H)).astype(np.float32)
    b = rng.normal(0.0, 0.02, E).astype(np.float32)
    if case == "ties":
        for e in range(0, E, 3):
            W[e + 1:e + 3] = W[e]
            b[e + 1:e + 3] = b[e]
    elif case == "nonfinite":
        W[5::7, 3] = np.nan
        W[2::9, 4] = np.inf
        W[1::11, 5] = -np.inf
    elif case == "three_visible":
        W[:, 7] = -np.inf
        W[[4, 40, 90], 7] = 0.0
    elif case == "all_nan":
        W[:, 0] = np.nan
    elif case == "zero":
        W[:] = 0.0
        b[:] = 0.0
        b[1::2] = -0.0
    return moe_data.bf16(W), moe_data.bf16(b)


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("k", [1, 4, 8])
@pytest.mark.parametrize("case", ["ties", "nonfinite", "three_visible", "all_nan", "zero"])
def test_mc_one_token_routing_prologue(gpu, orc, torch_mod, case, k, T):
    """One or two tokens on the matrix-core path route inside the gate_up
    launch (one token: one wave selects the top-k with packed key/index
    words and builds the plan of the k distinct experts; two: a wave per
    token, then the one-wave plan): indices, weights, gather map and expert
    offsets bit-identical to the exact path's router launch and to the
    oracle, on logits with ties, non-finite values, fewer visible experts
    than k, none visible and all zero; the output within the matrix-core
    tolerance of the exact path."""
    torch = torch_mod
    E, H, I = 128, 128, 128
    w = moe_data.make_layer(70 + k, E, H, I, bias="random")
    w["router_w"], w["router_b"] = _one_token_router(case, E, H, 80 + k)
    x = np.ones((T, H), np.float32)
    if T > 1:  # a second token with positive entries (the crafted columns keep their sign)
        x[1] = np.abs(np.random.default_rng(72).normal(1.0, 0.5, H)) + 0.1
    x = moe_data.bf16(x)
    _, res = moe_data.make_tokens(71, T, H)
    ex = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T, via_tables=False, exact=True)
    mc = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T, exact=False, tiled=ex.tiled, t=ex.t)
    dx, dr = dev(x, torch), dev(res, torch)
    out_mc = host(mc.layer.forward_prenormed(dx, dr))
    tr_mc = _trace_arrays(gpu, mc.layer, T, k, E, H, I, torch, False)
    out_ex = host(ex.layer.forward_prenormed(dx, dr))
    tr_ex = _trace_arrays(gpu, ex.layer, T, k, E, H, I, torch, False)
    torch.cuda.synchronize()
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    for name in ("idx", "gather_map"):
        assert np.array_equal(tr_mc[name], tr_ex[name]), (case, k, name, tr_mc[name], tr_ex[name])
        assert np.array_equal(tr_mc[name], tr[name]), (case, k, name)
    assert np.array_equal(tr_mc["w"].view(np.uint32), tr_ex["w"].view(np.uint32)), (case, k)
    assert np.array_equal(tr_mc["w"].view(np.uint32), tr["w"].view(np.uint32)), (case, k)
    rd = lambda p, n: gpu.copy_device_to_tensor(p, n * 4).cpu().numpy().view(np.int32)  # noqa
    tm, te = mc.layer.trace(), ex.layer.trace()
    assert np.array_equal(rd(tm.expert_offsets, E + 1), rd(te.expert_offsets, E + 1))
    assert np.array_equal(rd(tm.expert_counts, E), rd(te.expert_counts, E))
    na = int(rd(tm.n_active, 1)[0])
    assert na == int(rd(te.n_active, 1)[0]) == len(set(tr["idx"][tr["idx"] >= 0].tolist()))
    assert np.array_equal(rd(tm.active_experts, E)[:na], rd(te.active_experts, E)[:na])
    nslot = int((tr["idx"] >= 0).sum())
    assert np.array_equal(rd(tm.perm_token, nslot), rd(te.perm_token, nslot))
    assert np.array_equal(out_ex, ref)
    check_layer_out(out_mc, out_ex, f"routing prologue {case} k={k} T={T}")
    mc.layer.destroy()
    ex.layer.destroy()


@pytest.mark.parametrize("T", [127, 128])
def test_mc_decode_prefill_boundary(gpu, orc, torch_mod, pair120, T):
    """Either side of prefill_min_tokens at the GPT-OSS-120B shape: 127
    tokens (508 slots, the largest matrix-core decode step; experts with
    several 16-token chunks) and 128 (the grouped prefill GEMMs), against the
    exact decode kernels on the same weights: expert indices bit-exact,
    outputs within the tolerance, run-to-run deterministic."""
    torch = torch_mod
    w, ex, mc = pair120
    layer = DeviceLayer(gpu, torch, w, E120, K120, H120, I120, max_tokens=128, exact=False, tiled=ex.tiled, t=ex.t)
    assert layer.layer.cfg.prefill_min_tokens == 128
    cfg = gpu.default_config(E120, 128, prefill_min_tokens=0, decode_exact=True)
    exact = gpu.MoELayer().init(cfg, 0, ex.t["router_w"], ex.t.get("router_b"), ex.t.get("w1_bias"),
                                ex.t.get("w2_bias"), tiled=ex.tiled)
    x, res = moe_data.make_tokens(900 + T, T, H120)
    dx, dr = dev(x, torch), dev(res, torch)
    say("120B boundary T", T)
    out = host(layer.layer.forward_prenormed(dx, dr))
    idx = gpu.copy_device_to_tensor(layer.layer.trace().expert_indices, T * K120 * 4, torch.int32).cpu().numpy()
    out_ex = host(exact.forward_prenormed(dx, dr))
    idx_ex = gpu.copy_device_to_tensor(exact.trace().expert_indices, T * K120 * 4, torch.int32).cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(idx, idx_ex)
    check_layer_out(out, out_ex, f"120B T={T} vs exact")
    assert np.array_equal(out, host(layer.layer.forward_prenormed(dx, dr)))
    exact.destroy()


@pytest.mark.parametrize("k", [1, 2, 8])
@pytest.mark.parametrize("T", [1, 2, 8])
def test_mc_top_k_variants_gptoss20b(gpu, orc, torch_mod, k, T):
    """Top-k other than 4 at the GPT-OSS-20B shape (E=32, H=I=2880) on the
    matrix-core decode path (one and two tokens: top-k and plan inside the
    gate_up launch, operands staged in LDS; two tokens at k=8 give 16
    experts x 90 tiles, more than the resident work-groups, so work-groups
    restage for further items) against the exact path: indices and weights
    bit-exact, outputs within the tolerance; token 0 against the oracle."""
    torch = torch_mod
    E, H, I = 32, 2880, 2880
    w = moe_data.make_layer(950 + k, E, H, I, bias="random")
    ex = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=8, via_tables=False, exact=True)
    mc = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=8, exact=False, tiled=ex.tiled, t=ex.t)
    x, res = moe_data.make_tokens(960 + 10 * k + T, T, H)
    dx, dr = dev(x, torch), dev(res, torch)
    say("20B top-k", k, "T", T)
    out_mc = host(mc.layer.forward_prenormed(dx, dr))
    rd = lambda L, p, n, dt: gpu.copy_device_to_tensor(p, n * 4).cpu().numpy().view(dt)  # noqa: E731
    tr_mc = mc.layer.trace()
    idx_mc, w_mc = rd(mc, tr_mc.expert_indices, T * k, np.int32), rd(mc, tr_mc.expert_weights, T * k, np.float32)
    out_ex = host(ex.layer.forward_prenormed(dx, dr))
    tr_ex = ex.layer.trace()
    torch.cuda.synchronize()
    assert np.array_equal(idx_mc, rd(ex, tr_ex.expert_indices, T * k, np.int32))
    assert np.array_equal(w_mc.view(np.uint32), rd(ex, tr_ex.expert_weights, T * k, np.float32).view(np.uint32))
    check_layer_out(out_mc, out_ex, f"20B k={k} T={T} vs exact")
    assert np.array_equal(out_ex[:1], orc.moe_forward(w, x[:1], res[:1], E, k, H, I))


@pytest.mark.parametrize("T", [1, 3])
def test_mc_fp32_logits(gpu, orc, torch_mod, pair120, T):
    """fp32 router logits (logits_fp32 = 1) on the matrix-core decode path
    (one token: the gate_up launch selects from fp32 logits) against the
    oracle's fp32 routing: logits and indices bit-exact, weights bit-exact,
    outputs within the tolerance of the exact path."""
    torch = torch_mod
    w, ex, _ = pair120
    cfg = gpu.default_config(E120, 8, logits_fp32=True)
    cfg.top_k = K120
    mc = gpu.MoELayer().init(cfg, 0, ex.t["router_w"], ex.t.get("router_b"), ex.t.get("w1_bias"),
                             ex.t.get("w2_bias"), tiled=ex.tiled)
    cfg_ex = gpu.default_config(E120, 8, logits_fp32=True, decode_exact=True)
    exl = gpu.MoELayer().init(cfg_ex, 0, ex.t["router_w"], ex.t.get("router_b"), ex.t.get("w1_bias"),
                              ex.t.get("w2_bias"), tiled=ex.tiled)
    x, res = moe_data.make_tokens(980 + T, T, H120)
    dx, dr = dev(x, torch), dev(res, torch)
    out = host(mc.forward_prenormed(dx, dr))
    tr = mc.trace()
    rd = lambda p, n, dt: gpu.copy_device_to_tensor(p, n * 4).cpu().numpy().view(dt)  # noqa: E731
    logits = rd(tr.logits, T * E120, np.float32).reshape(T, E120)
    idx = rd(tr.expert_indices, T * K120, np.int32).reshape(T, K120)
    wts = rd(tr.expert_weights, T * K120, np.float32).reshape(T, K120)
    out_ex = host(exl.forward_prenormed(dx, dr))
    torch.cuda.synchronize()
    ref_logits = orc.router(x, w["router_w"], w["router_b"], logits_fp32=True)
    assert np.array_equal(logits.view(np.uint32), ref_logits.view(np.uint32))
    ridx, rw = orc.topk_softmax(ref_logits, K120)
    assert np.array_equal(idx, ridx) and np.array_equal(wts.view(np.uint32), rw.view(np.uint32))
    check_layer_out(out, out_ex, f"120B fp32 logits T={T} vs exact")
    mc.destroy()
    exl.destroy()


@pytest.mark.parametrize("T", [1, 2, 6])
def test_mc_forward_residual(gpu, orc, torch_mod, pair120, T):
    """The decode step's residual add + RMSNorm + MoE (forward_residual) on
    the matrix-core path: one and two tokens with the norm inside the
    router's launch (one token also routed inside gate_up), six with the
    norm in its own launch; the new residual bit-exact with the oracle, the
    expert indices with the exact path, outputs within the tolerance."""
    torch = torch_mod
    w, ex, _ = pair120
    norm_w = moe_data.bf16(np.random.default_rng(990).normal(1.0, 0.1, H120))
    dn = dev(norm_w, torch)
    layers = []
    for exact in (False, True):
        cfg = gpu.default_config(E120, 8, decode_exact=exact)
        cfg.top_k = K120
        layers.append(gpu.MoELayer().init(cfg, 0, ex.t["router_w"], ex.t.get("router_b"), ex.t.get("w1_bias"),
                                          ex.t.get("w2_bias"), moe_norm_weight=dn, tiled=ex.tiled))
    r, d = moe_data.make_tokens(995 + T, T, H120)
    outs, sums, idxs = [], [], []
    for L in layers:
        s_out = torch.empty((T, H120), dtype=torch.bfloat16, device="cuda")
        outs.append(host(L.forward_residual(dev(r, torch), dev(d, torch), residual_out=s_out)))
        sums.append(host(s_out))
        idxs.append(gpu.copy_device_to_tensor(L.trace().expert_indices, T * K120 * 4, torch.int32).cpu().numpy())
    torch.cuda.synchronize()
    _, ref_sum = orc.residual_rmsnorm(r, d, norm_w)
    assert np.array_equal(sums[0], ref_sum) and np.array_equal(sums[1], ref_sum)
    assert np.array_equal(idxs[0], idxs[1])
    check_layer_out(outs[0], outs[1], f"120B forward_residual T={T} mc vs exact")
    for L in layers:
        L.destroy()
