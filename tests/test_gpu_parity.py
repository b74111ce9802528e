"""GPU parity tests: the HIP library (through its C ABI) against the CPU oracle.

Tolerance: outputs within max-abs 2e-2 and mean-rel
1e-3 of the reference on bf16 outputs, expert indices bit-exact.  The layers
here run the exact decode kernels (decode_exact = 1), which follow the
oracle's summation order, so every comparison below first asserts the strict
result -- bit-identical bf16 / fp32 / int32 -- and the north-star tolerance
is therefore met with margin zero.  The matrix-core decode path (the default)
is checked in test_gpu_decode_mc.py.  Inputs are seeded synthetic data with
the BASELINE distributions (tests/moe_data.py).
"""
import os
import sys

import numpy as np
import pytest

import moe_data

pytestmark = pytest.mark.gpu

MAX_ABS_TOL = 2e-2
MEAN_REL_TOL = 1e-3


def say(*a):
    print("[gpu-test]", *a, flush=True)


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def dev(a, torch):
    """numpy -> device tensor (uint16 arrays become bfloat16)."""
    if a is None:
        return None
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def assert_bf16_parity(got, ref, what):
    c = moe_data.compare_bf16(got, ref)
    say(what, c)
    assert c["max_abs"] <= MAX_ABS_TOL and c["mean_rel"] <= MEAN_REL_TOL, (what, c)
    assert c["mismatches"] == 0, (what, c)


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------
def test_pack_and_dequant_all_codes_and_scales(gpu, orc, torch_mod):
    """Every e2m1 code times every e8m0 scale code (incl. 0 -> +-0, 255 -> inf
    and fp32-denormal products) through the gfx950 scaled fp4 conversion."""
    torch = torch_mod
    N, K = 256, 32
    packed = np.zeros((N, 16), np.uint8)
    packed[:, :8] = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8)
    packed[:, 8:] = np.arange(8 * N, dtype=np.uint32).reshape(N, 8).astype(np.uint8)
    scales = np.arange(256, dtype=np.uint8).reshape(N, 1)
    nib, sc = gpu.pack_tiled(dev(packed, torch), dev(scales, torch), N, K)
    out = host(gpu.dequant(nib, sc, N, K))
    ref = orc.mxfp4_dequant(packed, scales, N, K)
    bad = np.argwhere(out != ref)
    say("dequant mismatches", len(bad), bad[:8].tolist())
    assert len(bad) == 0


def test_swiglu_grid(gpu, orc, torch_mod):
    torch = torch_mod
    g = np.linspace(-40, 40, 2001, dtype=np.float32)
    u = np.linspace(-12, 12, 97, dtype=np.float32)
    G, U = np.meshgrid(g, u, indexing="ij")
    gu = np.stack([G.reshape(-1), U.reshape(-1)], axis=1).reshape(97, -1)  # rows of interleaved pairs
    gu = moe_data.bf16(gu)
    extra = moe_data.bf16(np.array([[np.inf, 0, -np.inf, 0, 7.0, 7.0, -7.0, -7.0, 1e-30, 3.0, -88.0, 1.0]], np.float32))
    for arr in (gu, extra):
        I = arr.shape[1] // 2
        out = host(gpu.swiglu(dev(arr, torch)))
        ref = orc.swiglu_rows(arr, I)
        assert np.array_equal(out, ref), np.argwhere(out != ref)[:8]


def _crafted_logits(T, E, seed):
    rng = np.random.default_rng(seed)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    q = T // 3
    lg[:q] = np.round(lg[:q] * 4) / 4             # exact ties
    if T > 6:
        lg[q, :] = np.nan                          # degenerate token
        lg[q + 1, ::5] = np.inf
        lg[q + 2, :] = -np.inf
        lg[q + 2, :3] = 0.5                        # only three visible
        lg[q + 3, ::2] = -0.0
        lg[q + 3, 1::2] = 0.0                      # +-0 ties
    return lg


@pytest.mark.parametrize("T", [1, 5, 8, 9, 300])
@pytest.mark.parametrize("k", [1, 2, 4, 8])
@pytest.mark.parametrize("fp32", [False, True])
def test_topk_softmax(gpu, orc, torch_mod, T, k, fp32):
    torch = torch_mod
    E = 128
    lg = _crafted_logits(T, E, 100 + T + k)
    if fp32:
        logits_np, lf = lg, lg
        logits = dev(lg, torch)
    else:
        logits_np = moe_data.bf16(lg)
        lf = orc.bf16_to_f32(logits_np)
        logits = dev(logits_np, torch)
    tpe = torch.zeros(E, dtype=torch.int32, device="cuda")
    idx, w = gpu.topk_softmax(logits, k, tokens_per_expert=tpe)
    ridx, rw = orc.topk_softmax(lf, k)
    assert np.array_equal(host(idx), ridx)
    assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    hist = np.bincount(ridx[ridx >= 0], minlength=E)
    assert np.array_equal(host(tpe), hist)


@pytest.mark.parametrize("T,E,shift", [(300, 32, 0), (300, 256, 0), (77, 36, 0), (300, 30, 0), (1000, 128, 1),
                                       (4100, 128, 0), (33, 4, 0), (50, 200, 0)])
@pytest.mark.parametrize("k", [1, 2, 4, 8])
@pytest.mark.parametrize("fp32", [False, True])
def test_topk_softmax_expert_counts(gpu, orc, torch_mod, T, E, shift, k, fp32):
    """The sixteen-lanes-a-token kernel (E % 4 == 0, logits aligned to its
    16- / 8-byte loads) over expert counts and ragged token counts, and the
    one-wave-a-token kernel it falls back to (E = 30, and logits one element
    off the load alignment), against the oracle."""
    torch = torch_mod
    if k > E:
        pytest.skip("k > E")
    lg = _crafted_logits(T, E, 7 * T + E + k)
    host_lg = lg if fp32 else moe_data.bf16(lg)
    lf = lg if fp32 else orc.bf16_to_f32(host_lg)
    flat = np.concatenate([np.zeros(shift, host_lg.dtype), host_lg.reshape(-1)])
    logits = dev(flat, torch)[shift:].view(T, E)
    tpe = torch.zeros(E, dtype=torch.int32, device="cuda")
    idx, w = gpu.topk_softmax(logits, k, tokens_per_expert=tpe)
    ridx, rw = orc.topk_softmax(lf, k)
    assert np.array_equal(host(idx), ridx)
    assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert np.array_equal(host(tpe), np.bincount(ridx[ridx >= 0], minlength=E))


MM_MIN_T = 64  # above this many tokens (and H % 32 == 0) the router runs on the matrix cores


def _mm_router_bound(orc, x, W, b):
    """fp64 logits and the fp32 error bound of any summation order: the K
    exact bf16 products and the bias, (K + 2) u (sum |x w| + |b|)."""
    xf = orc.bf16_to_f32(x).astype(np.float64)
    wf = orc.bf16_to_f32(W).astype(np.float64)
    bf = orc.bf16_to_f32(b).astype(np.float64)
    exact = xf @ wf.T + bf
    mag = np.abs(xf) @ np.abs(wf).T + np.abs(bf)
    return exact, (x.shape[1] + 2) * 2.0 ** -24 * mag


@pytest.mark.parametrize("T,fp32,E,H", [(1, False, 128, 2880), (8, False, 128, 2880), (64, False, 128, 2880),
                                         (9, True, 128, 2880), (4096, True, 128, 2880), (100, False, 20, 512),
                                         (300, True, 36, 4104), (130, True, 256, 2880), (65, True, 128, 2880),
                                         (1000, False, 128, 2880), (5, False, 30, 2880), (100, True, 30, 512),
                                         (70, False, 7, 192)])
def test_route_router_topk(gpu, orc, torch_mod, T, fp32, E, H):
    """Router + top-k; T=4096 fp32 is BASELINE config 1.
    Up to 64 tokens (and for H % 32 != 0: H = 4104, three chunks per chain)
    the logits follow the gemv_bf16 tree bit for bit, and so do the indices
    and weights.  Above 64 tokens they come from the matrix cores: asserted
    within the fp32 error bound of the exact (fp64) sum, deterministic, and a
    token's logits independent of the other tokens in the call; the indices
    and weights are exactly the oracle's top-k softmax of those logits, and
    against the oracle's own (tree) logits the indices differ only where
    two candidates for the k-th place lie within the bound of each other
    (none in these cases) with weights within 1e-6 (the config-1 bar).  The
    many-token cases also cover partial tiles (T, E not multiples of the
    tiles), a short hidden size and 256 experts; E = 30 and 7 (not a multiple
    of the four experts a tree work-group or a logit store covers) run on
    both orders."""
    torch = torch_mod
    k = 4
    rng = np.random.default_rng(T + E + H)
    x = moe_data.bf16(rng.normal(0, 1, (T, H)))
    W = moe_data.bf16(rng.normal(0, 0.02, (E, H)))
    b = moe_data.bf16(rng.normal(0, 0.02, E))
    say("route", T, fp32)
    logits, idx, w = gpu.route(dev(x, torch), dev(W, torch), dev(b, torch), k, logits_fp32=fp32)
    ref_l = orc.router(x, W, b, logits_fp32=fp32)
    got_l = host(logits)
    lf_ref = ref_l if fp32 else orc.bf16_to_f32(ref_l)
    ridx, rw = orc.topk_softmax(lf_ref, k)
    if T <= MM_MIN_T or H % 32:
        if fp32:
            assert np.array_equal(got_l.view(np.uint32), ref_l.view(np.uint32))
        else:
            assert np.array_equal(got_l, ref_l)
        assert np.array_equal(host(idx), ridx)
        assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    else:
        exact, bound = _mm_router_bound(orc, x, W, b)
        lg = got_l.astype(np.float64) if fp32 else orc.bf16_to_f32(got_l).astype(np.float64)
        # bf16 logits: one rounding of the fp32 value on top
        tol = bound if fp32 else bound + np.abs(exact) * 2.0 ** -8 + 2.0 ** -133
        err = np.abs(lg - exact)
        say("mm router logits", dict(max_err=float(err.max()), max_err_over_bound=float((err / tol).max())))
        assert np.all(err <= tol)
        # selection and weights: exactly the top-k softmax of the GPU's logits
        gidx, gw = orc.topk_softmax(lg.astype(np.float32), k)
        assert np.array_equal(host(idx), gidx)
        assert np.array_equal(host(w).view(np.uint32), gw.view(np.uint32))
        # against the oracle's tree logits: a token's selection can differ
        # only if its k-th and (k+1)-th exact logits lie within twice the bound
        srt = np.sort(exact, axis=1)[:, ::-1]
        tie = (srt[:, k - 1] - srt[:, k]) <= 2 * tol.max(axis=1)
        diff = np.any(host(idx) != ridx, axis=1)
        say("mm router vs tree selection", dict(tokens=T, near_ties=int(tie.sum()), differing=int(diff.sum())))
        assert not np.any(diff & ~tie)
        same = ~diff
        if fp32:  # config 1's bar: weights within 1e-6
            assert np.max(np.abs(host(w)[same] - rw[same]), initial=0.0) <= 1e-6
        else:  # bf16 logits: where the selected logits are the same bits, so are the weights
            sel_eq = np.all(np.take_along_axis(got_l, ridx, 1) == np.take_along_axis(ref_l, ridx, 1), axis=1) & same
            assert np.array_equal(host(w)[sel_eq].view(np.uint32), rw[sel_eq].view(np.uint32))
        # deterministic, and independent of the other tokens: the first
        # tokens alone give the same bits
        logits2, idx2, _ = gpu.route(dev(x, torch), dev(W, torch), dev(b, torch), k, logits_fp32=fp32)
        assert np.array_equal(host(logits2).view(np.uint8), got_l.view(np.uint8))
        h = max(MM_MIN_T + 1, T // 2)
        logits3, _, _ = gpu.route(dev(x[:h], torch), dev(W, torch), dev(b, torch), k, logits_fp32=fp32)
        assert np.array_equal(host(logits3).view(np.uint8), got_l[:h].view(np.uint8))
    # repeat: nothing carries over between calls
    logits2, idx2, w2 = gpu.route(dev(x, torch), dev(W, torch), dev(b, torch), k, logits_fp32=fp32)
    assert np.array_equal(host(idx2), host(idx))


@pytest.mark.parametrize("T,fp32", [(4096, True), (300, False), (64, False)])
def test_route_graph_replays(gpu, orc, torch_mod, T, fp32):
    """The router's launches (the matrix-core logits and the sixteen-lane
    top-k above 64 tokens, the tree below) captured in one hipGraph: every
    replay, with eager work and synchronisations between the replays and
    new inputs copied into the captured buffers, gives the eager call's
    bits."""
    torch = torch_mod
    E, H, k = 128, 2880, 4
    rng = np.random.default_rng(11 + T)
    xs = [moe_data.bf16(rng.normal(0, 1, (T, H))) for _ in range(3)]
    W = dev(moe_data.bf16(rng.normal(0, 0.02, (E, H))), torch)
    b = dev(moe_data.bf16(rng.normal(0, 0.02, E)), torch)
    x = dev(xs[0], torch)
    dt = torch.float32 if fp32 else torch.bfloat16
    logits = torch.empty((T, E), dtype=dt, device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    scratch = gpu.route_scratch(T, E, k)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gpu.route(x, W, b, k, logits_fp32=fp32, out=(logits, idx, w), scratch=scratch, stream=s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        gpu.route(x, W, b, k, logits_fp32=fp32, out=(logits, idx, w), scratch=scratch, stream=s)
    for rep, xn in enumerate(xs * 2):
        x.copy_(dev(xn, torch))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (host(logits).copy(), host(idx).copy(), host(w).copy())
        el, ei, ew = gpu.route(dev(xn, torch), W, b, k, logits_fp32=fp32)  # eager, fresh buffers
        torch.cuda.synchronize()
        assert np.array_equal(got[0].view(np.uint8), host(el).view(np.uint8)), rep
        assert np.array_equal(got[1], host(ei)), rep
        assert np.array_equal(got[2].view(np.uint32), host(ew).view(np.uint32)), rep
    del graph


@pytest.mark.parametrize("T,fp32,E,H", [(130, True, 128, 2880), (100, False, 20, 512), (9, True, 128, 2880),
                                         (300, False, 128, 2880)])
def test_route_null_bias_and_unaligned_logits(gpu, orc, torch_mod, T, fp32, E, H):
    """A null router bias is a zero bias: the same bits as an explicit zero
    bias on both logit orders (and, on the tree, the oracle's bits).  Logits
    one element off the 16- / 8-byte store alignment get the same bits, and
    the top-k over them (the one-wave-a-token kernel then) the same
    selections and weights."""
    torch = torch_mod
    k = 4
    rng = np.random.default_rng(3 * T + E)
    x = moe_data.bf16(rng.normal(0, 1, (T, H)))
    W = moe_data.bf16(rng.normal(0, 0.02, (E, H)))
    zero = np.zeros(E, np.uint16)
    xd, Wd = dev(x, torch), dev(W, torch)
    l0, i0, w0 = gpu.route(xd, Wd, None, k, logits_fp32=fp32)
    l1, i1, w1 = gpu.route(xd, Wd, dev(zero, torch), k, logits_fp32=fp32)
    assert np.array_equal(host(l0).view(np.uint8), host(l1).view(np.uint8))
    assert np.array_equal(host(i0), host(i1))
    assert np.array_equal(host(w0).view(np.uint32), host(w1).view(np.uint32))
    if T <= MM_MIN_T:
        ref = orc.router(x, W, zero, logits_fp32=fp32)
        assert np.array_equal(host(l0).view(np.uint8), ref.view(np.uint8))
    # logits at an odd element offset inside a larger buffer
    dt = torch.float32 if fp32 else torch.bfloat16
    buf = torch.full((T * E + 1,), 7.0, dtype=dt, device="cuda")
    lu = buf[1:].view(T, E)
    iu = torch.empty((T, k), dtype=torch.int32, device="cuda")
    wu = torch.empty((T, k), dtype=torch.float32, device="cuda")
    gpu.route(xd, Wd, None, k, logits_fp32=fp32, out=(lu, iu, wu))
    torch.cuda.synchronize()
    assert float(buf[0].item()) == 7.0
    assert np.array_equal(host(lu).view(np.uint8), host(l0).view(np.uint8))
    assert np.array_equal(host(iu), host(i0))
    assert np.array_equal(host(wu).view(np.uint32), host(w0).view(np.uint32))


# 6144 x 4 slots: the largest plan whose indices are staged in LDS; 8192 x 4:
# the plan reads them from global memory
@pytest.mark.parametrize("T,k,E", [(1, 4, 128), (64, 4, 128), (4096, 4, 128), (6144, 4, 128), (8192, 4, 128),
                                   (33, 2, 8), (7, 8, 32)])
def test_permute_plan(gpu, orc, torch_mod, T, k, E):
    torch = torch_mod
    rng = np.random.default_rng(T + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    if T > 8:
        idx[::9, -1] = -1
    p = gpu.permute_plan(dev(idx, torch), E)
    r = orc.plan(idx, E)
    for n in ("counts", "offsets", "gather_map"):
        assert np.array_equal(host(p[n]), r[n]), n
    nv = int((idx >= 0).sum())
    assert np.array_equal(host(p["perm_token"])[:nv], r["perm_token"][:nv])
    n = int(host(p["n_active"])[0])
    assert n == r["n_active"] and np.array_equal(host(p["active"])[:n], r["active"])
    # scatter of the reference (moe_permute.cu:84-124) from the same map
    H = 64
    x = moe_data.bf16(rng.normal(0, 1, (T, H)))
    perm = host(gpu.scatter_tokens(dev(x, torch), p["gather_map"], k))
    gm = r["gather_map"]
    for s in range(T * k):
        if gm[s] >= 0:
            assert np.array_equal(perm[gm[s]], x[s // k])


@pytest.mark.parametrize("N,K,M", [(5760, 2880, 1), (2880, 2880, 9), (128, 64, 3), (64, 96, 17), (192, 192, 8)])
def test_dense_mxfp4_gemv(gpu, orc, torch_mod, N, K, M):
    torch = torch_mod
    rng = np.random.default_rng(N * 7 + K + M)
    x = moe_data.bf16(rng.normal(0, 1, (M, K)))
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = rng.integers(119, 124, (N, K // 32), dtype=np.uint8)
    bias = moe_data.bf16(rng.normal(0, 0.5, N))
    nib, sc = gpu.pack_tiled(dev(packed, torch), dev(scales, torch), N, K)
    y = host(gpu.mxfp4_gemv(dev(x, torch), nib, sc, dev(bias, torch), N, K))
    ref = orc.mxfp4_gemv(x, packed, scales, bias, N, K)
    assert_bf16_parity(y, ref, f"gemv {N}x{K} M={M}")


def test_combine(gpu, orc, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(9)
    T, k, H = 37, 4, 2880
    y = moe_data.bf16(rng.normal(0, 40, (T * k, H)))
    res = moe_data.bf16(rng.normal(0, 1, (T, H)))
    gm = rng.permutation(T * k).astype(np.int32)
    gm[::11] = -1
    w = rng.dirichlet(np.ones(k), T).astype(np.float32)
    out = host(gpu.combine(dev(y, torch), dev(gm, torch), dev(w, torch), dev(res, torch), T, H, k))
    assert np.array_equal(out, orc.combine(y, gm, w, res, T, k, H))
    out = host(gpu.combine(dev(y, torch), dev(gm, torch), dev(w, torch), None, T, H, k))
    assert np.array_equal(out, orc.combine(y, gm, w, None, T, k, H))


# ---------------------------------------------------------------------------
# the fused layer
# ---------------------------------------------------------------------------
class DeviceLayer:
    """A layer on device copies of the oracle's weights.  exact: the exact
    decode kernels (bit-identical to the oracle) instead of the matrix-core
    ones; tiled: share another layer's tiled weights."""
    def __init__(self, gpu, torch, w, E, k, H, I, max_tokens, norm_w=None, via_tables=True, exact=True,
                 tiled=None, t=None):
        self.torch = torch
        self.t = t if t is not None else {n: dev(w[n], torch) for n in w if w[n] is not None}
        cfg = gpu.default_config(E, max_tokens, decode_exact=exact)
        cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, k
        self.norm = dev(norm_w, torch) if norm_w is not None else None
        self.layer = gpu.MoELayer()
        if tiled is not None:
            self.tiled = tiled
            self.layer.init(cfg, 0, self.t["router_w"], self.t.get("router_b"), self.t.get("w1_bias"),
                            self.t.get("w2_bias"), moe_norm_weight=self.norm, tiled=tiled)
        elif via_tables:
            mlp1 = ([self.t["w1_packed"][e] for e in range(E)], [self.t["w1_scales"][e] for e in range(E)])
            mlp2 = ([self.t["w2_packed"][e] for e in range(E)], [self.t["w2_scales"][e] for e in range(E)])
            self.layer.init(cfg, 0, self.t["router_w"], self.t.get("router_b"), self.t.get("w1_bias"),
                            self.t.get("w2_bias"), moe_norm_weight=self.norm, mlp1=mlp1, mlp2=mlp2)
        else:
            n1, s1 = gpu.tiled_size(2 * I, H)
            n2, s2 = gpu.tiled_size(H, I)
            tiled = [torch.empty(E * n, dtype=torch.uint8, device="cuda") for n in (n1, s1, n2, s2)]
            for e in range(E):
                gpu.pack_tiled(self.t["w1_packed"][e], self.t["w1_scales"][e], 2 * I, H,
                               tiled[0][e * n1:(e + 1) * n1], tiled[1][e * s1:(e + 1) * s1])
                gpu.pack_tiled(self.t["w2_packed"][e], self.t["w2_scales"][e], H, I,
                               tiled[2][e * n2:(e + 1) * n2], tiled[3][e * s2:(e + 1) * s2])
            self.tiled = tiled
            self.layer.init(cfg, 0, self.t["router_w"], self.t.get("router_b"), self.t.get("w1_bias"),
                            self.t.get("w2_bias"), moe_norm_weight=self.norm, tiled=tiled)


def _trace_arrays(gpu, layer, T, k, E, H, I, torch, with_gate_up):
    tr = layer.trace()
    S = T * k
    rd = lambda p, n, dt: gpu.copy_device_to_tensor(p, n * np.dtype(dt).itemsize).cpu().numpy().view(dt)  # noqa
    out = dict(idx=rd(tr.expert_indices, S, np.int32).reshape(T, k), w=rd(tr.expert_weights, S, np.float32).reshape(T, k),
               gather_map=rd(tr.gather_map, S, np.int32), act=rd(tr.act, S * I, np.uint16).reshape(S, I),
               y=rd(tr.expert_out, S * H, np.uint16).reshape(S, H))
    if with_gate_up:
        out["gate_up"] = rd(tr.gate_up, S * 2 * I, np.uint16).reshape(S, 2 * I)
    return out


@pytest.mark.parametrize("T", [1, 5, 8, 9, 40])
@pytest.mark.parametrize("bias", ["random", "none"])
def test_layer_small_with_intermediates(gpu, orc, torch_mod, T, bias):
    torch = torch_mod
    E, k, H, I = 8, 2, 128, 128
    w = moe_data.make_layer(20 + T, E, H, I, bias=bias)
    x, res = moe_data.make_tokens(20 + T, T, H)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=64)
    L.layer.set_trace_gate_up(True)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    torch.cuda.synchronize()
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    got = _trace_arrays(gpu, L.layer, T, k, E, H, I, torch, True)
    assert np.array_equal(got["idx"], tr["idx"])
    assert np.array_equal(got["w"].view(np.uint32), tr["w"].view(np.uint32))
    assert np.array_equal(got["gather_map"], tr["gather_map"])
    assert np.array_equal(got["gate_up"], tr["gate_up"])
    assert np.array_equal(got["act"], tr["act"])
    assert np.array_equal(got["y"], tr["y"])
    assert_bf16_parity(out, ref, f"layer small T={T} bias={bias}")


@pytest.mark.parametrize("T,E,H,I", [(40, 8, 320, 96), (20, 8, 640, 160), (64, 128, 128, 224), (3, 8, 320, 96)])
def test_layer_odd_part_counts(gpu, orc, torch_mod, T, E, H, I):
    """Products whose K splits into an odd number of parts (gate_up K = H:
    320 -> 5 parts of 2 blocks, 640 -> 5 of 4; down K = I: 96 -> 3 parts of
    1 block, 160 -> 5 of 1).  The exact kernels' work-group then has 64 x
    parts threads, which is not a multiple of the two-tile row group (128
    rows) taken above 64 slots, so the part-sum reduction's later passes emit
    rows other than the one each thread's prefetched bias belongs to.  The
    output tiles (N / 64 = 3, 5 or 7) leave the last row group one tile
    short.  I = 224 (7 blocks, one part: 64 threads) with up to 128 active
    experts also has more task records than threads.  T = 3 (12 slots, one
    tile per group) is the control.  Gate_up values, activations, expert
    outputs and the layer output are bit-exact."""
    torch = torch_mod
    k = 4
    w = moe_data.make_layer(70 + T + H, E, H, I, bias="random")
    x, res = moe_data.make_tokens(70 + T + H, T, H)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=64)
    L.layer.set_trace_gate_up(True)
    say("odd part counts", T, E, H, I)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    torch.cuda.synchronize()
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    got = _trace_arrays(gpu, L.layer, T, k, E, H, I, torch, True)
    assert np.array_equal(got["idx"], tr["idx"])
    assert np.array_equal(got["gate_up"], tr["gate_up"])
    assert np.array_equal(got["act"], tr["act"])
    assert np.array_equal(got["y"], tr["y"])
    assert_bf16_parity(out, ref, f"odd part counts T={T} H={H} I={I}")


def test_layer_golden_fixture(gpu, torch_mod):
    """The committed fixture (tests/golden/moe_tiny.npz) reproduced on the GPU."""
    torch = torch_mod
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "moe_tiny.npz"))
    E, k, H, I = (int(v) for v in d["shape"])
    w = {n: d[n] for n in ("router_w", "router_b", "w1_packed", "w1_scales", "w1_bias", "w2_packed",
                           "w2_scales", "w2_bias")}
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=8, via_tables=False)
    out = host(L.layer.forward_prenormed(dev(d["x"], torch), dev(d["residual"], torch)))
    assert_bf16_parity(out, d["out"], "golden fixture")


def test_layer_forward_with_rmsnorm(gpu, orc, torch_mod):
    torch = torch_mod
    E, k, H, I, T = 16, 4, 192, 128, 11
    w = moe_data.make_layer(31, E, H, I)
    x, _ = moe_data.make_tokens(31, T, H)
    norm_w = moe_data.bf16(np.random.default_rng(31).normal(1.0, 0.1, H))
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=16, norm_w=norm_w)
    out = host(L.layer.forward(dev(x, torch)))
    normed = orc.rmsnorm(x, norm_w)
    ref = orc.moe_forward(w, normed, x, E, k, H, I)
    assert_bf16_parity(out, ref, "forward (rmsnorm + moe)")


@pytest.mark.parametrize("T,H", [(1, 2880), (37, 192), (300, 4104)])
def test_fused_residual_rmsnorm_stage(gpu, orc, torch_mod, T, H):
    """fused_residual_rmsnorm_forward: normed and the bf16 sum bit-exact."""
    torch = torch_mod
    rng = np.random.default_rng(T + H)
    r = moe_data.bf16(rng.normal(0, 1, (T, H)))
    d = moe_data.bf16(rng.normal(0, 0.5, (T, H)))
    w = moe_data.bf16(rng.normal(1, 0.1, H))
    say("residual rmsnorm", T, H)
    normed, s = gpu.fused_residual_rmsnorm(dev(r, torch), dev(d, torch), dev(w, torch), 1e-5)
    rn, rs = orc.residual_rmsnorm(r, d, w, 1e-5)
    assert np.array_equal(host(normed), rn)
    assert np.array_equal(host(s), rs)


@pytest.mark.parametrize("T,E,H,I", [(1, 16, 192, 128), (4, 16, 192, 128), (5, 16, 192, 128), (8, 16, 192, 128),
                                     (9, 16, 192, 128), (64, 16, 192, 128), (100, 16, 192, 128),
                                     (2, 32, 2880, 2880), (8, 32, 2880, 2880), (64, 32, 2880, 2880),
                                     (9, 6, 128, 128), (40, 30, 192, 128)])
def test_layer_forward_residual(gpu, orc, torch_mod, T, E, H, I):
    """forward_residual = fused_residual_rmsnorm_forward + forward_prenormed:
    the new residual bit-exact, the router's logits bit-exact (the norm
    inside the router's launch up to 4 tokens, its own launch above), the
    layer output through the exact decode path bit-exact."""
    torch = torch_mod
    k = 4
    w = moe_data.make_layer(60 + T, E, H, I)
    res, delta = moe_data.make_tokens(60 + T, T, H)
    norm_w = moe_data.bf16(np.random.default_rng(60 + T).normal(1.0, 0.1, H))
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=128, norm_w=norm_w)
    say("forward_residual", T, E, H)
    res_out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    out = host(L.layer.forward_residual(dev(res, torch), dev(delta, torch), residual_out=res_out))
    torch.cuda.synchronize()
    rn, rs = orc.residual_rmsnorm(res, delta, norm_w)
    assert np.array_equal(host(res_out), rs)
    tr = L.layer.trace()
    logits = gpu.copy_device_to_tensor(tr.logits, T * E * 2).cpu().numpy().view(np.uint16).reshape(T, E)
    assert np.array_equal(logits, orc.router(rn, w["router_w"], w["router_b"], logits_fp32=False))
    ref = orc.moe_forward(w, rn, rs, E, k, H, I)
    assert_bf16_parity(out, ref, f"forward_residual T={T} E={E}")
    # without residual_out the sum stays in the layer's scratch; same output
    out2 = host(L.layer.forward_residual(dev(res, torch), dev(delta, torch)))
    assert np.array_equal(out2, out)
    if T == 1 and H == 192:
        # residual_out on the residual or the delta (in place, or one row
        # shifted) is refused before any launch; out in place on residual_out
        # is fine and gives the same result
        dr, dd = dev(res, torch), dev(delta, torch)
        for alias in (dr, dd):
            with pytest.raises(ValueError, match="residual_out overlaps"):
                L.layer.forward_residual(dr, dd, residual_out=alias)
        wide = torch.empty((T + 1, H), dtype=torch.bfloat16, device="cuda")
        wide[:T].copy_(dr)
        with pytest.raises(ValueError, match="residual_out overlaps"):
            gpu.check(gpu.lib.gptoss_moe_layer_forward_residual(
                L.layer._h, wide.data_ptr(), dd.data_ptr(), wide.data_ptr() + 2 * 8, res_out.data_ptr(), T,
                torch.cuda.current_stream().cuda_stream))
        same = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        assert np.array_equal(host(L.layer.forward_residual(dr, dd, residual_out=same, out=same)), out)


def test_layer_edge_cases(gpu, orc, torch_mod):
    torch = torch_mod
    E, k, H, I = 8, 8, 64, 64
    w = moe_data.make_layer(41, E, H, I)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=4)
    x, res = moe_data.make_tokens(41, 4, H)
    # T = 0 is a no-op; T above max_tokens is rejected
    L.layer.forward_prenormed(dev(x, torch)[:0], None, out=torch.empty((0, H), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        L.layer.forward_prenormed(dev(moe_data.make_tokens(1, 5, H)[0], torch), None)
    # k == E: every expert active for every token; residual NULL
    out = host(L.layer.forward_prenormed(dev(x, torch), None))
    ref = orc.moe_forward(w, x, None, E, k, H, I)
    assert_bf16_parity(out, ref, "k == E, no residual")


def test_layer_graph_replay(gpu, orc, torch_mod):
    """A forward captured in a HIP graph, replayed with new inputs, matches
    eager results bit for bit on every replay (no memset in the captured work)."""
    torch = torch_mod
    E, k, H, I, T = 16, 4, 128, 128, 8
    w = moe_data.make_layer(51, E, H, I)
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=T)
    xs = [moe_data.make_tokens(60 + i, T, H) for i in range(4)]
    eager = []
    for x, res in xs:
        eager.append(host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch))))
    sx = dev(xs[0][0], torch)
    sr = dev(xs[0][1], torch)
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
    assert np.array_equal(eager[1], orc.moe_forward(w, xs[1][0], xs[1][1], E, k, H, I))


# ---------------------------------------------------------------------------
# GPT-OSS shapes (BASELINE configs 0 and 2)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def gptoss120(gpu, torch_mod):
    say("building GPT-OSS-120B-shaped layer (E=128, H=I=2880)")
    E, k, H, I = 128, 4, 2880, 2880
    w = moe_data.make_layer(1234, E, H, I, bias="zero")
    L = DeviceLayer(gpu, torch_mod, w, E, k, H, I, max_tokens=64, via_tables=True)
    torch_mod.cuda.synchronize()
    return w, L


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_gptoss120b_decode_parity(gpu, orc, torch_mod, gptoss120, T):
    torch = torch_mod
    w, L = gptoss120
    E, k, H, I = 128, 4, 2880, 2880
    x, res = moe_data.make_tokens(500 + T, T, H)
    say("120B decode T", T)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    ref, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    got = _trace_arrays(gpu, L.layer, T, k, E, H, I, torch, False)
    assert np.array_equal(got["idx"], tr["idx"])
    assert np.array_equal(got["w"].view(np.uint32), tr["w"].view(np.uint32))
    assert np.array_equal(got["y"], tr["y"])
    assert_bf16_parity(out, ref, f"120B decode T={T}")
    out2 = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    assert np.array_equal(out, out2)  # run-to-run deterministic


def test_gptoss20b_decode_parity(gpu, orc, torch_mod):
    """BASELINE config 0 shape: E=32, k=4, H=I=2880, T=1, zero (non-null) biases."""
    torch = torch_mod
    E, k, H, I, T = 32, 4, 2880, 2880, 1
    w = moe_data.make_layer(77, E, H, I, bias="zero")
    L = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=1, via_tables=False)
    x, res = moe_data.make_tokens(77, T, H)
    out = host(L.layer.forward_prenormed(dev(x, torch), dev(res, torch)))
    ref = orc.moe_forward(w, x, res, E, k, H, I)
    assert_bf16_parity(out, ref, "20B decode T=1")


# ---------------------------------------------------------------------------
# The reference's C++ operator (gptoss::moe_layer_*, moe_layer.cu:1556-1615)
# through libgptoss_moe_compat.so, called by its mangled names as the
# reference's engine would link them.
# ---------------------------------------------------------------------------
_SHIM = {
    "create": "_ZN6gptoss16moe_layer_createEv",
    "destroy": "_ZN6gptoss17moe_layer_destroyEPNS_8MoELayerE",
    "init": "_ZN6gptoss14moe_layer_initEPNS_8MoELayerEiiiPNS_6EPCommEPKNS_12CublasHandleES6_P12ihipStream_tS8_"
            "PK14__hip_bfloat16SB_SB_SB_SB_PNS_11MXFP4WeightESD_PS9_SE_PiPfSF_SE_SF_SF_SF_SF_SE_SE_SE_SE_SE_SE_SE_"
            "SE_SE_P8ncclComm",
    "forward": "_ZN6gptoss17moe_layer_forwardEPNS_8MoELayerEPK14__hip_bfloat16PS2_iP12ihipStream_t",
    "prenormed": "_ZN6gptoss27moe_layer_forward_prenormedEPNS_8MoELayerEPK14__hip_bfloat16S4_PS2_iP12ihipStream_t",
    "max_tokens": "_ZN6gptoss20moe_layer_max_tokensEv",
}


def test_cpp_operator_shim_matches_c_abi(gpu, torch_mod, gptoss120):
    """The reference engine's calls, by mangled name, at its token counts:
    decode (1), a decode batch (64) and a prefill chunk (4096, above the
    old 256-token default; the shim's layers share one per-device workspace
    for the engine's 8192).  moe_layer_forward (RMSNorm inside) and
    moe_layer_forward_prenormed, bit for bit against the C ABI with the
    shim's configuration.  Two shim layers are created so that the second
    shares the first's workspace."""
    import ctypes
    torch = torch_mod
    w, L = gptoss120
    E, H = 128, 2880
    norm_w = moe_data.bf16(np.random.default_rng(5).normal(1.0, 0.1, H))
    # the operator shim runs the default configuration (matrix-core decode, grouped prefill)
    Lmc = DeviceLayer(gpu, torch, w, E, 4, H, H, max_tokens=4096, exact=False, t=L.t, via_tables=True,
                      norm_w=norm_w)
    lib = ctypes.CDLL(os.path.join(os.path.dirname(gpu.LIB_PATH), "libgptoss_moe_compat.so"))
    create = getattr(lib, _SHIM["create"])
    create.restype = ctypes.c_void_p
    destroy = getattr(lib, _SHIM["destroy"])
    destroy.argtypes = [ctypes.c_void_p]
    init = getattr(lib, _SHIM["init"])
    init.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 12 + \
        [ctypes.c_void_p] * 19 + [ctypes.c_void_p]
    init.restype = None
    fwd = getattr(lib, _SHIM["forward"])
    fwd.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p]
    fwd.restype = None
    pre = getattr(lib, _SHIM["prenormed"])
    pre.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p]
    pre.restype = None
    assert getattr(lib, _SHIM["max_tokens"])() == 8192

    class MXFP4Weight(ctypes.Structure):  # moe_layer.cu:585-589
        _fields_ = [("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("num_elements", ctypes.c_int)]

    mlp1 = (MXFP4Weight * E)()
    mlp2 = (MXFP4Weight * E)()
    for e in range(E):
        mlp1[e] = MXFP4Weight(L.t["w1_packed"][e].data_ptr(), L.t["w1_scales"][e].data_ptr(), 2 * H * H)
        mlp2[e] = MXFP4Weight(L.t["w2_packed"][e].data_ptr(), L.t["w2_scales"][e].data_ptr(), H * H)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    layers = []
    try:
        for _ in range(2):
            layer = create()
            assert layer
            layers.append(layer)
            # layer/device/gpu ids, EPComm, two BLAS handles, two streams, then the weights
            init(layer, 0, 0, 0, None, None, None, None, None, ptr(Lmc.norm), ptr(L.t["router_w"]),
                 ptr(L.t.get("router_b")), ptr(L.t.get("w1_bias")), ptr(L.t.get("w2_bias")),
                 ctypes.cast(mlp1, ctypes.c_void_p), ctypes.cast(mlp2, ctypes.c_void_p), *([None] * 19), None)
        stream = torch.cuda.current_stream().cuda_stream
        for T in (1, 64, 4096):
            x, res = moe_data.make_tokens(900 + T, T, H)
            dx, dr = dev(x, torch), dev(res, torch)
            for li, layer in enumerate(layers):
                say("C++ operator shim, layer", li, "T", T)
                out = torch.empty_like(dx)
                pre(layer, dx.data_ptr(), dr.data_ptr(), out.data_ptr(), T, stream)
                torch.cuda.synchronize()
                assert np.array_equal(host(out), host(Lmc.layer.forward_prenormed(dx, dr))), ("prenormed", T)
                out2 = torch.empty_like(dx)
                fwd(layer, dx.data_ptr(), out2.data_ptr(), T, stream)
                torch.cuda.synchronize()
                assert np.array_equal(host(out2), host(Lmc.layer.forward(dx))), ("forward", T)
    finally:
        for layer in layers:
            destroy(layer)
        Lmc.layer.destroy()


def test_shared_workspace(gpu, orc, torch_mod):
    """Layers of different shapes on one caller workspace, run one after
    another on one stream (the reference engine's scratch sharing), give the
    results of layers with their own scratch, at decode sizes and at a prefill
    size whose grouped kernels use the workspace's tile queue; a workspace
    that is too small or misaligned is refused."""
    torch = torch_mod
    shapes = [(16, 4, 128, 128), (8, 2, 192, 64)]
    own, shared = [], []
    need = 0
    cfgs = []
    for E, k, H, I in shapes:
        cfg = gpu.default_config(E, 160)
        cfg.hidden_size, cfg.intermediate_size, cfg.top_k = H, I, k
        cfgs.append(cfg)
        need = max(need, gpu.workspace_bytes(cfg))
    ws = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
    for (E, k, H, I), cfg in zip(shapes, cfgs):
        w = moe_data.make_layer(70 + E, E, H, I, bias="random")
        a = DeviceLayer(gpu, torch, w, E, k, H, I, max_tokens=160, exact=False, via_tables=False)
        b = gpu.MoELayer().init(cfg, 0, a.t["router_w"], a.t.get("router_b"), a.t.get("w1_bias"),
                                a.t.get("w2_bias"), tiled=a.tiled, workspace=ws[:need])
        own.append((a, w, H))
        shared.append(b)
    bad = gpu.MoELayer()
    with pytest.raises(ValueError, match="workspace of"):
        bad.init(cfgs[0], 0, own[0][0].t["router_w"], tiled=own[0][0].tiled, workspace=ws[:64])
    with pytest.raises(ValueError, match="aligned"):
        bad.init(cfgs[0], 0, own[0][0].t["router_w"], tiled=own[0][0].tiled, workspace=ws[8:8 + need])
    bad.destroy()
    for T in (1, 8, 150, 3):
        for (a, w, H), b in zip(own, shared):
            say("shared workspace T", T, "H", H)
            x, res = moe_data.make_tokens(80 + T, T, H)
            dx, dr = dev(x, torch), dev(res, torch)
            want = host(a.layer.forward_prenormed(dx, dr))
            assert np.array_equal(host(b.forward_prenormed(dx, dr)), want), (T, H)
    for b in shared:
        b.destroy()
    for a, _, _ in own:
        a.layer.destroy()
