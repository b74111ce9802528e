"""GPU: the decode paths against the reference's own arithmetic.

The oracle's expert_order = 1 restates, per active expert, the path the
reference takes and that path's summation order and rounding points: the
one-token fast path through fused_mxfp4_gemv (moe_layer.cu:1028-1098,
fused_mxfp4_gemv.cu:93-183), batches of one-token experts through the fused
GEMV with the bias inside, one-token experts of mixed batches through
gemv_bf16 over the dequantised weights (moe_layer.cu:1409-1411), and several-
token experts at hipBLASLt's rounding points with the canonical order standing
in for hipBLASLt's own (not vendored, so not restated).

Both decode paths of this build (the matrix-core default and the exact
kernels) are measured against it at BASELINE config 0 (E=32, T=1) and config
2 (E=128, B=1 and B=8).  Asserted: expert indices and routing weights bit-exact
and mean-rel <= 1e-3; no output further than one bf16
step of its token's largest output, and at most 2 % of outputs beyond 2e-2
(measured <= 1.2 %).  At these output magnitudes (|out| up to ~140, one bf16
step 0.125-0.5) the outputs beyond 2e-2 are those whose bf16 rounding lands
one step away in another summation order, so max-abs itself is reported, not
asserted.
"""
import numpy as np
import pytest

import moe_data
from test_gpu_parity import DeviceLayer, _trace_arrays, dev, host, say

pytestmark = pytest.mark.gpu

MEAN_REL_TOL = 1e-3
ROW_STEPS = 1.0
OVER_FRAC = 2e-2
H = I = 2880
K_TOP = 4


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _layers(gpu, torch, E, seed):
    say(f"building E={E} GPT-OSS-shaped layer (exact and matrix-core decode, shared tiled weights)")
    w = moe_data.make_layer(seed, E, H, I, bias="zero")
    ex = DeviceLayer(gpu, torch, w, E, K_TOP, H, I, max_tokens=8, via_tables=False, exact=True)
    mc = DeviceLayer(gpu, torch, w, E, K_TOP, H, I, max_tokens=8, exact=False, tiled=ex.tiled, t=ex.t)
    return w, ex, mc


@pytest.fixture(scope="module")
def layer20(gpu, torch_mod):
    return _layers(gpu, torch_mod, 32, 77)


@pytest.fixture(scope="module")
def layer120(gpu, torch_mod):
    return _layers(gpu, torch_mod, 128, 1234)


def _stats(got, ref):
    c = moe_data.mfma_stats(got, ref)
    return {k: c[k] for k in ("max_abs", "mean_rel", "mismatch_frac", "over_abs_frac", "max_ulps", "row_steps")}


@pytest.mark.parametrize("E,T", [(32, 1), (128, 1), (128, 8)])
def test_decode_vs_reference_order(gpu, orc, torch_mod, layer20, layer120, E, T):
    torch = torch_mod
    w, ex, mc = layer20 if E == 32 else layer120
    x, res = moe_data.make_tokens(700 + E + T, T, H)
    say(f"reference-order oracle, E={E} T={T}")
    ref_r, tr_r = orc.moe_forward(w, x, res, E, K_TOP, H, I, trace=True, order=1)
    ref_c = orc.moe_forward(w, x, res, E, K_TOP, H, I, order=0)
    say(f"E={E} T={T}: canonical vs reference order", _stats(ref_c, ref_r))
    dx, dr = dev(x, torch), dev(res, torch)
    for name, L in (("exact", ex), ("matrix-core", mc)):
        out = host(L.layer.forward_prenormed(dx, dr))
        torch.cuda.synchronize()
        got = _trace_arrays(gpu, L.layer, T, K_TOP, E, H, I, torch, False)
        assert np.array_equal(got["idx"], tr_r["idx"]), name
        assert np.array_equal(got["w"].view(np.uint32), tr_r["w"].view(np.uint32)), name
        s_r, s_c = _stats(out, ref_r), _stats(out, ref_c)
        say(f"E={E} T={T} {name} path vs reference order", s_r)
        say(f"E={E} T={T} {name} path vs canonical order", s_c)
        assert s_r["mean_rel"] <= MEAN_REL_TOL, (name, s_r)
        # whole-step moves only: at most one bf16 step of the token's largest
        # output, on a bounded fraction of outputs (measured <= 1.2 %)
        assert s_r["row_steps"] <= ROW_STEPS, (name, s_r)
        assert s_r["over_abs_frac"] <= OVER_FRAC, (name, s_r)
        if name == "exact":
            assert s_c["mismatch_frac"] == 0.0, s_c  # the exact kernels are the canonical order
