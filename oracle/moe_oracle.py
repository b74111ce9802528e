"""ctypes binding of the CPU oracle (oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The product library never
imports this module.  All arrays are numpy; bf16 values are uint16 bit
patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# GPTOSS_ORACLE_LIB: another build of the oracle (tests/sanitize's instrumented copy)
LIB_PATH = os.environ.get("GPTOSS_ORACLE_LIB") or os.path.join(HERE, "libmoe_oracle.so")

_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


class OrcCfg(ctypes.Structure):
    _fields_ = [("H", _I), ("E", _I), ("k", _I), ("I", _I), ("alpha", _F), ("limit", _F),
                ("logits_fp32", _I), ("topk_variant", _I), ("expert_order", _I)]


class OrcWeights(ctypes.Structure):
    _fields_ = [("router_w", _P), ("router_b", _P), ("w1_packed", _P), ("w1_scales", _P),
                ("w1_bias", _P), ("w2_packed", _P), ("w2_scales", _P), ("w2_bias", _P)]


class OrcTrace(ctypes.Structure):
    _fields_ = [("logits_bf16", _P), ("logits_f32", _P), ("idx", _P), ("w", _P),
                ("gather_map", _P), ("gate_up", _P), ("act", _P), ("y", _P)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = _F
        L.orc_f32_to_bf16.argtypes = [_F]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_e2m1.argtypes = [_I]
        L.orc_e2m1.restype = _F
        L.orc_e8m0.argtypes = [_I]
        L.orc_e8m0.restype = _F
        L.orc_expf.argtypes = [_F]
        L.orc_expf.restype = _F
        L.orc_swiglu.argtypes = [_F, _F, _F, _F]
        L.orc_swiglu.restype = _F
        L.orc_parts.argtypes = [_I]
        L.orc_parts.restype = _I
        L.orc_set_exp_mode.argtypes = [_I]
        L.orc_router.argtypes = [_P, _P, _P, _I, _I, _I, _P, _P]
        L.orc_topk_softmax.argtypes = [_P, _I, _I, _I, _I, _P, _P]
        L.orc_topk_softmax.restype = _I
        L.orc_plan.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P, _P]
        L.orc_plan.restype = _I
        L.orc_mxfp4_gemv.argtypes = [_P, _P, _I, _P, _P, _P, _I, _I, _P]
        L.orc_mxfp4_gemv_refkernel.argtypes = [_P, _I, _P, _P, _P, _I, _I, _P]
        L.orc_mxfp4_dequant.argtypes = [_P, _P, _I, _I, _P]
        L.orc_swiglu_rows.argtypes = [_P, _I, _I, _F, _F, _P]
        L.orc_combine.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P]
        L.orc_moe_forward.argtypes = [ctypes.POINTER(OrcCfg), ctypes.POINTER(OrcWeights), _P, _P, _I,
                                      _P, ctypes.POINTER(OrcTrace), _I]
        L.orc_moe_forward_routed.argtypes = [ctypes.POINTER(OrcCfg), ctypes.POINTER(OrcWeights), _P, _P, _I,
                                             _P, _P, _P, ctypes.POINTER(OrcTrace), _I]
        L.orc_moe_forward_routed.restype = None
        L.orc_rmsnorm.argtypes = [_P, _P, _I, _I, _F, _P]
        L.orc_residual_rmsnorm.argtypes = [_P, _P, _P, _I, _I, _F, _P, _P]
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# --------------------------------------------------------------------------
# numpy bf16 helpers (same rounding as orc_f32_to_bf16)
# --------------------------------------------------------------------------
def f32_to_bf16(a) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    qn = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, qn, r)


def bf16_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------
# wrappers
# --------------------------------------------------------------------------
def router(x, W, b, logits_fp32=False):
    T, H = x.shape
    E = W.shape[0]
    if logits_fp32:
        out = np.empty((T, E), np.float32)
        lib().orc_router(_ptr(x), _ptr(W), _ptr(b), T, E, H, None, _ptr(out))
    else:
        out = np.empty((T, E), np.uint16)
        lib().orc_router(_ptr(x), _ptr(W), _ptr(b), T, E, H, _ptr(out), None)
    return out


def topk_softmax(logits_f32, k, variant=0):
    logits_f32 = np.ascontiguousarray(logits_f32, np.float32)
    T, E = logits_f32.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    rc = lib().orc_topk_softmax(_ptr(logits_f32), T, E, k, variant, _ptr(idx), _ptr(w))
    if rc != 0:
        raise ValueError(f"orc_topk_softmax: unsupported k={k}")
    return idx, w


def plan(idx, E):
    idx = np.ascontiguousarray(idx, np.int32)
    T, k = idx.shape
    S = T * k
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    gmap = np.empty(S, np.int32)
    ptok = np.full(S, -1, np.int32)
    active = np.full(E, -1, np.int32)
    n = lib().orc_plan(_ptr(idx), T, k, E, _ptr(counts), _ptr(offsets), _ptr(gmap), _ptr(ptok), _ptr(active))
    return dict(counts=counts, offsets=offsets, gather_map=gmap, perm_token=ptok, active=active[:n], n_active=n)


def mxfp4_gemv(x, packed, scales, bias, N, K, xf=None):
    M = x.shape[0] if x is not None else xf.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().orc_mxfp4_gemv(_ptr(x), _ptr(xf), M, _ptr(packed), _ptr(scales), _ptr(bias), N, K, _ptr(y))
    return y


def mxfp4_gemv_refkernel(x, packed, scales, bias, N, K):
    M = x.shape[0]
    y = np.empty((M, N), np.uint16)
    lib().orc_mxfp4_gemv_refkernel(_ptr(x), M, _ptr(packed), _ptr(scales), _ptr(bias), N, K, _ptr(y))
    return y


def mxfp4_dequant(packed, scales, N, K):
    out = np.empty((N, K), np.uint16)
    lib().orc_mxfp4_dequant(_ptr(packed), _ptr(scales), N, K, _ptr(out))
    return out


def swiglu_rows(gate_up, I, alpha=1.702, limit=7.0):
    M = gate_up.shape[0]
    out = np.empty((M, I), np.uint16)
    lib().orc_swiglu_rows(_ptr(gate_up), M, I, alpha, limit, _ptr(out))
    return out


def combine(y, gather_map, w, residual, T, k, H):
    out = np.empty((T, H), np.uint16)
    lib().orc_combine(_ptr(y), _ptr(gather_map), _ptr(w), _ptr(residual), T, k, H, _ptr(out))
    return out


def rmsnorm(x, w, eps=1e-5):
    T, H = x.shape
    out = np.empty((T, H), np.uint16)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), T, H, eps, _ptr(out))
    return out


def residual_rmsnorm(r, d, w, eps=1e-5):
    """fused_residual_rmsnorm_forward: returns (normed, sum_out) bf16 bits."""
    T, H = r.shape
    normed = np.empty((T, H), np.uint16)
    sum_out = np.empty((T, H), np.uint16)
    lib().orc_residual_rmsnorm(_ptr(r), _ptr(d), _ptr(w), T, H, eps, _ptr(normed), _ptr(sum_out))
    return normed, sum_out


def set_exp_mode(mode: int) -> None:
    lib().orc_set_exp_mode(mode)


def moe_forward(weights: dict, x, residual, E, k, H, I, alpha=1.702, limit=7.0, logits_fp32=False,
                topk_variant=0, nthreads=0, trace=False, order=0):
    """Whole MoE layer.  weights: dict with router_w, router_b, w1_packed,
    w1_scales, w1_bias, w2_packed, w2_scales, w2_bias (numpy, expert-major).
    order 0: this build's canonical expert order; 1: the reference's own
    dispatch, orders and rounding points (orc_cfg.expert_order)."""
    T = x.shape[0]
    cfg = OrcCfg(H, E, k, I, alpha, limit, 1 if logits_fp32 else 0, topk_variant, order)
    wt = OrcWeights(*[_ptr(weights.get(n)) for n in
                      ("router_w", "router_b", "w1_packed", "w1_scales", "w1_bias",
                       "w2_packed", "w2_scales", "w2_bias")])
    out = np.empty((T, H), np.uint16)
    tr = None
    bufs = {}
    if trace:
        S = T * k
        bufs = dict(logits_bf16=np.empty((T, E), np.uint16), logits_f32=np.empty((T, E), np.float32),
                    idx=np.empty((T, k), np.int32), w=np.empty((T, k), np.float32),
                    gather_map=np.empty(S, np.int32), gate_up=np.empty((S, 2 * I), np.uint16),
                    act=np.empty((S, I), np.uint16), y=np.empty((S, H), np.uint16))
        tr = OrcTrace(*[_ptr(bufs[n]) for n in ("logits_bf16", "logits_f32", "idx", "w", "gather_map",
                                                  "gate_up", "act", "y")])
    lib().orc_moe_forward(ctypes.byref(cfg), ctypes.byref(wt), _ptr(x), _ptr(residual), T, _ptr(out),
                          ctypes.byref(tr) if tr is not None else None, nthreads)
    if trace:
        return out, bufs
    return out


def moe_forward_routed(weights: dict, x, residual, idx, w, E, k, H, I, alpha=1.702, limit=7.0, nthreads=0,
                       trace=False, order=0):
    """The layer's expert half with the routing given (idx int32 [T][k],
    w float32 [T][k]); weights as moe_forward (router entries unused)."""
    T = x.shape[0]
    cfg = OrcCfg(H, E, k, I, alpha, limit, 0, 0, order)
    wt = OrcWeights(*[_ptr(weights.get(n)) for n in
                      ("router_w", "router_b", "w1_packed", "w1_scales", "w1_bias",
                       "w2_packed", "w2_scales", "w2_bias")])
    idx = np.ascontiguousarray(idx, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty((T, H), np.uint16)
    tr = None
    bufs = {}
    if trace:
        S = T * k
        bufs = dict(gather_map=np.empty(S, np.int32), gate_up=np.empty((S, 2 * I), np.uint16),
                    act=np.empty((S, I), np.uint16), y=np.empty((S, H), np.uint16))
        tr = OrcTrace(None, None, None, None, *[_ptr(bufs[n]) for n in ("gather_map", "gate_up", "act", "y")])
    lib().orc_moe_forward_routed(ctypes.byref(cfg), ctypes.byref(wt), _ptr(x), _ptr(residual), T, _ptr(idx),
                                 _ptr(w), _ptr(out), ctypes.byref(tr) if tr is not None else None, nthreads)
    if trace:
        return out, bufs
    return out
