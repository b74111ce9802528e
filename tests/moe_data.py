"""Seeded synthetic MoE inputs with the BASELINE value distributions.

MXFP4 nibble bytes uniform over 0..255 (codes uniform over the 16 e2m1
values), e8m0 scales uniform over {119..123} (2^-8..2^-4), router weight and
bias bf16(N(0, 0.02)), activations and residual bf16(N(0, 1)) from
independent streams, expert biases zero-filled (but passed, non-null) unless
`bias="random"`.  Arrays are numpy, expert-major, in the reference layout
(packed [N][K/2], low nibble = even k; scales [N][K/32])."""
from __future__ import annotations

import numpy as np

import moe_oracle as orc


def bf16(a) -> np.ndarray:
    return orc.f32_to_bf16(np.asarray(a, dtype=np.float32))


def make_layer(seed: int, E: int, H: int, I: int, bias: str = "zero") -> dict:
    rng = np.random.default_rng(seed)
    w = dict(
        router_w=bf16(rng.normal(0.0, 0.02, (E, H))),
        router_b=bf16(rng.normal(0.0, 0.02, E)),
        w1_packed=rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8),
        w1_scales=rng.integers(119, 124, (E, 2 * I, H // 32), dtype=np.uint8),
        w2_packed=rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8),
        w2_scales=rng.integers(119, 124, (E, H, I // 32), dtype=np.uint8),
    )
    if bias == "zero":
        w["w1_bias"] = np.zeros((E, 2 * I), np.uint16)
        w["w2_bias"] = np.zeros((E, H), np.uint16)
    elif bias == "random":
        w["w1_bias"] = bf16(rng.normal(0.0, 0.5, (E, 2 * I)))
        w["w2_bias"] = bf16(rng.normal(0.0, 0.5, (E, H)))
    else:
        w["w1_bias"] = None
        w["w2_bias"] = None
    return w


def make_tokens(seed: int, T: int, H: int):
    rx = np.random.default_rng([seed, 1])
    rr = np.random.default_rng([seed, 2])
    return bf16(rx.normal(0.0, 1.0, (T, H))), bf16(rr.normal(0.0, 1.0, (T, H)))


def ulp_bf16(v) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (for scale-aware error reports)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def compare_bf16(got, ref) -> dict:
    """max-abs, mean-rel and mismatch count of two bf16 bit arrays."""
    g = orc.bf16_to_f32(got).astype(np.float64)
    r = orc.bf16_to_f32(ref).astype(np.float64)
    d = np.abs(g - r)
    denom = np.maximum(np.abs(r), 1e-6)
    return dict(max_abs=float(d.max(initial=0.0)), mean_rel=float((d / denom).mean()) if d.size else 0.0,
                mismatches=int((np.asarray(got) != np.asarray(ref)).sum()),
                max_ulps=float((d / ulp_bf16(r)).max(initial=0.0)))


def zipf_routing(seed: int, T: int, E: int, k: int, s: float = 1.1):
    """Skewed routing (BASELINE prefill config): expert popularity
    p(e) ~ (pi(e)+1)^-s for a seeded permutation pi, k distinct experts per
    token drawn without replacement (Gumbel top-k, in draw order), weights =
    softmax of k sorted N(0,1) draws, descending.  Returns int32 [T][k] and
    float32 [T][k]."""
    rng = np.random.default_rng([seed, 3])
    pi = rng.permutation(E)
    logp = -s * np.log(pi + 1.0)
    keys = logp[None, :] + rng.gumbel(size=(T, E))
    top = np.argpartition(-keys, k - 1, axis=1)[:, :k]
    order = np.argsort(-np.take_along_axis(keys, top, axis=1), axis=1, kind="stable")
    idx = np.take_along_axis(top, order, axis=1).astype(np.int32)
    z = -np.sort(-rng.normal(size=(T, k)), axis=1)
    w = np.exp(z - z[:, :1])
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


def mfma_stats(got, ref) -> dict:
    """Agreement of a matrix-core (reordered fp32 sum) result with the
    canonical one: NaN positions, max-abs, mean-rel, the fraction of bf16
    values that differ and the largest difference in bf16 ulps of the
    reference (one rounding step = 1)."""
    g = orc.bf16_to_f32(got).astype(np.float64)
    r = orc.bf16_to_f32(ref).astype(np.float64)
    nan_ok = bool(np.array_equal(np.isnan(g), np.isnan(r)))
    f = np.isfinite(r) & np.isfinite(g)
    inf_ok = bool(np.array_equal(g[~np.isnan(r) & ~f], r[~np.isnan(r) & ~f]))
    d = np.abs(g[f] - r[f])
    denom = np.maximum(np.abs(r[f]), 1e-6)
    return dict(nan_ok=nan_ok, inf_ok=inf_ok, max_abs=float(d.max(initial=0.0)),
                mean_rel=float((d / denom).mean()) if d.size else 0.0,
                mismatch_frac=float((np.asarray(got) != np.asarray(ref)).mean()) if d.size else 0.0,
                over_abs_frac=float((d > 2e-2).mean()) if d.size else 0.0,
                max_ulps=float((d / ulp_bf16(r[f])).max(initial=0.0)),
                # largest difference beyond one bf16 step of the reference
                max_excess=float((d - ulp_bf16(r[f])).max(initial=0.0)),
                # norm-wise relative error ||got - ref|| / ||ref||
                norm_rel=float(np.sqrt((d * d).sum() / max((r[f] ** 2).sum(), 1e-300))) if d.size else 0.0,
                # largest difference in bf16 steps at the largest magnitude
                # of its row (token): a reordered sum moves an output by a
                # few steps of the values it adds, whatever the output's size
                row_steps=_row_steps(g, r))


def _row_steps(g, r) -> float:
    if g.ndim != 2 or g.size == 0:
        return 0.0
    f = np.isfinite(r) & np.isfinite(g)
    rowmax = np.where(f, np.abs(r), 0.0).max(axis=1, keepdims=True)
    d = np.where(f, np.abs(g - r), 0.0)
    return float((d / ulp_bf16(rowmax)).max(initial=0.0))
