"""CPU tests that pin the oracle (oracle/moe_oracle.c) before it is trusted.

Each oracle function is checked against something other than its own
formula: the reference's known-answer vector (BUGFIX_REPORT.md:108-121), the
e2m1 / e8m0 definitions evaluated independently, torch's bf16 rounding, fp64
mathematics with error bounds, brute force on small inputs, structural
invariants, and hand-computed cancellation cases that only the reference's
summation trees produce.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import moe_data

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------
# MXFP4 decode
# ---------------------------------------------------------------------------
def test_bugfix_report_vector(orc):
    """BUGFIX_REPORT.md:108-121: bytes aa b8 11 a8 with scale 122 decode to
    [-0.03125, -0.03125, -0.0, -0.046875, 0.015625, 0.015625, -0.0, -0.03125]."""
    with open(os.path.join(GOLDEN, "bugfix_mxfp4_vector.json")) as f:
        g = json.load(f)
    packed = np.zeros((1, 16), np.uint8)
    packed[0, :4] = [int(b, 16) for b in g["packed_bytes"]]
    scales = np.array([[g["scale"]]], np.uint8)
    out = orc.bf16_to_f32(orc.mxfp4_dequant(packed, scales, 1, 32))[0, :8]
    exp = np.array(g["expected"], np.float32)
    assert np.array_equal(out, exp)
    assert np.array_equal(np.signbit(out), np.signbit(exp))  # -0.0 entries keep their sign


def _e2m1_spec(code):
    """OCP MX e2m1: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0."""
    s = -1.0 if code & 8 else 1.0
    e = (code >> 1) & 3
    m = code & 1
    mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1.0 + m / 2.0)
    return s * mag


def test_e2m1_e8m0_exhaustive(orc):
    L = orc.lib()
    for c in range(16):
        v = L.orc_e2m1(c)
        assert v == _e2m1_spec(c) and math.copysign(1, v) == math.copysign(1, _e2m1_spec(c))
    for s in range(256):
        v = L.orc_e8m0(s)
        if s == 0:
            assert v == 0.0                 # register rule: code << 23 (fused_mxfp4_gemv.cu:42-44)
        elif s == 255:
            assert math.isinf(v)
        else:
            assert v == 2.0 ** (s - 127)
    # the product of every code and scale (all 4096 pairs) through dequant
    packed = np.zeros((256, 16), np.uint8)
    packed[:, :8] = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    out = orc.bf16_to_f32(orc.mxfp4_dequant(packed, scales, 256, 32)).astype(np.float64)
    for s in range(1, 255):
        for c in range(16):
            exp = _e2m1_spec(c) * 2.0 ** (s - 127)
            with np.errstate(over="ignore"):
                exp32 = float(orc.bf16_to_f32(orc.f32_to_bf16(np.array([exp], np.float32)))[0])
            assert out[s, c] == exp32, (s, c)


def test_bf16_rounding_matches_torch(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e-38, 2000).astype(np.float32),
        (rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -3.4e38], np.float32),
    ])
    vals = vals[~np.isnan(vals)]
    ours = orc.f32_to_bf16(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    # C entry point agrees with the numpy helper
    L = orc.lib()
    for v in vals[:2000]:
        assert L.orc_f32_to_bf16(float(v)) == orc.f32_to_bf16(np.float32(v))[()]


# ---------------------------------------------------------------------------
# exp and SwiGLU
# ---------------------------------------------------------------------------
def _ulp32(x):
    return np.spacing(np.abs(np.float32(x))).astype(np.float64)


def test_expf_accuracy(orc):
    L = orc.lib()
    xs = np.concatenate([np.linspace(-87.0, 88.0, 40001), np.random.default_rng(1).uniform(-20, 20, 20000),
                         np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    worst = 0.0
    for x in xs:
        got = L.orc_expf(float(x))
        exact = math.exp(float(x))
        worst = max(worst, abs(got - exact) / float(_ulp32(exact)))
    assert worst <= 2.0, worst
    assert L.orc_expf(0.0) == 1.0
    assert L.orc_expf(float("inf")) == float("inf")
    assert L.orc_expf(float("-inf")) == 0.0
    assert math.isnan(L.orc_expf(float("nan")))
    assert L.orc_expf(89.0) == float("inf")
    assert L.orc_expf(-104.0) == 0.0


def test_swiglu_closed_form(orc):
    L = orc.lib()
    alpha, limit = 1.702, 7.0
    g = np.linspace(-30, 30, 601).astype(np.float32)
    u = np.linspace(-12, 12, 49).astype(np.float32)
    for gv in g:
        for uv in u[::6]:
            got = L.orc_swiglu(float(gv), float(uv), alpha, limit)
            gc = min(float(gv), limit)
            uc = min(max(float(uv), -limit), limit)
            arg = float(np.float32(-np.float32(alpha)) * np.float32(gc))  # the fp32 product of swiglu.cu:27
            exact = (uc + 1.0) * gc / (1.0 + math.exp(arg))
            assert abs(got - exact) <= 8 * float(_ulp32(exact)) + 1e-30, (gv, uv, got, exact)
    # clamps: gate only from above, up symmetric
    assert L.orc_swiglu(100.0, 0.0, alpha, limit) == L.orc_swiglu(7.0, 0.0, alpha, limit)
    assert L.orc_swiglu(1.0, 100.0, alpha, limit) == L.orc_swiglu(1.0, 7.0, alpha, limit)
    assert L.orc_swiglu(1.0, -100.0, alpha, limit) == L.orc_swiglu(1.0, -7.0, alpha, limit)
    assert L.orc_swiglu(-100.0, 0.0, alpha, limit) != L.orc_swiglu(-7.0, 0.0, alpha, limit)


# ---------------------------------------------------------------------------
# router (gemv_bf16 tree)
# ---------------------------------------------------------------------------
def test_router_vs_fp64(orc):
    T, E, H = 16, 32, 2880
    rng = np.random.default_rng(2)
    x = moe_data.bf16(rng.normal(0, 1, (T, H)))
    W = moe_data.bf16(rng.normal(0, 0.02, (E, H)))
    b = moe_data.bf16(rng.normal(0, 0.02, E))
    lf = orc.router(x, W, b, logits_fp32=True).astype(np.float64)
    xd = orc.bf16_to_f32(x).astype(np.float64)
    Wd = orc.bf16_to_f32(W).astype(np.float64)
    exact = xd @ Wd.T + orc.bf16_to_f32(b).astype(np.float64)
    bound = (H * 2.0 ** -24) * (np.abs(xd) @ np.abs(Wd).T) * 1.01 + 1e-7
    assert np.all(np.abs(lf - exact) <= bound)
    lb = orc.router(x, W, b, logits_fp32=False)
    assert np.array_equal(lb, orc.f32_to_bf16(lf.astype(np.float32)))
    # transposed / swapped operands would break the bound for a non-symmetric case
    assert not np.allclose(lf[:, :16], (xd @ Wd.T)[:, :16][::-1], atol=1e-3)


def _norm_fp64(s64, w64, eps):
    inv = 1.0 / np.sqrt(np.mean(s64 * s64, axis=1, keepdims=True) + eps)
    return s64 * inv * w64


def _within_one_bf16_ulp(got_bits, exact, orc):
    got = orc.bf16_to_f32(got_bits).astype(np.float64)
    # one bf16 ulp of the exact value (8 significant bits), floor for tiny values
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -120))) - 7)
    return np.all(np.abs(got - exact) <= ulp)


def test_rmsnorm_vs_fp64(orc):
    """rmsnorm.cu:47-83: out = x / sqrt(mean(x^2) + eps) * w.  fp32 with the
    gemv tree is within one bf16 ulp of the fp64 value; a dropped eps, a sum
    instead of a mean or a missing weight fails."""
    T, H, eps = 6, 2880, 1e-5
    rng = np.random.default_rng(31)
    x = moe_data.bf16(rng.normal(0, 1, (T, H)))
    x[5] = moe_data.bf16(rng.normal(0, 1e-3, H))  # small row: eps matters at 1e-5 relative
    w = moe_data.bf16(rng.normal(1, 0.1, H))
    out = orc.rmsnorm(x, w, eps)
    exact = _norm_fp64(orc.bf16_to_f32(x).astype(np.float64), orc.bf16_to_f32(w).astype(np.float64), eps)
    assert _within_one_bf16_ulp(out, exact, orc)
    assert not _within_one_bf16_ulp(out, _norm_fp64(orc.bf16_to_f32(x).astype(np.float64),
                                                   orc.bf16_to_f32(w).astype(np.float64), 1e-2), orc)


def test_residual_rmsnorm(orc):
    """fused_residual_rmsnorm_forward (rmsnorm.cu:224-337): sum_out = bf16(r + d)
    (fp32 add), normed from the fp32 sum.  With d = 0 it is rmsnorm of r bit
    for bit; otherwise within one bf16 ulp of fp64; symmetric in r and d."""
    T, H, eps = 5, 2880, 1e-5
    rng = np.random.default_rng(32)
    r = moe_data.bf16(rng.normal(0, 1, (T, H)))
    d = moe_data.bf16(rng.normal(0, 0.5, (T, H)))
    w = moe_data.bf16(rng.normal(1, 0.1, H))
    normed, sum_out = orc.residual_rmsnorm(r, d, w, eps)
    s32 = orc.bf16_to_f32(r) + orc.bf16_to_f32(d)  # fp32 sum, as the kernel
    ref_sum = torch.from_numpy(s32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(sum_out, ref_sum)
    s64 = orc.bf16_to_f32(r).astype(np.float64) + orc.bf16_to_f32(d).astype(np.float64)
    assert _within_one_bf16_ulp(normed, _norm_fp64(s64, orc.bf16_to_f32(w).astype(np.float64), eps), orc)
    n2, s2 = orc.residual_rmsnorm(d, r, w, eps)
    assert np.array_equal(n2, normed) and np.array_equal(s2, sum_out)
    z = np.zeros_like(r)
    n0, s0 = orc.residual_rmsnorm(r, z, w, eps)
    assert np.array_equal(n0, orc.rmsnorm(r, w, eps))
    assert np.array_equal(s0, r)


def test_router_tree_cancellation(orc):
    """Only the gemv_bf16_kernel tree gives 1.0 here: thread 0 holds 1,
    thread 1 holds 2^24, thread 16 holds -2^24.  The xor-16 butterfly step adds
    1 + (-2^24) first (exact), the xor-1 step then adds 2^24: result 1.  A
    sequential sum would round 1 + 2^24 to 2^24 and return 0."""
    H = 2880
    x = np.zeros((1, H), np.float32)
    W = np.zeros((1, H), np.float32)
    x[0, 0], W[0, 0] = 1.0, 1.0                  # chunk 0 -> thread 0
    x[0, 8], W[0, 8] = 2.0 ** 12, 2.0 ** 12      # chunk 1 -> thread 1
    x[0, 128], W[0, 128] = -(2.0 ** 12), 2.0 ** 12  # chunk 16 -> thread 16
    lf = orc.router(orc.f32_to_bf16(x), orc.f32_to_bf16(W), None, logits_fp32=True)
    assert lf[0, 0] == 1.0
    # a second wave (threads 64..127): its sum is added after wave 0's
    x2 = np.zeros((1, H), np.float32)
    x2[0, 0], x2[0, 8 * 64] = 2.0 ** 24, 1.0
    W2 = np.zeros((1, H), np.float32)
    W2[0, 0], W2[0, 8 * 64] = 1.0, 1.0
    lf2 = orc.router(orc.f32_to_bf16(x2), orc.f32_to_bf16(W2), None, logits_fp32=True)
    assert lf2[0, 0] == 2.0 ** 24  # (2^24) + 1 rounds to even


# ---------------------------------------------------------------------------
# top-k softmax
# ---------------------------------------------------------------------------
def _brute_topk(lg, k):
    v = np.where(np.isfinite(lg) & (lg > -np.finfo(np.float32).max), lg, -np.inf)
    out_i, out_v = [], []
    for row in v:
        order = sorted(range(len(row)), key=lambda e: (-row[e], e))
        sel = [e for e in order if np.isfinite(row[e])][:k]
        vals = [row[e] for e in sel]
        while len(sel) < k:
            sel.append(-1)
            vals.append(-np.inf)
        out_i.append(sel)
        out_v.append(vals)
    return np.array(out_i, np.int32), np.array(out_v, np.float64)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_topk_brute_force(orc, k):
    rng = np.random.default_rng(10 + k)
    T, E = 300, 128
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    lg[:100] = np.round(lg[:100] * 4) / 4            # many exact ties
    lg[100:120] = 0.0
    lg[100:120, ::3] = -0.0                           # +0 and -0 are a tie
    lg[120:140, ::5] = np.nan                         # sanitised away
    lg[140:160, ::7] = np.inf
    lg[160:170, :] = np.nan                           # fully degenerate
    lg[170:180, :] = -np.inf
    lg[170:180, :2] = 1.0                             # only two visible experts
    idx, w = orc.topk_softmax(lg, k)
    bi, bv = _brute_topk(lg, k)
    degenerate = np.all(bi == -1, axis=1)
    assert np.array_equal(idx[~degenerate], bi[~degenerate])
    assert np.array_equal(idx[degenerate], np.tile(np.arange(k, dtype=np.int32), (int(degenerate.sum()), 1)))
    assert np.allclose(w[degenerate], 1.0 / k)
    ok = ~degenerate
    ex = np.where(bi >= 0, np.exp(bv - bv[:, :1]), 0.0)
    ref_w = ex / ex.sum(axis=1, keepdims=True)
    assert np.max(np.abs(w[ok] - ref_w[ok])) <= 1e-6
    assert np.all(np.abs(w[ok].sum(axis=1) - 1.0) <= 1e-6)
    assert np.all(np.diff(w[ok], axis=1) <= 0)
    assert np.all(w[ok][bi[ok] == -1] == 0.0)


def test_topk_variants_sum_order(orc):
    """v1 sums ((e0+e1)+e2)+e3, v2 (e0+e2)+(e1+e3): both within 1 ulp."""
    rng = np.random.default_rng(5)
    lg = rng.normal(0, 1, (2000, 128)).astype(np.float32)
    i1, w1 = orc.topk_softmax(lg, 4, variant=1)
    i2, w2 = orc.topk_softmax(lg, 4, variant=2)
    assert np.array_equal(i1, i2)
    assert np.max(np.abs(w1 - w2)) <= 2 * np.finfo(np.float32).eps
    assert np.any(w1 != w2)  # the two orders really differ somewhere
    # variant 0 follows the launcher (T <= 8 -> v1, else v2)
    i0, w0 = orc.topk_softmax(lg[:8], 4, variant=0)
    assert np.array_equal(w0, w1[:8])
    i0, w0 = orc.topk_softmax(lg[:9], 4, variant=0)
    assert np.array_equal(w0, w2[:9])


# ---------------------------------------------------------------------------
# dispatch plan
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T,k,E", [(1, 4, 128), (64, 4, 128), (4096, 4, 128), (33, 2, 8), (7, 8, 32)])
def test_plan_invariants(orc, T, k, E):
    rng = np.random.default_rng(T * 31 + k)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    if T > 8:
        idx[::9, -1] = -1                                 # dropped slots
    p = orc.plan(idx, E)
    flat = idx.reshape(-1)
    valid = flat >= 0
    assert np.array_equal(p["counts"], np.bincount(flat[valid], minlength=E))
    assert p["offsets"][0] == 0 and np.array_equal(np.diff(p["offsets"]), p["counts"])
    gm = p["gather_map"]
    assert np.all(gm[~valid] == -1)
    assert np.array_equal(np.sort(gm[valid]), np.arange(valid.sum()))  # bijection
    for e in range(E):
        slots = np.nonzero(flat == e)[0]
        assert np.array_equal(gm[slots], p["offsets"][e] + np.arange(len(slots)))  # stable, in range
    assert np.array_equal(p["perm_token"][gm[valid]], np.nonzero(valid)[0] // k)
    assert np.array_equal(p["active"], np.nonzero(p["counts"])[0])


# ---------------------------------------------------------------------------
# MXFP4 products
# ---------------------------------------------------------------------------
def _dequant_f64(packed, scales, N, K, orc):
    return orc.bf16_to_f32(orc.mxfp4_dequant(packed, scales, N, K)).astype(np.float64)


@pytest.mark.parametrize("N,K", [(64, 64), (128, 2880), (64, 96)])
def test_mxfp4_gemv_vs_fp64(orc, N, K):
    rng = np.random.default_rng(N + K)
    M = 3
    x = moe_data.bf16(rng.normal(0, 1, (M, K)))
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = rng.integers(119, 124, (N, K // 32), dtype=np.uint8)
    bias = moe_data.bf16(rng.normal(0, 0.5, N))
    y = orc.bf16_to_f32(orc.mxfp4_gemv(x, packed, scales, bias, N, K)).astype(np.float64)
    Wd = _dequant_f64(packed, scales, N, K, orc)
    xd = orc.bf16_to_f32(x).astype(np.float64)
    exact = xd @ Wd.T + orc.bf16_to_f32(bias)
    bound = K * 2.0 ** -24 * (np.abs(xd) @ np.abs(Wd).T) * 1.01 + moe_data.ulp_bf16(exact) * 0.5 + 1e-30
    assert np.all(np.abs(y - exact) <= bound)
    # the reference kernel's order lands within the same bound and differs by at most 1 bf16 ulp
    yr = orc.bf16_to_f32(orc.mxfp4_gemv_refkernel(x, packed, scales, bias, N, K)).astype(np.float64)
    assert np.all(np.abs(yr - exact) <= bound)
    assert np.all(np.abs(yr - y) <= moe_data.ulp_bf16(exact) * 1.01)


def test_mxfp4_canonical_part_order(orc):
    """Canonical dot: K=192 (6 blocks) -> 6 parts added in part order.
    Part 0 = 2^24, part 1 = 1, part 2 = 1, part 3 = -2^24: the sequential part
    sum is 0 (2^24 + 1 rounds back to 2^24 twice, then -2^24); a pairwise
    tree ((p0+p1)+(p2+p3)) would give 1."""
    K, N = 192, 64
    assert orc.lib().orc_parts(K) == 6
    x = np.zeros((1, K), np.float32)
    # weights: code 2 (= 1.0) at chosen k, scale 127 (= 1.0)
    packed = np.zeros((N, K // 2), np.uint8)
    scales = np.full((N, K // 32), 127, np.uint8)
    for k_, xv in [(0, 2.0 ** 24), (32, 1.0), (64, 1.0), (96, -(2.0 ** 24))]:
        x[0, k_] = xv
        packed[:, k_ // 2] = 0x02  # low nibble (even k) = code 2 -> 1.0
    y = orc.bf16_to_f32(orc.mxfp4_gemv(orc.f32_to_bf16(x), packed, scales, None, N, K))
    assert np.all(y == 0.0)  # sequential part order: the two +1 are absorbed by 2^24


def _unit_weights(N, K, ks):
    """MXFP4 rows with weight 1.0 (code 2, scale 127) at the elements ks, 0 elsewhere."""
    packed = np.zeros((N, K // 2), np.uint8)
    for k_ in ks:
        packed[:, k_ // 2] |= np.uint8(0x02 << (4 * (k_ & 1)))
    return packed, np.full((N, K // 32), 127, np.uint8)


@pytest.mark.parametrize("case", [
    # (element: x value) -> expected output, derived by hand from
    # fused_mxfp4_gemv.cu:93-183 at K = 2880 (360 uint32 chunks of 8 elements;
    # thread tid takes chunks tid and tid + 256; warp = tid // 64).
    # Warps are added in order from 0: ((2^24 + 1) + 1) - 2^24 = 0 (a pairwise
    # tree over the warps would give 2).
    ({0: 2.0 ** 24, 512: 1.0, 1024: 1.0, 1536: -(2.0 ** 24)}, 0.0),
    # Inside a warp the xor butterfly pairs thread l with l + 32 first:
    # (2^24 - 2^24) + (1 + 1) = 2 (an ascending sum over threads gives 1).
    ({0: 2.0 ** 24, 8: 1.0, 256: -(2.0 ** 24), 264: 1.0}, 2.0),
    # Thread 0 adds its chunks 0 and 256 first: (2^24 + 1) rounds to 2^24,
    # then thread 32's -2^24 cancels it: 0 (a split of chunk 256 to another
    # thread would leave the 1).
    ({0: 2.0 ** 24, 2048: 1.0, 256: -(2.0 ** 24)}, 0.0),
    # Inside a chunk, products are added in pairs before the chunk sum:
    # (2^24 + 1) -> 2^24, (1 - 2^24) exact, sum 1 (an element chain gives 0).
    ({0: 2.0 ** 24, 1: 1.0, 2: 1.0, 3: -(2.0 ** 24)}, 1.0),
])
def test_mxfp4_refkernel_order(orc, case):
    """The restatement of the reference's fused MXFP4 GEMV order, pinned by
    cancellation cases whose results a different order changes."""
    vals, want = case
    N, K = 64, 2880
    x = np.zeros((1, K), np.float32)
    for k_, v in vals.items():
        x[0, k_] = v
    packed, scales = _unit_weights(N, K, vals)
    y = orc.bf16_to_f32(orc.mxfp4_gemv_refkernel(orc.f32_to_bf16(x), packed, scales, None, N, K))
    assert np.all(y == want), (vals, y[:4])


# ---------------------------------------------------------------------------
# combine
# ---------------------------------------------------------------------------
def test_combine_one_hot_and_linear(orc):
    rng = np.random.default_rng(7)
    T, k, H = 5, 4, 64
    y = moe_data.bf16(rng.normal(0, 30, (T * k, H)))
    res = moe_data.bf16(rng.normal(0, 1, (T, H)))
    gm = np.arange(T * k, dtype=np.int32)
    w = np.zeros((T, k), np.float32)
    w[:, 1] = 1.0
    out = orc.combine(y, gm, w, res, T, k, H)
    expect = orc.f32_to_bf16(orc.bf16_to_f32(y[1::k]) + orc.bf16_to_f32(res))
    assert np.array_equal(out, expect)
    w = rng.dirichlet(np.ones(k), T).astype(np.float32)
    out = orc.bf16_to_f32(orc.combine(y, gm, w, res, T, k, H)).astype(np.float64)
    exact = np.einsum("tk,tkh->th", w.astype(np.float64),
                      orc.bf16_to_f32(y).reshape(T, k, H).astype(np.float64)) + orc.bf16_to_f32(res)
    assert np.all(np.abs(out - exact) <= moe_data.ulp_bf16(exact) * 0.51 + 1e-4)
    gm2 = gm.copy()
    gm2[::3] = -1  # dropped slots contribute nothing
    out2 = orc.bf16_to_f32(orc.combine(y, gm2, w, None, T, k, H)).astype(np.float64)
    w2 = w.reshape(-1).copy()
    w2[::3] = 0
    exact2 = np.einsum("tk,tkh->th", w2.reshape(T, k).astype(np.float64),
                       orc.bf16_to_f32(y).reshape(T, k, H).astype(np.float64))
    assert np.all(np.abs(out2 - exact2) <= moe_data.ulp_bf16(exact2) * 0.51 + 1e-4)


# ---------------------------------------------------------------------------
# whole layer against an fp64 restatement with the same rounding points
# ---------------------------------------------------------------------------
def _layer_fp64(w, x, res, E, k, H, I, orc, fast_one=False):
    """The layer in fp64 with bf16 roundings at the reference's points.
    fast_one: the one-token fast path's points (moe_layer.cu:1028-1098):
    bf16 gate_up before its bias, bf16 down product before its bias."""
    xd = orc.bf16_to_f32(x).astype(np.float64)
    logits = xd @ orc.bf16_to_f32(w["router_w"]).astype(np.float64).T + orc.bf16_to_f32(w["router_b"])
    logits_b = orc.bf16_to_f32(orc.f32_to_bf16(logits.astype(np.float32))).astype(np.float64)
    T = x.shape[0]
    out = np.zeros((T, H))

    def rnd(v):
        return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)

    for t in range(T):
        order = sorted(range(E), key=lambda e: (-logits_b[t, e], e))[:k]
        v = logits_b[t, order]
        p = np.exp(v - v[0])
        p /= p.sum()
        acc = np.zeros(H)
        for s, e in enumerate(order):
            W1 = _dequant_f64(w["w1_packed"][e], w["w1_scales"][e], 2 * I, H, orc)
            b1 = orc.bf16_to_f32(w["w1_bias"][e]).astype(np.float64)
            if fast_one:
                gu = rnd(xd[t] @ W1.T) + b1
            else:
                gu = rnd(xd[t] @ W1.T + b1)
            g = np.minimum(gu[0::2], 7.0)
            u = np.clip(gu[1::2], -7.0, 7.0)
            a = (u + 1) * g / (1 + np.exp(-1.702 * g))
            a = orc.bf16_to_f32(orc.f32_to_bf16(a.astype(np.float32))).astype(np.float64)
            W2 = _dequant_f64(w["w2_packed"][e], w["w2_scales"][e], H, I, orc)
            b2 = orc.bf16_to_f32(w["w2_bias"][e]).astype(np.float64)
            yy = rnd(rnd(a @ W2.T) + b2) if fast_one else rnd(a @ W2.T + b2)
            acc += p[s] * yy
        out[t] = acc + orc.bf16_to_f32(res[t])
    return orc.bf16_to_f32(orc.f32_to_bf16(out.astype(np.float32))).astype(np.float64)


def test_layer_tiny_vs_fp64(orc):
    E, k, H, I, T = 8, 2, 64, 64, 6
    w = moe_data.make_layer(3, E, H, I, bias="random")
    x, res = moe_data.make_tokens(3, T, H)
    out = orc.bf16_to_f32(orc.moe_forward(w, x, res, E, k, H, I)).astype(np.float64)
    ref = _layer_fp64(w, x, res, E, k, H, I, orc)
    rel = np.abs(out - ref) / np.maximum(np.abs(ref), 1e-3)
    assert rel.mean() <= 1e-3
    assert np.all(np.abs(out - ref) <= 2 * moe_data.ulp_bf16(ref) + 1e-6)
    assert (out == ref).mean() > 0.9


@pytest.mark.parametrize("T", [1, 12])
def test_layer_reference_order_vs_fp64(orc, T):
    """order=1 (the reference's dispatch and rounding points) stays within two
    bf16 steps of the fp64 layer, like the canonical order."""
    E, k, H, I = 8, 2, 64, 64
    # one token: random biases, at the fast path's rounding points; several
    # tokens: zero biases, where every path's rounding points coincide
    w = moe_data.make_layer(13 + T, E, H, I, bias="random" if T == 1 else "zero")
    x, res = moe_data.make_tokens(13 + T, T, H)
    out = orc.bf16_to_f32(orc.moe_forward(w, x, res, E, k, H, I, order=1)).astype(np.float64)
    ref = _layer_fp64(w, x, res, E, k, H, I, orc, fast_one=T == 1)
    rel = np.abs(out - ref) / np.maximum(np.abs(ref), 1e-3)
    assert rel.mean() <= 1e-3
    assert np.all(np.abs(out - ref) <= 2 * moe_data.ulp_bf16(ref) + 1e-6)


def _f32(a):
    return np.asarray(a, np.float32)


def test_layer_reference_order_one_token(orc):
    """The one-token fast path (moe_layer.cu:1028-1098) in order=1, checked
    stage by stage against the oracle's single-matrix primitives: gate_up is
    the fused GEMV with no bias; the SwiGLU takes bf16(gate_up) + bias in fp32;
    the down output is bf16(bf16(GEMV) + bias); the combine starts from the
    residual and adds w_k * y_k in slot order."""
    E, k, H, I = 8, 4, 256, 128
    w = moe_data.make_layer(21, E, H, I, bias="random")
    x, res = moe_data.make_tokens(21, 1, H)
    out, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True, order=1)
    L = orc.lib()
    gm = tr["gather_map"]
    acc = orc.bf16_to_f32(res[0]).copy()
    for s in range(k):
        e, p = int(tr["idx"][0, s]), int(gm[s])
        gu = orc.mxfp4_gemv_refkernel(x, w["w1_packed"][e], w["w1_scales"][e], None, 2 * I, H)[0]
        assert np.array_equal(tr["gate_up"][p], gu)
        gb = orc.bf16_to_f32(gu) + orc.bf16_to_f32(w["w1_bias"][e])      # fp32 sum, not rounded
        act = np.array([L.orc_swiglu(float(gb[2 * i]), float(gb[2 * i + 1]), 1.702, 7.0) for i in range(I)],
                       np.float32)
        assert np.array_equal(tr["act"][p], orc.f32_to_bf16(act))
        yd = orc.mxfp4_gemv_refkernel(tr["act"][p:p + 1], w["w2_packed"][e], w["w2_scales"][e], None, H, I)[0]
        y = orc.f32_to_bf16(orc.bf16_to_f32(yd) + orc.bf16_to_f32(w["w2_bias"][e]))
        assert np.array_equal(tr["y"][p], y)
        # fma(w, y, acc): the product is exact in fp64 and so is its sum with acc here
        acc = _f32(np.float64(tr["w"][0, s]) * orc.bf16_to_f32(y).astype(np.float64) + acc.astype(np.float64))
    assert np.array_equal(out[0], orc.f32_to_bf16(acc))


def test_layer_reference_order_dispatch(orc):
    """order=1 with several tokens picks the reference's path per active
    expert (moe_layer.cu:1282-1417).  Routing: experts 0-7 one token each
    (batch 0: all one-token -> fused GEMV, bias inside), expert 8 four tokens
    and 9-12 one each (batch 1, mixed -> hipBLASLt stand-in for 8, gemv_bf16
    over the dequantised weights for 9-12, each then a separate bias add).
    Every expert's rows are checked against the oracle's primitives."""
    E, k, H, I, T = 16, 4, 256, 128, 4
    w = moe_data.make_layer(22, E, H, I, bias="random")
    x, res = moe_data.make_tokens(22, T, H)
    idx = np.array([[0, 1, 8, 9], [2, 3, 8, 10], [4, 5, 8, 11], [6, 7, 8, 12]], np.int32)
    wts = np.full((T, k), 0.25, np.float32)
    out, tr = orc.moe_forward_routed(w, x, res, idx, wts, E, k, H, I, trace=True, order=1)
    gm = tr["gather_map"]

    def round_then_bias(prod_f32, b):
        return orc.f32_to_bf16(orc.bf16_to_f32(orc.f32_to_bf16(prod_f32)) + orc.bf16_to_f32(b))

    for t in range(T):
        for s in range(k):
            e, p = int(idx[t, s]), int(gm[t * k + s])
            P1, S1, B1 = w["w1_packed"][e], w["w1_scales"][e], w["w1_bias"][e]
            P2, S2, B2 = w["w2_packed"][e], w["w2_scales"][e], w["w2_bias"][e]
            a = tr["act"][p:p + 1]
            if e < 8:
                gu = orc.mxfp4_gemv_refkernel(x[t:t + 1], P1, S1, B1, 2 * I, H)[0]
                y = orc.mxfp4_gemv_refkernel(a, P2, S2, B2, H, I)[0]
            elif e == 8:
                gu = round_then_bias(orc.bf16_to_f32(orc.mxfp4_gemv(x[t:t + 1], P1, S1, None, 2 * I, H))[0], B1)
                y = round_then_bias(orc.bf16_to_f32(orc.mxfp4_gemv(a, P2, S2, None, H, I))[0], B2)
            else:
                dq1 = orc.mxfp4_dequant(P1, S1, 2 * I, H)
                dq2 = orc.mxfp4_dequant(P2, S2, H, I)
                gu = round_then_bias(orc.router(x[t:t + 1], dq1, None, logits_fp32=True)[0], B1)
                y = round_then_bias(orc.router(a, dq2, None, logits_fp32=True)[0], B2)
            assert np.array_equal(tr["gate_up"][p], gu), (t, s, e)
            assert np.array_equal(tr["act"][p], orc.swiglu_rows(gu[None], I)[0]), (t, s, e)
            assert np.array_equal(tr["y"][p], y), (t, s, e)
    assert np.array_equal(out, orc.combine(tr["y"], gm, wts, res, T, k, H))


def test_layer_threads_deterministic(orc):
    E, k, H, I, T = 16, 4, 128, 64, 9
    w = moe_data.make_layer(4, E, H, I)
    x, res = moe_data.make_tokens(4, T, H)
    a = orc.moe_forward(w, x, res, E, k, H, I, nthreads=1)
    b = orc.moe_forward(w, x, res, E, k, H, I, nthreads=7)
    assert np.array_equal(a, b)


def test_golden_fixture(orc):
    """Regression of the oracle against the committed fixture written by
    tests/golden/make_golden.py (E=8, k=2, H=I=128, T=5, random biases)."""
    d = np.load(os.path.join(GOLDEN, "moe_tiny.npz"))
    w = {n: d[n] for n in ("router_w", "router_b", "w1_packed", "w1_scales", "w1_bias",
                           "w2_packed", "w2_scales", "w2_bias")}
    E, k, H, I = (int(v) for v in d["shape"])
    out, tr = orc.moe_forward(w, d["x"], d["residual"], E, k, H, I, trace=True)
    assert np.array_equal(out, d["out"])
    assert np.array_equal(tr["idx"], d["idx"])
    assert np.array_equal(tr["w"], d["w"])


def test_layer_routed_matches_forward_and_is_per_token(orc):
    """The routed entry (expert half with the routing given) reproduces the
    full forward on its own routing, and each token's output depends only on
    that token: a subset of tokens run alone gives the same rows."""
    E, k, H, I, T = 16, 4, 128, 96, 23
    w = moe_data.make_layer(8, E, H, I, bias="random")
    x, res = moe_data.make_tokens(8, T, H)
    out, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    routed = orc.moe_forward_routed(w, x, res, tr["idx"], tr["w"], E, k, H, I)
    assert np.array_equal(routed, out)
    sel = np.array([0, 5, 6, 17, 22])
    sub = orc.moe_forward_routed(w, x[sel], res[sel], tr["idx"][sel], tr["w"][sel], E, k, H, I)
    assert np.array_equal(sub, out[sel])


def test_zipf_routing_shape():
    """Prefill routing generator: k distinct experts per token, weights a
    descending distribution, expert loads skewed (Zipf 1.1 over 128)."""
    idx, w = moe_data.zipf_routing(3, 4096, 128, 4)
    assert idx.shape == (4096, 4) and idx.dtype == np.int32
    s = np.sort(idx, axis=1)
    assert (s[:, 1:] != s[:, :-1]).all() and idx.min() >= 0 and idx.max() < 128
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6) and (np.diff(w, axis=1) <= 0).all()
    counts = np.bincount(idx.ravel(), minlength=128)
    assert counts.sum() == 4096 * 4 and counts.max() > 2000 and counts.min() < 40
