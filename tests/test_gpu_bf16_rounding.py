"""GPU: the fp32 -> bf16 rounding every kernel's output goes through.

The kernels round with gfx950's packed conversion (`static_cast<__bf16>`
and its two-lane vector form, v_cvt_pk_bf16_f32): round to nearest even,
NaN kept quiet with its sign and leading payload bits.  These tests pin that
on the device against the oracle's integer form (orc.f32_to_bf16, itself
pinned against torch in test_oracle.py), bit for bit, through two stage
entry points:

  * gptoss_moe_combine_forward with one slot, expert row 1.0 and no
    residual: out = bf16(fma(w, 1, 0)) = bf16(w) for any fp32 w (the scalar
    conversion of the combine kernels), over random bit patterns, ties and
    near-ties at every exponent, denormals, infinities, the largest finite
    values (which round to inf) and NaN payloads;
  * gptoss_moe_grouped_mxfp4_gemm with weights 1.0 picking three K
    positions, one per 32-element block: each output is a + b + c where a, b
    and c are the three bf16 pieces of a target fp32 value v (top, middle
    and low 8 significant bits), every partial sum exact, so the output is
    bf16(v) through the prefill epilogue's two-lane conversion.

A toolchain or rounding-mode change that moved any of these would move every
bf16 output of the library.
"""
import numpy as np
import pytest

from test_gpu_parity import dev, host, say

pytestmark = pytest.mark.gpu


def _edge_bits(rng, n_random):
    """fp32 bit patterns: random ones, then ties / near ties at every
    exponent (both signs, even and odd bf16 mantissa), denormals, the values
    around the largest finite one, infinities and NaN payloads."""
    parts = [rng.integers(0, 2 ** 32, n_random, dtype=np.uint64).astype(np.uint32)]
    exps = np.arange(0, 255, dtype=np.uint32)
    for low in (0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF, 0x4000, 0xC000):
        for odd in (0, 1):
            for hi_m in (0x00, 0x35, 0x7E):
                m = (np.uint32(hi_m) << 17) | (np.uint32(odd) << 16) | np.uint32(low)
                for sign in (0, 1):
                    parts.append((np.uint32(sign) << 31) | (exps << 23) | m)
    parts.append(np.array([0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7E8000, 0x7F7F0000,
                           0x7F800000, 0xFF800000, 0x00000000, 0x80000000, 0x00000001, 0x80000001,
                           0x00008000, 0x00018000, 0x007FFFFF, 0x00800000], np.uint32))
    # NaN payloads: quiet and signalling, payload bits above and below bit 16
    pay = rng.integers(1, 2 ** 22, 4096, dtype=np.uint64).astype(np.uint32)
    for q in (0, 1):
        for sign in (0, 1):
            parts.append((np.uint32(sign) << 31) | np.uint32(0x7F800000) | (np.uint32(q) << 22) | pay)
    return np.concatenate(parts)


def test_combine_rounds_like_the_oracle(gpu, orc):
    import torch
    rng = np.random.default_rng(2024)
    bits = _edge_bits(rng, 1 << 20)
    # token q: one slot, weight w[q], expert row q of eight 1.0 values
    n, Hs = bits.size, 8
    w = bits.view(np.float32).reshape(n, 1)
    y = torch.full((n, Hs), 1.0, dtype=torch.bfloat16, device="cuda")
    gm = torch.arange(n, dtype=torch.int32, device="cuda")
    out = host(gpu.combine(y, gm, dev(w, torch), None, n, Hs, 1))
    torch.cuda.synchronize()
    # the fma's own result: -0 * 1 + 0 = +0, a signalling NaN comes back quiet
    acc = bits.copy()
    acc[acc == 0x80000000] = 0
    nan = ((acc & 0x7F800000) == 0x7F800000) & ((acc & 0x7FFFFF) != 0)
    acc[nan] |= 0x00400000
    want = orc.f32_to_bf16(acc.view(np.float32))
    got = out[:, 0]
    assert np.all(out == got[:, None])
    bad = np.nonzero(got != want)[0]
    say("combine bf16 rounding", dict(values=int(n), mismatches=int(bad.size),
                                      first=[(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i])))
                                             for i in bad[:5]]))
    assert bad.size == 0


def _pieces(v):
    """v (fp32) as a + b + c, three bf16 values holding its top, middle and
    low 8 significant bits (exact: the pieces cover v's 24 bits)."""
    u = v.view(np.uint32)
    a = (u & 0xFFFF0000).view(np.float32)
    r1 = (v.astype(np.float64) - a.astype(np.float64)).astype(np.float32)
    b = (r1.view(np.uint32) & 0xFFFF0000).view(np.float32)
    c = (r1.astype(np.float64) - b.astype(np.float64)).astype(np.float32)
    assert np.all((c.view(np.uint32) & 0xFFFF) == 0)
    assert np.array_equal(a.astype(np.float64) + b + c, v.astype(np.float64))
    return [(p.view(np.uint32) >> 16).astype(np.uint16) for p in (a, b, c)]


def test_grouped_epilogue_rounds_like_the_oracle(gpu, orc):
    import torch
    rng = np.random.default_rng(7)
    N, K = 64, 96
    rows = 200
    # target values: random finite patterns with biased exponent 20..254 (every
    # piece a normal bf16), ties and near ties among them, and values that
    # round up to inf
    n = rows * 32
    u = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    e = rng.integers(20, 255, n).astype(np.uint32)
    u = (u & 0x807FFFFF) | (e << 23)
    lows = np.array([0x8000, 0x7FFF, 0x8001, 0x0000], np.uint32)
    sel = rng.integers(0, 2, n).astype(bool)
    u[sel] = (u[sel] & 0xFFFF0000) | lows[rng.integers(0, 4, int(sel.sum()))]
    u[:8] = [0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7E8000, 0xFF7F8000, 0x4B800000, 0xCB808000]
    v = u.view(np.float32).reshape(rows, 32)
    a, b, c = _pieces(v.reshape(-1))
    x = np.zeros((rows, K), np.uint16)
    x[:, 0:32] = a.reshape(rows, 32)
    x[:, 32:64] = b.reshape(rows, 32)
    x[:, 64:96] = c.reshape(rows, 32)
    # weights: row n holds e2m1 1.0 (code 2) at element n % 32 of each block,
    # scale code 127 (2^0); two experts share them
    nib = np.zeros((N, K), np.uint8)
    for nn in range(N):
        nib[nn, [nn % 32, 32 + nn % 32, 64 + nn % 32]] = 2
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    scales = np.full((N, K // 32), 127, np.uint8)
    E = 2
    tn, ts = [], []
    for _ in range(E):
        p, s = gpu.pack_tiled(dev(packed, torch), dev(scales, torch), N, K)
        tn.append(p)
        ts.append(s)
    tn, ts = torch.cat(tn), torch.cat(ts)
    offsets = dev(np.array([0, 130, rows], np.int32), torch)  # a full 128-row tile, then partial ones
    out = host(gpu.grouped_mxfp4_gemm(dev(x, torch), offsets, tn, ts, N, K, rows))
    torch.cuda.synchronize()
    want = orc.f32_to_bf16(v)
    got = np.concatenate([out[:, :32], out[:, 32:]])
    bad = np.argwhere(got != np.concatenate([want, want]))
    say("grouped epilogue bf16 rounding", dict(values=int(got.size), mismatches=int(len(bad))))
    assert len(bad) == 0
