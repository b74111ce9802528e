"""GPU: how gfx950's matrix cores sum the products of one instruction.

This pins the hardware fact behind the prefill's choice of bf16 products
over the block-scaled f8f6f4 ones.  One wave runs one instruction from a
zero accumulator on operands whose exact sum is known (the probe library,
tests/hw/mfma_probe.hip, built by build()):

  * v_mfma_f32_16x16x32_bf16: 256 + 2^-9 comes back exactly.  Every
    product fits fp32, and the sum keeps every bit an fp32 sum keeps.
  * v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 x e4m3, and e2m1 x e4m3, scales
    2^0): 256 + 2^-9 comes back as 256.  The small product is dropped: the
    instruction aligns products to the largest of their group and keeps
    fewer bits below it than fp32 would.

The sums are built so that only row r, column c products at K = 0 and 1 are
non-zero (lanes 0..15 hold K 0..15 of both operands), so every output
element of the 16x16 tile is the same two-term sum.
"""
import ctypes
import os

import numpy as np
import pytest

from test_gpu_parity import say

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))

E4M3_ONE, E4M3_256, E4M3_2M9 = 0x38, 0x78, 0x01   # 1.0, 2^8, 2^-9 (the smallest subnormal)
E4M3_2M4 = 0x18                                    # 2^-4
BF16 = {1.0: 0x3F80, 256.0: 0x4380, 2.0 ** -9: 0x3B00}
E2M1_ONE = 0x2


@pytest.fixture(scope="module")
def probe():
    import torch  # noqa: F401  (the probe binds to torch's HIP runtime)
    path = os.path.join(HERE, "hw", "libmfma_probe.so")
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    P = ctypes.c_void_p
    lib.mfma_probe_bf16.argtypes = [P, P, P]
    lib.mfma_probe_f8f6f4.argtypes = [P, P, P, P, ctypes.c_int, P]
    return lib


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bf16_sum(probe, x0, x1):
    import torch
    a = np.zeros((64, 8), np.uint16)
    b = np.zeros((64, 8), np.uint16)
    a[:16, 0], a[:16, 1] = BF16[x0], BF16[x1]       # A[r, 0] = x0, A[r, 1] = x1
    b[:16, 0] = b[:16, 1] = BF16[1.0]               # B[0, c] = B[1, c] = 1
    d = torch.zeros((64, 4), dtype=torch.float32, device="cuda")
    assert probe.mfma_probe_bf16(_dev(a.view(np.uint32)).data_ptr(), _dev(b.view(np.uint32)).data_ptr(),
                                 d.data_ptr()) == 0
    return d.cpu().numpy()


def _f8f6f4_sum(probe, b0, b1, a_fp4):
    """A = 1.0 at K 0 and 1 (e4m3 or e2m1), B = b0, b1 (e4m3 codes) there."""
    import torch
    a = np.zeros((64, 32), np.uint8)
    b = np.zeros((64, 32), np.uint8)
    if a_fp4:
        a[:16, 0] = E2M1_ONE | (E2M1_ONE << 4)       # lanes 0..15: row l, K 0..31; K0 low nibble
    else:
        a[:16, 0] = a[:16, 1] = E4M3_ONE              # lanes 0..15: K 0..15 (bytes 0..15)
    b[:16, 0], b[:16, 1] = b0, b1
    scales = np.full(64, 0x7F7F7F7F, np.uint32)      # e8m0 127: 2^0
    d = torch.zeros((64, 4), dtype=torch.float32, device="cuda")
    sa, sb = _dev(scales), _dev(scales)
    assert probe.mfma_probe_f8f6f4(_dev(a.view(np.uint32)).data_ptr(), _dev(b.view(np.uint32)).data_ptr(),
                                   sa.data_ptr(), sb.data_ptr(), 1 if a_fp4 else 0, d.data_ptr()) == 0
    return d.cpu().numpy()


def test_bf16_products_sum_in_fp32(probe):
    d = _bf16_sum(probe, 256.0, 2.0 ** -9)
    say("bf16 16x16x32: 256 + 2^-9 ->", float(d[0, 0]))
    assert np.all(d == np.float32(256.0 + 2.0 ** -9))
    assert np.all(_bf16_sum(probe, 1.0, 256.0) == np.float32(257.0))


@pytest.mark.parametrize("a_fp4", [0, 1], ids=["e4m3xe4m3", "e2m1xe4m3"])
def test_block_scaled_products_drop_low_bits(probe, a_fp4):
    d = _f8f6f4_sum(probe, E4M3_256, E4M3_2M9, a_fp4)
    d2 = _f8f6f4_sum(probe, E4M3_256, E4M3_2M4, a_fp4)
    ctl = _f8f6f4_sum(probe, E4M3_2M9, E4M3_2M9, a_fp4)
    say(f"f8f6f4 16x16x128 a_fp4={a_fp4}: 256 + 2^-9 ->", float(d[0, 0]), " 256 + 2^-4 ->", float(d2[0, 0]),
        " 2^-9 + 2^-9 ->", float(ctl[0, 0]))
    # the small operand alone is exact (control), next to 256 it is lost
    assert np.all(ctl == np.float32(2.0 ** -8))
    assert np.all(d == np.float32(256.0))
    # 2^-4, 12 binades below 256, survives: the loss is of low bits, not of
    # the smaller product as such
    assert np.all(d2 == np.float32(256.0 + 2.0 ** -4))
