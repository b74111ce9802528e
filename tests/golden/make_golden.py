"""Writes tests/golden/moe_tiny.npz: a small MoE layer (E=8, k=2, H=I=128,
T=5, random biases) and the oracle's output, idx and weights for it.  The
fixture pins the oracle against accidental change and gives the GPU tests a
committed expected output.  Run: python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
sys.path.insert(0, os.path.join(HERE, ".."))

import moe_data  # noqa: E402
import moe_oracle as orc  # noqa: E402


def main():
    E, k, H, I, T = 8, 2, 128, 128, 5
    w = moe_data.make_layer(11, E, H, I, bias="random")
    x, res = moe_data.make_tokens(11, T, H)
    out, tr = orc.moe_forward(w, x, res, E, k, H, I, trace=True)
    np.savez_compressed(os.path.join(HERE, "moe_tiny.npz"), shape=np.array([E, k, H, I]), x=x, residual=res,
                        out=out, idx=tr["idx"], w=tr["w"], **w)


if __name__ == "__main__":
    main()
