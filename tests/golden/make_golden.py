"""Writes the committed golden vectors of the CPU-runnable configuration
B=1, H=1, L=128 (u ~ N(0,1) seed 0, k ~ N(0,1)/sqrt(L) seed 1, numpy PCG64):
config1.npz holds u, k and y = the fp64 causal convolution, plus the reference
generator's first sequence (seed 88172645463325252) with its fp64 convolution.
Run from the repository root: python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402


def main():
    L = 128
    u = np.random.default_rng(0).standard_normal((1, 1, L)).astype(np.float32)
    k = (np.random.default_rng(1).standard_normal((1, L)) / np.sqrt(L)).astype(np.float32)
    y = oracle.direct_conv(u, k)
    ur, kr = oracle.ref_inputs(1, 1, L)
    yr = oracle.direct_conv(ur, kr)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1.npz")
    np.savez(out, u=u, k=k, y=y, ref_u=ur, ref_k=kr, ref_y=yr)
    print("wrote", out)


if __name__ == "__main__":
    main()
