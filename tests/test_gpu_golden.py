"""The committed configuration-1 fixtures (B=1, H=1, L=128: tests/golden/config1.npz, the
build's seeded generator and the reference's generator, with their fp64 direct
convolutions) through the HIP path: sffft_spectrum + sffft_conv_f32 / sffft_conv_bf16 on
every one-sequence plan of L = 128 (B = 1 has no pair), against the stored outputs at the
bounds of the fp32 (5e-4) and bf16 (3e-3) I/O types. The oracle's own check of these
fixtures is tests/test_oracle.py::test_golden_vectors."""
import os

import numpy as np
import pytest

import oracle
import sffft_amd as sf

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz")


@pytest.mark.parametrize("which", ["build", "reference"])
def test_config1_golden_through_hip(dev, which):
    import torch

    g = np.load(GOLDEN)
    u, k, y = (g["u"], g["k"], g["y"]) if which == "build" else (g["ref_u"], g["ref_k"], g["ref_y"])
    L = u.shape[-1]
    assert u.shape == (1, 1, L) and L == 128
    plans = [p for p in sf.plans(L) if p.seqs == 1]
    plans.append(sf.default_plan(L, "fp32", 1))
    assert plans
    for plan in plans:
        for acc, bound32, bound16 in ((0, 5e-4, 3e-3), (1, 2e-3, 6e-3)):
            p = sf.make_plan(plan.name(), plan.waves, acc=acc, cached=1, seqs=1, mode=plan.mode,
                             channels=plan.channels)
            kf = sf.spectrum(torch.from_numpy(k).to(dev), L, p)
            ud = torch.from_numpy(u).to(dev)
            y32 = sf.conv(ud, kf, p).cpu().numpy()
            y16 = sf.conv(sf.to_bf16(ud), kf, p).float().cpu().numpy()
            e32, e16 = oracle.rel_l2(y32, y), oracle.rel_l2(y16, y)
            print(f"config1 {which} {p!r}: fp32 {e32:.3e} bf16 {e16:.3e}", flush=True)
            assert np.isfinite(e32) and e32 <= bound32, (which, repr(p), e32)
            assert np.isfinite(e16) and e16 <= bound16, (which, repr(p), e16)
