"""Parity of the fused HIP convolution (through the C ABI) with the fp64 oracle.

Bounds (relative L2 over all outputs, against the fp64 convolution of the fp32
inputs): <= 5e-4 for fp32 I/O with fp32 accumulation, <= 3e-3 for bf16 I/O
(which includes the bf16 rounding of inputs and outputs, as in src/sffft.cu:395).
fp16 accumulation is held to the reference smoke-test caps: 2e-3 (fp32 I/O) and
6e-3 (bf16 I/O) (tests/precision_smoke.sh:62,73).

Two sequences per transform (seqs=2) pack a pair of rows as the real and imaginary
parts of one transform. The fp16 rounding noise that a single real row sheds into
the discarded imaginary output then lands on the second row, so the error is about
1.2x the one-row error. Pair plans are held to the same bounds as every other plan.
"""
import numpy as np
import pytest

import oracle
import sffft_amd as sf

pytestmark = pytest.mark.gpu

BOUND = {("fp32", 0): 5e-4, ("bf16", 0): 3e-3, ("fp32", 1): 2e-3, ("bf16", 1): 6e-3}


def bound(io, acc, seqs=1):
    """The bound of an I/O type and accumulation, whatever the sequences per transform."""
    return BOUND[(io, acc)]


def _run(dev, u, k, plan, io):
    import torch

    L = u.shape[-1]
    kd = torch.from_numpy(k).to(dev)
    kf = sf.spectrum(kd, L, plan)
    ud = torch.from_numpy(u).to(dev)
    if io == "bf16":
        ud = sf.to_bf16(ud)
    y = sf.conv(ud, kf, plan)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


def _cases():
    for L in sf.LENGTHS:
        for p in sf.plans(L):
            yield L, p


@pytest.mark.parametrize("L,plan", list(_cases()), ids=lambda x: repr(x) if not isinstance(x, int) else f"L{x}")
def test_conv_matches_oracle(dev, L, plan):
    # wave plans: 26 pairs, so wavefronts take several pairs and the last workgroup
    # is partly idle; workgroup plans: 16 sequences (8 pairs)
    B, H = (4, 13) if plan.mode == 1 else (2, 8)
    u, k = oracle.gen_inputs(B, H, L, seed=L)
    ref = oracle.conv(u, k)
    for io in ("fp32", "bf16"):
        print(f"case L={L} {plan!r} io={io}", flush=True)
        y = _run(dev, u, k, plan, io)
        err = oracle.rel_l2(y, ref)
        print(f"  rel_l2={err:.3e}", flush=True)
        assert np.isfinite(err) and err <= bound(io, 0, plan.seqs), (L, repr(plan), io, err)


@pytest.mark.parametrize("L", sf.LENGTHS)
def test_legacy_and_fp16_accumulation(dev, L):
    B, H = 2, 2
    u, k = oracle.gen_inputs(B, H, L, seed=7 * L)
    ref = oracle.conv(u, k)
    for base in sf.plans(L)[:2]:
        for cached in (0, 1):
            for acc in (0, 1):
                p = base.replace(cached=cached, acc=acc)
                for io in ("fp32", "bf16"):
                    print(f"case L={L} {p!r} io={io}", flush=True)
                    err = oracle.rel_l2(_run(dev, u, k, p, io), ref)
                    print(f"  rel_l2={err:.3e}", flush=True)
                    assert np.isfinite(err) and err <= bound(io, acc, p.seqs), (L, repr(p), io, err)
