"""Parity at the full benchmark configurations, through the C ABI:

- B=8, H=768, L=1024, fp32 I/O, 64x32 (wave pipeline, the benchmark workload);
- B=8, H=768, L=2048, bf16 I/O, 16x16x16, fp32 and fp16 accumulation;
- B=8, H=768, L=8192, fp32 and bf16 I/O, 32x32x16;
- B=4, H=1536, L=16384, bf16 I/O, 32x32x32, a long filter made of 16 decaying
  sinusoids per channel.

Sampled sequences are compared with the fp64 oracle (direct convolution up to
L=2048, FFT convolution above) to the parity bounds of test_gpu_parity.py. The
whole batch is checked through properties that hold bit for bit at any size:

- each output row depends only on its own input row and channel, so swapping two
  batch pairs, or two channels together with their filters, permutes the output
  exactly;
- two launches on the same inputs give identical bits.
"""
import numpy as np
import pytest

import oracle
import sffft_amd as sf

from test_gpu_parity import bound

pytestmark = pytest.mark.gpu

NSAMPLE = 48


def sinusoid_filters(H, L, seed, dev):
    """k[h, n] = sum_{i<16} A_hi sin(w_hi n) exp(-a_h n): w ~ U(0, pi), A ~ N(0, 1),
    a_h log-uniform in [1e-4, 1e-2] (numpy PCG64 draws; evaluated in float64 on the
    device, 128 channels at a time)."""
    import torch

    rng = np.random.default_rng(seed)
    w = torch.from_numpy(rng.uniform(0.0, np.pi, (H, 16))).to(dev)
    amp = torch.from_numpy(rng.standard_normal((H, 16))).to(dev)
    alpha = torch.from_numpy(np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), H))).to(dev)
    n = torch.arange(L, dtype=torch.float64, device=dev)
    k = torch.empty((H, L), dtype=torch.float64, device=dev)
    for h in range(0, H, 128):
        s = slice(h, h + 128)
        k[s] = (amp[s, :, None] * torch.sin(w[s, :, None] * n)).sum(1) * torch.exp(-alpha[s, None] * n)
    return k.float().cpu().numpy()


def decaying_filters(H, L, decay, seed):
    n = np.arange(L, dtype=np.float64)
    return (np.random.default_rng(seed).standard_normal((H, L)) * np.exp(-n / decay) / np.sqrt(L)).astype(np.float32)


def run(u32, kf, plan, io):
    import torch

    u = sf.to_bf16(u32) if io == "bf16" else u32
    y = sf.conv(u, kf, plan)
    torch.cuda.synchronize()
    return y


def sampled_error(u32, k, y, B, H, L):
    """rel-L2 of NSAMPLE evenly spread sequences against the fp64 oracle (the bf16
    error includes the I/O rounding, measured against the fp32 input)."""
    import torch

    idx = np.linspace(0, B * H - 1, NSAMPLE).astype(np.int64)
    ti = torch.from_numpy(idx).to(u32.device)
    us = u32.reshape(B * H, L)[ti].cpu().numpy()
    ys = y.float().reshape(B * H, L)[ti].cpu().numpy()
    ks = k[idx % H]
    ref = oracle.conv(us[None], ks)[0]
    return oracle.rel_l2(ys, ref)


CONFIGS = [
    # (B, H, L, plan spec, waves, seqs, mode, channels, io list, acc list, filter)
    (8, 768, 1024, "64x32", 12, 2, 1, 3, ("fp32",), (0,), "decay256"),
    (8, 768, 2048, "16x16x16", 4, 2, 0, 1, ("bf16",), (0, 1), "decay256"),
    (8, 768, 8192, "32x32x16", 4, 2, 0, 1, ("fp32", "bf16"), (0,), "decay2048"),
    (4, 1536, 16384, "32x32x32", 8, 2, 0, 1, ("bf16",), (0,), "sines"),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"B{c[0]}_H{c[1]}_L{c[2]}_{c[3]}")
def test_full_size_config(dev, cfg):
    import torch

    B, H, L, spec, waves, seqs, mode, channels, ios, accs, filt = cfg
    if filt == "sines":
        k = sinusoid_filters(H, L, seed=5, dev=dev)
    else:
        k = decaying_filters(H, L, 256.0 if filt == "decay256" else 2048.0, seed=L + 1)
    g = torch.Generator(device=dev).manual_seed(L)
    u32 = torch.randn(B, H, L, device=dev, generator=g)
    kd = torch.from_numpy(k).to(dev)
    for acc in accs:
        plan = sf.make_plan(spec, waves, acc=acc, cached=1, seqs=seqs, mode=mode, channels=channels)
        assert sf.plan_check(L, plan) == 0, repr(plan)
        kf = sf.spectrum(kd, L, plan)
        for io in ios:
            print(f"case B={B} H={H} L={L} {plan!r} io={io}", flush=True)
            y = run(u32, kf, plan, io)
            err = sampled_error(u32, k, y, B, H, L)
            print(f"  sampled rel_l2={err:.3e}", flush=True)
            assert np.isfinite(err) and err <= bound(io, acc, seqs), (L, repr(plan), io, err)

            # determinism
            assert torch.equal(run(u32, kf, plan, io), y)

            # swapping batch pairs 0 <-> last permutes the output exactly
            order = list(range(B))
            order[0], order[1], order[B - 2], order[B - 1] = B - 2, B - 1, 0, 1
            p = torch.tensor(order, device=dev)
            yp = run(u32[p].contiguous(), kf, plan, io)
            assert torch.equal(yp, y[p]), "batch-pair swap"

            # swapping two channels (input rows and filters) permutes the output exactly
            h1, h2 = 1, H - 2
            order = list(range(H))
            order[h1], order[h2] = h2, h1
            q = torch.tensor(order, device=dev)
            kq = sf.spectrum(kd[q].contiguous(), L, plan)
            yq = run(u32[:, q].contiguous(), kq, plan, io)
            assert torch.equal(yq, y[:, q]), "channel swap"
