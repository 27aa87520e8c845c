"""Parity at the full benchmark configurations, through the C ABI:

- B=8, H=768, L=1024, 64x32 (wave pipeline, the benchmark workload), fp32 and bf16 I/O;
- B=8, H=768, L=2048: 16x16x16 with bf16 I/O, fp32 and fp16 accumulation, and the
  default 64x64 wave plan in both I/O types;
- B=8, H=768, L=4096: the default plan 32x16x16 with 4 wavefronts, fp32 and bf16 I/O;
- B=8, H=768, L=8192: 32x32x16 (the default, 8 wavefronts, and 4) in fp32 and bf16 I/O,
  and 64x16x16 (held to 128 VGPRs) in bf16;
- B=4, H=1536, L=16384, 32x32x32 (the default, 8 wavefronts, and 16) in bf16 and fp32
  I/O, a long filter made of 16 decaying sinusoids per channel.

Every B*H*L output is compared with the fp64 oracle (src/sffft.cu:394-399): the direct
convolution up to L=2048, the fp64 FFT convolution above it, itself cross-checked
against the direct sum on sequences {0, BH/2, BH-1} as src/sffft.cu:376 does. The
bounds are those of test_gpu_parity.py. The whole batch is also checked through
properties that hold bit for bit at any size:

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


def reference(u32, k, B, H, L):
    """fp64 convolution of every sequence; beyond L = 2048 the FFT convolution, whose
    agreement with the direct sum on sequences {0, BH/2, BH-1} is asserted here."""
    u_np = u32.cpu().numpy()
    if L <= 2048:
        return oracle.direct_conv(u_np, k)
    ref = oracle.fft_conv(u_np, k)
    seqs = [0, B * H // 2, B * H - 1]
    x = oracle.rel_l2(ref.reshape(B * H, L)[seqs], oracle.direct_conv_seqs(u_np, k, seqs))
    print(f"  oracle fft vs direct on {seqs}: {x:.2e}", flush=True)
    assert x <= 1e-12, x
    return ref


CONFIGS = [
    # (B, H, L, filter, [(plan spec, waves, seqs, mode, channels, acc, io list), ...])
    (8, 768, 1024, "decay256", [("64x32", 12, 2, 1, 3, 0, ("fp32", "bf16"))]),
    (8, 768, 2048, "decay256", [("16x16x16", 4, 2, 0, 1, 0, ("bf16",)), ("16x16x16", 4, 2, 0, 1, 1, ("bf16",)),
                                ("64x64", 12, 2, 1, 3, 0, ("fp32", "bf16"))]),
    (8, 768, 4096, "decay2048", [("32x16x16", 4, 2, 0, 1, 0, ("fp32", "bf16"))]),
    (8, 768, 8192, "decay2048", [("32x32x16", 8, 2, 0, 1, 0, ("fp32", "bf16")),
                                 ("32x32x16", 4, 2, 0, 1, 0, ("fp32", "bf16")),
                                 ("64x16x16", 8, 2, 0, 1, 0, ("bf16",))]),
    (4, 1536, 16384, "sines", [("32x32x32", 8, 2, 0, 1, 0, ("bf16", "fp32")),
                               ("32x32x32", 16, 2, 0, 1, 0, ("bf16", "fp32"))]),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"B{c[0]}_H{c[1]}_L{c[2]}")
def test_full_size_config(dev, cfg):
    import torch

    B, H, L, filt, plans = cfg
    if filt == "sines":
        k = sinusoid_filters(H, L, seed=5, dev=dev)
    else:
        k = decaying_filters(H, L, 256.0 if filt == "decay256" else 2048.0, seed=L + 1)
    g = torch.Generator(device=dev).manual_seed(L)
    u32 = torch.randn(B, H, L, device=dev, generator=g)
    kd = torch.from_numpy(k).to(dev)
    ref = reference(u32, k, B, H, L)
    for spec, waves, seqs, mode, channels, acc, ios in plans:
        plan = sf.make_plan(spec, waves, acc=acc, cached=1, seqs=seqs, mode=mode, channels=channels)
        assert sf.plan_check(L, plan) == 0, repr(plan)
        kf = sf.spectrum(kd, L, plan)
        for io in ios:
            print(f"case B={B} H={H} L={L} {plan!r} io={io}", flush=True)
            y = run(u32, kf, plan, io)
            err = oracle.rel_l2(y.float().cpu().numpy(), ref)
            print(f"  rel_l2 over all {B * H * L} outputs = {err:.3e} (bound {bound(io, acc)})", flush=True)
            assert np.isfinite(err) and err <= bound(io, acc), (L, repr(plan), io, err)

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
            del y, yp, yq
