"""Parity of the multi-pass convolution (mode-2 plans, sffft_conv_long_*) with the fp64
oracle, through the C ABI.

Every compiled plan (column radix 16, 32 or 64 with row plans 16x16, 32x32, 64x32 and
64x64, L = 2048 .. 131072) runs both I/O types on seeded inputs and is compared over all
outputs with the oracle's fp64 FFT convolution (direct convolution at L = 2048). Bounds
are those of the fused kernel: 5e-4 for fp32 I/O (the pass-A input enters as an fp16
value plus its remainder) and 3e-3 for bf16 I/O, whose error includes the rounding of
inputs and outputs. The circular convolution, an operation the reference does not have,
has its own fp32 bound (see its test).

At the plans' own small L the result must also agree with the single-pass kernel to
the same bound, and the bench configurations run at full B=8, H=768 through the
bit-exact properties of test_gpu_configs.py (permutation of pairs and channels,
repeatability) on sampled sequences.
"""
import numpy as np
import pytest

import oracle
import sffft_amd as sf

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 5e-4, "bf16": 3e-3}


def _cases():
    for L in (2048, 4096, 8192, 16384) + sf.LONG_LENGTHS:
        for nc in (16, 32, 64):
            for rows in ((16, 16), (32, 32), (64, 32), (64, 64)):
                if nc * rows[0] * rows[1] == 2 * L:
                    yield L, f"{nc}x{rows[0]}x{rows[1]}"


def _run(dev, u, k, plan, io, work=None):
    import torch

    L = u.shape[-1]
    kf = sf.spectrum(torch.from_numpy(k).to(dev), L, plan)
    ud = torch.from_numpy(u).to(dev)
    if io == "bf16":
        ud = sf.to_bf16(ud)
    y = sf.conv(ud, kf, plan, work=work)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("L,spec", list(_cases()))
def test_long_conv_matches_oracle(dev, L, spec):
    plan = sf.long_plan(spec)
    # B=6 (three pairs per channel: a workgroup's last row slot idle), H=3; fewer rows
    # at the longest lengths
    B, H = (6, 3) if L <= 16384 else (4, 2)
    u, k = oracle.gen_inputs(B, H, L, seed=L + plan.r0)
    ref = oracle.conv(u, k)
    for io in ("fp32", "bf16"):
        print(f"case L={L} {spec} io={io} B={B} H={H}", flush=True)
        y = _run(dev, u, k, plan, io)
        err = oracle.rel_l2(y, ref)
        print(f"  rel_l2={err:.3e}", flush=True)
        assert np.isfinite(err) and err <= BOUND[io], (L, spec, io, err)


def test_long_matches_single_pass(dev):
    # one pair per channel (B=2): the row pass's workgroups take rows of different channels
    L, B, H = 8192, 2, 5
    u, k = oracle.gen_inputs(B, H, L, seed=11)
    ref = oracle.conv(u, k)
    a = _run(dev, u, k, sf.long_plan("64x16x16"), "fp32")
    b = _run(dev, u, k, sf.default_plan(L, "fp32", B), "fp32")
    assert oracle.rel_l2(a, ref) <= 5e-4 and oracle.rel_l2(b, ref) <= 5e-4
    assert oracle.rel_l2(a, b.astype(np.float64)) <= 1e-3


def test_long_workspace_reuse_and_delta(dev):
    """A caller's workspace is reused across calls (it is fully rewritten), and closed
    forms hold: a unit impulse at n = 0 in u returns k itself; a shifted impulse returns
    the shifted filter (the oracle is not involved)."""
    import torch

    L, B, H = 32768, 2, 2
    plan = sf.long_plan("64x32x32")
    rng = np.random.default_rng(5)
    k = (rng.standard_normal((H, L)) * np.exp(-np.arange(L) / 4096.0) / np.sqrt(L)).astype(np.float32)
    u = np.zeros((B, H, L), np.float32)
    u[0, :, 0] = 1.0
    u[1, :, 777] = 1.0
    work = torch.full((sf.work_bytes(B, H, L, plan),), 0x7f, dtype=torch.uint8, device=dev)
    y1 = _run(dev, u, k, plan, "fp32", work=work)
    y2 = _run(dev, u, k, plan, "fp32", work=work)
    assert np.array_equal(y1, y2)
    exp = np.zeros((B, H, L))
    exp[0] = k
    exp[1, :, 777:] = k[:, :L - 777]
    assert oracle.rel_l2(y1, exp) <= 5e-4


def test_long_chunks_agree(dev):
    """The batch runs in chunks of whole channels sized by the workspace: one channel per
    chunk, a ragged last chunk (2 of 5 channels) and the whole batch give the same bits."""
    import torch

    L, B, H = 32768, 4, 5
    plan = sf.long_plan("32x64x32")
    u, k = oracle.gen_inputs(B, H, L, seed=21)
    per = (B // 2) * 2 * L * 4
    outs = []
    for nch in (1, 3, H):
        work = torch.empty(nch * per + 8, dtype=torch.uint8, device=dev)  # a few spare bytes are ignored
        outs.append(_run(dev, u, k, plan, "fp32", work=work))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    assert oracle.rel_l2(outs[0], oracle.conv(u, k)) <= 5e-4


def test_long_full_batch_properties(dev):
    """B=8, H=768, L=32768 fp32 with the default plan: sampled sequences against the
    oracle; swapping two batch pairs permutes the output bit for bit; two launches
    agree bit for bit."""
    import torch

    L, B, H = 32768, 8, 768
    plan = sf.default_plan(L, "fp32", B)
    g = torch.Generator(device=dev).manual_seed(3)
    u = torch.randn((B, H, L), generator=g, device=dev, dtype=torch.float32)
    n = torch.arange(L, device=dev, dtype=torch.float32)
    k = torch.randn((H, L), generator=g, device=dev) * torch.exp(-n / 2048.0) / L ** 0.5
    kf = sf.spectrum(k, L, plan)
    work = torch.empty(sf.work_bytes(B, H, L, plan), dtype=torch.uint8, device=dev)
    y = sf.conv(u, kf, plan, work=work)
    y2 = sf.conv(u, kf, plan, work=work)
    us = u[[2, 3, 0, 1, 4, 5, 6, 7]].contiguous()
    ys = sf.conv(us, kf, plan, work=work)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(ys, y[[2, 3, 0, 1, 4, 5, 6, 7]])
    rng = np.random.default_rng(0)
    hs = rng.choice(H, 12, replace=False)
    for b in (0, 5):
        us_np = u[b, hs].cpu().numpy()[None]
        ref = oracle.conv(us_np, k[hs].cpu().numpy())
        err = oracle.rel_l2(y[b, hs].cpu().numpy()[None], ref)
        print(f"  b={b} sampled rel_l2={err:.3e}", flush=True)
        assert err <= 5e-4


@pytest.mark.parametrize("N,spec", [(8192, "32x16x16"), (65536, "64x32x32"), (131072, "32x64x64")])
def test_circular_conv_matches_oracle(dev, N, spec):
    """Circular convolution of period N (sffft_circconv_long_*): every output against the fp64
    circular convolution, both I/O types; with a zero second half of u and a zero-padded filter
    it equals the causal convolution.

    fp32 bound 6e-4: with no zero half in the transform input, each fp16 rounding carries about
    twice the noise energy per unit of output signal of the causal case (4.2e-4 there, so about
    sqrt(2) x 4.2e-4 here), with the same arithmetic."""
    import torch

    plan = sf.long_plan(spec)
    B, H = 4, 3
    rng = np.random.default_rng(N)
    u = rng.standard_normal((B, H, N)).astype(np.float32)
    k = (rng.standard_normal((H, N)) * np.exp(-np.arange(N) / (N / 8)) / np.sqrt(N)).astype(np.float32)
    ref = oracle.circ_conv(u, k[None])
    kf = sf.spectrum_circular(torch.from_numpy(k).to(dev), plan)
    for io in ("fp32", "bf16"):
        ud = torch.from_numpy(u).to(dev)
        if io == "bf16":
            ud = sf.to_bf16(ud)
        y = sf.circconv(ud, kf, plan).float().cpu().numpy()
        err = oracle.rel_l2(y, ref)
        print(f"case circular N={N} {spec} io={io} rel_l2={err:.3e}", flush=True)
        assert np.isfinite(err) and err <= (6e-4 if io == "fp32" else BOUND[io]), (N, spec, io, err)
    L = N // 2
    uc = u.copy()
    uc[..., L:] = 0
    kc = k.copy()
    kc[:, L:] = 0
    kfc = sf.spectrum_circular(torch.from_numpy(kc).to(dev), plan)
    y = sf.circconv(torch.from_numpy(uc).to(dev), kfc, plan).cpu().numpy()
    ref_causal = oracle.conv(uc[..., :L].copy(), kc[:, :L].copy())
    assert oracle.rel_l2(y[..., :L], ref_causal) <= 5e-4


@pytest.mark.parametrize("L,plan_of", [
    (128, lambda L: sf.default_plan(L)),
    (256, lambda L: sf.make_plan("16x32", 12, seqs=2, mode=1, channels=3)),
    (512, lambda L: sf.make_plan("64x16", 12, seqs=2, mode=1, channels=3)),
    (1024, lambda L: sf.default_plan(L)),
    (2048, lambda L: sf.default_plan(L)),
    (4096, lambda L: sf.default_plan(L)),
    (32768, lambda L: sf.default_plan(L))],
    ids=["L128-wave16x16", "L256-wave16x32", "L512-wave64x16", "L1024-wave", "L2048-wave64x64-spectraL2",
         "L4096-workgroup", "L32768-multipass"])
def test_complex_input_conv(dev, L, plan_of):
    """Complex causal convolution (sffft_spectrum_complex + a pair plan): complex u and complex
    k, every output against numpy's fp64 complex convolution. The wave plans run their
    whole-spectrum instantiation: R0 = 16 (one strip split at lane 8 in the Hermitian form),
    R1 = 32 with R0 = 16, 64x16, and 64x64 (whole spectra read through L2, first-kind
    fragments only). The same spectrum gathered from torch's natural-order spectrum
    (sffft_spectrum_from_natural_complex) agrees with it to fp32 rounding."""
    import torch

    plan = plan_of(L)
    Bc, H = 3, 4
    rng = np.random.default_rng(L + 1)
    x = (rng.standard_normal((Bc, H, L)) + 1j * rng.standard_normal((Bc, H, L))).astype(np.complex64)
    env = np.exp(-np.arange(L) / (L / 8)) / np.sqrt(L)
    k = ((rng.standard_normal((H, L)) + 1j * rng.standard_normal((H, L))) * env).astype(np.complex64)
    kd = torch.from_numpy(k).to(dev)
    kf = sf.spectrum_complex(kd, L, plan)
    if L <= 16384:
        kc = torch.fft.fft(torch.cat([kd, torch.zeros_like(kd)], 1), dim=1)  # zero-padded to 2L
        kf_nat = sf.spectrum_from_natural(kc, L, plan, complex_filter=True)
        # the spectrum's own transform and rocFFT's differ in their last bits: compare as values
        assert torch.allclose(torch.view_as_real(kf_nat), torch.view_as_real(kf), rtol=1e-5, atol=1e-6)
    y = sf.complex_conv(torch.from_numpy(x).to(dev), kf, plan).cpu().numpy().astype(np.complex128)
    x64, k64 = x.astype(np.complex128), k.astype(np.complex128)
    if L <= 4096:
        ref = np.stack([np.stack([np.convolve(x64[b, h], k64[h])[:L] for h in range(H)]) for b in range(Bc)])
    else:  # the same convolution through numpy's fp64 FFT, zero-padded to 2L (no wrap-around)
        ref = np.fft.ifft(np.fft.fft(x64, 2 * L) * np.fft.fft(k64, 2 * L)[None], axis=-1)[..., :L]
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    print(f"case complex L={L} {plan!r} rel_l2={err:.3e}", flush=True)
    assert err <= 5e-4, (L, repr(plan), err)
