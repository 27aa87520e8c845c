"""The PyTorch operators over the C ABI (sffft_amd/torch_ops.py).

CPU: schemas, fake-tensor shape propagation, the tuned default plans, and the identities behind
the gradients (the adjoint of causal convolution is flip o causal_conv o flip, and equally the
same convolution with the conjugate spectrum, which the backward passes run), checked against
brute-force anti-causal correlations.
GPU: bit equality with the C-ABI path, torch.library.opcheck, the gradient against the oracle,
the spectrum cache, torch.compile and graph capture.
"""
import gc
import weakref

import numpy as np
import pytest
import torch

import oracle
import sffft_amd as sf
from sffft_amd import torch_ops


def test_schemas():
    assert str(torch.ops.sffft.conv.default._schema) == "sffft::conv(Tensor u, Tensor kf, int[] plan) -> Tensor"
    assert str(torch.ops.sffft.spectrum.default._schema) == \
        "sffft::spectrum(Tensor k, int[] plan, bool conj=False) -> Tensor"
    # registered from C++ (libsffft_torch.so): GPU kernels and autograd, no Python wrapper
    for op in (torch.ops.sffft.conv.default, torch.ops.sffft.spectrum.default):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA")
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Autograd")


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    p = torch_ops.plan_fields(sf.default_plan(1024))
    with FakeTensorMode():
        k = torch.empty(768, 1024, device="cuda")
        kf = torch.ops.sffft.spectrum(k, p)
        y = torch.ops.sffft.conv(torch.empty(8, 768, 1024, device="cuda", dtype=torch.bfloat16), kf, p)
        assert kf.shape == (768, 2048) and kf.dtype == torch.complex64
        assert y.shape == (8, 768, 1024) and y.dtype == torch.bfloat16


@pytest.mark.parametrize("L", sf.LENGTHS + sf.LONG_LENGTHS)
def test_default_plans_are_compiled(L):
    for io in ("fp32", "bf16"):
        for B in (8, 7):
            if L in sf.LONG_LENGTHS and B % 2:
                with pytest.raises(ValueError):  # multi-pass plans take pairs of sequences
                    sf.default_plan(L, io, B)
                continue
            p = sf.default_plan(L, io, B)
            assert sf.plan_check(L, p) == 0, (L, io, B, p)
            assert B % p.seqs == 0


def test_adjoint_is_flipped_causal_convolution():
    rng = np.random.default_rng(3)
    B, H, L = 2, 3, 64
    dy = rng.standard_normal((B, H, L)).astype(np.float32)
    k = rng.standard_normal((H, L)).astype(np.float32)
    # brute force: du[b,h,m] = sum_{n >= m} dy[b,h,n] k[h,n-m]
    du = np.zeros((B, H, L))
    for m in range(L):
        for n in range(m, L):
            du[:, :, m] += dy[:, :, n].astype(np.float64) * k[None, :, n - m]
    got = oracle.direct_conv(dy[:, :, ::-1].copy(), k)[:, :, ::-1]
    assert np.abs(got - du).max() < 1e-9 * np.abs(du).max()
    # a plausible mistake (no output flip) fails the same check
    wrong = oracle.direct_conv(dy[:, :, ::-1].copy(), k)
    assert np.abs(wrong - du).max() > 1e-3 * np.abs(du).max()


def test_correlation_is_convolution_with_the_conjugate_spectrum():
    """The adjoint the backward passes run: with N = 2L zero padding,
    sum_{n >= m} x[n] k[n - m] = IDFT_N(DFT_N(x) * conj(DFT_N(k)))[m] for m < L, i.e. the causal
    convolution machinery with the filter's spectrum conjugated (no time reversal)."""
    rng = np.random.default_rng(9)
    L = 40
    N = 2 * L
    x = rng.standard_normal(L)
    k = rng.standard_normal(L)
    corr = np.array([sum(x[n] * k[n - m] for n in range(m, L)) for m in range(L)])
    X = np.fft.fft(x, N)
    K = np.fft.fft(k, N)
    got = np.fft.ifft(X * np.conj(K))[:L]
    assert np.abs(got.imag).max() < 1e-12 and np.abs(got.real - corr).max() < 1e-12 * np.abs(corr).max()
    # the plain spectrum gives the causal convolution instead (the mistake this guards against)
    wrong = np.fft.ifft(X * K)[:L].real
    assert np.abs(wrong - corr).max() > 1e-3 * np.abs(corr).max()


def test_filter_gradient_is_flipped_causal_convolution():
    """dk[h,j] = sum_b sum_{n>=j} dy[b,h,n] u[b,h,n-j] equals flip(causal_conv(flip(dy), u))
    summed over b, with u as a per-sequence filter: the identity filter_grad runs on."""
    rng = np.random.default_rng(5)
    B, H, L = 3, 2, 48
    dy = rng.standard_normal((B, H, L)).astype(np.float32)
    u = rng.standard_normal((B, H, L)).astype(np.float32)
    dk = np.zeros((H, L))
    for j in range(L):
        for n in range(j, L):
            dk[:, j] += (dy[:, :, n].astype(np.float64) * u[:, :, n - j]).sum(0)
    # one channel per (b, h) sequence, batch of one
    r = oracle.direct_conv(dy[:, :, ::-1].reshape(1, B * H, L).copy(), u.reshape(B * H, L))
    got = r.reshape(B, H, L)[:, :, ::-1].sum(0)
    assert np.abs(got - dk).max() < 1e-9 * np.abs(dk).max()
    # plausible mistakes (no output flip; u and dy exchanged) fail the same check
    wrong = r.reshape(B, H, L).sum(0)
    assert np.abs(wrong - dk).max() > 1e-3 * np.abs(dk).max()
    r2 = oracle.direct_conv(u[:, :, ::-1].reshape(1, B * H, L).copy(), dy.reshape(B * H, L))
    wrong2 = r2.reshape(B, H, L)[:, :, ::-1].sum(0)
    assert np.abs(wrong2 - dk).max() > 1e-3 * np.abs(dk).max()


# ---- GPU ----------------------------------------------------------------------------------

def _inputs(dev, B, H, L, seed):
    u, k = oracle.gen_inputs(B, H, L, seed=seed)
    return torch.from_numpy(u).to(dev), torch.from_numpy(k).to(dev), u, k


@pytest.mark.gpu
@pytest.mark.parametrize("L,io", [(1024, "fp32"), (4096, "bf16"), (32768, "fp32")])
def test_ops_match_the_c_abi(dev, L, io):
    u, k, _, _ = _inputs(dev, 4, 13, L, seed=L)
    if io == "bf16":
        u = u.to(torch.bfloat16)
    plan = sf.default_plan(L, io, 4)
    p = torch_ops.plan_fields(plan)
    kf = torch.ops.sffft.spectrum(k, p)
    assert torch.equal(torch.view_as_real(kf), torch.view_as_real(sf.spectrum(k, L, plan)))
    assert torch.equal(torch.ops.sffft.conv(u, kf, p), sf.conv(u, kf, plan))
    # the conjugate spectrum is the conjugate of the spectrum, value for value
    kc = torch.ops.sffft.spectrum(k, p, True)
    assert torch.equal(torch.view_as_real(kc), torch.view_as_real(torch.conj_physical(kf)))


@pytest.mark.gpu
def test_opcheck(dev):
    u, k, _, _ = _inputs(dev, 2, 3, 256, seed=1)
    p = torch_ops.plan_fields(sf.default_plan(256, "fp32", 2))
    kf = torch.ops.sffft.spectrum(k, p)
    torch.library.opcheck(torch.ops.sffft.spectrum.default, (k, p))
    torch.library.opcheck(torch.ops.sffft.spectrum.default, (k, p, True))
    torch.library.opcheck(torch.ops.sffft.conv.default, (u, kf, p))
    torch.library.opcheck(torch.ops.sffft.conv.default, (u.clone().requires_grad_(), kf, p))


@pytest.mark.gpu
@pytest.mark.parametrize("L", [512, 4096, 32768])
def test_input_gradient(dev, L):
    B, H = (4, 5) if L <= 16384 else (2, 3)
    u, k, _, k_np = _inputs(dev, B, H, L, seed=11)
    w = torch.randn(B, H, L, device=dev, generator=torch.Generator(device=dev).manual_seed(2))
    lc = torch_ops.LongConv()
    u.requires_grad_()
    (lc(u, k) * w).sum().backward()
    # du[b,h,m] = sum_{n>=m} w[b,h,n] k[h,n-m], in fp64
    w_np = w.cpu().numpy()
    ref = oracle.conv(w_np[:, :, ::-1].copy(), k_np)[:, :, ::-1]
    err = oracle.rel_l2(u.grad.cpu().numpy(), ref)
    print(f"L={L} input-gradient rel_l2={err:.3e}", flush=True)
    assert err <= 5e-4


@pytest.mark.gpu
@pytest.mark.parametrize("L,io", [(512, "fp32"), (4096, "fp32"), (1024, "bf16"), (32768, "fp32")])
def test_filter_gradient(dev, L, io):
    B, H = (4, 5) if L <= 16384 else (2, 3)
    u, k, u_np, k_np = _inputs(dev, B, H, L, seed=13)
    if io == "bf16":
        u = u.to(torch.bfloat16)
        u_np = u.float().cpu().numpy()
    w = torch.randn(B, H, L, device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    k.requires_grad_()
    u.requires_grad_()
    lc = torch_ops.LongConv()
    (lc(u, k).float() * w).sum().backward()
    # dk[h,j] = sum_b sum_{n>=j} w[b,h,n] u[b,h,n-j] in fp64 (the identity is pinned on the CPU)
    w_np = w.cpu().numpy()
    r = oracle.conv(w_np[:, :, ::-1].reshape(1, B * H, L).copy(), u_np.reshape(B * H, L))
    ref = r.reshape(B, H, L)[:, :, ::-1].sum(0)
    err = oracle.rel_l2(k.grad.cpu().numpy(), ref)
    print(f"L={L} {io} filter-gradient rel_l2={err:.3e}", flush=True)
    assert err <= (5e-4 if io == "fp32" else 3e-3)
    assert u.grad is not None and u.grad.dtype == u.dtype


@pytest.mark.gpu
def test_spectrum_op_has_no_gradient(dev):
    _, k, _, _ = _inputs(dev, 2, 3, 256, seed=4)
    k.requires_grad_()
    p = torch_ops.plan_fields(sf.default_plan(256, "fp32", 2))
    kf = torch.ops.sffft.spectrum(k, p)
    with pytest.raises(RuntimeError, match="no gradient"):
        torch.view_as_real(kf).sum().backward()


@pytest.mark.gpu
def test_filter_training_step_refreshes_spectrum(dev):
    u, k, _, _ = _inputs(dev, 2, 3, 1024, seed=8)
    k.requires_grad_()
    lc = torch_ops.LongConv()
    opt = torch.optim.SGD([k], lr=0.1)
    y0 = lc(u, k)
    y0.square().sum().backward()
    opt.step()
    assert lc.spectra_computed == 1
    y1 = lc(u, k)  # the optimizer changed k in place: a new spectrum
    assert lc.spectra_computed == 2 and not torch.equal(y0, y1)
    y2 = lc(u, k)
    assert lc.spectra_computed == 2 and torch.equal(y1, y2)


@pytest.mark.gpu
def test_spectrum_cache(dev):
    u, k, _, _ = _inputs(dev, 2, 3, 1024, seed=5)
    lc = torch_ops.LongConv()
    y1 = lc(u, k)
    y2 = lc(u, k)
    assert lc.spectra_computed == 1 and torch.equal(y1, y2)
    k.mul_(2.0)  # in place: the version moves, the spectrum is recomputed
    y3 = lc(u, k)
    assert lc.spectra_computed == 2
    assert torch.allclose(y3, 2 * y1, rtol=0, atol=1e-5 * float(y1.abs().max()))
    k2 = k.clone()
    lc(u, k2)
    assert lc.spectra_computed == 3
    # a freed filter drops its entry; a dropped LongConv releases its spectra even while
    # the filters it has seen live on
    del k2
    gc.collect()
    assert len(lc._cache) == 1
    kf = weakref.ref(lc._cache[id(k)][2])
    owner = weakref.ref(lc)
    del lc
    gc.collect()
    assert owner() is None and kf() is None
    assert k.is_cuda  # the filter itself is untouched


@pytest.mark.gpu
def test_longconv_without_gradients(dev):
    """LongConv with and without autograd recording gives the operator's outputs bit for bit, and
    a plan set on the layer replaces its cached default."""
    u, k, _, _ = _inputs(dev, 4, 5, 1024, seed=8)
    lc = torch_ops.LongConv()
    with torch.no_grad():
        y_fast = lc(u, k)
    p = torch_ops.plan_fields(lc.plan_for(u))
    y_op = torch.ops.sffft.conv(u, torch.ops.sffft.spectrum(k, p), p)
    ur = u.clone().requires_grad_()
    y_grad = lc(ur, k)
    assert not y_fast.requires_grad and y_grad.requires_grad
    assert torch.equal(y_fast, y_op) and torch.equal(y_grad.detach(), y_op)
    lc.plan = sf.make_plan("32x32", 4, seqs=2, mode=1, channels=1)
    assert lc.plan_for(u.to(torch.bfloat16)).waves == 4 and lc.plan_for(u).r0 == 32


@pytest.mark.gpu
def test_torch_compile(dev):
    u, k, _, _ = _inputs(dev, 2, 6, 512, seed=6)
    p = torch_ops.plan_fields(sf.default_plan(512, "fp32", 2))

    def f(u, k):
        return torch.ops.sffft.conv(u * 2.0, torch.ops.sffft.spectrum(k, p), p)

    eager = f(u, k)
    compiled = torch.compile(f, fullgraph=True, backend="aot_eager")(u, k)
    assert torch.equal(compiled, eager)


@pytest.mark.gpu
def test_graph_capture(dev):
    u, k, _, _ = _inputs(dev, 4, 6, 1024, seed=7)
    p = torch_ops.plan_fields(sf.default_plan(1024, "fp32", 4))
    kf = torch.ops.sffft.spectrum(k, p)
    eager = torch.ops.sffft.conv(u, kf, p)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = torch.ops.sffft.conv(u, kf, p)
    for i in range(3):
        y.zero_()
        torch.ops.sffft.conv(u * 0.5, kf, p)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
