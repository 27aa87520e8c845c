"""Race check of the fused kernels (the debug-barrier build the reference's __syncwarp-only
hand-off calls for, src/sffft.cu:273-279).

The wave pipeline passes data between the lanes of one wavefront through LDS (the row
loads' operand transpose, the output staging) and lets the pair loads of the first channel
stay in flight across the workgroup barrier; the workgroup kernel overwrites a row of LDS
its wavefront has just read. The product library relies on a wavefront's LDS operations
completing in issue order for these. libsffft_debug.so is the same source built with
SFFFT_DEBUG_BARRIERS, where each of those places waits for every outstanding LDS operation
(and the prologue for every load). Both libraries run every compiled plan on the same
inputs, through the C ABI, and must agree bit for bit: a result that depended on the
timing of one of those hand-offs would differ.
"""
import ctypes

import numpy as np
import pytest

import oracle
import sffft_amd as sf

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def run_with(lib, u, k, plan, complex_filter=False):
    """Spectrum and convolution through the given library's C ABI on the current stream."""
    import torch

    B, H, L = u.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    kf = torch.empty((H, 2 * L), dtype=torch.complex64, device=u.device)
    work = torch.empty_like(kf)
    if complex_filter:
        kr, ki = k.real.contiguous(), k.imag.contiguous()
        rc = lib.sffft_spectrum_complex(_ptr(kr), _ptr(ki), H, L, ctypes.byref(plan), _ptr(kf), _ptr(work), stream)
    else:
        rc = lib.sffft_spectrum(_ptr(k), H, L, ctypes.byref(plan), _ptr(kf), _ptr(work), stream)
    assert rc == 0, rc
    y = torch.empty_like(u)
    io = "f32" if u.dtype == torch.float32 else "bf16"
    if plan.mode == 2:
        wb = lib.sffft_work_bytes(B, H, L, ctypes.byref(plan))
        w = torch.empty(wb, dtype=torch.uint8, device=u.device)
        rc = getattr(lib, f"sffft_conv_long_{io}")(_ptr(u), _ptr(kf), _ptr(y), _ptr(w), wb, B, H, L,
                                                     ctypes.byref(plan), stream)
    else:
        name = f"sffft_conv_complex_{io}" if complex_filter else f"sffft_conv_{io}"
        rc = getattr(lib, name)(_ptr(u), _ptr(kf), _ptr(y), B, H, L, ctypes.byref(plan), stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return kf, y


@pytest.fixture(scope="module")
def libs():
    return sf.lib(), sf.load_library(sf.DEBUG_LIB_PATH)


def _cases():
    for L in sf.LENGTHS:
        for i, p in enumerate(sf.plans(L)):
            for acc in ((0, 1) if i < 2 else (0,)):
                yield L, p.replace(acc=acc)
    yield 32768, sf.default_plan(32768)


@pytest.mark.parametrize("L,plan", list(_cases()), ids=lambda x: repr(x) if not isinstance(x, int) else f"L{x}")
def test_debug_barrier_build_is_bit_identical(dev, libs, L, plan):
    import torch

    B, H = (4, 13) if plan.mode == 1 else (2, 5)
    u32, k = oracle.gen_inputs(B, H, L, seed=L + 3)
    kd = torch.from_numpy(k).to(dev)
    ud = torch.from_numpy(u32).to(dev)
    for io in ("fp32", "bf16"):
        print(f"case L={L} {plan!r} io={io}", flush=True)
        u = sf.to_bf16(ud) if io == "bf16" else ud
        kf0, y0 = run_with(libs[0], u, kd, plan)
        kf1, y1 = run_with(libs[1], u, kd, plan)
        assert torch.equal(torch.view_as_real(kf0), torch.view_as_real(kf1))
        assert torch.equal(y0, y1), (L, repr(plan), io)


@pytest.mark.parametrize("L", [1024, 2048])
def test_debug_barrier_build_full_batch(dev, libs, L):
    """The benchmark batch (B=8, H=768, three channels per workgroup, one pair per wavefront,
    every CU busy), where the first channel's loads cross the workgroup barrier."""
    import torch

    plan = sf.default_plan(L, "fp32", 8)
    g = torch.Generator(device=dev).manual_seed(L)
    u = torch.randn(8, 768, L, device=dev, generator=g)
    k = torch.randn(768, L, device=dev, generator=g) * torch.exp(-torch.arange(L, device=dev) / 256.0) / L ** 0.5
    for io in ("fp32", "bf16"):
        x = sf.to_bf16(u) if io == "bf16" else u
        _, y0 = run_with(libs[0], x, k, plan)
        _, y1 = run_with(libs[1], x, k, plan)
        assert torch.equal(y0, y1), (L, io)


def test_debug_barrier_build_complex_filter(dev, libs):
    """The wave pipeline's whole-spectrum instantiation (complex filters)."""
    import torch

    L = 1024
    plan = sf.default_plan(L, "fp32", 8)
    rng = np.random.default_rng(9)
    u = torch.from_numpy(rng.standard_normal((6, 7, L)).astype(np.float32)).to(dev)
    k = torch.from_numpy((rng.standard_normal((7, L)) + 1j * rng.standard_normal((7, L))).astype(np.complex64)).to(dev)
    _, y0 = run_with(libs[0], u, k, plan, complex_filter=True)
    _, y1 = run_with(libs[1], u, k, plan, complex_filter=True)
    assert torch.equal(y0, y1)
