"""sffft_spectrum_noalloc, the entry point that allocates nothing (no counterpart in the
reference; for callers that cannot call hipMalloc): through the C ABI, its output must be
bit-identical to sffft_spectrum's (same kernels, workspace from the library's static
scratch instead of the caller's buffer) on consecutive calls of decreasing size, the first
ones large enough to run in several chunks of channels, whatever the previous call left in
the scratch."""
import ctypes

import numpy as np
import pytest

import sffft_amd as sf

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def spectra(k, L, plan):
    import torch

    H = k.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ref = torch.full((H, 2 * L), 7.0 + 3.0j, dtype=torch.complex64, device=k.device)
    work = torch.empty_like(ref)
    assert sf.lib().sffft_spectrum(_ptr(k), H, L, ctypes.byref(plan), _ptr(ref), _ptr(work), stream) == 0
    got = torch.full((H, 2 * L), -5.0 - 1.0j, dtype=torch.complex64, device=k.device)
    assert sf.lib().sffft_spectrum_noalloc(_ptr(k), H, L, ctypes.byref(plan), _ptr(got), stream) == 0
    torch.cuda.synchronize()
    return ref, got


CALLS = [  # (L, H, plan): decreasing sizes; chunks = ceil(H / (32 MiB / (2L * 8)))
    (32768, 70, lambda L: sf.default_plan(L)),        # multi-pass plan, 2 chunks of 64 channels
    (16384, 300, lambda L: sf.default_plan(L)),       # workgroup plan, 3 chunks of 128
    (2048, 2100, lambda L: sf.default_plan(L)),       # wave plan: Hermitian halves, 3 chunks of 1024
    (1024, 5, lambda L: sf.default_plan(L)),          # one chunk
    (128, 3, lambda L: sf.make_plan("16x16", 2, seqs=1)),
]


def test_noalloc_spectrum_matches_the_allocating_entry(dev):
    import torch

    for L, H, plan_of in CALLS:
        plan = plan_of(L)
        chunk = min(H, SCRATCH_BYTES // (2 * L * 8))
        print(f"case noalloc spectrum L={L} H={H} {plan!r} chunks={-(-H // chunk)}", flush=True)
        k = torch.from_numpy(np.random.default_rng(L + H).standard_normal((H, L)).astype(np.float32)).to(dev)
        ref, got = spectra(k, L, plan)
        assert torch.equal(torch.view_as_real(got), torch.view_as_real(ref)), (L, H, repr(plan))


def test_noalloc_spectrum_argument_errors(dev):
    import torch

    k = torch.zeros(2, 1024, device=dev)
    kf = torch.empty(2, 2048, dtype=torch.complex64, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    plan = sf.default_plan(1024)
    f = sf.lib().sffft_spectrum_noalloc
    assert f(None, 2, 1024, ctypes.byref(plan), _ptr(kf), stream) == sf.SFFFT_EINVAL
    assert f(_ptr(k), 0, 1024, ctypes.byref(plan), _ptr(kf), stream) == sf.SFFFT_EINVAL
    assert f(_ptr(k), 2, 1000, ctypes.byref(plan), _ptr(kf), stream) == sf.SFFFT_EINVAL
