"""Standalone transforms (sffft_fft_c2c, sffft_fft2_c2c) and the 2-D circular convolution
(sffft_circconv2d_f32) through the C ABI. The reference lists these as not exposed
(README.md:174), so there is no reference output to match: results are checked against
numpy's fp64 FFT, against closed forms (delta, constant, pure tones, which fix the sign
convention independently of numpy) and, for the convolution, against a brute-force fp64
direct sum. Each stage is evaluated in fp64 and stored as complex64, so the bound is a
relative L2 error of 1e-6 (transforms) and 1e-5 (convolution)."""
import numpy as np
import pytest

import sffft_amd as sf

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def crandn(rng, *shape):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)


@pytest.mark.parametrize("batch,N", [(3, 2), (5, 4), (7, 16), (4, 64), (3, 128), (6, 1024), (2, 4096), (3, 8192),
                                     (2, 65536), (1, 1 << 20), (1, 1 << 22), (1, 1 << 24)])
def test_fft_matches_numpy(batch, N):
    """Up to N = 2^24, whose six radix-16 stages fill the stage table exactly."""
    print(f"fft batch={batch} N={N}", flush=True)
    x = crandn(np.random.default_rng(N + batch), batch, N)
    X = sf.fft(torch.from_numpy(x).to(DEV)).cpu().numpy()
    ref = np.fft.fft(x.astype(np.complex128), axis=1)
    assert rel(X, ref) <= 1e-6
    xi = sf.fft(torch.from_numpy(X).to(DEV), inverse=True, scale=1.0 / N).cpu().numpy()
    assert rel(xi, x) <= 1e-6
    Xi = sf.fft(torch.from_numpy(x).to(DEV), inverse=True).cpu().numpy()
    assert rel(Xi, np.fft.ifft(x.astype(np.complex128), axis=1) * N) <= 1e-6


@pytest.mark.parametrize("N", [8, 512, 4096])
def test_fft_closed_forms(N):
    n = np.arange(N)
    delta = np.zeros((1, N), np.complex64)
    delta[0, 0] = 1
    const = np.ones((1, N), np.complex64)
    f = 3 % N
    tone = np.exp(2j * np.pi * f * n / N).astype(np.complex64)[None]
    X = sf.fft(torch.from_numpy(np.concatenate([delta, const, tone])).to(DEV)).cpu().numpy()
    assert np.abs(X[0] - 1).max() <= 1e-6
    e0 = np.zeros(N)
    e0[0] = N
    assert np.abs(X[1] - e0).max() <= 1e-6 * N
    ef = np.zeros(N)
    ef[f] = N  # forward sign -1: exp(+2 pi i f n / N) lands in bin f
    assert np.abs(X[2] - ef).max() <= 2e-6 * N
    Xi = sf.fft(torch.from_numpy(tone).to(DEV), inverse=True).cpu().numpy()
    ei = np.zeros(N)
    ei[(N - f) % N] = N  # inverse sign +1: the tone lands in bin -f
    assert np.abs(Xi[0] - ei).max() <= 2e-6 * N


@pytest.mark.parametrize("batch,N", [(3, 2), (64, 16), (9, 256), (5, 1024), (4, 2048), (3, 4096), (3, 8192),
                                     (2, 16384)])
def test_one_pass_matches_staged_path_bitwise(batch, N):
    """Contiguous sequences of N <= 16384 take the one-pass kernel (every stage in LDS); the
    same values as the columns of a matrix take the staged kernels. The stages do the
    same arithmetic, so the two agree bit for bit, forward and inverse with a scale."""
    print(f"one-pass vs staged batch={batch} N={N}", flush=True)
    x = crandn(np.random.default_rng(3 * N + batch), batch, N)
    rows = torch.from_numpy(x).to(DEV)
    cols = torch.from_numpy(np.ascontiguousarray(x.T)).to(DEV)
    for inverse, scale in ((False, 1.0), (True, 1.0 / N)):
        a = sf.fft(rows, inverse=inverse, scale=scale).cpu().numpy()
        b = np.ascontiguousarray(sf.fft(cols, inverse=inverse, scale=scale, dim=0).cpu().numpy().T)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (N, inverse)


@pytest.mark.parametrize("batch,N", [(2, 1 << 15), (3, 1 << 16), (2, 1 << 17), (2, 1 << 19), (2, 1 << 20),
                                     (2, 1 << 21), (2, 1 << 24)])
def test_two_pass_matches_staged_path_bitwise(batch, N):
    """Contiguous sequences of 16384 < N <= 2^24 take the two-pass kernels (the first stages
    on N1-point columns, then N2-point blocks, written in natural order); the same values as
    the columns of a matrix take one launch per stage. Same arithmetic in the same order:
    bit-identical, forward and inverse with a scale."""
    print(f"two-pass vs staged batch={batch} N={N}", flush=True)
    x = crandn(np.random.default_rng(N + 7 * batch), batch, N)
    rows = torch.from_numpy(x).to(DEV)
    cols = torch.from_numpy(np.ascontiguousarray(x.T)).to(DEV)
    for inverse, scale in ((False, 1.0), (True, 1.0 / N)):
        a = sf.fft(rows, inverse=inverse, scale=scale).cpu().numpy()
        b = np.ascontiguousarray(sf.fft(cols, inverse=inverse, scale=scale, dim=0).cpu().numpy().T)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (N, inverse)


@pytest.mark.parametrize("batch,N,stride,dist", [(3, 128, 2, 256), (3, 128, 3, 1), (2, 4096, 3, 12288),
                                                  (4, 256, 4, 1)])
def test_fft_layout_family_edges(batch, N, stride, dist):
    """The edges of the two layout families sffft_fft_c2c takes: whole sequences exactly
    N * stride apart, and sequences interleaved exactly batch * dist per element step. Gaps
    in the layout stay untouched."""
    import ctypes

    print(f"fft layout batch={batch} N={N} stride={stride} dist={dist}", flush=True)
    extent = (batch - 1) * dist + (N - 1) * stride + 1
    rng = np.random.default_rng(N + stride)
    buf = crandn(rng, extent)
    idx = np.array([[b * dist + n * stride for n in range(N)] for b in range(batch)])
    x = torch.from_numpy(buf).to(DEV)
    X = torch.full_like(x, complex(7.0, -3.0))
    work = torch.empty(max(sf.lib().sffft_fft_work_bytes(batch, N), 16), dtype=torch.uint8, device=DEV)
    rc = sf.lib().sffft_fft_c2c(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(X.data_ptr()),
                                ctypes.c_void_p(work.data_ptr()), work.numel(), batch, N, stride, dist, 0, 1.0,
                                ctypes.c_void_p(0))
    assert rc == sf.SFFFT_OK, sf.strerror(rc)
    out = X.cpu().numpy()
    ref = np.fft.fft(buf[idx].astype(np.complex128), axis=1)
    assert rel(out[idx], ref) <= 1e-6
    untouched = np.ones(extent, bool)
    untouched[idx.reshape(-1)] = False
    assert np.all(out[untouched] == np.complex64(complex(7.0, -3.0)))


@pytest.mark.parametrize("L", [128, 1024, 8192, 16384, 32768])
def test_spectrum_matches_fp64_dft(L):
    """sffft_spectrum against the same kernel-order gather (sffft_spectrum_from_natural)
    applied to numpy's fp64 DFT of the zero-padded filters, rounded to complex64, for every
    compiled plan. Up to N = 16384 the spectrum runs the one-pass transform above, beyond it
    the two-pass transform with the spectrum's own rows as workspace (L = 16384: workgroup
    plans; L = 32768: multi-pass plans)."""
    print(f"spectrum L={L}", flush=True)
    H = 7
    k = np.random.default_rng(L + 1).standard_normal((H, L)).astype(np.float32)
    nat = np.fft.fft(np.pad(k.astype(np.float64), ((0, 0), (0, L))), axis=1).astype(np.complex64)
    kd = torch.from_numpy(k).to(DEV)
    nat_d = torch.from_numpy(nat).to(DEV)
    for plan in sf.plans(L):
        got = sf.spectrum(kd, L, plan).cpu().numpy()
        ref = sf.spectrum_from_natural(nat_d, L, plan).cpu().numpy()
        assert rel(got, ref) <= 1e-6, (L, plan, rel(got, ref))


def test_fft_in_place_and_columns():
    rng = np.random.default_rng(7)
    x = crandn(rng, 4, 2048)
    t = torch.from_numpy(x).to(DEV)
    sf.fft(t, out=t)
    assert rel(t.cpu().numpy(), np.fft.fft(x.astype(np.complex128), axis=1)) <= 1e-6
    for N, C in ((128, 5), (4096, 3), (32, 64)):
        m = crandn(rng, N, C)
        X = sf.fft(torch.from_numpy(m).to(DEV), dim=0).cpu().numpy()
        assert rel(X, np.fft.fft(m.astype(np.complex128), axis=0)) <= 1e-6


@pytest.mark.parametrize("shape", [(3, 64, 128), (2, 256, 32), (1, 2, 4096), (2, 128, 128), (1, 4, 2)])
def test_fft2_matches_numpy(shape):
    print(f"fft2 shape={shape}", flush=True)
    x = crandn(np.random.default_rng(sum(shape)), *shape)
    t = torch.from_numpy(x).to(DEV)
    X = sf.fft2(t).cpu().numpy()
    ref = np.fft.fft2(x.astype(np.complex128))
    assert rel(X, ref) <= 1e-6
    P = shape[1] * shape[2]
    sf.fft2(torch.from_numpy(X).to(DEV), inverse=True, scale=1.0 / P, out=t)  # t overwritten
    assert rel(t.cpu().numpy(), x) <= 1e-6
    sf.fft2(t, out=t)  # in place
    assert rel(t.cpu().numpy(), ref) <= 1e-6


def circ2_direct(u, k):
    B, H, N0, N1 = u.shape
    y = np.zeros((B, H, N0, N1))
    for a in range(N0):
        for c in range(N1):
            y += u[:, :, a, c][:, :, None, None] * np.roll(np.roll(k, a, axis=1), c, axis=2)[None]
    return y


def test_circconv2d_brute_force():
    rng = np.random.default_rng(11)
    u = rng.standard_normal((2, 3, 4, 8)).astype(np.float32)
    k = rng.standard_normal((3, 4, 8)).astype(np.float32)
    y = sf.circconv2d(torch.from_numpy(u).to(DEV), torch.from_numpy(k).to(DEV)).cpu().numpy()
    assert rel(y, circ2_direct(u.astype(np.float64), k.astype(np.float64))) <= 1e-5


@pytest.mark.parametrize("shape", [(2, 3, 64, 128), (1, 2, 256, 256), (4, 1, 16, 1024)])
def test_circconv2d_matches_fp64_fft(shape):
    print(f"circconv2d shape={shape}", flush=True)
    rng = np.random.default_rng(shape[2])
    u = rng.standard_normal(shape).astype(np.float32)
    k = (rng.standard_normal(shape[1:]) / np.sqrt(shape[2] * shape[3])).astype(np.float32)
    y = sf.circconv2d(torch.from_numpy(u).to(DEV), torch.from_numpy(k).to(DEV)).cpu().numpy()
    ref = np.fft.ifft2(np.fft.fft2(u.astype(np.float64)) * np.fft.fft2(k.astype(np.float64))[None]).real
    assert rel(y, ref) <= 1e-5
