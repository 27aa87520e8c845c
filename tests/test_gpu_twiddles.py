"""Direct pins of the twiddle factors, the reference's twid() (src/sffft.cu:106-113):
w^e = exp(-2 pi i e / N) with e the product of an index and a frequency digit.

- The wave pipeline's fp32 tables (built in fp64 on the host, read back through
  sffft_twiddle_table), and their fp16 form for the fp16-accumulation kernels (within half
  an fp16 ulp). Every entry of TW1 = sc0 w^(m k0) and TW2 = sc0 sc1 w^(k0 n1) at its
  slot of the documented layout (tile, lane (c, g), value v; m = 16 mt + 4 g + v,
  k0 = 16 nt + c for TW1, k0 = 16 s + 4 g + v, n1 = 16 t + c for TW2), against numpy's fp64
  cos/sin of the exact angle: within one fp32 rounding, |err| <= 2^-24 |w|.
- The workgroup kernel's in-register twiddles: v_sin/v_cos of the exactly reduced angle in
  revolutions, a three-step complex recurrence over the four values of a lane, and the
  row-to-row recurrence of its phase-2 loop. sffft_twiddle_probe evaluates them on the GPU
  with the kernel's own code; against fp64 exp(-2 pi i e / N), max |err| <= 4e-6 for the base
  values and <= 1.2e-5 after 15 row steps (the longest chain in a kernel is 7).

Budget: one fp16 rounding, of which a two-stage transform has three and a three-stage one
five, has a relative error up to 2^-11 = 4.9e-4, so the in-register twiddles use at most
about 2.5% of one rounding. The bounds discriminate: a wrong sign of the angle (a
conjugation) or an exponent one step off (2 pi / N >= 1.9e-4 at N = 32768) is more than 15
times the bound; the planted versions of both, applied to the fp64 reference on the CPU,
fail the same comparisons.
"""
import ctypes

import numpy as np
import pytest

import sffft_amd as sf

pytestmark = pytest.mark.gpu

BASE_BOUND = 4e-6
ROWS_BOUND = 1.2e-5
ROWS = 15


def _wave_reference(r0, r1):
    """(TW1, TW2) as complex128 [tile][lane][v] from the definition, and the scales."""
    N, ST, MT = r0 * r1, r0 // 16, r1 // 16
    sc0, sc1 = 1 / np.sqrt(r0), 1 / np.sqrt(r1)
    lane = np.arange(64)
    c, g = lane & 15, lane >> 4
    v = np.arange(4)
    tw1 = np.empty((MT * ST, 64, 4), np.complex128)
    for mt in range(MT):
        for nt in range(ST):
            m = 16 * mt + 4 * g[:, None] + v[None]
            k0 = (16 * nt + c)[:, None]
            tw1[mt * ST + nt] = sc0 * np.exp(-2j * np.pi * ((m * k0) % N) / N)
    tw2 = np.empty((ST * MT, 64, 4), np.complex128)
    for s in range(ST):
        for t in range(MT):
            k0 = 16 * s + 4 * g[:, None] + v[None]
            n1 = (16 * t + c)[:, None]
            tw2[s * MT + t] = sc0 * sc1 * np.exp(-2j * np.pi * ((k0 * n1) % N) / N)
    return tw1, tw2


def _unpack(raw, ntiles, split):
    """Table floats -> complex64 [tile][lane][v] of the split or paired layout (tw_index)."""
    f4 = raw.reshape(-1, 4)
    out = np.empty((ntiles, 64, 4), np.complex64)
    for tile in range(ntiles):
        for q in range(2):
            idx = (tile * 2 + q) * 64 + np.arange(64) if split else (tile * 64 + np.arange(64)) * 2 + q
            out[tile, :, 2 * q] = f4[idx, 0] + 1j * f4[idx, 1]
            out[tile, :, 2 * q + 1] = f4[idx, 2] + 1j * f4[idx, 3]
    return out


def _unpack_h(raw, ntiles):
    """fp16 table (layout 2): h8 per (tile, lane) = [wr0..wr3 | wi0..wi3]."""
    h = raw.reshape(ntiles, 64, 8).astype(np.float64)
    return h[..., :4] + 1j * h[..., 4:]


def _fp16_rounding_ok(got, want):
    tol = 2.0 ** -11 * np.abs(want) * (1 + 1e-6) + 2.0 ** -25  # half an ulp, subnormals included
    return bool(np.all(np.abs(got.real - want.real) <= tol) and np.all(np.abs(got.imag - want.imag) <= tol))


def _fp32_rounding_ok(got, want):
    tol = 2.0 ** -24 * np.abs(want) * (1 + 1e-6) + 1e-30
    return bool(np.all(np.abs(got.real - want.real) <= tol) and np.all(np.abs(got.imag - want.imag) <= tol))


def _table_plans():
    seen = set()
    for L in sf.LENGTHS:
        for p in sf.plans(L):
            if p.mode == 1 and (p.r0, p.r1) not in seen:
                seen.add((p.r0, p.r1))
                yield p.r0, p.r1, not (p.r0 == 64 and p.r1 == 64)  # the wave kernels' layout
    for L in sf.LONG_LENGTHS:  # the multi-pass row pass: paired layout of its row plan
        for p in sf.plans(L):
            if (p.r1, p.r2, False) not in seen:
                seen.add((p.r1, p.r2, False))
                yield p.r1, p.r2, False


@pytest.mark.parametrize("r0,r1,split", list(_table_plans()))
def test_wave_twiddle_tables(r0, r1, split):
    N = r0 * r1
    raw = np.zeros(N * 4, np.float32)
    rc = sf.lib().sffft_twiddle_table(r0, r1, 1 if split else 0, raw.ctypes.data_as(ctypes.c_void_p), raw.nbytes)
    assert rc == sf.SFFFT_OK, sf.strerror(rc)
    ntiles = (r0 // 16) * (r1 // 16)
    got1 = _unpack(raw[:2 * N], ntiles, split)
    got2 = _unpack(raw[2 * N:], ntiles, split)
    want1, want2 = _wave_reference(r0, r1)
    err = max(np.abs(got1 - want1).max(), np.abs(got2 - want2).max())
    print(f"twiddle table {r0}x{r1} split={split}: max |err| {err:.2e}", flush=True)
    assert _fp32_rounding_ok(got1, want1) and _fp32_rounding_ok(got2, want2), (r0, r1, split)
    # planted mistakes in the reference fail the same check
    assert not _fp32_rounding_ok(got1, np.conj(want1))
    assert not _fp32_rounding_ok(got1, want1 * np.exp(-2j * np.pi / N))  # exponent one step off


@pytest.mark.parametrize("r0,r1", sorted({(r0, r1) for r0, r1, split in _table_plans() if split or r0 == r1 == 64}))
def test_wave_twiddle_tables_fp16(r0, r1):
    """The fp16 tables of the fp16-accumulation wave kernels: the same values rounded to
    fp16, within half an fp16 ulp of the fp64 definition."""
    N = r0 * r1
    raw = np.zeros(N * 4, np.float16)
    rc = sf.lib().sffft_twiddle_table(r0, r1, 2, raw.ctypes.data_as(ctypes.c_void_p), raw.nbytes)
    assert rc == sf.SFFFT_OK, sf.strerror(rc)
    ntiles = (r0 // 16) * (r1 // 16)
    got1, got2 = _unpack_h(raw[:2 * N], ntiles), _unpack_h(raw[2 * N:], ntiles)
    want1, want2 = _wave_reference(r0, r1)
    print(f"fp16 twiddle table {r0}x{r1}: max |err| {max(np.abs(got1 - want1).max(), np.abs(got2 - want2).max()):.2e}",
          flush=True)
    assert _fp16_rounding_ok(got1, want1) and _fp16_rounding_ok(got2, want2), (r0, r1)
    assert not _fp16_rounding_ok(got1, np.conj(want1))
    assert not _fp16_rounding_ok(got1, want1 * np.exp(-2j * np.pi / N))


def _probe(dev, N, q, sc):
    import torch

    qd = torch.from_numpy(q.astype(np.int32)).to(dev)
    out = torch.empty((len(q), ROWS + 1, 4, 2), dtype=torch.float32, device=dev)
    rc = sf.lib().sffft_twiddle_probe(N, sf._ptr(qd), len(q), ROWS, sc, sf._ptr(out), sf._stream())
    assert rc == sf.SFFFT_OK, sf.strerror(rc)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    return o[..., 0] + 1j * o[..., 1]


@pytest.mark.parametrize("N", [256, 512, 1024, 2048, 4096, 8192, 16384, 32768])
def test_workgroup_kernel_twiddles(dev, N):
    rng = np.random.default_rng(N)
    n = 4096
    q = np.stack([rng.integers(0, N * 32, n), rng.integers(0, N, n), rng.integers(0, N, n),
                  rng.integers(0, N, n)], 1)
    # the reduction boundaries and the quarter and eighth turns
    special = [0, 1, N // 8, N // 4, N // 2 - 1, N // 2, N // 2 + 1, 3 * N // 4, N - 1]
    q[:len(special), 0] = special
    q[len(special):2 * len(special), 1] = special
    sc = float(np.float32(1 / np.sqrt(32.0)))  # a stage scale, as the kernel passes
    got = _probe(dev, N, q, sc) / sc  # compared as values of unit size
    e0, st, f0, fs = (q[:, i, None].astype(np.int64) for i in range(4))
    v = np.arange(4)[None]
    e = (e0 + st * v) % N
    f = (f0 + fs * v) % N
    r = np.arange(ROWS + 1)[None, :, None]
    want = np.exp(-2j * np.pi * ((e[:, None] + r * f[:, None]) % N) / N)
    base = np.abs(got[:, 0] - want[:, 0]).max()
    rows = np.abs(got - want).max()
    print(f"in-register twiddles N={N}: base max |err| {base:.2e}, after {ROWS} row steps {rows:.2e}", flush=True)
    assert base <= BASE_BOUND and rows <= ROWS_BOUND, (base, rows)
    # planted mistakes in the reference fail: conjugated angle, exponent one step off
    assert np.abs(got[:, 0] - np.conj(want[:, 0])).max() > 15 * BASE_BOUND
    assert np.abs(got[:, 0] - np.exp(-2j * np.pi * ((e + 1) % N) / N)).max() > 15 * BASE_BOUND
