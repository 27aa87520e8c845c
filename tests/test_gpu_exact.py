"""Bit-exact checks of the pure index and byte work on the GPU, through the C ABI:

- sffft_spectrum_from_natural (the replacement of permuteK, src/sffft.cu:283-288) on
  index-coded spectra: every output slot holds exactly the scaled value of the frequency
  the kernel order assigns to it, for every compiled plan of every mode (workgroup
  kernel, wave pipeline with its Hermitian half spectrum, multi-pass rows);
- the half spectrum of a wave plan equals, value for value, the whole spectrum that
  sffft_spectrum_complex writes for the same real filter and a zero imaginary part;
- sffft_to_bf16 (src/sffft.cu:306,364) against IEEE round-to-nearest-even on a bit
  pattern sweep, ties, overflow, infinities and NaNs;
- the device DFT coefficient table (the cached DFT matrices, src/sffft.cu:349-362): every
  complex and real-input fragment against fp16(fp32(cos)), fp16(fp32(sin)) of the exact
  angle from numpy.
"""
import numpy as np
import pytest

import sffft_amd as sf

pytestmark = pytest.mark.gpu


def last_stage_scale(p):
    """The factor the gather folds in: 1/sqrt(R) of the last forward radix; square wave
    plans and square multi-pass row plans carry 1/R (their shared twiddle table's factor)."""
    R = p.r2 if p.r2 > 1 else p.r1
    if p.mode == 2:
        return np.float32(1.0 / R if p.r1 == p.r2 else 1.0 / np.sqrt(R))
    if p.mode == 1 and p.r0 == p.r1:
        return np.float32(1.0 / R)
    return np.float32(1.0 / np.sqrt(R))


def kernel_order(p):
    """(frequency, conjugated) of every complex slot of one channel's kernel-order spectrum,
    from the digit order of src/sffft.cu:283-288 (frequency f = d0 + R0 d1 + R0 R1 d2) and
    each kernel's consumption order; frequency -1 marks padding."""
    r0, r1, r2 = p.r0, p.r1, p.r2
    N = r0 * r1 * r2
    out = []
    if p.mode == 1:  # Hermitian half (WavePlan::hs_index)
        MT = r1 // 16
        pitch = 8 * MT + 1
        for k0 in range(r0 // 2 + 1):
            for rem in range(pitch):
                for e in range(2):
                    if rem == pitch - 1:
                        out.append((-1, False))
                        continue
                    g, q, kt = rem & 3, (rem >> 2) & 1, rem >> 3
                    k1 = 16 * kt + 4 * g + 2 * q + e
                    if k0 == r0 // 2:
                        out.append((k0 + r0 * (r1 - 1 - k1), True))
                    else:
                        out.append((k0 + r0 * k1, False))
        return out
    for idx in range(N):
        if p.mode == 2:  # row k1 of the column radix r0, each row in the wave order over r1 x r2
            NR = r1 * r2
            row, i = divmod(idx, NR)
            e, lane, rest = i & 1, (i >> 1) & 63, i >> 7
            q, tile, MT = rest & 1, rest >> 1, r2 // 16
            c, g = lane & 15, lane >> 4
            a0 = 16 * (tile // MT) + c
            a1 = 16 * (tile % MT) + 4 * g + 2 * q + e
            out.append((row + r0 * (a0 + r1 * a1), False))
            continue
        v, lane, rest = idx & 3, (idx >> 2) & 63, idx >> 8
        c, g = lane & 15, lane >> 4
        if r2 == 1:
            T1 = r1 // 16
            mt, s = rest % T1, rest // T1
            k0, k1, k2 = 16 * s + c, 16 * mt + 4 * g + v, 0
        else:
            T1, T2 = r1 // 16, r2 // 16
            mt, t1 = rest % T2, (rest // T2) % T1
            k0, k1, k2 = rest // (T2 * T1), 16 * t1 + c, 16 * mt + 4 * g + v
        out.append((k0 + r0 * k1 + r0 * r1 * k2, False))
    return out


def all_plans():
    for L in sf.LENGTHS:
        for p in sf.plans(L):
            yield L, p
    for L in sf.LONG_LENGTHS:
        for p in sf.plans(L):
            yield L, p


@pytest.mark.parametrize("L,plan", list(all_plans()), ids=lambda x: repr(x) if not isinstance(x, int) else f"L{x}")
def test_spectrum_from_natural_is_the_digit_permutation(dev, L, plan):
    import torch

    H, N = 3, 2 * L
    f = np.arange(N, dtype=np.float32)
    h = np.arange(H, dtype=np.float32)[:, None]
    kc = np.empty((H, N), np.complex64)
    kc.real = f[None] + 1.0  # frequency code: exact integers below 2^24
    kc.imag = np.broadcast_to(-(h + 1.0) * np.float32(1 << 20), (H, N))  # channel code
    kc_d = torch.from_numpy(kc).to(dev)
    kf = sf.spectrum_from_natural(kc_d, L, plan).cpu().numpy()
    order = kernel_order(plan)
    n = len(order)
    sc = last_stage_scale(plan)
    freq = np.array([o[0] for o in order])
    conj = np.array([o[1] for o in order])
    assert kf.shape == (H, N), "one row per channel"
    for ch in range(H):
        got = kf[ch, :n]
        # a Hermitian half leaves the rest of its channel's row zero
        assert np.all(kf[ch, n:] == 0), (L, plan)
        pad = freq < 0
        assert np.all(got[pad] == 0), "padding slots are zero"
        fr = freq[~pad]
        re = kc[ch, fr].real.astype(np.float32) * sc
        im = np.where(conj[~pad], -kc[ch, fr].imag.astype(np.float32), kc[ch, fr].imag.astype(np.float32)) * sc
        assert np.array_equal(got[~pad].real.view(np.uint32), re.astype(np.float32).view(np.uint32)), (L, plan)
        assert np.array_equal(got[~pad].imag.view(np.uint32), im.astype(np.float32).view(np.uint32)), (L, plan)
    # every frequency appears: the whole spectrum, or for the Hermitian half every
    # frequency or its partner N - f
    seen = set(int(x) for x in freq[freq >= 0])
    if plan.mode == 1:
        assert all(x in seen or (N - x) % N in seen for x in range(N))
    else:
        assert seen == set(range(N))


@pytest.mark.parametrize("L", [128, 256, 512, 1024, 2048])
def test_half_spectrum_matches_whole_spectrum(dev, L):
    import torch

    H = 5
    k = torch.from_numpy(np.random.default_rng(L).standard_normal((H, L)).astype(np.float32)).to(dev)
    for plan in [p for p in sf.plans(L) if p.mode == 1]:
        half = sf.spectrum(k, L, plan).cpu().numpy()
        whole = sf.spectrum_complex(torch.complex(k, torch.zeros_like(k)), L, plan).cpu().numpy()
        order = kernel_order(plan)
        n = len(order)
        # the whole spectrum's order (sp_index): tile (s, kt), float4 q, lane (c, g), value e
        MT = plan.r1 // 16
        pos = {}
        for idx in range(2 * L):
            e, lane, rest = idx & 1, (idx >> 1) & 63, idx >> 7
            q, tile = rest & 1, rest >> 1
            c, g = lane & 15, lane >> 4
            k0 = 16 * (tile // MT) + c
            k1 = 16 * (tile % MT) + 4 * g + 2 * q + e
            pos[k0 + plan.r0 * k1] = idx
        for ch in range(H):
            got = half[ch, :n]
            assert np.all(half[ch, n:] == 0)
            for i, (fr, cj) in enumerate(order):
                if fr < 0:
                    continue
                w = whole[ch, pos[fr]]
                w = np.conj(w) if cj else w
                # equal values (the whole spectrum adds i * 0 for the zero imaginary filter,
                # which may turn a -0.0 into +0.0)
                assert got[i] == w, (plan, ch, i, got[i], w)


def bf16_rne(x):
    """IEEE binary32 -> bfloat16 round to nearest, ties to even, on the bit pattern; NaNs
    stay NaN (quiet)."""
    b = x.view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return r, nan


def test_to_bf16_round_to_nearest_even(dev):
    import torch

    rng = np.random.default_rng(3)
    bits = np.concatenate([
        rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
        # ties: the 16 dropped bits are exactly half, with even and odd kept parts
        (rng.integers(0, 2 ** 16, 4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000,
        # just below and above a tie
        (rng.integers(0, 2 ** 16, 4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x7FFF,
        (rng.integers(0, 2 ** 16, 4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8001,
        np.array([0, 0x80000000, 0x7F800000, 0xFF800000,            # zeros, infinities
                  0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF,   # overflow to inf and not
                  0x00000001, 0x00008000, 0x00018000, 0x807FFFFF,   # subnormals
                  0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FFFFFFF], np.uint32)])  # NaNs
    x = bits.view(np.float32)
    y = sf.to_bf16(torch.from_numpy(x).to(dev)).cpu().view(torch.int16).numpy().view(np.uint16)
    want, nan = bf16_rne(x)
    assert np.array_equal(y[~nan], want[~nan])
    yn = y[nan]
    assert np.all((yn & 0x7F80) == 0x7F80) and np.all((yn & 0x007F) != 0), "NaN stays NaN"



def test_dft_table_fragments():
    """CF[R][a][b][kind] lane (r, g) slot v holds [cos t | sin t] (kind 0) or [-sin t | cos t]
    (kind 1) of t = 2 pi ((16a + r)(16b + 4g + v) mod R) / R; RI[R][nt][kind] lane (c, g)
    slot j holds cos t (kind 0) or -sin t (kind 1) of t = 2 pi (n0 (16nt + c) mod R) / R,
    n0 = 4g + j (j < 4) or 16 + 4g + j - 4, and zero for n0 >= R/2. Each value is rounded to
    fp32 and then to fp16, as in the reference's table (src/sffft.cu:349-362). The second
    kind's -sin is the rounded sin with its sign bit flipped, which the wave pipeline's
    first-kind-only layout relies on."""
    t = sf.dft_table().reshape(-1, 8)  # units of one lane's 8 halves
    assert t.shape[0] == 3584
    lane = np.arange(64)
    r, g = lane & 15, lane >> 4

    def h(x):
        return x.astype(np.float32).astype(np.float16).view(np.uint16)

    for R, cf, ri in ((16, 0, 128), (32, 256, 768), (64, 1024, 3072)):
        T = R // 16
        for a in range(T):
            for b in range(T):
                f = a * T + b
                e = ((16 * a + r)[:, None] * (16 * b + 4 * g[:, None] + np.arange(4)[None])) % R
                c, sn = h(np.cos(2 * np.pi * e / R)), h(np.sin(2 * np.pi * e / R))
                k0 = t[cf + 2 * f * 64: cf + 2 * f * 64 + 64]
                k1 = t[cf + (2 * f + 1) * 64: cf + (2 * f + 1) * 64 + 64]
                np.testing.assert_array_equal(k0[:, :4], c)
                np.testing.assert_array_equal(k0[:, 4:], sn)
                np.testing.assert_array_equal(k1[:, :4], sn ^ 0x8000)
                np.testing.assert_array_equal(k1[:, 4:], c)
        j = np.arange(8)
        n0 = np.where(j < 4, 4 * g[:, None] + j[None], 16 + 4 * g[:, None] + j[None] - 4)
        for nt in range(T):
            e = (n0 * (16 * nt + r)[:, None]) % R
            zero = n0 >= R // 2
            c = np.where(zero, 0, h(np.cos(2 * np.pi * e / R)))
            msn = np.where(zero, 0, h(np.sin(2 * np.pi * e / R)) ^ 0x8000)
            np.testing.assert_array_equal(t[ri + 2 * nt * 64: ri + 2 * nt * 64 + 64], c)
            np.testing.assert_array_equal(t[ri + (2 * nt + 1) * 64: ri + (2 * nt + 1) * 64 + 64], msn)
