"""The C ABI of libsffft.so: every symbol declared in include/sffft.h is exported,
and the host-side checks (plans, sizes, argument validation) behave without a GPU."""
import ctypes
import re

import pytest

import sffft_amd as sf


def declared_functions():
    text = open(sf.HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(sffft_[a-z0-9_]+)\s*\(", text, re.M)))


@pytest.mark.parametrize("path", [sf.LIB_PATH, sf.DEBUG_LIB_PATH], ids=["product", "debug-barriers"])
def test_every_declared_symbol_is_exported(path):
    names = declared_functions()
    assert len(names) >= 16
    lib = ctypes.CDLL(path)
    for n in names:
        assert hasattr(lib, n), n


@pytest.mark.parametrize("L", sf.LENGTHS)
def test_registry(L):
    plans = sf.plans(L)
    assert plans
    for p in plans:
        assert p.r0 * p.r1 * p.r2 == 2 * L
        assert sf.plan_check(L, p) == sf.SFFFT_OK
        assert sf.plan_check(L, p.replace(acc=1, cached=0)) == sf.SFFFT_OK
        assert 0 < sf.lds_bytes(L, p) <= 163840
    assert sf.plan_check(L, plans[0].replace(waves=17)) == sf.SFFFT_EINVAL


def test_plan_validation():
    P = sf.make_plan
    assert sf.plan_check(1024, P("64x32", 4)) == sf.SFFFT_OK
    assert sf.plan_check(1024, P("64x16", 4)) == sf.SFFFT_EINVAL       # product != 2L
    assert sf.plan_check(1024, P("128x16", 4)) == sf.SFFFT_EINVAL      # radix 128
    assert sf.plan_check(1000, P("64x32", 4)) == sf.SFFFT_EINVAL       # L not a power of two
    assert sf.plan_check(1024, P("64x32", 4, seqs=3)) == sf.SFFFT_EINVAL
    assert sf.plan_check(1024, P("64x32", 4, acc=2)) == sf.SFFFT_EINVAL
    assert sf.plan_check(2048, P("16x16x16", 32)) == sf.SFFFT_EINVAL   # waves
    assert sf.plan_check(1024, P("64x32", 1)) == sf.SFFFT_ENOPLAN      # valid, not compiled
    assert sf.plan_check(1024, P("64x32", 12, seqs=2, mode=1, channels=3)) == sf.SFFFT_OK
    assert sf.plan_check(1024, P("64x32", 12)) == sf.SFFFT_EINVAL       # 12 waves: mode 1 only
    assert sf.plan_check(1024, P("64x32", 12, seqs=1, mode=1, channels=3)) == sf.SFFFT_EINVAL  # pairs only
    assert sf.plan_check(4096, P("32x16x16", 4, seqs=2, mode=1)) == sf.SFFFT_EINVAL  # two-stage only
    assert sf.plan_check(1024, P("64x32", 4, channels=2)) == sf.SFFFT_EINVAL  # channels: mode 1 only
    # LDS of a wave plan: tables (DFT fragments, two twiddle tables) + one Hermitian half
    # spectrum per channel (33 columns k0 = 0..32 of 2*8+1 float4, the three channels in whole
    # 1 KB runs) + a 16-row operand scratch per wavefront
    half = 33 * 17 * 16
    assert sf.lds_bytes(1024, P("64x32", 12, seqs=2, mode=1, channels=3)) == (32768 + 8192 + 32768 +
                                                                            (3 * half + 1023) // 1024 * 1024 +
                                                                            12 * 16 * 36 * 4)
    # 64x64, 12 wavefronts, 3 channels: both fragment kinds (32 KB) do not fit beside the
    # spectra, the first kind (16 KB) does; one shared twiddle table
    half = 33 * 33 * 16
    assert sf.lds_bytes(2048, P("64x64", 12, seqs=2, mode=1, channels=3)) == (16384 + 32768 +
                                                                            (3 * half + 1023) // 1024 * 1024 +
                                                                            12 * 16 * 68 * 4) == 154624
    assert sf.lds_bytes(1024, P("64x16", 4)) == 0


def test_conv_argument_errors_need_no_gpu():
    p = sf.make_plan("64x32", 4, seqs=2)
    lib = sf.lib()
    null = ctypes.c_void_p(0)
    good = ctypes.c_void_p(1 << 20)
    assert lib.sffft_conv_f32(null, good, good, 8, 768, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL
    assert lib.sffft_conv_f32(good, good, good, 7, 768, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL  # B odd
    assert lib.sffft_conv_f32(ctypes.c_void_p((1 << 20) + 4), good, good, 8, 768, 1024, ctypes.byref(p),
                              null) == sf.SFFFT_EINVAL  # misaligned rows
    assert lib.sffft_conv_bf16(good, good, good, 0, 768, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL
    assert lib.sffft_spectrum(good, 768, 1024, ctypes.byref(p), good, good, null) == sf.SFFFT_EINVAL  # kf == work
    # the whole-spectrum gather serves pair plans only, and kc and kf must differ
    f = lib.sffft_spectrum_from_natural_complex
    assert f(good, 768, 1024, ctypes.byref(sf.make_plan("64x32", 4, seqs=1)), ctypes.c_void_p(1 << 30),
             null) == sf.SFFFT_EINVAL
    assert f(good, 768, 1024, ctypes.byref(p), good, null) == sf.SFFFT_EINVAL
    assert f(null, 768, 1024, ctypes.byref(p), good, null) == sf.SFFFT_EINVAL
    assert f(good, 768, 1000, ctypes.byref(p), ctypes.c_void_p(1 << 30), null) == sf.SFFFT_EINVAL
    assert sf.lib().sffft_spectrum_bytes(768, 1024) == 768 * 2048 * 8
    # the dispatch floor checks its shape like conv, before any HIP call
    assert lib.sffft_dispatch_floor(0, 768, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL
    assert lib.sffft_dispatch_floor(7, 768, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL  # B odd
    assert lib.sffft_dispatch_floor(8, 768, 1000, ctypes.byref(p), null) == sf.SFFFT_EINVAL  # L
    for shape in ((0, 256, 0), (256, 0, 0), (256, 96, 0), (256, 1088, 0), (256, 256, 163841)):
        assert lib.sffft_dispatch_floor_shape(*shape, null) == sf.SFFFT_EINVAL, shape


def test_strerror():
    assert sf.strerror(sf.SFFFT_OK) == "success"
    assert "invalid" in sf.strerror(sf.SFFFT_EINVAL)


def _long_plans_all():
    for L in (2048, 4096, 8192, 16384) + sf.LONG_LENGTHS:
        for nc in (16, 32, 64):
            for rows in ((16, 16), (32, 32), (64, 32), (64, 64)):
                if nc * rows[0] * rows[1] == 2 * L:
                    yield L, sf.long_plan(f"{nc}x{rows[0]}x{rows[1]}")


def test_long_plans_registry():
    # every compiled multi-pass plan: column radix in {16, 32, 64} with one of four row plans
    cases = list(_long_plans_all())
    assert len(cases) == 12
    for L, p in cases:
        assert sf.plan_check(L, p) == sf.SFFFT_OK, (L, p)
        NR = p.r1 * p.r2
        frags = ((p.r1 // 16) ** 2 + (0 if p.r1 == p.r2 else (p.r2 // 16) ** 2)) * 64 * 16
        assert sf.lds_bytes(L, p) == frags + (1 if p.r1 == p.r2 else 2) * NR * 8
        per_channel = 4 * 2 * L * 4  # B/2 pairs of 2L complex fp16 points
        assert sf.work_bytes(8, 768, L, p) == min(768, (96 << 20) // per_channel) * per_channel
        assert sf.work_bytes(8, 3, L, p) == min(3, (96 << 20) // per_channel) * per_channel
    for L in sf.LONG_LENGTHS:
        listed = sf.plans(L)
        assert listed and all(q.mode == 2 and q.r0 * q.r1 * q.r2 == 2 * L for q in listed)
        assert repr(sf.default_plan(L)) in [repr(q) for q in listed]
    assert sf.lib().sffft_plan_count(262144) == 0
    assert sf.lib().sffft_spectrum_bytes(768, 131072) == 768 * 262144 * 8


def test_long_plan_validation():
    P, LP = sf.make_plan, sf.long_plan
    assert sf.plan_check(65536, LP("32x64x64")) == sf.SFFFT_OK
    assert sf.plan_check(65536, LP("32x64x64").replace(acc=1)) == sf.SFFFT_EINVAL     # fp32 accumulation only
    assert sf.plan_check(65536, LP("32x64x64").replace(cached=0)) == sf.SFFFT_EINVAL  # table fragments only
    assert sf.plan_check(65536, LP("32x64x64").replace(seqs=1)) == sf.SFFFT_EINVAL    # pairs only
    assert sf.plan_check(65536, LP("32x64x64").replace(waves=8)) == sf.SFFFT_EINVAL
    assert sf.plan_check(65536, LP("64x32x64")) == sf.SFFFT_ENOPLAN                   # row plan not compiled
    assert sf.plan_check(65536, LP("64x64x64")) == sf.SFFFT_EINVAL                    # product != 2L
    assert sf.plan_check(65536, P("32x64x64", 8)) == sf.SFFFT_EINVAL                  # single-pass beyond 16384
    assert sf.plan_check(262144, LP("64x64x64")) == sf.SFFFT_EINVAL                   # beyond 131072
    assert sf.work_bytes(7, 768, 65536, LP("32x64x64")) == 0                          # odd B
    assert sf.work_bytes(8, 768, 1024, sf.make_plan("64x32", 4, seqs=2)) == 0         # not multi-pass


def test_long_conv_argument_errors_need_no_gpu():
    p = sf.long_plan("32x64x64")
    lib = sf.lib()
    null = ctypes.c_void_p(0)
    L, B, H = 65536, 8, 4
    need = sf.work_bytes(B, H, L, p)
    assert need == H * (B // 2) * 2 * L * 4  # four channels fit one 96 MiB chunk
    io = B * H * L * 4
    u, kf, y, w = (ctypes.c_void_p((1 << 40) + i * (1 << 34)) for i in range(4))
    f = lib.sffft_conv_long_f32
    assert f(u, kf, y, null, need, B, H, L, ctypes.byref(p), null) == sf.SFFFT_EINVAL          # no workspace
    assert f(u, kf, y, w, need // H - 1, B, H, L, ctypes.byref(p), null) == sf.SFFFT_EINVAL    # < one channel
    assert f(u, kf, y, w, need, 7, H, L, ctypes.byref(p), null) == sf.SFFFT_EINVAL            # B odd
    assert f(u, kf, y, ctypes.c_void_p((1 << 40) + 8), need, B, H, L, ctypes.byref(p),
             null) == sf.SFFFT_EINVAL                                                         # misaligned
    assert f(u, kf, y, ctypes.c_void_p((1 << 40) + io - 16), need, B, H, L, ctypes.byref(p),
             null) == sf.SFFFT_EINVAL                                                         # overlaps u
    assert f(u, kf, y, w, need, B, H, 1024, ctypes.byref(p), null) == sf.SFFFT_EINVAL          # plan vs L
    single = sf.make_plan("64x32", 4, seqs=2)
    assert f(u, kf, y, w, need, B, H, 1024, ctypes.byref(single), null) == sf.SFFFT_EINVAL     # not mode 2
    # the single-pass entry points refuse a multi-pass plan (it needs a workspace)
    assert lib.sffft_conv_f32(u, kf, y, B, H, L, ctypes.byref(p), null) == sf.SFFFT_EINVAL
    assert lib.sffft_dispatch_floor(B, H, L, ctypes.byref(p), null) == sf.SFFFT_EINVAL
