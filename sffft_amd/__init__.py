"""MI355X fused causal long convolution: Python binding of libsffft.so.

y[b,h,n] = sum_{m<=n} u[b,h,m] * k[h,n-m] in one fused HIP launch per batch.

This module is a thin ctypes layer over the C ABI declared in include/sffft.h
(the drop-in boundary). torch supplies device memory and the current stream;
every computation runs in libsffft.so. There is no fallback: if the library is
missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsffft.so")
# The race-check build (every wavefront-level LDS hand-off a real wait), for tests only.
DEBUG_LIB_PATH = os.path.join(_HERE, "libsffft_debug.so")
CLI_PATH = os.path.join(_HERE, "sffft")
ROCFFT_LIB_PATH = os.path.join(_HERE, "libsffft_rocfft.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "sffft.h")

SFFFT_OK, SFFFT_EINVAL, SFFFT_ENOPLAN, SFFFT_EHIP, SFFFT_ENOTFOUND, SFFFT_ESCRATCH = 0, 1, 2, 3, 4, 5
LENGTHS = (128, 256, 512, 1024, 2048, 4096, 8192, 16384)
# multi-pass plans (mode 2) beyond one CU's LDS
LONG_LENGTHS = (32768, 65536, 131072)


class Plan(ctypes.Structure):
    """sffft_plan: N = 2L = r0*r1*r2 (r2 = 1 for two-stage plans). mode 0: one
    workgroup per transform; mode 1: one wavefront per pair of sequences, `channels`
    channels per workgroup; mode 2: multi-pass, column radix r0 and row plan r1 x r2,
    with a workspace (conv_long)."""

    _fields_ = [
        ("r0", ctypes.c_int),
        ("r1", ctypes.c_int),
        ("r2", ctypes.c_int),
        ("waves", ctypes.c_int),
        ("acc", ctypes.c_int),
        ("cached", ctypes.c_int),
        ("seqs", ctypes.c_int),
        ("mode", ctypes.c_int),
        ("channels", ctypes.c_int),
    ]

    def name(self) -> str:
        return f"{self.r0}x{self.r1}" + (f"x{self.r2}" if self.r2 > 1 else "")

    def replace(self, **kw) -> "Plan":
        d = {f: getattr(self, f) for f, _ in self._fields_}
        d.update(kw)
        return Plan(**d)

    def __repr__(self) -> str:
        return (f"Plan({self.name()}, waves={self.waves}, acc={self.acc}, cached={self.cached}, "
                f"seqs={self.seqs}, mode={self.mode}, channels={self.channels})")


class Candidate(ctypes.Structure):
    _fields_ = [
        ("method", ctypes.c_char_p),
        ("io", ctypes.c_char_p),
        ("config", ctypes.c_char_p),
        ("ms", ctypes.c_double),
        ("rel_err", ctypes.c_double),
    ]


class SffftError(RuntimeError):
    def __init__(self, code: int, what: str):
        detail = lib().sffft_last_error().decode() if code == SFFFT_EHIP else ""
        super().__init__(f"{what}: {strerror(code)} (code {code}) {detail}".rstrip())
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libsffft.so (built in-tree by `make -C sffft_amd`)."""
    global _lib
    if _lib is None:
        _lib = load_library(LIB_PATH)
    return _lib


def load_library(path: str) -> ctypes.CDLL:
    """Loads a build of the C ABI from `path` with the argument types of include/sffft.h."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C sffft_amd` "
                           "(or __graft_entry__.build())")
    # PyTorch ships its own HIP runtime under the same soname as /opt/rocm's.
    # Import it first so the library binds to the runtime torch uses: two HIP
    # runtimes in one process do not share devices, memory or streams.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(path)
    P = ctypes.POINTER(Plan)
    vp, ci, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sigs = {
        "sffft_plan_check": (ci, [ci, P]),
        "sffft_plan_lds_bytes": (sz, [ci, P]),
        "sffft_plan_occupancy": (ci, [ci, P, ctypes.POINTER(ci)]),
        "sffft_plan_count": (ci, [ci]),
        "sffft_plan_get": (ci, [ci, ci, P, ctypes.c_char_p, sz]),
        "sffft_spectrum_bytes": (sz, [ci, ci]),
        "sffft_spectrum": (ci, [vp, ci, ci, P, vp, vp, vp]),
        "sffft_spectrum_conj": (ci, [vp, ci, ci, P, vp, vp, vp]),
        "sffft_spectrum_from_natural": (ci, [vp, ci, ci, P, vp, vp]),
        "sffft_spectrum_from_natural_complex": (ci, [vp, ci, ci, P, vp, vp]),
        "sffft_spectrum_noalloc": (ci, [vp, ci, ci, P, vp, vp]),
        "sffft_conv_f32": (ci, [vp, vp, vp, ci, ci, ci, P, vp]),
        "sffft_conv_bf16": (ci, [vp, vp, vp, ci, ci, ci, P, vp]),
        "sffft_conv_complex_f32": (ci, [vp, vp, vp, ci, ci, ci, P, vp]),
        "sffft_conv_complex_bf16": (ci, [vp, vp, vp, ci, ci, ci, P, vp]),
        "sffft_work_bytes": (sz, [ci, ci, ci, P]),
        "sffft_conv_long_f32": (ci, [vp, vp, vp, vp, sz, ci, ci, ci, P, vp]),
        "sffft_conv_long_bf16": (ci, [vp, vp, vp, vp, sz, ci, ci, ci, P, vp]),
        "sffft_spectrum_circular": (ci, [vp, ci, ci, P, vp, vp, vp]),
        "sffft_spectrum_complex": (ci, [vp, vp, ci, ci, P, vp, vp, vp]),
        "sffft_circconv_long_f32": (ci, [vp, vp, vp, vp, sz, ci, ci, ci, P, vp]),
        "sffft_circconv_long_bf16": (ci, [vp, vp, vp, vp, sz, ci, ci, ci, P, vp]),
        "sffft_fft_work_bytes": (sz, [ci, ci]),
        "sffft_fft_c2c": (ci, [vp, vp, vp, sz, ci, ci, ctypes.c_longlong, ctypes.c_longlong, ci,
                               ctypes.c_float, vp]),
        "sffft_fft2_work_bytes": (sz, [ci, ci, ci]),
        "sffft_fft2_c2c": (ci, [vp, vp, vp, sz, ci, ci, ci, ci, ctypes.c_float, vp]),
        "sffft_circconv2d_work_bytes": (sz, [ci, ci, ci, ci]),
        "sffft_circconv2d_f32": (ci, [vp, vp, vp, vp, sz, ci, ci, ci, ci, vp]),
        "sffft_to_bf16": (ci, [vp, vp, sz, vp]),
        "sffft_dispatch_floor": (ci, [ci, ci, ci, P, vp]),
        "sffft_dispatch_floor_shape": (ci, [ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp]),
        "sffft_dft_table": (ci, [vp, sz]),
        "sffft_twiddle_probe": (ci, [ci, vp, ci, ci, ctypes.c_float, vp, vp]),
        "sffft_twiddle_table": (ci, [ci, ci, ci, vp, sz]),
        "sffft_select_candidate": (ci, [ctypes.POINTER(Candidate), ci, ctypes.c_double, ctypes.c_char_p]),
        "sffft_relative_l2": (ctypes.c_double, [ctypes.c_double, ctypes.c_double]),
        "sffft_strerror": (ctypes.c_char_p, [ci]),
        "sffft_last_error": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


def strerror(code: int) -> str:
    return lib().sffft_strerror(code).decode()


def _check(code: int, what: str) -> None:
    if code != SFFFT_OK:
        raise SffftError(code, what)


def plans(L: int) -> List[Plan]:
    """Compiled plans for length L (acc=0, cached=1); vary acc/cached/seqs as needed."""
    out = []
    for i in range(lib().sffft_plan_count(L)):
        p = Plan()
        _check(lib().sffft_plan_get(L, i, ctypes.byref(p), None, 0), "sffft_plan_get")
        out.append(p)
    return out


def make_plan(spec: str, waves: int, acc: int = 0, cached: int = 1, seqs: int = 1, mode: int = 0,
              channels: int = 1) -> Plan:
    r = [int(x) for x in spec.split("x")]
    r += [1] * (3 - len(r))
    return Plan(r[0], r[1], r[2], waves, acc, cached, seqs, mode, channels)


# Tuned plan per (L, I/O) at B=8, H=768 (spec, waves, seqs, mode, channels): wave plans up to
# L=2048, workgroup plans beyond. A pair of sequences per transform is ~30% less accurate than
# one sequence; with fp32 I/O the three-stage pair plans measure 4.2e-4 to 4.7e-4 rel-L2
# (bound 5e-4) and run 1.5x to 1.8x faster than one-sequence plans (3.2e-4 to 3.8e-4).
# Callers that need more margin pass a one-sequence plan (ODD_BATCH_PLANS).
DEFAULT_PLANS = {
    (128, "fp32"): ("16x16", 4, 2, 1, 1), (128, "bf16"): ("16x16", 4, 2, 1, 1),
    (256, "fp32"): ("32x16", 4, 2, 1, 1), (256, "bf16"): ("32x16", 4, 2, 1, 1),
    (512, "fp32"): ("32x32", 4, 2, 1, 1), (512, "bf16"): ("32x32", 4, 2, 1, 1),
    (1024, "fp32"): ("64x32", 12, 2, 1, 3), (1024, "bf16"): ("64x32", 12, 2, 1, 3),
    (2048, "fp32"): ("64x64", 12, 2, 1, 3), (2048, "bf16"): ("64x64", 12, 2, 1, 3),
    (4096, "fp32"): ("32x16x16", 4, 2, 0, 1), (4096, "bf16"): ("32x16x16", 4, 2, 0, 1),
    (8192, "fp32"): ("32x32x16", 8, 2, 0, 1), (8192, "bf16"): ("32x32x16", 8, 2, 0, 1),
    (16384, "fp32"): ("32x32x32", 8, 2, 0, 1), (16384, "bf16"): ("32x32x32", 8, 2, 0, 1),
}
# Multi-pass plans (mode 2): column radix x row plan, measured at B=8, H=768
LONG_DEFAULT_PLANS = {32768: "64x32x32", 65536: "64x64x32", 131072: "64x64x64"}
# One sequence per transform (workgroup kernel) for an odd batch
ODD_BATCH_PLANS = {128: ("16x16", 2), 256: ("32x16", 2), 512: ("32x32", 2), 1024: ("64x32", 4),
                   2048: ("16x16x16", 8), 4096: ("32x16x16", 8), 8192: ("32x32x16", 4), 16384: ("32x32x32", 8)}


def long_plan(spec: str) -> Plan:
    """A multi-pass plan "NCxR0xR1": column radix NC, row plan R0 x R1."""
    return make_plan(spec, 4, acc=0, cached=1, seqs=2, mode=2, channels=1)


def default_plan(L: int, io: str = "fp32", B: int = 8, acc: int = 0) -> Plan:
    """The tuned plan for length L and I/O type; pairs of sequences need an even B.
    Beyond L = 16384 the plan is multi-pass (mode 2), which needs an even B and acc = 0."""
    if L in LONG_DEFAULT_PLANS:
        if B % 2 or acc:
            raise ValueError(f"L={L}: multi-pass plans take pairs of sequences (even B) and fp32 accumulation")
        return long_plan(LONG_DEFAULT_PLANS[L])
    spec, waves, seqs, mode, channels = DEFAULT_PLANS[(L, io)]
    if seqs == 2 and B % 2:
        spec, waves = ODD_BATCH_PLANS[L]
        seqs, mode, channels = 1, 0, 1
    return make_plan(spec, waves, acc=acc, cached=1, seqs=seqs, mode=mode, channels=channels)


def plan_check(L: int, plan: Plan) -> int:
    return lib().sffft_plan_check(L, ctypes.byref(plan))


def lds_bytes(L: int, plan: Plan) -> int:
    return lib().sffft_plan_lds_bytes(L, ctypes.byref(plan))


def occupancy(L: int, plan: Plan) -> int:
    n = ctypes.c_int(0)
    _check(lib().sffft_plan_occupancy(L, ctypes.byref(plan), ctypes.byref(n)), "sffft_plan_occupancy")
    return n.value


def select_candidate(cands: List[Tuple[str, str, str, float, float]], max_error: float, io: str) -> int:
    arr = (Candidate * max(1, len(cands)))()
    keep = []
    for i, (m, o, c, ms, err) in enumerate(cands):
        b = [m.encode(), o.encode(), c.encode()]
        keep.append(b)
        arr[i] = Candidate(b[0], b[1], b[2], ms, err)
    return lib().sffft_select_candidate(arr, len(cands), max_error, io.encode())


def relative_l2(squared_error: float, squared_reference: float) -> float:
    return lib().sffft_relative_l2(squared_error, squared_reference)


# ---- torch-facing helpers (device memory and streams come from torch) ----------
_raw_stream = None


def _stream():
    """The current device's current stream. torch's C accessors, when this torch has them,
    skip building a Stream object (about a microsecond and a half of every call)."""
    global _raw_stream
    if _raw_stream is None:
        import torch

        c = torch._C
        if hasattr(c, "_cuda_getCurrentRawStream") and hasattr(c, "_cuda_getDevice"):
            _raw_stream = lambda: c._cuda_getCurrentRawStream(c._cuda_getDevice())  # noqa: E731
        else:
            _raw_stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    return ctypes.c_void_p(_raw_stream())


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _check_spectrum(kf, u, H: int, N: int) -> None:
    """kf must be the [H, N] complex64 spectrum buffer of u's H channels (row h is channel h),
    contiguous and on u's device: the kernels read H rows of N values from its start."""
    import torch

    if not (kf.is_cuda and kf.dtype == torch.complex64 and kf.is_contiguous() and kf.device == u.device
            and tuple(kf.shape) == (H, N)):
        raise ValueError(f"kf must be a contiguous complex64 [H, 2L] = [{H}, {N}] tensor on {u.device} "
                         f"(a spectrum of this call's channels), got {tuple(kf.shape)} {kf.dtype} on {kf.device}")


def spectrum(k, L: int, plan: Plan, work=None, conj: bool = False):
    """Kernel-order filter spectrum [H, 2L] complex64 from the real filter k [H, L] (fp32, cuda);
    with conj, the conjugate spectrum (sffft_spectrum_conj), on which sffft_conv_* computes the
    anti-causal correlation sum_{n>=m} x[n] k[n-m] instead of the causal convolution."""
    import torch

    assert k.is_cuda and k.dtype == torch.float32 and k.dim() == 2 and k.shape[1] == L
    k = k.contiguous()
    H = k.shape[0]
    kf = torch.empty((H, 2 * L), dtype=torch.complex64, device=k.device)
    if work is None:
        work = torch.empty_like(kf)
    fn = lib().sffft_spectrum_conj if conj else lib().sffft_spectrum
    _check(fn(_ptr(k), H, L, ctypes.byref(plan), _ptr(kf), _ptr(work), _stream()), "sffft_spectrum")
    return kf


def spectrum_from_natural(kc, L: int, plan: Plan, complex_filter: bool = False):
    """Kernel-order spectrum from the unnormalised natural-order spectrum kc [H, 2L] complex64 of
    a real filter; with complex_filter, of any filter (the whole spectrum of
    sffft_spectrum_from_natural_complex, for complex_conv)."""
    import torch

    assert kc.is_cuda and kc.dtype == torch.complex64 and kc.shape[1] == 2 * L
    kc = kc.contiguous()
    kf = torch.empty_like(kc)
    fn = lib().sffft_spectrum_from_natural_complex if complex_filter else lib().sffft_spectrum_from_natural
    _check(fn(_ptr(kc), kc.shape[0], L, ctypes.byref(plan), _ptr(kf), _stream()), "sffft_spectrum_from_natural")
    return kf


def work_bytes(B: int, H: int, L: int, plan: Plan) -> int:
    """Workspace bytes of a multi-pass (mode 2) plan; 0 for the other modes."""
    return lib().sffft_work_bytes(B, H, L, ctypes.byref(plan))


def conv(u, kf, plan: Plan, out=None, work=None):
    """y = causal_conv(u, k) for u [B, H, L] fp32 or bf16 (cuda), kf from spectrum().
    Multi-pass plans (mode 2) use `work` (a cuda tensor of at least work_bytes() bytes),
    or allocate one for the call."""
    import torch

    assert u.is_cuda and u.dim() == 3
    u = u.contiguous()
    B, H, L = u.shape
    _check_spectrum(kf, u, H, 2 * L)
    y = torch.empty_like(u) if out is None else out
    if plan.mode == 2:
        return conv_long(u, kf, plan, y, work)
    if u.dtype == torch.float32:
        fn = lib().sffft_conv_f32
    elif u.dtype == torch.bfloat16:
        fn = lib().sffft_conv_bf16
    else:
        raise TypeError(f"unsupported dtype {u.dtype}")
    _check(fn(_ptr(u), _ptr(kf), _ptr(y), B, H, L, ctypes.byref(plan), _stream()), "sffft_conv")
    return y


def conv_long(u, kf, plan: Plan, out=None, work=None):
    """Multi-pass convolution (sffft_conv_long_*): three launches on the current stream."""
    import torch

    u = u.contiguous()
    B, H, L = u.shape
    _check_spectrum(kf, u, H, 2 * L)
    y = torch.empty_like(u) if out is None else out
    nbytes = work_bytes(B, H, L, plan)
    if work is None:
        work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=u.device)
    if u.dtype == torch.float32:
        fn = lib().sffft_conv_long_f32
    elif u.dtype == torch.bfloat16:
        fn = lib().sffft_conv_long_bf16
    else:
        raise TypeError(f"unsupported dtype {u.dtype}")
    wb = work.numel() * work.element_size()
    _check(fn(_ptr(u), _ptr(kf), _ptr(y), _ptr(work), wb, B, H, L, ctypes.byref(plan), _stream()),
           "sffft_conv_long")
    return y


def spectrum_complex(k, L: int, plan: Plan, work=None):
    """Kernel-order spectrum [H, 2L] of the complex filters k [H, L] (complex64, cuda) for a pair
    plan (seqs = 2). conv(u, kf, plan) then computes the complex causal convolution of the
    sequences whose real and imaginary planes are batch rows 2b' and 2b'+1 of u (see
    complex_conv)."""
    import torch

    assert k.is_cuda and k.dtype == torch.complex64 and k.dim() == 2 and k.shape[1] == L
    kr = k.real.contiguous()
    ki = k.imag.contiguous()
    H = k.shape[0]
    kf = torch.empty((H, 2 * L), dtype=torch.complex64, device=k.device)
    if work is None:
        work = torch.empty_like(kf)
    _check(lib().sffft_spectrum_complex(_ptr(kr), _ptr(ki), H, L, ctypes.byref(plan), _ptr(kf), _ptr(work),
                                        _stream()), "sffft_spectrum_complex")
    return kf


def complex_conv(x, kf, plan: Plan):
    """Complex causal convolution of x [Bc, H, L] complex64 (cuda) with the filters of
    spectrum_complex(): the planes are interleaved as batch rows (2b', 2b'+1) = (Re, Im) of x[b'],
    convolved by sffft_conv_complex_f32 (conv_long for multi-pass plans), and reassembled."""
    import torch

    Bc, H, L = x.shape
    _check_spectrum(kf, x, H, 2 * L)
    u = torch.stack([x.real, x.imag], 1).reshape(2 * Bc, H, L).contiguous()
    if plan.mode == 2:
        y = conv_long(u, kf, plan)
    else:
        y = torch.empty_like(u)
        _check(lib().sffft_conv_complex_f32(_ptr(u), _ptr(kf), _ptr(y), 2 * Bc, H, L, ctypes.byref(plan),
                                            _stream()), "sffft_conv_complex_f32")
    y = y.reshape(Bc, 2, H, L)
    return torch.complex(y[:, 0], y[:, 1])


def spectrum_circular(k, plan: Plan, work=None):
    """Spectrum [H, N] complex64 of the unpadded filters k [H, N] (fp32, cuda) for a circular
    convolution of period N = r0*r1*r2 with a multi-pass plan."""
    import torch

    assert k.is_cuda and k.dtype == torch.float32 and k.dim() == 2
    k = k.contiguous()
    H, N = k.shape
    kf = torch.empty((H, N), dtype=torch.complex64, device=k.device)
    if work is None:
        work = torch.empty_like(kf)
    _check(lib().sffft_spectrum_circular(_ptr(k), H, N, ctypes.byref(plan), _ptr(kf), _ptr(work), _stream()),
           "sffft_spectrum_circular")
    return kf


def circconv(u, kf, plan: Plan, out=None, work=None):
    """y[b,h,n] = sum_m u[b,h,m] k[h,(n-m) mod N] for u [B, H, N] fp32 or bf16 (cuda), kf from
    spectrum_circular(); a multi-pass plan, B even."""
    import torch

    u = u.contiguous()
    B, H, N = u.shape
    y = torch.empty_like(u) if out is None else out
    nbytes = work_bytes(B, H, N // 2, plan)
    if work is None:
        work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=u.device)
    if u.dtype == torch.float32:
        fn = lib().sffft_circconv_long_f32
    elif u.dtype == torch.bfloat16:
        fn = lib().sffft_circconv_long_bf16
    else:
        raise TypeError(f"unsupported dtype {u.dtype}")
    wb = work.numel() * work.element_size()
    _check(fn(_ptr(u), _ptr(kf), _ptr(y), _ptr(work), wb, B, H, N, ctypes.byref(plan), _stream()),
           "sffft_circconv_long")
    return y


def _work(nbytes: int, device):
    import torch

    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def fft(x, inverse: bool = False, scale: float = 1.0, dim: int = -1, out=None):
    """Unnormalised complex transform of x (complex64, cuda) along `dim`:
    X[k] = scale * sum_n x[n] exp(-/+ 2 pi i n k / N), minus sign forward, plus inverse.
    dim -1 on any shape, or dim 0 of a 2-D tensor (its columns, read in place with
    stride = columns). N a power of two in [2, 2^24]. `out` may be x."""
    import torch

    assert x.is_cuda and x.dtype == torch.complex64
    x = x.contiguous()
    if dim in (-1, x.dim() - 1):
        N = x.shape[-1]
        batch, stride, dist = x.numel() // N, 1, N
    elif dim == 0 and x.dim() == 2:
        N, batch = x.shape
        stride, dist = batch, 1
    else:
        raise ValueError("fft: dim must be the last dimension, or 0 of a 2-D tensor")
    X = torch.empty_like(x) if out is None else out
    assert X.shape == x.shape and X.dtype == x.dtype and X.is_contiguous()
    work = _work(lib().sffft_fft_work_bytes(batch, N), x.device)
    _check(lib().sffft_fft_c2c(_ptr(x), _ptr(X), _ptr(work), work.numel(), batch, N, stride, dist, int(inverse),
                               scale, _stream()), "sffft_fft_c2c")
    return X


def fft2(x, inverse: bool = False, scale: float = 1.0, out=None):
    """Unnormalised 2-D transform over the last two dimensions of x [..., N0, N1]
    (complex64, cuda), signs as fft(). `out` may be x."""
    import torch

    assert x.is_cuda and x.dtype == torch.complex64 and x.dim() >= 2
    x = x.contiguous()
    N0, N1 = x.shape[-2:]
    batch = x.numel() // (N0 * N1)
    X = torch.empty_like(x) if out is None else out
    assert X.shape == x.shape and X.dtype == x.dtype and X.is_contiguous()
    work = _work(lib().sffft_fft2_work_bytes(batch, N0, N1), x.device)
    _check(lib().sffft_fft2_c2c(_ptr(x), _ptr(X), _ptr(work), work.numel(), batch, N0, N1, int(inverse), scale,
                                _stream()), "sffft_fft2_c2c")
    return X


def circconv2d(u, k):
    """2-D circular convolution of period (N0, N1): u [B, H, N0, N1], k [H, N0, N1], fp32 cuda."""
    import torch

    assert u.is_cuda and u.dtype == torch.float32 and k.dtype == torch.float32 and u.dim() == 4
    u, k = u.contiguous(), k.contiguous()
    B, H, N0, N1 = u.shape
    assert tuple(k.shape) == (H, N0, N1)
    y = torch.empty_like(u)
    work = _work(lib().sffft_circconv2d_work_bytes(B, H, N0, N1), u.device)
    _check(lib().sffft_circconv2d_f32(_ptr(u), _ptr(k), _ptr(y), _ptr(work), work.numel(), B, H, N0, N1, _stream()),
           "sffft_circconv2d_f32")
    return y


def to_bf16(x):
    import torch

    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    _check(lib().sffft_to_bf16(_ptr(x.contiguous()), _ptr(y), x.numel(), _stream()), "sffft_to_bf16")
    return y


def dispatch_floor(B: int, H: int, L: int, plan: Plan) -> None:
    """Launches the body-less kernel with the launch shape of conv() for this plan."""
    _check(lib().sffft_dispatch_floor(B, H, L, ctypes.byref(plan), _stream()), "sffft_dispatch_floor")


def dispatch_floor_shape(grid: int, block: int, lds_bytes: int) -> None:
    """The body-less kernel with an explicit launch shape (sffft_dispatch_floor_shape)."""
    _check(lib().sffft_dispatch_floor_shape(grid, block, lds_bytes, _stream()), "sffft_dispatch_floor_shape")


def dft_table():
    import numpy as np

    buf = (ctypes.c_uint16 * (57344 // 2))()
    _check(lib().sffft_dft_table(buf, 57344), "sffft_dft_table")
    return np.frombuffer(buf, dtype=np.uint16).copy()


class RocfftPipeline:
    """The rocFFT comparator of the driver (libsffft_rocfft.so; the reference's cuFFT
    pipeline, src/sffft.cu:289-305,365-371): pad -> R2C -> multiply by the half spectrum / N
    -> C2R -> slice, on the current torch stream. Measurement infrastructure, not part of
    the drop-in boundary."""

    _rlib = None

    def __init__(self, B: int, H: int, L: int, k):
        import torch

        if RocfftPipeline._rlib is None:
            lib()  # binds the HIP runtime torch uses first
            R = ctypes.CDLL(ROCFFT_LIB_PATH)
            vp, ci = ctypes.c_void_p, ctypes.c_int
            R.sffft_rocfft_create.argtypes = [ci, ci, ci, vp, ctypes.POINTER(vp)]
            R.sffft_rocfft_filter.argtypes = [vp, vp, vp]
            R.sffft_rocfft_full.argtypes = [vp, vp, vp]
            R.sffft_rocfft_core.argtypes = [vp]
            R.sffft_rocfft_destroy.argtypes = [vp]
            RocfftPipeline._rlib = R
        self.R = RocfftPipeline._rlib
        self.h = ctypes.c_void_p()
        rc = self.R.sffft_rocfft_create(B, H, L, _stream(), ctypes.byref(self.h))
        if rc:
            raise RuntimeError(f"sffft_rocfft_create failed ({rc})")
        assert k.is_cuda and k.dtype == torch.float32 and tuple(k.shape) == (H, L)
        self.k = k.contiguous()
        if self.R.sffft_rocfft_filter(self.h, _ptr(self.k), None):
            raise RuntimeError("sffft_rocfft_filter failed")

    def full(self, u, y) -> None:
        if self.R.sffft_rocfft_full(self.h, _ptr(u), _ptr(y)):
            raise RuntimeError("sffft_rocfft_full failed")

    def core(self) -> None:
        if self.R.sffft_rocfft_core(self.h):
            raise RuntimeError("sffft_rocfft_core failed")

    def close(self) -> None:
        if self.h:
            self.R.sffft_rocfft_destroy(self.h)
            self.h = ctypes.c_void_p()


# Sources the convolution kernels (wave pipeline, workgroup kernel, multi-pass passes) are
# compiled from, with the build flags: a profile summary measured on a build of other
# sources does not describe this one. (The host code, the spectrum preparation and the
# standalone transforms, in api.hip and transforms.hpp, are not part of those kernels.)
# The sources each kernel family is compiled from, and the build flags (Makefile): the
# single-pass kernels (plan modes 0 and 1, conv_inst.hip) and the multi-pass kernels
# (mode 2, long_inst.hip, which also include the single-pass headers).
SINGLE_PASS_SOURCES = ("csrc/fftconv.hpp", "csrc/fftconv_wave.hpp", "csrc/registry.hpp", "csrc/plans.def",
                       "csrc/conv_inst.hip", "Makefile")
MULTI_PASS_SOURCES = SINGLE_PASS_SOURCES + ("csrc/longconv.hpp", "csrc/long_inst.hip")


def _code_only(rel: str, text: str) -> str:
    """The source without its comments (C++ // and /* */, Makefile #), blank lines and
    indentation, so that an edit of comments or layout does not change the stamp of an
    unchanged kernel."""
    import re

    if rel.endswith("Makefile"):
        text = re.sub(r"(?m)^\s*#.*$", "", text)
    else:
        text = re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))
    return "\n".join(line.strip() for line in text.splitlines() if line.strip())


def kernel_sources_sha(mode: int = 1) -> str:
    """First 16 hex digits of the sha256 over the code (comments removed) of the sources
    and build flags of the kernel family that runs plans of this mode (0 and 1:
    single-pass, 2: multi-pass)."""
    import hashlib

    h = hashlib.sha256()
    for rel in MULTI_PASS_SOURCES if mode == 2 else SINGLE_PASS_SOURCES:
        with open(os.path.join(_HERE, rel)) as f:
            h.update(rel.encode() + b"\0" + _code_only(rel, f.read()).encode() + b"\0")
    return h.hexdigest()[:16]


def loaded_library_paths() -> List[str]:
    """Shared objects of this package mapped into the process (for load checks)."""
    out = []
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if _HERE in line and line.rstrip().endswith(".so"):
                    out.append(line.split()[-1])
    except OSError:
        pass
    return sorted(set(out))
