"""CPU oracle for the fused causal long convolution (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker. The product (sffft_amd, libsffft.so)
never imports, links or calls it.

Python bindings of oracle/liboracle.so (oracle/oracle.c, built by `make -C oracle`);
each function documents the reference lines it restates and how it is pinned.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
REF_SELECTION_LIB = os.path.join(_HERE, "_ref", "libref_selection.so")
REF_SELECTION_TEST = os.path.join(_HERE, "_ref", "selection_test")
DEFAULT_SEED = 88172645463325252  # src/sffft.cu:308

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
        ci = ctypes.c_int
        L.oracle_ref_inputs.argtypes = [ctypes.c_uint64, ci, ci, ci, ctypes.c_double, f32p, f32p]
        L.oracle_direct_conv.argtypes = [f32p, f32p, f64p, ci, ci, ci, ci]
        L.oracle_direct_conv_seqs.argtypes = [f32p, f32p, f64p, ci, ci, i64p, ci]
        L.oracle_fft_conv.argtypes = [f32p, f32p, f64p, ci, ci, ci, ci]
        L.oracle_spectrum_p_order.argtypes = [f32p, ci, ci, ci, ci, f64p]
        L.oracle_fourstep_conv.argtypes = [f64p, f64p, ci, ci, ci, ci, ci, f64p]
        L.oracle_round_f16.argtypes = [ctypes.c_double]
        L.oracle_round_f16.restype = ctypes.c_double
        L.oracle_relative_l2.argtypes = [ctypes.c_double, ctypes.c_double]
        L.oracle_relative_l2.restype = ctypes.c_double
        _lib = L
    return _lib


def threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def ref_inputs(B, H, L, seed=DEFAULT_SEED, input_scale=1.0):
    """Reference generator (src/sffft.cu:308-310,339-341): u [B,H,L], k [H,L] fp32."""
    u = np.empty((B, H, L), np.float32)
    k = np.empty((H, L), np.float32)
    lib().oracle_ref_inputs(seed, B, H, L, input_scale, u, k)
    return u, k


def direct_conv(u, k, nthreads=None):
    """fp64 direct causal convolution (src/sffft.cu:377) of u [B,H,L] with k [H,L]."""
    u = np.ascontiguousarray(u, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    B, H, L = u.shape
    y = np.empty((B, H, L), np.float64)
    lib().oracle_direct_conv(u, k, y, B, H, L, nthreads or threads())
    return y


def direct_conv_seqs(u, k, seqs):
    """fp64 direct convolution of selected sequences s = b*H + h (src/sffft.cu:376)."""
    u = np.ascontiguousarray(u, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    H, L = k.shape
    s = np.ascontiguousarray(seqs, np.int64)
    y = np.empty((len(s), L), np.float64)
    lib().oracle_direct_conv_seqs(u.reshape(-1), k, y, H, L, s, len(s))
    return y


def fft_conv(u, k, nthreads=None):
    """fp64 FFT causal convolution of every sequence (cross-checked against direct_conv)."""
    u = np.ascontiguousarray(u, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    B, H, L = u.shape
    y = np.empty((B, H, L), np.float64)
    lib().oracle_fft_conv(u, k, y, B, H, L, nthreads or threads())
    return y


def conv(u, k):
    """fp64 reference: direct convolution up to L=2048, FFT convolution above."""
    return direct_conv(u, k) if u.shape[-1] <= 2048 else fft_conv(u, k)


def circ_conv(u, k):
    """fp64 circular convolution of period N over the last axis, y[..., n] = sum_m u[..., m]
    k[..., (n - m) mod N], via numpy's FFT. The reference has no circular convolution
    (README.md:174); this checker is pinned against the brute-force sum in
    tests/test_oracle.py."""
    u = np.asarray(u, np.float64)
    k = np.asarray(k, np.float64)
    return np.fft.ifft(np.fft.fft(u, axis=-1) * np.fft.fft(k, axis=-1), axis=-1).real


def spectrum_p_order(k_row, r0, r1, r2=1):
    """Unnormalised spectrum of one zero-padded filter row in the reference digit order
    (src/sffft.cu:283-288): complex128 array of length 2L."""
    k_row = np.ascontiguousarray(k_row, np.float32)
    L = k_row.shape[0]
    out = np.empty(4 * L, np.float64)
    lib().oracle_spectrum_p_order(k_row, L, r0, r1, r2, out)
    return out[0::2] + 1j * out[1::2]


def fourstep_conv(x, kf_p_order, r0, r1, r2=1, mode=0):
    """Four-step schedule of the reference (Appendix A of the build notes; src/sffft.cu:137-241):
    mode 0 fp64, 1 fp16 storage emulation, 2 plus fp16-rounded raw accumulators."""
    x = np.ascontiguousarray(x, np.float64)
    L = x.shape[0]
    kf = np.ascontiguousarray(np.stack([kf_p_order.real, kf_p_order.imag], -1).reshape(-1), np.float64)
    y = np.empty(L, np.float64)
    lib().oracle_fourstep_conv(x, kf, L, r0, r1, r2, mode, y)
    return y


def round_f16(x: float) -> float:
    """IEEE binary16 round-to-nearest-even of a double (overflow to +-inf)."""
    return lib().oracle_round_f16(x)


def relative_l2(squared_error, squared_reference):
    """src/selection.h:26-29."""
    return lib().oracle_relative_l2(squared_error, squared_reference)


def rel_l2(y, ref) -> float:
    """||y - ref||_2 / ||ref||_2 over all elements (src/sffft.cu:394-399)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return relative_l2(float(np.sum((y - ref) ** 2)), float(np.sum(ref ** 2)))


class _OCand(ctypes.Structure):
    _fields_ = [("method", ctypes.c_char_p), ("io", ctypes.c_char_p), ("config", ctypes.c_char_p),
                ("ms", ctypes.c_double), ("rel_err", ctypes.c_double)]


def select_candidate(cands, max_error, io):
    """src/selection.h:13-24; returns an index or -1."""
    f = lib().oracle_select_candidate
    f.restype = ctypes.c_int
    arr = (_OCand * max(1, len(cands)))()
    keep = []
    for i, (m, o, c, ms, err) in enumerate(cands):
        b = (m.encode(), o.encode(), c.encode())
        keep.append(b)
        arr[i] = _OCand(b[0], b[1], b[2], ms, err)
    f.argtypes = [ctypes.POINTER(_OCand), ctypes.c_int, ctypes.c_double, ctypes.c_char_p]
    return f(arr, len(cands), max_error, io.encode())


def gen_inputs(B, H, L, seed=0, decay=None, dtype=np.float32):
    """Synthetic inputs of the benchmark configurations: u ~ N(0,1) [B,H,L];
    k[h,n] ~ N(0,1) * exp(-n/decay) / sqrt(L) [H,L] (numpy PCG64, seeds seed / seed+1)."""
    decay = decay or max(1.0, L / 4)
    u = np.random.default_rng(seed).standard_normal((B, H, L), dtype=np.float32)
    n = np.arange(L, dtype=np.float64)
    k = (np.random.default_rng(seed + 1).standard_normal((H, L)) * np.exp(-n / decay) / np.sqrt(L)).astype(dtype)
    return u.astype(dtype), k
