"""Selector and relative-error semantics (src/selection.h:8-29), checked three ways:
the reference's own known-answer test compiled from its sources (oracle/_ref), the
reference header itself through a C shim, and libsffft's C ABI and the oracle
against the 17 asserts of tests/selection_test.cpp and random candidate sets."""
import math
import os
import random
import subprocess
import ctypes

import pytest

import oracle
import sffft_amd as sf

NAN, INF = math.nan, math.inf
CANDS = [("strict", "fp32", "p0", 2.0, 0.0004), ("relaxed", "fp32", "p1", 1.0, 0.003),
         ("bf16", "bf16", "p2", 0.5, 0.006), ("nan_error", "fp32", "p3", 0.01, NAN),
         ("inf_error", "fp32", "p4", 0.01, INF), ("nan_time", "fp32", "p5", NAN, 0),
         ("zero_time", "fp32", "p6", 0, 0), ("negative_error", "fp32", "p7", 0.01, -1)]
# (candidate list, max_error, io) -> expected index (tests/selection_test.cpp:17-31)
KAT = [(CANDS, 0.001, "fp32", 0), (CANDS, 0.01, "fp32", 1), (CANDS, 0.01, "bf16", 2), (CANDS, 0.01, "any", 2),
       (CANDS, 0.0004, "fp32", 0), (CANDS, 0.0001, "fp32", -1), (CANDS, 0.001, "bf16", -1),
       (CANDS, NAN, "fp32", -1), (CANDS, INF, "fp32", -1), (CANDS, -1, "fp32", -1), (CANDS, 0, "fp32", -1),
       (CANDS, 0.01, "unknown", -1), ([], 0.01, "fp32", -1),
       (CANDS + [("tie", "fp32", "p8", 1.0, 0.002)], 0.01, "fp32", 8)]


def _ref_select():
    if not os.path.exists(oracle.REF_SELECTION_LIB):
        return None
    L = ctypes.CDLL(oracle.REF_SELECTION_LIB)
    f = L.ref_select_candidate
    f.restype = ctypes.c_int
    sp = ctypes.POINTER(ctypes.c_char_p)
    dp = ctypes.POINTER(ctypes.c_double)
    f.argtypes = [sp, sp, sp, dp, dp, ctypes.c_int, ctypes.c_double, ctypes.c_char_p]
    L.ref_relative_l2.restype = ctypes.c_double
    L.ref_relative_l2.argtypes = [ctypes.c_double, ctypes.c_double]

    def select(cands, max_error, io):
        n = len(cands)
        arr = lambda i: (ctypes.c_char_p * max(1, n))(*[c[i].encode() for c in cands])  # noqa: E731
        num = lambda i: (ctypes.c_double * max(1, n))(*[c[i] for c in cands])  # noqa: E731
        return f(arr(0), arr(1), arr(2), num(3), num(4), n, max_error, io.encode())

    return select, L.ref_relative_l2


@pytest.mark.parametrize("case", range(len(KAT)))
def test_known_answers(case):
    cands, max_error, io, want = KAT[case]
    assert oracle.select_candidate(cands, max_error, io) == want
    assert sf.select_candidate(cands, max_error, io) == want
    ref = _ref_select()
    if ref:
        assert ref[0](cands, max_error, io) == want


def test_relative_l2():
    for f in (oracle.relative_l2, sf.relative_l2):
        assert f(0, 0) == 0 and math.isinf(f(1, 0)) and f(1, 100) == 0.1


def test_random_candidate_sets_agree_with_reference_header():
    ref = _ref_select()
    rng = random.Random(1234)
    vals = [NAN, INF, -INF, 0.0, -1e-9, 1e-4, 3e-4, 5e-4, 1e-3, 2e-3]
    for _ in range(400):
        n = rng.randint(0, 9)
        cands = [(f"m{i}", rng.choice(["fp32", "bf16", "any"]), f"c{i}",
                  rng.choice([NAN, 0.0, -1.0, 0.01, 0.02, 0.02, 0.05, INF]), rng.choice(vals)) for i in range(n)]
        me = rng.choice([NAN, INF, -1.0, 0.0, 1e-4, 5e-4, 1e-3, 3e-3])
        io = rng.choice(["fp32", "bf16", "any", "fp16"])
        a = oracle.select_candidate(cands, me, io)
        assert sf.select_candidate(cands, me, io) == a
        if ref:
            assert ref[0](cands, me, io) == a


def test_reference_known_answer_binary():
    if not os.path.exists(oracle.REF_SELECTION_TEST):
        pytest.skip("reference tree not present when the oracle was built")
    r = subprocess.run([oracle.REF_SELECTION_TEST], capture_output=True, text=True, timeout=30)
    assert r.returncode == 0 and r.stdout.startswith("PASS")
