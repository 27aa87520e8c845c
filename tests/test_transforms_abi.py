"""Argument checks and workspace sizes of the standalone transforms; every call here is
rejected before any HIP call, so no GPU is needed."""
import ctypes

import sffft_amd as sf


def test_work_bytes():
    lib = sf.lib()
    assert lib.sffft_fft_work_bytes(4, 16) == 0  # one stage: no workspace
    assert lib.sffft_fft_work_bytes(4, 128) == 4 * 128 * 8
    assert lib.sffft_fft_work_bytes(4, 96) == 0  # not a power of two: rejected
    assert lib.sffft_fft_work_bytes(1, 1 << 25) == 0
    # the largest length: six radix-16 stages (the stage table holds exactly six), so it is
    # accepted and staged through a workspace of one sequence
    assert lib.sffft_fft_work_bytes(1, 1 << 24) == (1 << 24) * 8
    assert lib.sffft_fft_work_bytes(1, 1 << 21) == (1 << 21) * 8
    assert lib.sffft_fft_work_bytes(0, 64) == 0
    assert lib.sffft_fft2_work_bytes(2, 16, 8) == 0
    assert lib.sffft_fft2_work_bytes(2, 64, 128) == 2 * 64 * 128 * 8
    assert lib.sffft_circconv2d_work_bytes(2, 3, 64, 128) == (2 * 3 + 3 + 2 * 3) * 64 * 128 * 8
    assert lib.sffft_circconv2d_work_bytes(2, 3, 64, 100) == 0


def test_argument_errors_need_no_gpu():
    lib = sf.lib()
    E = sf.SFFFT_EINVAL
    null = ctypes.c_void_p(0)
    x, X, w = (ctypes.c_void_p((1 << 40) + i * (1 << 34)) for i in range(3))
    f = lib.sffft_fft_c2c
    assert f(null, X, w, 1 << 20, 2, 128, 1, 128, 0, 1.0, null) == E           # null input
    assert f(x, X, w, 1 << 20, 2, 96, 1, 96, 0, 1.0, null) == E                # N not a power of two
    assert f(x, X, w, 1 << 20, 2, 1, 1, 1, 0, 1.0, null) == E                  # N < 2
    assert f(x, X, w, 1 << 40, 1, 1 << 25, 1, 0, 0, 1.0, null) == E           # N > 2^24
    assert f(x, X, w, 1 << 40, 1 << 12, 1 << 20, 1, 1 << 20, 0, 1.0, null) == E  # batch * N > 2^31
    assert f(x, X, w, 1 << 20, 2, 128, 0, 128, 0, 1.0, null) == E              # stride 0
    assert f(x, X, w, 1 << 20, 2, 128, 1, 0, 0, 1.0, null) == E                # sequences alias
    assert f(x, X, w, 1 << 20, 2, 128, 1, 1, 0, 1.0, null) == E                # overlapping sequences
    assert f(x, X, w, 1 << 20, 4, 128, 2, 128, 0, 1.0, null) == E              # dist < N * stride, stride < batch
    assert f(x, X, w, 1 << 20, 4, 128, 3, 1, 0, 1.0, null) == E                # interleaved, stride < batch * dist
    assert f(x, ctypes.c_void_p((1 << 40) + 8), w, 1 << 20, 2, 128, 1, 128, 0, 1.0, null) == E  # x, X overlap
    assert f(x, X, w, 1 << 20, 2, 128, 1, 128, 2, 1.0, null) == E              # inverse not 0/1
    assert f(x, X, w, 2 * 128 * 8 - 8, 2, 128, 1, 128, 0, 1.0, null) == E      # workspace too small
    assert f(x, X, null, 1 << 20, 2, 128, 1, 128, 0, 1.0, null) == E           # workspace missing
    assert f(x, X, ctypes.c_void_p((1 << 40) + 8), 1 << 20, 2, 128, 1, 128, 0, 1.0, null) == E  # overlaps x
    assert f(ctypes.c_void_p((1 << 40) + 4), X, w, 1 << 20, 2, 128, 1, 128, 0, 1.0, null) == E  # misaligned
    g = lib.sffft_fft2_c2c
    assert g(x, X, w, 1 << 20, 2, 64, 100, 0, 1.0, null) == E                  # N1 not a power of two
    assert g(x, X, w, 10, 2, 64, 128, 0, 1.0, null) == E                       # workspace too small
    assert g(x, ctypes.c_void_p((1 << 40) + 64), w, 1 << 20, 2, 64, 128, 0, 1.0, null) == E  # partial overlap
    c = lib.sffft_circconv2d_f32
    need = lib.sffft_circconv2d_work_bytes(2, 3, 64, 128)
    assert c(x, X, ctypes.c_void_p((1 << 40) + (1 << 36)), w, need - 8, 2, 3, 64, 128, null) == E  # too small
    assert c(x, X, ctypes.c_void_p((1 << 40) + 64), w, need, 2, 3, 64, 128, null) == E           # y overlaps u
    assert c(x, X, ctypes.c_void_p((1 << 40) + (1 << 36)), w, need, 2, 3, 64, 96, null) == E     # N1 invalid


def test_layout_families():
    """sffft_fft_c2c takes two layout families: whole sequences one after another
    (dist >= N * stride) and sequences interleaved within one element step (stride >=
    batch * dist). Layouts between them are rejected before any HIP call, including
    non-overlapping ones."""
    lib = sf.lib()
    E = sf.SFFFT_EINVAL
    null = ctypes.c_void_p(0)
    x, X, w = (ctypes.c_void_p((1 << 40) + i * (1 << 34)) for i in range(3))
    f = lib.sffft_fft_c2c

    def disjoint(batch, N, stride, dist):
        addrs = {b * dist + n * stride for b in range(batch) for n in range(N)}
        return len(addrs) == batch * N

    # between the families, yet one-to-one: 3 sequences of 4 at stride 2, 5 apart
    assert disjoint(3, 4, 2, 5)
    assert f(x, X, w, 1 << 20, 3, 4, 2, 5, 0, 1.0, null) == E
    # the same with N = 128 (the workspace path): the odd distance interleaves the middle
    # sequence's elements between the others', and an overlapping one
    assert disjoint(3, 128, 2, 129)
    assert f(x, X, w, 1 << 20, 3, 128, 2, 129, 0, 1.0, null) == E
    assert not disjoint(3, 128, 2, 4)
    assert f(x, X, w, 1 << 20, 3, 128, 2, 4, 0, 1.0, null) == E
    # the edges of the two families are accepted: tests/test_gpu_transforms.py runs them
