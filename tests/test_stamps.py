"""The kernel-source stamps that tie a profile summary to the build it measured
(bench.py copies a summary's HBM traffic into its line only for an equal stamp)."""
import os

import bench
import sffft_amd as sf


def test_stamp_per_kernel_family():
    assert sf.kernel_sources_sha(0) == sf.kernel_sources_sha(1)  # both single-pass
    assert sf.kernel_sources_sha(1) != sf.kernel_sources_sha(2)
    assert len(sf.kernel_sources_sha(2)) == 16
    # the multi-pass kernels include the single-pass headers
    assert set(sf.SINGLE_PASS_SOURCES) < set(sf.MULTI_PASS_SOURCES)
    for rel in sf.MULTI_PASS_SOURCES:
        assert os.path.exists(os.path.join(os.path.dirname(sf.__file__), rel)), rel


def test_code_only_ignores_comments_and_layout():
    a = "int f(int x) {  // first\n  return x + 1; /* two\n lines */\n}\n"
    b = "// header\nint f(int x) {\n\n        return x + 1;\n}  // end\n"
    assert sf._code_only("csrc/a.hpp", a) == sf._code_only("csrc/a.hpp", b)
    assert sf._code_only("csrc/a.hpp", a) != sf._code_only("csrc/a.hpp", a.replace("x + 1", "x + 2"))
    m1 = "# flags\nHIPFLAGS ?= -O3\n\nall: x\n"
    m2 = "HIPFLAGS ?= -O3\n# the default target\nall: x\n"
    assert sf._code_only("Makefile", m1) == sf._code_only("Makefile", m2)
    assert sf._code_only("Makefile", m1) != sf._code_only("Makefile", m1.replace("-O3", "-O2"))


def test_profiled_traffic_needs_the_same_stamp():
    plan = sf.default_plan(1024, "fp32", 8)
    workload = "B=8 H=768 L=1024 fp32"
    assert bench.profiled_traffic(workload, plan, "0" * 16) is None
    # a committed summary exists for the benchmark workload; with this build's stamp it
    # either matches (profiled build) or the line reports null
    got = bench.profiled_traffic(workload, plan, sf.kernel_sources_sha(plan.mode))
    assert got is None or got > 0
