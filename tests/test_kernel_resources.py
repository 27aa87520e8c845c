"""The compiler's resource report of the built kernels: no kernel of a default plan spills.

A spill puts per-lane scratch traffic into a kernel whose budget is HBM bytes, and the
register allocation of these kernels moves with small source changes (a one-line mask of
the lane index once raised the 64x32 wave kernel from 151 VGPRs to a 24-value spill). The
build keeps hipcc's `-Rpass-analysis=kernel-resource-usage` report of every length beside
its object (sffft_amd/_build/conv_L<L>.o.resources); this test reads it, so it needs no GPU.
"""
import glob
import os
import re

import pytest

import sffft_amd as sf

BUILD = os.path.join(os.path.dirname(sf.LIB_PATH), "_build")


def reports(build=BUILD):
    """{mangled kernel name: {field: value}} over every length's report in `build` (a
    field's bracketed unit, as in `ScratchSize [bytes/lane]`, is dropped from its name)."""
    out = {}
    for path in sorted(glob.glob(os.path.join(build, "conv_L*.o.resources"))):
        cur = None
        for line in open(path):
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                cur = out.setdefault(m.group(1), {})
                continue
            m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\w+) \[", line)
            if m and cur is not None:
                cur[m.group(1).strip()] = m.group(2)
    return out


def mangled_prefix(L, io, acc):
    """Mangled-name prefix of the kernel the default plan of (L, io) launches with real
    filters and cached DFT tables."""
    spec, waves, seqs, mode, channels = sf.DEFAULT_PLANS[(L, io)]
    radices = "".join(f"ELi{r}" for r in spec.split("x"))[1:]
    t = "f" if io == "fp32" else "t"
    if mode == 1:
        return (f"_ZN5sffft19fftconv_wave_kernelINS_8WavePlanI{radices}EEELi{waves}ELi{channels}E"
                f"{t}Lb1ELb{acc}ELb1E")
    return f"_ZN5sffft14fftconv_kernelINS_4PlanI{radices}EEELi{waves}ELi{seqs}E{t}Lb1ELb{acc}E"


@pytest.fixture(scope="module")
def rep():
    r = reports()
    if not r:
        pytest.skip("no resource reports: build with `make -C sffft_amd` first")
    return r


@pytest.mark.parametrize("acc", [0, 1])
@pytest.mark.parametrize("key", sorted(sf.DEFAULT_PLANS))
def test_default_plans_do_not_spill(rep, key, acc):
    L, io = key
    prefix = mangled_prefix(L, io, acc)
    hits = {n: v for n, v in rep.items() if n.startswith(prefix)}
    assert len(hits) == 1, (key, acc, prefix, sorted(hits))
    (name, v), = hits.items()
    assert int(v["VGPRs Spill"]) == 0 and int(v["ScratchSize"]) == 0, (key, acc, v)
    # the wave plans sized their workgroups for these occupancies (one workgroup of 12
    # wavefronts per CU at L = 1024 and 2048, several of 4 below)
    if sf.DEFAULT_PLANS[key][3] == 1 and L >= 1024:
        assert int(v["Occupancy"]) >= 3, (key, acc, v)


def test_report_parser_reads_a_spill():
    """The parser on a report of the form hipcc writes, with a spill planted."""
    text = ("csrc/fftconv_wave.hpp:581:1: remark: Function Name: _ZN5sffft19k [-Rpass-analysis=kernel-resource-usage]\n"
            "csrc/fftconv_wave.hpp:581:1: remark:     VGPRs: 168 [-Rpass-analysis=kernel-resource-usage]\n"
            "csrc/fftconv_wave.hpp:581:1: remark:     ScratchSize [bytes/lane]: 100 [-Rpass-analysis=kernel-resource-usage]\n"
            "csrc/fftconv_wave.hpp:581:1: remark:     VGPRs Spill: 24 [-Rpass-analysis=kernel-resource-usage]\n")
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        open(os.path.join(d, "conv_L1.o.resources"), "w").write(text)
        r = reports(d)
    assert r == {"_ZN5sffft19k": {"VGPRs": "168", "ScratchSize": "100", "VGPRs Spill": "24"}}
