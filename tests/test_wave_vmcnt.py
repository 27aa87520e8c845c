"""The wave-pipeline kernels wait for their LDS table copies with an explicit
vector-memory count (fftconv_wave.hpp: the copies, then the first pair's loads, then
`s_waitcnt vmcnt(pair_load_issues)` and a raw `s_barrier`). That is only correct if
the compiled code issues exactly that many loads after the last copy and does not
wait for fewer. This test compiles the device code of every length and checks each
wave kernel's prologue in the gfx950 assembly (no GPU needed)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "sffft_amd", "csrc", "conv_inst.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-fno-slp-vectorize", "-mllvm", "-amdgpu-mfma-vgpr-form", "--cuda-device-only", "-S"]


def kernels(asm):
    lines = asm.split("\n")
    starts = [i for i, l in enumerate(lines) if re.match(r"^_ZN5sffft19fftconv_wave_kernel\S+:", l)]
    for st in starts:
        body = []
        for l in lines[st + 1:]:
            if l.startswith(".Lfunc_end"):
                break
            t = l.strip()
            if t and not t.startswith((";", ".")):
                body.append(t)
        yield lines[st].split(":")[0], body


@pytest.mark.parametrize("L", [128, 256, 512, 1024, 2048])
def test_prologue_waits_for_the_copies_only(L, tmp_path):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    out = tmp_path / f"c{L}.s"
    subprocess.run([HIPCC if os.path.exists(HIPCC) else "hipcc"] + FLAGS + [f"-DSFFFT_INST_L={L}", SRC, "-o",
                    str(out)], check=True, capture_output=True, timeout=600)
    n = 0
    for name, body in kernels(out.read_text()):
        n += 1
        bi = next(i for i, t in enumerate(body) if t.startswith("s_barrier"))
        pre = body[:bi]
        last_copy = max(i for i, t in enumerate(pre) if t.startswith("global_load_lds"))
        loads = [t for t in pre[last_copy + 1:] if t.split()[0].startswith(("global_load", "buffer_load"))]
        waits = [int(m.group(1)) for t in pre if t.startswith("s_waitcnt")
                 for m in [re.search(r"vmcnt\((\d+)\)", t)] if m]
        expect = min(len(loads), 63)
        assert loads, name
        # correctness: the active path waits until at most `expect` operations are in
        # flight, i.e. every copy has landed (a larger count alone would not be enough)
        assert expect in waits, (name, len(loads), waits)
        assert all(w <= expect for w in waits), (name, len(loads), waits)
        # overlap: only the idle path (no pair for this wave) drains the counter
        assert waits.count(0) <= 1, (name, len(loads), waits)
    assert n > 0
