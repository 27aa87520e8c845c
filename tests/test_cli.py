"""CLI validation of the `sffft` driver (mirrors tests/precision_smoke.sh:20-35 of
the reference): argument errors exit 1 before any GPU work, --help exits 0."""
import os
import subprocess

import pytest

import sffft_amd as sf

CASES_EXIT1 = [
    ["--max-error", v] for v in ("nan", "inf", "0", "-1", "1e-999", "garbage")
] + [
    ["--max-error"], ["--io", "unknown"], ["--seed", "0"], ["--seed", "-1"], ["--input-scale", "inf"],
    ["--input-scale", "0"], ["--allocator", "unknown"], ["--allocator"], ["--kernel", "unknown"], ["--kernel"],
    ["0", "1", "128"], ["1", "0", "128"], ["1", "1", "129"], ["2147483647", "2", "128"],
    ["1", "1", "32768"], ["1", "1", "64"], ["1", "2", "3", "4"], ["x"], ["--seed", "12abc"],
    ["--input-scale", "1e39"],
]


def run(args):
    if not os.path.exists(sf.CLI_PATH):
        pytest.fail(f"{sf.CLI_PATH} is not built (make -C sffft_amd)")
    return subprocess.run([sf.CLI_PATH] + args, capture_output=True, text=True, timeout=60)


def test_help_exits_zero():
    r = run(["--help"])
    assert r.returncode == 0 and "Usage: sffft" in r.stdout


@pytest.mark.parametrize("args", CASES_EXIT1, ids=lambda a: " ".join(a) or "empty")
def test_invalid_arguments_exit_one(args):
    assert run(args).returncode == 1


@pytest.mark.parametrize("B,H,L,extra", [(2, 3, 128, []), (1, 5, 1024, ["--seed", "42"]),
                                         (2, 2, 256, ["--seed", "12345", "--input-scale", "25000"])])
def test_driver_inputs_are_the_reference_generator(tmp_path, B, H, L, extra):
    """The driver's calibration inputs are bit-identical to the oracle's restatement of the
    reference generator (src/sffft.cu:308-310,339-341) for the same seed and scale."""
    import numpy as np

    import oracle

    path = tmp_path / "inputs.bin"
    r = run([str(B), str(H), str(L), "--dump-inputs", str(path)] + extra)
    assert r.returncode == 0, r.stderr
    raw = np.fromfile(path, np.float32)
    assert raw.size == B * H * L + H * L
    seed = int(extra[extra.index("--seed") + 1]) if "--seed" in extra else oracle.DEFAULT_SEED
    scale = float(extra[extra.index("--input-scale") + 1]) if "--input-scale" in extra else 1.0
    u, k = oracle.ref_inputs(B, H, L, seed=seed, input_scale=scale)
    assert np.array_equal(raw[:B * H * L].view(np.uint32), u.reshape(-1).view(np.uint32))
    assert np.array_equal(raw[B * H * L:].view(np.uint32), k.reshape(-1).view(np.uint32))


def test_dump_inputs_needs_a_length(tmp_path):
    assert run(["1", "1", "--dump-inputs", str(tmp_path / "x")]).returncode == 1
    assert run(["1", "1", "128", "--dump-inputs"]).returncode == 1
