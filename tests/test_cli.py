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
