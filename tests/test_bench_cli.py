"""bench.py's command line: the cases it must refuse before touching a GPU."""

import subprocess
import sys
from pathlib import Path

import pytest

BENCH = Path(__file__).resolve().parent.parent / "bench.py"


def _run(*args):
    return subprocess.run([sys.executable, str(BENCH), *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args,message", [
    (["--gpus", "2"], "one GPU only"),
    (["--gpus", "8", "--steps", "5"], "one GPU only"),
    (["--steps", "0"], "--steps must be >= 1"),
    (["--warmup", "-1"], "--steps must be >= 1 and --warmup >= 0"),
    (["--legs", "decode,nope"], "unknown legs ['nope']"),
])
def test_bench_refuses_before_any_gpu_work(args, message):
    r = _run(*args)
    assert r.returncode == 1
    assert message in r.stderr
    assert r.stdout == ""  # no JSON line for a refused run


def test_bench_help_lists_every_leg():
    r = _run("--help")
    assert r.returncode == 0
    for leg in ("decode", "lm", "layer", "prefill", "batch", "fx", "q4c", "group"):
        assert leg in r.stdout
