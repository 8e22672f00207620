"""CPU checks of bench.py's command-line contract: this build measures one
GPU, so --gpus above 1 exits with status 2 and a message naming the reason
before a model is built or a GPU touched; --help lists the measurement modes
(the default decode/TTFT line, --speculative and --verify)."""

import subprocess
import sys
from pathlib import Path

BENCH = Path(__file__).resolve().parent.parent / "bench.py"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(BENCH), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_help_lists_the_modes():
    r = subprocess.run([sys.executable, str(BENCH), "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for flag in ("--steps", "--warmup", "--speculative", "--verify", "--verify-tokens"):
        assert flag in r.stdout
