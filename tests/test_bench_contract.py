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


def test_embedded_draft_policy():
    """The speculative line's draft-weight policy (bench.embed_draft) on the
    CPU oracle at a small shape: with the target's later layers mixed in at 0
    the target computes the draft's function, so their greedy choices agree
    step for step (the rescaled norms are the only difference); at mix 1 the
    later layers are ordinary random layers and the agreement is gone."""
    import importlib.util

    import numpy as np

    import oracle_lib
    import plamo_hip

    spec = importlib.util.spec_from_file_location("bench", BENCH)
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    agreement = {}
    for mix in (0.0, 1.0):
        d = plamo_hip.Synthetic(64, 4, 4, 2, 16, 128, 300, tied=1, seed=5, window=64,
                                global_capacity=128, pattern=2)
        t = plamo_hip.Synthetic(192, 15, 12, 4, 16, 384, 300, tied=1, seed=6, window=64,
                                global_capacity=128, pattern=2)
        di, ti = d.instance(), t.instance()
        try:
            assert bench.embed_draft(ti, di, mix) > 0
            prompt = [int(x) for x in np.random.default_rng(1).integers(0, 300, 20)]
            assert oracle_lib.prefill(di, prompt) and oracle_lib.prefill(ti, prompt)
            same = 0
            for _ in range(40):
                a, b = int(np.argmax(di.logits())), int(np.argmax(ti.logits()))
                same += a == b
                assert oracle_lib.forward(di, b) and oracle_lib.forward(ti, b)
            agreement[mix] = same
        finally:
            for x in (di, ti):
                x.close()
            d.close()
            t.close()
    assert agreement[0.0] >= 38 and agreement[1.0] <= 10, agreement
