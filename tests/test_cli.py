"""The Linux command-line host (plamo-3-translate.c_amd/plamo-hip, built from
csrc/cli.c) on the CPU: usage and argument errors with the reference CLI's
exit codes (runtime/cli.c:129-141: 0 done, 1 failure, 2 usage; counts without
sign or leading zero, runtime/cli.c:23-31), a missing model directory, ids
outside the checkpoint's vocabulary (rejected before the GPU is opened), and
a real checkpoint on a host without a GPU, where the backend's open fails
cleanly with its message. Decoding through the host is a GPU test
(test_gpu_cli.py)."""

import os
import subprocess
from pathlib import Path

import pytest

import checkpoint_writer
from parity import plamo_hip

CLI = Path(__file__).resolve().parent.parent / "plamo-3-translate.c_amd" / "plamo-hip"


def run(*args, env=None):
    if not CLI.exists():
        pytest.fail(f"{CLI} is not built (make -C plamo-3-translate.c_amd/csrc)")
    return subprocess.run([str(CLI), *args], capture_output=True, text=True, timeout=120,
                          env=env, stdin=subprocess.DEVNULL)


def test_usage_and_argument_errors():
    r = run("--help")
    assert r.returncode == 0 and r.stdout.startswith("usage: plamo-hip")
    r = run()
    assert r.returncode == 0 and r.stdout.startswith("usage: plamo-hip")
    for bad in (["--max-tokens", "0", "5"], ["--max-tokens", "4097", "5"],
                ["--max-tokens", "07", "5"], ["--max-tokens", "+5", "5"],
                ["--speculative-tokens", "17", "5"], ["--frobnicate", "x", "5"],
                ["5x"], ["-5"], ["4294967296"], ["--model"], ["--max-tokens", "3"]):
        r = run(*bad)
        assert r.returncode == 2, bad
        assert r.stderr.startswith("usage: plamo-hip"), bad


def test_missing_model_directory(tmp_path):
    r = run("--model", str(tmp_path / "absent"), "1", "2")
    assert r.returncode == 1
    assert "config.json" in r.stderr
    env = {k: v for k, v in os.environ.items() if k != "PLAMO_MODEL_DIR"}
    r = run("3", env=env)
    assert r.returncode == 1 and r.stderr


def test_checkpoint_on_a_host_without_gpu(tmp_path):
    syn = plamo_hip.Synthetic(256, 2, 2, 1, 128, 512, 300, window=4, global_capacity=32,
                              pattern=2, seed=3)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    r = run("--model", str(directory), "5", "299,300")
    assert r.returncode == 2 and "outside the vocabulary" in r.stderr
    r = run("--model", str(directory), "--max-tokens", "3", "5,17", "42")
    if r.returncode == 0:
        pytest.skip("a GPU is visible: decoding is covered by test_gpu_cli.py")
    assert r.returncode == 1
    assert "MI355X" in r.stderr
    assert r.stdout == ""


def test_worker_startup_without_gpu(tmp_path):
    """--worker reports a failed start as the reference worker does
    (runtime/worker.c:413-420): one error event, status 1. Ids on the command
    line are a usage error in worker mode."""
    r = run("--worker", "5")
    assert r.returncode == 2 and r.stderr.startswith("usage: plamo-hip")
    syn = plamo_hip.Synthetic(256, 2, 2, 1, 128, 512, 300, window=4, global_capacity=32,
                              pattern=2, seed=3)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=1)
    finally:
        syn.close()
    r = run("--worker", "--model", str(directory))
    if r.returncode == 0:
        pytest.skip("a GPU is visible: the worker is covered by test_gpu_cli.py")
    assert r.returncode == 1
    import json
    event = json.loads(r.stdout)
    assert event["event"] == "error" and event["code"] == "startup_failed"
    assert "MI355X" in event["message"]
