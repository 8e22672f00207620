"""The reference's own front-ends on Linux, on the CPU: runtime/cli.c (the
`plamo` command) and runtime/worker.c (the persistent `plamo-worker`) compile
unchanged with -Werror against include/ and link with libplamo_hip.so and the
reference engine (tests/engine_link/Makefile). Their one Darwin header,
<sys/qos.h>, is stood in for by tests/engine_link/darwin/sys/qos.h.

What runs without a GPU: the CLI's argument handling and exit codes
(runtime/cli.c:11-21, 38-104: 0 for --help, 2 for usage errors, 1 for engine
errors), its tokenizer-only mode (TEXT alone prints the prompt ids without
loading weights, runtime/cli.c:114-125), and the worker's tokenizer-only
protocol (runtime/worker.c:1-4, 427-489): the ready event, op 2 tokenize
frames, op 3 cancel frames between requests, NUL rejection, malformed frames
and end of input. The tokenizer is the engine-link test's stand-in
(tests/engine_link/host_stubs.c).

Skipped where the reference checkout is absent (its sources are compiled where
they lie, never copied)."""

import json
import os
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

import plamo_hip

ROOT = Path(__file__).resolve().parents[1]
HERE = ROOT / "tests" / "engine_link"
REF = Path("/root/reference/runtime")

pytestmark = pytest.mark.skipif(
    not (REF / "cli.c").exists() or shutil.which("gcc") is None or shutil.which("make") is None,
    reason="the reference checkout (runtime/cli.c) or gcc/make is not available")

PREFIX = [[20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 29, 23],
          [20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 30, 23]]


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    out = tmp_path_factory.mktemp("frontends")
    r = subprocess.run(["make", "-C", str(HERE), f"REF={REF}", f"OUT={out}", "-B"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return out


@pytest.fixture
def vocab_dir(tmp_path):
    (tmp_path / "tokenizer.jsonl").write_text("300\n")
    return tmp_path


def env(directory):
    return dict(os.environ, LD_LIBRARY_PATH=str(plamo_hip.LIB_PATH.parent),
                PLAMO_MODEL_DIR=str(directory))


def toy_ids(text: str, vocab: int = 300):
    return [32 + b % (vocab - 32) for b in text.encode()]


def frame(op, direction=0, max_tokens=0, body=b""):
    return struct.pack("<4I", op, direction, max_tokens, len(body)) + body


def test_frontends_compile_unchanged(built):
    """cli.c and worker.c see the library's headers through the shims and the
    Linux <sys/qos.h>; both link with --no-undefined."""
    for source in ("cli.c", "worker.c"):
        r = subprocess.run(["gcc", "-std=gnu11", "-fsyntax-only", "-H", f"-I{HERE / 'shim'}",
                            "-I-", f"-I{ROOT / 'include'}", f"-I{REF}", f"-I{HERE / 'darwin'}",
                            str(REF / source)], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stderr
        names = {Path(line.split()[-1]).name for line in r.stderr.splitlines()
                 if line.startswith(".")}
        assert {"plamo_backend.h", "plamo_model.h", "qos.h"} <= names, (source, names)
    assert (built / "plamo").exists() and (built / "plamo-worker").exists()
    for binary in ("plamo", "plamo-worker"):
        r = subprocess.run(["nm", "-u", str(built / binary)], capture_output=True, text=True)
        undefined = {line.split()[-1].split("@")[0] for line in r.stdout.splitlines()}
        # The backend, the hook trampolines and the draft interface come from the library.
        assert {"plamo_metal_open", "plamo_forward", "plamo_argmax"} <= undefined


def test_cli_usage_and_exit_codes(built, vocab_dir):
    cli = built / "plamo"
    e = env(vocab_dir)
    r = subprocess.run([str(cli), "--help"], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 0 and r.stdout.startswith("usage: plamo")
    r = subprocess.run([str(cli)], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 0 and r.stdout.startswith("usage: plamo")
    for bad in (["--max-tokens", "0", "x"], ["--max-tokens", "4097", "x"], ["--threads", "65", "x"],
                ["--backend", "cuda", "x"], ["--memory", "swap", "x"], ["-j"], ["-x", "y"],
                ["a", "b"], ["-g", "a", "-j", "b"], ["--threads"]):
        r = subprocess.run([str(cli), *bad], capture_output=True, text=True, env=e, timeout=30)
        assert r.returncode == 2 and r.stderr.startswith("usage: plamo"), bad
    # A missing model is an engine error: exit 1 with the engine's message.
    r = subprocess.run([str(cli), "-j", "hi"], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 1
    assert r.stderr.splitlines()[-1].startswith("plamo: missing or invalid weight files")


def test_cli_tokenizes_without_weights(built, vocab_dir):
    e = env(vocab_dir)
    r = subprocess.run([str(built / "plamo"), "hi"], capture_output=True, text=True, env=e,
                       timeout=30)
    assert r.returncode == 0, r.stderr
    assert [int(x) for x in r.stdout.split()] == toy_ids("hi")
    # After `--` a leading dash is text (runtime/cli.c:53-56, 100-103).
    r = subprocess.run([str(built / "plamo"), "--", "-x"], capture_output=True, text=True, env=e,
                       timeout=30)
    assert r.returncode == 0 and [int(x) for x in r.stdout.split()] == toy_ids("-x")


def test_worker_tokenizer_only_protocol(built, vocab_dir):
    requests = (frame(2, 1, 0, b"hi") + frame(3) + frame(2, 2, 0, b"ok") + frame(2, 0, 0, b"a\0b")
                + frame(2, 0, 0, b"plain"))
    r = subprocess.run([str(built / "plamo-worker"), "--tokenizer-only"], input=requests,
                       capture_output=True, env=env(vocab_dir), timeout=30)
    assert r.returncode == 0, r.stderr  # end of input ends the worker cleanly
    events = [json.loads(line) for line in r.stdout.decode().splitlines()]
    ready = events[0]
    assert ready["event"] == "ready" and ready["protocol"] == 1
    assert ready["memory"]["mode"] == "tokenizer" and ready["compute"]["backend"] == "cpu"
    assert ready["model"] == "plamo-3-translate-custom"
    assert events[1] == {"event": "tokenized", "prompt_tokens": 15,
                         "token_ids": PREFIX[0] + toy_ids("hi") + [17]}
    # The cancel frame between requests is consumed silently.
    assert events[2]["token_ids"] == PREFIX[1] + toy_ids("ok") + [17]
    assert events[3] == {"event": "error", "code": "invalid_input",
                         "message": "NUL characters are not supported"}
    assert events[4]["token_ids"] == toy_ids("plain")
    assert len(events) == 5


@pytest.mark.parametrize("requests,message", [
    (frame(7), "invalid request frame"),
    (struct.pack("<4I", 2, 0, 0, 16385), "invalid request frame"),
    (struct.pack("<2I", 2, 0), "incomplete request header"),
    (struct.pack("<4I", 2, 0, 0, 10) + b"abc", "incomplete text"),
])
def test_worker_protocol_errors(built, vocab_dir, requests, message):
    r = subprocess.run([str(built / "plamo-worker"), "--tokenizer-only"], input=requests,
                       capture_output=True, env=env(vocab_dir), timeout=30)
    assert r.returncode == 1
    events = [json.loads(line) for line in r.stdout.decode().splitlines()]
    assert events[0]["event"] == "ready"
    assert events[-1] == {"event": "error", "code": "protocol_error", "message": message}


def test_worker_arguments_and_startup_failure(built, vocab_dir):
    worker = str(built / "plamo-worker")
    e = env(vocab_dir)
    r = subprocess.run([worker, "--help"], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 0 and r.stdout.startswith("usage: plamo-worker")
    for bad in (["--threads", "0"], ["--backend", "x"], ["--memory", "x"], ["--bogus"]):
        r = subprocess.run([worker, *bad], capture_output=True, text=True, env=e, timeout=30)
        assert r.returncode == 64, bad
    # The draft peer serves only the 0.8b / 2b profiles (runtime/worker.c:385-390).
    r = subprocess.run([worker, "--draft-peer"], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 64
    # No weights: a startup_failed event and exit 1.
    r = subprocess.run([worker], capture_output=True, text=True, env=e, timeout=30)
    assert r.returncode == 1
    event = json.loads(r.stdout.splitlines()[-1])
    assert event["event"] == "error" and event["code"] == "startup_failed"
