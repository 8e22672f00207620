"""The reference's own front-ends driving the library on the GPU.

tests/engine_link/_build/plamo and plamo-worker are runtime/cli.c and
runtime/worker.c compiled unchanged (with runtime/engine.c and
runtime/prompt_cache.c) against include/ and libplamo_hip.so; only <sys/qos.h>
and the tokenizer are stood in for (tests/engine_link/darwin,
tests/engine_link/host_stubs.c). They are built by __graft_entry__.build()
where the reference checkout exists and shipped prebuilt.

- `plamo -j/-e/-g TEXT` (runtime/cli.c:104-131): one request, no prompt
  cache, tokens printed as the tokenizer decodes them ("<id>" here).
- `plamo-worker` (runtime/worker.c:380-489): prepares both translation
  prefixes, reports ready, serves translate frames with prefill, token and
  done events, and a cancel frame that arrives during generation.
- `plamo-worker --draft-peer` (runtime/worker.c:197-318) over a checkpoint of
  the 0.8b profile's shape (the peer refuses other models): reset, proposal
  and acceptance frames, where an acceptance below the forwarded count rolls
  the KV rows back on the host (plamo_draft_restore) and the backend must pick
  the edit up, and an acceptance one past it forwards the last proposal.

Every generated or proposed id must equal the oracle's greedy sequence over
the same checkpoint and prompt ids, with the GPU backend open (no CPU
fallback)."""

import json
import os
import re
import select
import struct
import subprocess
import time
from pathlib import Path

import numpy as np
import pytest

import checkpoint_writer
from parity import oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

BUILD = Path(__file__).resolve().parent / "engine_link" / "_build"
CLI, WORKER = BUILD / "plamo", BUILD / "plamo-worker"
PREFIX = [[20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 29, 23],
          [20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 30, 23]]
DRAFT_MAGIC = 0x504C4431

needs_build = pytest.mark.skipif(not (CLI.exists() and WORKER.exists()),
                                 reason="the front-ends were not built (needs the reference "
                                        "checkout at build time)")


def toy_prompt(text: str, direction: int, vocab: int):
    """The stand-in tokenizer's ids (tests/engine_link/host_stubs.c)."""
    ids = [32 + b % (vocab - 32) for b in text.encode()]
    return PREFIX[direction - 1] + ids + [17] if direction else ids


def oracle_greedy(directory, prompt, max_tokens):
    ck = plamo_hip.Checkpoint(directory)
    cpu = ck.instance()
    try:
        assert oracle_lib.prefill(cpu, prompt)
        out = []
        token = int(np.argmax(cpu.logits()))
        while len(out) < max_tokens and token not in (1, 16):
            out.append(token)
            if len(out) == max_tokens:
                break
            assert oracle_lib.forward(cpu, token)
            token = int(np.argmax(cpu.logits()))
        return out
    finally:
        cpu.close()
        ck.close()


def frame(op, a=0, b=0, body=b""):
    return struct.pack("<4I", op, a, b, len(body)) + body


class Pipe:
    """A worker process with bounded reads of its stdout."""

    def __init__(self, args, env):
        self.p = subprocess.Popen(args, stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                  stderr=subprocess.PIPE, env=env)
        self.buf = b""

    def send(self, data):
        self.p.stdin.write(data)
        self.p.stdin.flush()

    def read(self, n, timeout=120):
        deadline = time.monotonic() + timeout
        while len(self.buf) < n:
            left = deadline - time.monotonic()
            ready, _, _ = select.select([self.p.stdout], [], [], max(left, 0))
            if not ready:
                raise TimeoutError(f"worker silent for {timeout} s")
            chunk = os.read(self.p.stdout.fileno(), 1 << 16)
            if not chunk:
                raise EOFError(f"worker ended: {self.p.wait()} {self.p.stderr.read().decode()}")
            self.buf += chunk
        out, self.buf = self.buf[:n], self.buf[n:]
        return out

    def event(self, timeout=120):
        deadline = time.monotonic() + timeout
        while b"\n" not in self.buf:
            ready, _, _ = select.select([self.p.stdout], [], [],
                                        max(deadline - time.monotonic(), 0))
            if not ready:
                raise TimeoutError(f"worker silent for {timeout} s")
            chunk = os.read(self.p.stdout.fileno(), 1 << 16)
            if not chunk:
                raise EOFError(f"worker ended: {self.p.wait()} {self.p.stderr.read().decode()}")
            self.buf += chunk
        line, self.buf = self.buf.split(b"\n", 1)
        return json.loads(line)

    def close(self, timeout=60):
        self.p.stdin.close()
        try:
            return self.p.wait(timeout)
        except subprocess.TimeoutExpired:
            self.p.kill()
            self.p.wait()
            raise


@pytest.fixture(scope="module")
def small_checkpoint(tmp_path_factory):
    syn = plamo_hip.Synthetic(512, 4, 8, 2, 64, 1024, 1000, window=16, global_capacity=256,
                              pattern=2, seed=37)
    try:
        directory = checkpoint_writer.write(tmp_path_factory.mktemp("fe") / "ck", syn, shards=2)
    finally:
        syn.close()
    (directory / "tokenizer.jsonl").write_text("1000\n")
    return directory


def lib_env(directory):
    return dict(os.environ, PLAMO_MODEL_DIR=str(directory),
                LD_LIBRARY_PATH=str(plamo_hip.LIB_PATH.parent))


@needs_build
def test_reference_cli_translates_on_gpu(small_checkpoint):
    env = lib_env(small_checkpoint)
    for flag, direction, text, max_tokens in (("-j", 1, "The CLI is unchanged.", 10),
                                              ("-e", 2, "Other direction.", 10),
                                              ("-g", 0, "raw prompt", 6)):
        say(f"plamo {flag}, {max_tokens} tokens")
        r = subprocess.run([str(CLI), "--backend", "metal", "--max-tokens", str(max_tokens), flag,
                            text], capture_output=True, text=True, timeout=120, env=env)
        assert r.returncode == 0, r.stderr
        printed = [int(v) for v in re.findall(r"<(\d+)>", r.stdout)]
        assert r.stdout.endswith("\n") and "".join(f"<{i}>" for i in printed) == r.stdout[:-1]
        expected = oracle_greedy(small_checkpoint, toy_prompt(text, direction, 1000), max_tokens)
        assert printed == expected, (printed, expected)
    # --backend auto takes the GPU as well (runtime/engine.c:180-185).
    r = subprocess.run([str(CLI), "--max-tokens", "4", "-j", "auto"], capture_output=True,
                       text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    assert [int(v) for v in re.findall(r"<(\d+)>", r.stdout)] == oracle_greedy(
        small_checkpoint, toy_prompt("auto", 1, 1000), 4)


@needs_build
def test_reference_worker_serves_on_gpu(small_checkpoint):
    say("plamo-worker start")
    w = Pipe([str(WORKER), "--backend", "metal", "--memory", "resident"],
             lib_env(small_checkpoint))
    try:
        ready = w.event()
        assert ready["event"] == "ready", ready
        assert ready["compute"]["backend"] == "metal" and ready["memory"]["mode"] == "resident"
        assert ready["compute"]["cpu_fallbacks"] == 0 and ready["compute"]["errors"] == 0
        # Both fixed prefixes were prefilled on the GPU and captured at prepare.
        assert ready["prompt_cache"]["en_ja_tokens"] == 12
        assert ready["prompt_cache"]["ja_en_tokens"] == 12
        for direction, text, max_tokens in ((1, "first request", 8), (2, "second request", 8),
                                            (1, "third, en-ja again", 8), (0, "raw", 5)):
            say(f"plamo-worker translate direction {direction}")
            w.send(frame(1, direction, max_tokens, text.encode()))
            prompt = toy_prompt(text, direction, 1000)
            event = w.event()
            assert event["event"] == "prefill" and event["prompt_tokens"] == len(prompt)
            ids = []
            while True:
                event = w.event()
                if event["event"] != "token":
                    break
                ids.append(int(re.fullmatch(r"<(\d+)>", bytes.fromhex(event["hex"]).decode())[1]))
            assert event["event"] == "done", event
            assert event["usage"]["prompt_tokens"] == len(prompt)
            assert event["usage"]["completion_tokens"] == len(ids)
            assert event["usage"]["cached_prompt_tokens"] == (12 if direction else 0)
            assert event["compute"]["cpu_fallbacks"] == 0 and event["compute"]["errors"] == 0
            assert ids == oracle_greedy(small_checkpoint, prompt, max_tokens), direction
        # A cancel frame already waiting when the first token is ready ends the
        # request with no token (runtime/worker.c:114-126).
        say("plamo-worker cancel")
        w.send(frame(1, 1, 8, b"cancel me") + frame(3))
        assert w.event()["event"] == "prefill"
        event = w.event()
        assert event["event"] == "done" and event["finish_reason"] == "cancelled", event
        assert event["usage"]["completion_tokens"] == 0
        w.send(frame(2, 2, 0, b"tok"))
        assert w.event()["token_ids"] == toy_prompt("tok", 2, 1000)
        assert w.close() == 0
    finally:
        if w.p.poll() is None:
            w.p.kill()
            w.p.wait()


@needs_build
def test_reference_draft_peer_on_gpu(tmp_path):
    """The 0.8b profile's shape: hidden 1536, 16 layers, 16 query heads over one
    KV head, MLP 6144, vocabulary 107520 (tools/profiles/0.8b/config.json)."""
    say("draft peer: writing a 0.8b-shaped checkpoint")
    syn = plamo_hip.Synthetic(1536, 16, 16, 1, 128, 6144, 107520, window=2048, global_capacity=1024,
                              pattern=8, embedding_std=1.0, seed=808)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    (directory / "tokenizer.jsonl").write_text("107520\n")
    oracle_lib.load().oracle_set_threads(16)
    vocab = 107520

    def greedy_after(history, first, count):
        """The peer's proposal: ids[0] = first, then each id the argmax after
        forwarding the one before, until `count` ids or an EOS id (1 or 16),
        which is included (runtime/worker.c:244-290)."""
        ids = [first]
        if first in (1, 16) or count == 1:
            return ids
        ck = plamo_hip.Checkpoint(directory)
        cpu = ck.instance()
        try:
            assert oracle_lib.prefill(cpu, history + [first])
            while True:
                ids.append(int(np.argmax(cpu.logits())))
                if len(ids) == count or ids[-1] in (1, 16):
                    return ids
                assert oracle_lib.forward(cpu, ids[-1])
        finally:
            cpu.close()
            ck.close()

    say("draft peer: start")
    w = Pipe([str(WORKER), "--draft-peer"], lib_env(directory))
    reply = struct.Struct("<18I")
    try:
        assert struct.unpack("<4I", w.read(16)) == (DRAFT_MAGIC, 1, vocab, 16)

        def call(data):
            w.send(data)
            ok, count, *ids = reply.unpack(w.read(reply.size))
            return ok, ids[:count]

        text = "draft peer request"
        say("draft peer: reset")
        assert call(frame(1, 1, 0, text.encode()))[0] == 1
        history = toy_prompt(text, 1, vocab)
        first = oracle_greedy(directory, history, 1)[0]
        rounds = ((first, 6, 3),     # roll back 2 of 5 forwarded steps on the host
                  (None, 5, 5),      # accept one past the forwarded count: forward the last
                  (None, 4, 3),      # accept exactly the forwarded steps: no rollback
                  (None, 6, 1))      # keep only the first id
        for i, (start, count, accepted) in enumerate(rounds):
            if start is None:  # a token the target chose against the draft
                start = (history[-1] * 7919 + 13) % vocab
            say(f"draft peer: proposal {i} of {count} from {start}")
            ok, ids = call(frame(2, start, count))
            assert ok == 1
            assert ids == greedy_after(history, start, count), i
            assert call(frame(3, accepted))[0] == 1
            history = history + ids[:accepted]
        # A new request resets the peer on the other prefix.
        say("draft peer: reset to direction 2")
        assert call(frame(1, 2, 0, b"again"))[0] == 1
        history = toy_prompt("again", 2, vocab)
        ok, ids = call(frame(2, 5, 4))
        assert ok == 1 and ids == greedy_after(history, 5, 4)
        assert call(frame(3, 2))[0] == 1
        assert w.close() == 0
    finally:
        if w.p.poll() is None:
            w.p.kill()
            w.p.wait()
