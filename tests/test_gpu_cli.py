"""The Linux command-line host end to end on the GPU: a real-format
checkpoint (config.json + BF16 safetensors shards, tests/checkpoint_writer.py)
opened by plamo_model_open, decoded greedily by plamo-hip (the engine's loop,
runtime/engine.c:514-566; EOS ids 1 and 16 stop without being printed), and
the printed ids compared with the oracle's greedy sequence over the same
checkpoint. The same checkpoint as its own in-process draft must print the
same ids (speculation never changes the output) and have proposals
accepted."""

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import checkpoint_writer
from parity import oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

CLI = Path(__file__).resolve().parent.parent / "plamo-3-translate.c_amd" / "plamo-hip"


def test_cli_greedy_and_self_draft_match_oracle(tmp_path):
    syn = plamo_hip.Synthetic(512, 4, 8, 2, 64, 1024, 1000, window=8, global_capacity=256,
                              pattern=2, seed=29)
    try:
        directory = str(checkpoint_writer.write(tmp_path / "ck", syn, shards=2))
    finally:
        syn.close()
    prompt = [17, 230, 5, 999, 42, 7, 300]
    max_tokens = 12
    ck = plamo_hip.Checkpoint(directory)
    cpu = ck.instance()
    try:
        assert oracle_lib.prefill(cpu, prompt)
        expected = []
        token = int(np.argmax(cpu.logits()))
        while len(expected) < max_tokens and token not in (1, 16):
            expected.append(token)
            if len(expected) == max_tokens:
                break
            assert oracle_lib.forward(cpu, token)
            token = int(np.argmax(cpu.logits()))
    finally:
        cpu.close()
        ck.close()
    ids = [str(t) for t in prompt]
    say("plamo-hip greedy")
    r = subprocess.run([str(CLI), "--model", directory, "--max-tokens", str(max_tokens), *ids],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert [int(v) for v in r.stdout.split()] == expected
    say("plamo-hip with the checkpoint as its own draft")
    r = subprocess.run([str(CLI), "--model", directory, "--draft", directory, "--max-tokens",
                        str(max_tokens), "--speculative-tokens", "4", ",".join(ids)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert [int(v) for v in r.stdout.split()] == expected
    m = re.search(r"speculative (\d+) batches, (\d+) proposed, (\d+) accepted", r.stderr)
    assert m, r.stderr
    batches, proposed, accepted = (int(g) for g in m.groups())
    assert batches > 0 and proposed > 0 and accepted > 0, r.stderr


def frame(op, direction=0, max_tokens=0, text=b""):
    """A request of the reference worker's protocol (runtime/worker.c:1-4)."""
    import struct
    return struct.pack("<4I", op, direction, max_tokens, len(text)) + text


class Worker:
    """plamo-hip --worker with a reader thread, so a silent worker fails the
    test by timeout instead of hanging it."""

    def __init__(self, *args):
        import queue
        import threading
        self.p = subprocess.Popen([str(CLI), "--worker", *args], stdin=subprocess.PIPE,
                                  stdout=subprocess.PIPE, stderr=subprocess.PIPE)
        self.lines = queue.Queue()

        def pump():
            for line in self.p.stdout:
                self.lines.put(line)
            self.lines.put(None)
        threading.Thread(target=pump, daemon=True).start()

    def send(self, data):
        self.p.stdin.write(data)
        self.p.stdin.flush()

    def event(self, timeout=120):
        import json
        line = self.lines.get(timeout=timeout)
        assert line is not None, self.p.stderr.read().decode()
        return json.loads(line)

    def generation(self):
        """Events of one generate request: (prefill, token ids, done)."""
        prefill = self.event()
        assert prefill["event"] == "prefill", prefill
        ids = []
        while True:
            e = self.event()
            if e["event"] != "token":
                return prefill, ids, e
            ids.append(e["token_id"])

    def finish(self, timeout=60):
        self.p.stdin.close()
        return self.p.wait(timeout=timeout)


def test_worker_protocol(tmp_path):
    """The worker frames and events of runtime/worker.c:427-489 over the ids-only
    host: ready, tokenize, two generations with the oracle's greedy ids (the
    request reset between them, runtime/engine.c:447), an id outside the
    vocabulary (error, the worker goes on), a cancel frame queued behind a
    request (finish "cancelled"), end of input (status 0) and a malformed frame
    (protocol_error, status 1)."""
    syn = plamo_hip.Synthetic(512, 4, 8, 2, 64, 1024, 1000, window=8, global_capacity=256,
                              pattern=2, seed=29)
    try:
        directory = str(checkpoint_writer.write(tmp_path / "ck", syn, shards=2))
    finally:
        syn.close()
    prompt = [17, 230, 5, 999, 42, 7, 300]
    ck = plamo_hip.Checkpoint(directory)
    cpu = ck.instance()
    try:
        assert oracle_lib.prefill(cpu, prompt)
        expected = []
        token = int(np.argmax(cpu.logits()))
        while len(expected) < 12 and token not in (1, 16):
            expected.append(token)
            if len(expected) == 12:
                break
            assert oracle_lib.forward(cpu, token)
            token = int(np.argmax(cpu.logits()))
    finally:
        cpu.close()
        ck.close()
    text = " ".join(map(str, prompt)).encode()
    say("worker: ready, tokenize, generate twice")
    w = Worker("--model", directory)
    try:
        ready = w.event()
        assert ready["event"] == "ready" and ready["protocol"] == 1, ready
        assert ready["model"] == "plamo-3-translate-custom"
        assert ready["compute"]["cpu_fallbacks"] == 0
        w.send(frame(2, text=b"17,230\n5"))
        assert w.event() == {"event": "tokenized", "prompt_tokens": 3, "token_ids": [17, 230, 5]}
        for _ in range(2):
            w.send(frame(1, 0, 12, text))
            prefill, ids, done = w.generation()
            assert prefill["prompt_tokens"] == len(prompt)
            assert done["event"] == "done", done
            assert ids == expected
            assert done["usage"]["completion_tokens"] == len(expected)
            assert done["compute"]["errors"] == 0 and done["compute"]["cpu_fallbacks"] == 0
        w.send(frame(1, 0, 4, b"5 1000"))
        e = w.event()
        assert e["event"] == "error" and e["code"] == "invalid_input", e
        say("worker: cancel queued behind a request")
        w.send(frame(1, 0, 4096, text) + frame(3))
        _, ids, done = w.generation()
        assert done["event"] == "done" and done["finish_reason"] == "cancelled", done
        assert ids == []
        assert w.finish() == 0
    finally:
        if w.p.poll() is None:
            w.p.kill()
    say("worker: malformed frame")
    w = Worker("--model", directory)
    try:
        assert w.event()["event"] == "ready"
        w.send(frame(9, 0, 0))
        e = w.event()
        assert e["event"] == "error" and e["code"] == "protocol_error", e
        assert w.p.wait(timeout=60) == 1
    finally:
        if w.p.poll() is None:
            w.p.kill()
