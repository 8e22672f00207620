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
