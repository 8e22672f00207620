"""The head groupings and widths of the reference's published profiles,
through the checkpoint loader, on the GPU against the oracle.

tools/profiles/*/config.json of the reference:

  0.8b  hidden 1536, 16 query heads over 1 KV head (group 16), MLP 6144
  2b    hidden 2560, 24 over 4 (group 6), attention width 3072 above hidden
  8b    hidden 4096, 32 over 4 (group 8), MLP 16384
  31b   hidden 5120, 64 over 8 (group 8), attention width 8192, MLP 25600,
        tied embedding and head

all with head dim 128, vocabulary 107520 and a 2048-row sliding window. Each
case writes a two-layer checkpoint of that shape (layer 0 sliding, layer 1
global with YaRN; tests/checkpoint_writer.py), opens it with the C binder,
prefills a prompt (prompt attention on the matrix cores at that group), runs
decode steps (the captured graph with attention fused into the O projection)
and a verify of three candidates committed against sequential oracle
forwards, with the reference's gate (tests/metal_decode.c:192-216) on state,
logits and every layer's K / V / rotated K rows.
"""

import numpy as np
import pytest

import checkpoint_writer
from parity import compare, gate, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

PROFILES = {  # (hidden, qh, kh, intermediate, tied)
    "0.8b": (1536, 16, 1, 6144, 0),
    "2b": (2560, 24, 4, 10240, 0),
    "8b": (4096, 32, 4, 16384, 0),
    "31b": (5120, 64, 8, 25600, 1),
}


@pytest.fixture(scope="module", autouse=True)
def threads():
    oracle_lib.load().oracle_set_threads(16)


@pytest.mark.parametrize("name", list(PROFILES))
def test_profile_grouping_through_checkpoint(name, tmp_path):
    hidden, qh, kh, inter, tied = PROFILES[name]
    say(f"profile {name}: writing a 2-layer checkpoint")
    syn = plamo_hip.Synthetic(hidden, 2, qh, kh, 128, inter, 107520, window=2048,
                              global_capacity=1024, pattern=2, tied=tied, embedding_std=1.0,
                              seed=4000 + qh)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    ck = plamo_hip.Checkpoint(directory)
    gpu, cpu = ck.instance(pinned=True), ck.instance()
    be = plamo_hip.Backend(ck)
    try:
        L = gpu.model.count
        rng = np.random.default_rng(qh)
        prompt = rng.integers(0, 107520, size=45).tolist()
        say(f"profile {name}: prefill {len(prompt)} tokens")
        assert be.prefill(gpu, prompt) == 1
        assert oracle_lib.prefill(cpu, prompt)
        compare(gpu, cpu)
        token = int(np.argmax(cpu.logits()))
        for step in range(3):
            say(f"profile {name}: decode step {step}")
            before = be.info().dispatches
            assert be.forward(gpu, token) == 1
            assert oracle_lib.forward(cpu, token)
            compare(gpu, cpu)
            token = int(np.argmax(cpu.logits()))
            # Embedding, four kernels per layer (QKV, attention fused with
            # O, gate/up, down) and the head: the fused decode step.
            assert be.info().dispatches - before == 2 + 4 * L
        base = cpu.snapshot()
        ids = [token] + rng.integers(0, 107520, size=2).tolist()
        states, logits = [], []
        for t in ids:
            assert oracle_lib.forward(cpu, t)
            states.append(cpu.state().copy())
            logits.append(cpu.logits().copy())
        say(f"profile {name}: verify {len(ids)} candidates")
        r, nxt = be.verify(gpu, ids)
        assert r == 1
        for i in range(len(ids)):
            assert be.commit(gpu, i) == 1
            gate(gpu.state().copy(), states[i], f"verified state {i}")
            gate(gpu.logits().copy(), logits[i], f"verified logits {i}")
            top2 = np.sort(logits[i])[-2:]
            if top2[1] - top2[0] >= 1e-3:
                assert nxt[i] == int(np.argmax(logits[i]))
        compare(gpu, cpu)
        del base
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    finally:
        be.close()
        gpu.close()
        cpu.close()
        ck.close()
