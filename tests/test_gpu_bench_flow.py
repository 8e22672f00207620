"""Oracle parity on the flow and at the shapes the bench measures.

C4 at full depth, 32 layers and the 100000-token
head, with bench.py's own seed and prompt ids: the 12-token template prefix is
prefilled on the GPU and captured (runtime/prompt_cache.c:15-56); each
request resets the model, restores that prefix (runtime/prompt_cache.c:
62-82) and prefills the 69-, 116- or 443-token body of the 81-, 128- or
455-token prompt (the TTFT runs), then takes 8 greedy steps on the decode
graph writing the pinned host arrays in place (the timed decode). The oracle
prefills each whole prompt from a reset model. Greedy ids must agree except
after a step whose oracle top-2 logit gap is below 1e-3 (BASELINE.json north
star); state, logits and every layer's K / V / rotated K rows pass the
reference's gate (tests/metal_decode.c:192-216).

C5 with 2 of its 60 layers and the tied 100000 x 6144 head: a
real 455-token prefill, decode steps, then verify of 5 candidates (the
speculative batch) committed against sequential oracle forwards, and a
rejected suffix (tests/metal_decode.c:309-365 at this width).
"""

import numpy as np
import pytest

import prompt_cache
from parity import compare, gate, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

BENCH_SEED = 20261201  # bench.py: the synthetic target's seed
PREFIX = 12


@pytest.fixture(scope="module", autouse=True)
def threads():
    oracle_lib.load().oracle_set_threads(16)


@pytest.fixture(scope="module")
def c4():
    shape = {k: v for k, v in plamo_hip.CONFIGS["c4"].items() if k != "tied"}
    syn = plamo_hip.Synthetic(**shape, seed=BENCH_SEED)
    gpu, cpu = syn.instance(pinned=True), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        prompt = np.random.default_rng(7).integers(0, shape["vocab"], size=455)
        prompt = prompt.astype(np.uint32).tolist()
        say("c4: prefix prefill and capture")
        assert be.prefill(gpu, prompt[:PREFIX]) == 1
        snap = prompt_cache.capture(gpu, prompt[:PREFIX])
        assert snap is not None
        yield be, gpu, cpu, prompt, snap
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    finally:
        be.close()
        gpu.close()
        cpu.close()
        syn.close()


def greedy_steps(be, gpu, cpu, steps, label):
    token = prompt_cache.greedy(cpu)
    for step in range(steps):
        top2 = np.sort(cpu.logits())[-2:]
        if top2[1] - top2[0] >= 1e-3:
            assert prompt_cache.greedy(gpu) == token, f"{label}: greedy id at step {step}"
        assert be.forward(gpu, token) == 1
        assert oracle_lib.forward(cpu, token)
        gate(gpu.state().copy(), cpu.state().copy(), f"{label} step {step} state")
        gate(gpu.logits().copy(), cpu.logits().copy(), f"{label} step {step} logits")
        token = prompt_cache.greedy(cpu)


@pytest.mark.parametrize("n", [81, 128, 455])
def test_c4_full_depth_restored_prefix(c4, n):
    be, gpu, cpu, prompt, snap = c4
    say(f"c4: {n}-token prompt, {PREFIX} restored, {n - PREFIX} prefilled")
    gpu.reset()
    assert prompt_cache.restore(snap, gpu, prompt[:n]) == PREFIX
    assert be.prefill(gpu, prompt[PREFIX:n]) == 1
    cpu.reset()
    assert oracle_lib.prefill(cpu, prompt[:n])
    compare(gpu, cpu)
    say(f"c4: {n}-token prompt, 8 greedy steps")
    greedy_steps(be, gpu, cpu, 8, f"c4 {n}")
    compare(gpu, cpu)


def test_c5_prefill_455_tied_head_and_verify():
    cfg = dict(plamo_hip.CONFIGS["c5"], layers=2)
    tied = cfg.pop("tied")
    syn = plamo_hip.Synthetic(**cfg, tied=tied, pattern=2, seed=BENCH_SEED)
    gpu, cpu = syn.instance(pinned=True), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        rng = np.random.default_rng(11)
        prompt = rng.integers(0, cfg["vocab"], size=455).tolist()
        say("c5: 455-token prefill")
        assert be.prefill(gpu, prompt) == 1
        assert oracle_lib.prefill(cpu, prompt)
        compare(gpu, cpu)
        greedy_steps(be, gpu, cpu, 2, "c5")
        compare(gpu, cpu)
        base = cpu.snapshot()
        first = prompt_cache.greedy(cpu)
        ids = [first] + rng.integers(0, cfg["vocab"], size=4).tolist()
        states, logits = [], []
        for t in ids:
            assert oracle_lib.forward(cpu, t)
            states.append(cpu.state().copy())
            logits.append(cpu.logits().copy())
        say("c5: verify 5 candidates, commit all")
        gbase = gpu.snapshot()
        r, nxt = be.verify(gpu, ids)
        assert r == 1
        for i in range(5):
            top2 = np.sort(logits[i])[-2:]
            if top2[1] - top2[0] >= 1e-3:
                assert nxt[i] == int(np.argmax(logits[i])), f"candidate {i}"
            assert be.commit(gpu, i) == 1
            gate(gpu.state().copy(), states[i], f"verified state {i}")
            gate(gpu.logits().copy(), logits[i], f"verified logits {i}")
        compare(gpu, cpu)
        say("c5: verify 5 candidates, commit 2, then a different token")
        cpu.restore(base)
        for t in ids[:2]:
            assert oracle_lib.forward(cpu, t)
        assert oracle_lib.forward(cpu, 12)
        gpu.restore(gbase)
        be.invalidate()
        assert be.verify(gpu, ids)[0] == 1
        for i in range(2):
            assert be.commit(gpu, i) == 1
        assert be.forward(gpu, 12) == 1
        assert be.commit(gpu, 2) == 0
        compare(gpu, cpu)
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    finally:
        be.close()
        gpu.close()
        cpu.close()
        syn.close()
