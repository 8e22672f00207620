"""GPU parity at the BASELINE.json shapes, on the default decode path (the
captured graph of the bench) and the prompt/verify paths.

C1: one layer, hidden 2048, 16/4 heads of 128, MLP 8192, KV
pre-filled with 512 (then 254) rows of raw K/V ~ N(0,1) (rotations rebuilt by
the first step on both sides); then decode steps and a prompt.
C2 in full: 16 layers, vocab 100000, a 32-token prompt and 64
greedy steps; the greedy ids must match the oracle's except after a step whose
oracle top-2 logit gap is below 1e-3, and every
step's logits pass the reference gate.
C3 shapes with 2 of its 24 layers (one local, one global YaRN
layer): attention width 2048 under hidden 2560, the 10240-column down
projection; the engine's flow of a 12-token prefix restored from the prompt
cache, then the 116- and 443-token suffixes of the 128- and 455-token prompts,
then decode steps.
C4 shapes with 4 of its 32 layers and the full 100000-token
head: the 16K-column down projection and the fused attention at group 4.
C5 shapes with 2 of its 60 layers and the tied head: six query
heads per KV head, O and down at 6144 and 24576 columns; decode over a
455-row prefix, then verify of 1-5 candidates (the token GEMV) and 6-16
(the skinny GEMM) committed against sequential oracle forwards
(tests/metal_decode.c:309-365 at this width).
"""

import numpy as np
import pytest

import prompt_cache
from parity import compare, gate, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def threads():
    oracle_lib.load().oracle_set_threads(16)


def run_pair(syn, steps, prompt, fill=0, pinned=False):
    gpu, cpu = syn.instance(pinned=pinned), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        if fill:
            gpu.fill_kv(fill, 7)
            cpu.fill_kv(fill, 7)
        if prompt:
            assert be.prefill(gpu, prompt) == 1
            assert oracle_lib.prefill(cpu, prompt)
            compare(gpu, cpu)
        token = int(np.argmax(cpu.logits())) if prompt else 3
        for step in range(steps):
            say(f"step {step}")
            assert be.forward(gpu, token) == 1
            assert oracle_lib.forward(cpu, token)
            compare(gpu, cpu)
            token = int(np.argmax(cpu.logits()))
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    finally:
        be.close()
        gpu.close()
        cpu.close()


def test_c1_single_layer_prefilled_kv():
    cfg = plamo_hip.CONFIGS["c1"]
    syn = plamo_hip.Synthetic(**cfg, embedding_std=1.0, seed=101)
    try:
        run_pair(syn, steps=6, prompt=None, fill=512)
        # 255 -> 257 rows: four splits per KV head merged by the O projection,
        # then five merged by the last attention block.
        run_pair(syn, steps=3, prompt=None, fill=254)
        run_pair(syn, steps=3, prompt=[3, 9, 1, 15, 0, 7, 2, 11, 4, 5, 13, 6, 8], fill=0)
    finally:
        syn.close()


def test_c4_shapes_four_layers():
    # Pinned host arrays: the decode graph writes logits, state, normalized
    # state and the new K/V rows into them in place (the bench's setup). The
    # 100000-row head of the headline config, then pageable host arrays (the
    # graph stages the step's outputs in a device outbox).
    say("c4 four layers, vocab 100000")
    cfg = dict(plamo_hip.CONFIGS["c4"], layers=4)
    syn = plamo_hip.Synthetic(**cfg, pattern=4, seed=202)
    try:
        run_pair(syn, steps=4, prompt=list(range(5, 5 + 69 * 7, 7)), pinned=True)
        run_pair(syn, steps=2, prompt=list(range(3, 3 + 20 * 5, 5)))
    finally:
        syn.close()


def test_c3_prefix_restore_and_prompts():
    # runtime/engine.c:358-381: the 12-token template prefix is prefilled once
    # and captured (runtime/prompt_cache.c); each request resets the model,
    # restores the prefix rows and prefills the rest of its prompt. The oracle
    # prefills the whole prompt from a reset model.
    cfg = dict(plamo_hip.CONFIGS["c3"], layers=2, vocab=1000)
    syn = plamo_hip.Synthetic(**cfg, pattern=2, seed=606)
    gpu, cpu = syn.instance(pinned=True), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        rng = np.random.default_rng(128)
        prefix = rng.integers(0, cfg["vocab"], size=12).tolist()
        assert be.prefill(gpu, prefix) == 1
        snap = prompt_cache.capture(gpu, prefix)
        assert snap is not None
        for total in (128, 455):
            say(f"c3 prompt {total} ({total - 12} after the restored prefix)")
            ids = prefix + rng.integers(0, cfg["vocab"], size=total - 12).tolist()
            gpu.reset()
            cpu.reset()
            assert prompt_cache.restore(snap, gpu, ids) == 12
            assert be.prefill(gpu, ids[12:]) == 1
            assert oracle_lib.prefill(cpu, ids)
            compare(gpu, cpu)
            token = prompt_cache.greedy(cpu)
            for step in range(3):
                assert be.forward(gpu, token) == 1
                assert oracle_lib.forward(cpu, token)
                compare(gpu, cpu)
                token = prompt_cache.greedy(cpu)
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    finally:
        be.close()
        gpu.close()
        cpu.close()
        syn.close()


def test_c5_decode_and_verify_over_455_rows():
    cfg = dict(plamo_hip.CONFIGS["c5"], layers=2, vocab=500)
    syn = plamo_hip.Synthetic(**cfg, pattern=2, embedding_std=1.0, seed=707)
    gpu, cpu = syn.instance(pinned=True), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        # 455 prefix rows of raw K/V ~ N(0,1); the first step rebuilds the
        # rotations (eager), the next ones run the captured graph.
        gpu.fill_kv(455, 9)
        cpu.fill_kv(455, 9)
        token = 7
        for step in range(3):
            say(f"c5 decode step {step}")
            assert be.forward(gpu, token) == 1
            assert oracle_lib.forward(cpu, token)
            compare(gpu, cpu)
            token = prompt_cache.greedy(cpu)
        base = cpu.snapshot()
        ids = [(i * 37 + 11) % cfg["vocab"] for i in range(16)]
        for count in (1, 2, 3, 4, 5, 6, 8, 16):
            say(f"c5 verify {count} candidates over {base['layers'][0][3]} rows")
            cpu.restore(base)
            states, logits, gold = [], [], []
            for i in range(count):
                assert oracle_lib.forward(cpu, ids[i])
                states.append(cpu.state().copy())
                logits.append(cpu.logits().copy())
                gold.append(int(np.argmax(cpu.logits())))
            # The oracle's rows replace the GPU's at unchanged counters: an
            # edit the backend is told about (include/plamo_draft.h).
            gpu.restore(base)
            be.invalidate()
            r, nxt = be.verify(gpu, ids[:count])
            assert r == 1
            for i in range(count):
                top2 = np.sort(logits[i])[-2:]
                if top2[1] - top2[0] >= 1e-3:
                    assert nxt[i] == gold[i], f"candidate {i}"
                assert be.commit(gpu, i) == 1
                gate(gpu.state().copy(), states[i], f"verified state {i}")
                gate(gpu.logits().copy(), logits[i], f"verified logits {i}")
            compare(gpu, cpu)
            assert be.commit(gpu, count) == 0
            if count == 5:
                # A rejected suffix: three commits, then an ordinary step.
                cpu.restore(base)
                for i in range(3):
                    assert oracle_lib.forward(cpu, ids[i])
                assert oracle_lib.forward(cpu, 12)
                gpu.restore(base)
                be.invalidate()
                assert be.verify(gpu, ids[:count])[0] == 1
                for i in range(3):
                    assert be.commit(gpu, i) == 1
                assert be.forward(gpu, 12) == 1
                assert be.commit(gpu, 3) == 0
                compare(gpu, cpu)
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
        assert info.verification_batches >= 9
    finally:
        be.close()
        gpu.close()
        cpu.close()
        syn.close()


def test_c2_greedy_64_steps():
    cfg = plamo_hip.CONFIGS["c2"]
    syn = plamo_hip.Synthetic(**cfg, seed=303)
    gpu, cpu = syn.instance(), syn.instance()
    be = plamo_hip.Backend(syn)
    try:
        rng = np.random.default_rng(32)
        prompt = rng.integers(0, cfg["vocab"], size=32).tolist()
        assert be.prefill(gpu, prompt) == 1
        assert oracle_lib.prefill(cpu, prompt)
        compare(gpu, cpu, kv=False)
        token = int(np.argmax(cpu.logits()))
        diverged = False
        for step in range(64):
            lg = cpu.logits().copy()
            top2 = np.sort(lg)[-2:]
            g_tok = int(np.argmax(gpu.logits()))
            if not diverged:
                if g_tok != token:
                    # Allowed only where the oracle's own top-2 gap is tiny.
                    assert top2[1] - top2[0] < 1e-3, f"step {step}: {g_tok} vs {token}"
                    diverged = True
                    break
            assert be.forward(gpu, token) == 1
            assert oracle_lib.forward(cpu, token)
            gate(gpu.logits().copy(), cpu.logits().copy(), f"step {step} logits")
            gate(gpu.state().copy(), cpu.state().copy(), f"step {step} state")
            token = int(np.argmax(cpu.logits()))
            if step % 8 == 0:
                say(f"greedy step {step}: token {token}")
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        gpu.close()
        cpu.close()
        syn.close()


def test_long_context_split_attention():
    # Contexts past 1024 rows split a KV head over several blocks whose
    # partials are merged by the last one; 1023 -> 1025 crosses the boundary.
    syn = plamo_hip.Synthetic(512, 2, 8, 2, 128, 1024, 500, window=4096, global_capacity=8192,
                              pattern=2, embedding_std=1.0, seed=404)
    try:
        run_pair(syn, steps=3, prompt=None, fill=1023)
        run_pair(syn, steps=3, prompt=None, fill=3000)
    finally:
        syn.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_short_context_graph_boundary(pinned):
    # Below 256 rows in every layer a decode step runs the short-context graph
    # (32-row attention blocks over at most 256 allocated rows); the step whose
    # count reaches 256 switches to the general graph. 250 -> 262 crosses it,
    # with the allocation grown to 512 rows first (a longer prompt earlier in
    # the request), as the bench's decode runs after its 455-token prompts.
    syn = plamo_hip.Synthetic(512, 2, 8, 2, 128, 1024, 500, window=4096, global_capacity=8192,
                              pattern=2, embedding_std=1.0, seed=405)
    try:
        run_pair(syn, steps=12, prompt=None, fill=250, pinned=pinned)
        gpu, cpu = syn.instance(pinned=pinned), syn.instance()
        be = plamo_hip.Backend(syn)
        try:
            prompt = [(j * 13 + 5) % 500 for j in range(300)]
            assert be.prefill(gpu, prompt) == 1  # allocation grows past 256 rows
            gpu.reset()
            cpu.reset()
            assert be.prefill(gpu, prompt[:200]) == 1
            assert oracle_lib.prefill(cpu, prompt[:200])
            token = int(np.argmax(cpu.logits()))
            for step in range(60):
                assert be.forward(gpu, token) == 1
                assert oracle_lib.forward(cpu, token)
                compare(gpu, cpu)
                token = int(np.argmax(cpu.logits()))
            info = be.info()
            assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
        finally:
            be.close()
            gpu.close()
            cpu.close()
    finally:
        syn.close()


def test_eager_decode_matches_graph(monkeypatch):
    """PLAMO_HIP_EAGER_DECODE=1 (read when the backend opens) launches the
    decode step's kernels one by one instead of replaying the captured graph:
    the same kernels with the same arguments, so logits, states and the
    appended KV rows are bit-identical to the graph's, in the short-context
    graph's range and past it."""
    cfg = dict(plamo_hip.CONFIGS["c4"], layers=2, vocab=1000)
    syn = plamo_hip.Synthetic(**cfg, pattern=2, seed=808)
    runs = []
    try:
        for eager in ("", "1"):
            say(f"eager={eager!r}")
            monkeypatch.setenv("PLAMO_HIP_EAGER_DECODE", eager)
            gpu = syn.instance(pinned=True)
            be = plamo_hip.Backend(syn)
            monkeypatch.delenv("PLAMO_HIP_EAGER_DECODE")
            try:
                gpu.fill_kv(250, 5)
                token, out = 3, []
                for step in range(10):  # rows 251..260 cross the 256-row boundary
                    assert be.forward(gpu, token) == 1
                    out.append((gpu.logits().copy(), gpu.state().copy(), gpu.normalized().copy()))
                    token = int(np.argmax(out[-1][0]))
                kv = [gpu.kv(i, w).copy() for i in range(cfg["layers"])
                      for w in ("k", "v", "rot")]
                info = be.info()
                assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
                runs.append((out, kv))
            finally:
                be.close()
                gpu.close()
    finally:
        syn.close()
    (graph_out, graph_kv), (eager_out, eager_kv) = runs
    for a, b in zip(graph_out, eager_out):
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
    for x, y in zip(graph_kv, eager_kv):
        assert np.array_equal(x, y)
