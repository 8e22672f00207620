"""GPU checks of speculative decoding with the in-process draft.

The reference speculates through a draft peer process (runtime/draft.c,
runtime/worker.c:198-317) and the engine loop runtime/engine.c:514-566;
include/plamo_draft.h provides both in-process. Speculation must never change
the output: every speculative run is compared token by token with plain
greedy decoding on the GPU and with the CPU oracle, where the oracle's top-2
logit gap below 1e-3 is the only allowed divergence (the greedy-match bar of
the decode benchmark). Draft internals are checked against the oracle too:
proposals are the draft model's greedy continuation, and after a rollback
(device rewind or host checkpoint) the draft continues as if the rejected
steps had never run.
"""

import ctypes

import numpy as np
import pytest

import prompt_cache
from parity import compare, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

EOS = (1, 16)


def model(seed=5, window=128, vocab=640, layers=4):
    # Layers alternate sliding (capacity window + 1) and global.
    return plamo_hip.Synthetic(256, layers, 4, 2, 128, 512, vocab, window=window,
                               global_capacity=256, pattern=2, seed=seed)


def oracle_greedy(inst, prompt, max_tokens):
    """Greedy tokens as the engine emits them, and each step's top-2 gap."""
    inst.reset()
    assert oracle_lib.prefill(inst, prompt)
    tokens, gaps = [], []
    while len(tokens) < max_tokens:
        logits = inst.logits().astype(np.float64)
        top = np.sort(logits)[-2:]
        gaps.append(float(top[1] - top[0]))
        t = prompt_cache.greedy(inst)
        if t in EOS:
            break
        tokens.append(t)
        if len(tokens) == max_tokens:
            break
        assert oracle_lib.forward(inst, t)
    return tokens, gaps


def same_tokens(got, want, gaps, name):
    for i, (g, w) in enumerate(zip(got, want)):
        if g != w:
            assert gaps[i] < 1e-3, f"{name}: token {i} is {g}, oracle {w} (gap {gaps[i]:.3g})"
            return
    assert len(got) == len(want), f"{name}: {len(got)} tokens, oracle {len(want)}"


def gpu_decode(be, inst, prompt, max_tokens, draft=None, block=0):
    inst.reset()
    assert be.prefill(inst, prompt) == 1
    return plamo_hip.decode(be, inst, prompt, max_tokens, draft=draft, block=block)


def clean(backend):
    info = backend.info()
    assert info.errors == 0, info.note.decode()
    assert info.cpu_fallbacks == 0


PROMPT = [3, 9, 27, 81, 243, 89, 267, 161, 483, 169, 507, 241, 83, 249, 107, 321, 323, 329, 347,
          401]


@pytest.mark.parametrize("pinned", [False, True])
def test_rewind_matches_shorter_history(pinned):
    s = model()
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    lib = plamo_hip.load()
    try:
        say(f"rewind pinned={pinned}")
        assert be.prefill(a, PROMPT) == 1
        assert oracle_lib.prefill(b, PROMPT)
        for t in (5, 6, 7, 8, 9):
            assert be.forward(a, t) == 1
        before = a.counts()
        assert lib.plamo_hip_rewind(be.handle, a.model_ptr, 0) == 1
        assert lib.plamo_hip_rewind(be.handle, a.model_ptr, 3) == 1
        assert a.counts() == [c - 3 for c in before]
        for i in range(a.model.count):
            assert a.rotation(i).processed_count == a.cache(i).count
            assert a.layer(i).mixer.contents.gqa.contents.tokens == a.cache(i).count
        for t in (5, 6):
            assert oracle_lib.forward(b, t)
        for t in (40, 41, 42):
            assert be.forward(a, t) == 1
            assert oracle_lib.forward(b, t)
            compare(a, b)
        # More steps than rows: refused, nothing changed.
        counts = a.counts()
        assert lib.plamo_hip_rewind(be.handle, a.model_ptr, min(counts) + 1) == 0
        assert a.counts() == counts
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


def test_rewind_refuses_a_full_sliding_window():
    s = model(window=8)
    a, b = s.instance(), s.instance()
    be = plamo_hip.Backend(s)
    lib = plamo_hip.load()
    try:
        assert be.prefill(a, PROMPT) == 1
        counts = a.counts()
        assert counts[0] == 9  # the sliding layer is full
        assert lib.plamo_hip_rewind(be.handle, a.model_ptr, 1) == 0
        assert a.counts() == counts
        # A host edit since the last call is not rewound either.
        a.rotation(1).processed_count = 0
        assert lib.plamo_hip_rewind(be.handle, a.model_ptr, 1) == 0
        assert oracle_lib.prefill(b, PROMPT)
        b.rotation(1).processed_count = 0
        assert be.forward(a, 12) == 1 and oracle_lib.forward(b, 12)
        compare(a, b)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


def test_draft_proposals_and_rollback_follow_the_draft_model():
    # The draft's proposals are its own greedy continuation; after accept the
    # draft holds exactly the consumed ids (runtime/worker.c:298-311).
    s = model(seed=8)
    d_inst, o = s.instance(), s.instance()
    draft = plamo_hip.Draft(s, d_inst)
    try:
        assert draft.reset_ids(PROMPT) == 1
        P = len(PROMPT)
        assert d_inst.counts() == [P] * 4
        assert draft.propose(12, 0) == [] and draft.propose(12, 17) == []
        assert draft.propose(640, 4) == []  # outside the vocabulary
        ids = draft.propose(12, 4)
        assert len(ids) == 4 and ids[0] == 12
        assert draft.propose(12, 4) == []  # one open proposal at a time
        assert d_inst.counts() == [P + 3] * 4
        assert oracle_lib.prefill(o, PROMPT)
        assert oracle_lib.forward(o, 12)
        for j in range(1, 4):
            assert ids[j] == prompt_cache.greedy(o), f"proposal {j}"
            if j < 3:
                assert oracle_lib.forward(o, ids[j])
        assert draft.accept(5) == 0  # more than proposed
        # accept 2 of 4: one device rewind.
        draft.accept(2)
        st = draft.stats()
        assert st.device_rewinds == 1 and st.horizon == 8 and st.accepted_tokens == 1
        assert d_inst.counts() == [P + 2] * 4
        assert draft.accept(1) == 0  # nothing open
        # Next proposal continues from PROMPT + ids[:2].
        nxt = draft.propose(33, 4)
        o.reset()
        assert oracle_lib.prefill(o, PROMPT + ids[:2])
        assert oracle_lib.forward(o, 33)
        assert nxt[1] == prompt_cache.greedy(o)
        # Everything consumed plus the unforwarded last id: one more draft step.
        draft.accept(4)
        assert d_inst.counts() == [P + 2 + 4] * 4
        o.reset()
        assert oracle_lib.prefill(o, PROMPT + ids[:2] + nxt)
        compare(d_inst, o)
        st = draft.stats()
        assert st.proposals == 2 and st.proposed_tokens == 6 and st.horizon == 16
    finally:
        draft.close()
        d_inst.close()
        o.close()
        s.close()


def test_margin_stop(monkeypatch):
    # runtime/worker.c:239-264: with a minimum margin no confident draft can
    # reach, proposals stop after the minimum token count.
    monkeypatch.setenv("PLAMO_DRAFT_MIN_MARGIN", "1e9")
    monkeypatch.setenv("PLAMO_DRAFT_MIN_TOKENS", "2")
    s = model(seed=8)
    d_inst = s.instance()
    draft = plamo_hip.Draft(s, d_inst)
    try:
        assert draft.reset_ids(PROMPT) == 1
        ids = draft.propose(12, 16)
        assert len(ids) == 2
        assert draft.accept(2)
        assert draft.stats().horizon == 8  # fewer than requested
    finally:
        draft.close()
        d_inst.close()
        s.close()


@pytest.mark.parametrize("kind", ["same", "other", "sliding"])
def test_speculative_decode_matches_greedy(kind):
    # same: the draft is the target's own weights (every proposal accepted);
    # other: an unrelated draft (mostly rejected: device rewinds);
    # sliding: unrelated and an 8-row window that fills during decoding
    # (rollbacks through the host checkpoint).
    window = 8 if kind == "sliding" else 128
    target = model(seed=5, window=window)
    source = target if kind == "same" else model(seed=11, window=window)
    a, o, d_inst = target.instance(), target.instance(), source.instance()
    be = plamo_hip.Backend(target)
    draft = plamo_hip.Draft(source, d_inst)
    max_tokens = 48
    try:
        say(f"speculative {kind}")
        want, gaps = oracle_greedy(o, PROMPT, max_tokens)
        plain, r0, _ = gpu_decode(be, a, PROMPT, max_tokens)
        same_tokens(plain, want, gaps, "plain")
        assert r0.speculative_batches == 0 and r0.completion_tokens == len(plain)
        spec, r, alive = gpu_decode(be, a, PROMPT, max_tokens, draft=draft)
        assert alive
        same_tokens(spec, want, gaps, "speculative")
        assert spec == plain
        st = draft.stats()
        say(f"  {len(spec)} tokens, {r.speculative_batches} batches, "
            f"{r.accepted_tokens}/{r.proposed_tokens} accepted, rewinds {st.device_rewinds}, "
            f"restores {st.host_restores}")
        assert r.speculative_batches == st.proposals > 0
        assert r.proposed_tokens == st.proposed_tokens and r.accepted_tokens == st.accepted_tokens
        assert r.completion_tokens == len(spec)
        if kind == "same":
            assert r.accepted_tokens >= r.proposed_tokens - 1
            assert r.speculative_batches < len(spec) // 4
        else:
            assert r.accepted_tokens < r.proposed_tokens
            if kind == "other":
                assert st.device_rewinds > 0
            else:
                assert st.host_restores > 0
        # The target's state after speculation equals plain decoding's: every
        # emitted token but a final one cut by max_tokens was forwarded.
        o.reset()
        assert oracle_lib.prefill(o, PROMPT)
        for t in (spec if r.finish == 1 else spec[:-1]):
            assert oracle_lib.forward(o, t)
        compare(a, o)
        clean(be)
    finally:
        draft.close()
        be.close()
        for inst in (a, o, d_inst):
            inst.close()
        target.close()
        if source is not target:
            source.close()


def test_decode_loop_contract(monkeypatch):
    s = model(seed=5)
    small = model(seed=5, vocab=320)
    a, d_inst, d2 = s.instance(), s.instance(), small.instance()
    be = plamo_hip.Backend(s)
    lib = plamo_hip.load()
    try:
        plain, _, _ = gpu_decode(be, a, PROMPT, 20)
        # A cancelling callback stops the request (runtime/engine.c:412-415).
        a.reset()
        assert be.prefill(a, PROMPT) == 1
        got, r, _ = plamo_hip.decode(be, a, PROMPT, 20, cancel_after=5)
        assert got == plain[:5] and r.finish == 2 and r.completion_tokens == 4
        # A draft whose vocabulary differs is dropped; decoding goes on.
        draft = plamo_hip.Draft(small, d2)
        got, r, alive = gpu_decode(be, a, PROMPT, 20, draft=draft)
        assert not alive and draft.handle.value is None
        assert got == plain and r.speculative_batches == 0
        # The reference entry points: an installed proposer is handed out once,
        # PLAMO_SPECULATIVE=0 opts out (runtime/draft.c:95-98), and reset
        # tokenizes through the callback.
        draft = plamo_hip.Draft(s, d_inst)
        lib.plamo_hip_draft_install(draft.handle)
        monkeypatch.setenv("PLAMO_SPECULATIVE", "0")
        assert not lib.plamo_draft_open()
        monkeypatch.delenv("PLAMO_SPECULATIVE")
        handle = lib.plamo_draft_open()
        assert handle == draft.handle.value
        assert not lib.plamo_draft_open()
        ids = (ctypes.c_uint32 * len(PROMPT))(*PROMPT)
        seen = []

        def tokenize(_ctx, text, direction, out):
            seen.append((text, direction))
            out[0] = ids
            return len(PROMPT)

        fn = plamo_hip.TOKENIZE_FN(tokenize)
        assert lib.plamo_draft_reset(handle, b"text", 1) == 0  # no tokenizer yet
        lib.plamo_hip_draft_set_tokenizer(handle, fn, None)
        assert lib.plamo_draft_reset(handle, b"text", 3) == 0  # direction 0..2
        assert lib.plamo_draft_reset(handle, "日本語".encode(), 2) == 1
        assert seen == [("日本語".encode(), 2)]
        assert d_inst.counts() == [len(PROMPT)] * 4
        out = (ctypes.c_uint32 * 16)()
        assert lib.plamo_draft_propose(handle, plain[0], 4, out) == 4
        assert list(out)[1:4] == plain[1:4]  # the same weights: the target's greedy tokens
        assert lib.plamo_draft_accept(handle, 4) == 1
        draft.close()
        clean(be)
    finally:
        be.close()
        for inst in (a, d_inst, d2):
            inst.close()
        s.close()
        small.close()
