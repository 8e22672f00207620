"""CPU checks of the draft interface (include/plamo_draft.h).

The rollback and horizon cases restate the reference's own draft test
(tests/draft.c): the KV checkpoint is exercised at every truncation boundary
of a 20-row sliding cache against independently appended rows
(tests/draft.c:74-106), and the proposal horizon follows the sequence its
client test observes through a fake peer (tests/draft.c:58-93). Nothing here
needs a GPU: checkpoint and restore edit host arrays only.
"""

import ctypes

import numpy as np
import pytest

import plamo_hip

DRAFT_MAX = plamo_hip.DRAFT_MAX


class OneLayer:
    """A one-layer model whose cache is `capacity` rows of `width` floats
    (tests/draft.c:80-87)."""

    def __init__(self, capacity=20, width=3, sliding=1):
        self.k = np.zeros(capacity * width, np.float32)
        self.v = np.zeros(capacity * width, np.float32)
        f = plamo_hip.f32p
        self.cache = plamo_hip.Cache(self.k.ctypes.data_as(f), self.v.ctypes.data_as(f), capacity,
                                     0, width, sliding)
        self.rotation = plamo_hip.Rotation(cache=ctypes.pointer(self.cache), processed_count=99,
                                           scale_bits=123)
        self.gqa = plamo_hip.Gqa()
        self.mixer = plamo_hip.Mixer(cache=ctypes.pointer(self.cache),
                                     rotation=ctypes.pointer(self.rotation),
                                     gqa=ctypes.pointer(self.gqa))
        self.layer = plamo_hip.Layer(mixer=ctypes.pointer(self.mixer))
        self.layers = (ctypes.POINTER(plamo_hip.Layer) * 1)(ctypes.pointer(self.layer))
        self.model = plamo_hip.Model(layers=self.layers, count=1)

    def append(self, token):
        """A decode step's cache write: shift a full window, then append the
        row token*100 + j (K) and its negation (V) (tests/draft.c:9-20)."""
        c, w = self.cache, self.cache.width
        if c.count == c.capacity:
            self.k[: (c.count - 1) * w] = self.k[w: c.count * w].copy()
            self.v[: (c.count - 1) * w] = self.v[w: c.count * w].copy()
            c.count -= 1
        row = np.arange(w, dtype=np.float32) + token * 100
        self.k[c.count * w: (c.count + 1) * w] = row
        self.v[c.count * w: (c.count + 1) * w] = -row
        c.count += 1


def test_rollback_every_truncation_boundary(hip):
    # tests/draft.c:74-106: initial 0..20 rows in a 20-row window, 0..16
    # processed steps, every accepted prefix (several evictions, a window
    # already full).
    for initial in range(21):
        for processed in range(17):
            for accepted in range(processed + 1):
                got, want = OneLayer(), OneLayer()
                for i in range(initial):
                    got.append(i)
                    want.append(i)
                s = hip.plamo_draft_checkpoint(ctypes.byref(got.model), 16)
                assert s
                try:
                    for i in range(processed):
                        got.append(initial + i)
                    for i in range(accepted):
                        want.append(initial + i)
                    assert not hip.plamo_draft_restore(s, processed, processed + 1)
                    assert hip.plamo_draft_restore(s, processed, accepted)
                finally:
                    hip.plamo_draft_checkpoint_free(s)
                n = want.cache.count
                case = (initial, processed, accepted)
                assert got.cache.count == n, case
                w = got.cache.width
                assert got.k[: n * w].tobytes() == want.k[: n * w].tobytes(), case
                assert got.v[: n * w].tobytes() == want.v[: n * w].tobytes(), case
                assert got.rotation.processed_count == 0 and got.rotation.scale_bits == 0, case
                assert got.gqa.tokens == n, case


def test_rollback_rejected_arguments(hip):
    m = OneLayer()
    for i in range(5):
        m.append(i)
    assert not hip.plamo_draft_checkpoint(ctypes.byref(m.model), 0)
    assert not hip.plamo_draft_checkpoint(ctypes.byref(m.model), DRAFT_MAX + 1)
    small = OneLayer(capacity=4)
    assert not hip.plamo_draft_checkpoint(ctypes.byref(small.model), 8)  # capacity < limit
    s = hip.plamo_draft_checkpoint(ctypes.byref(m.model), 4)
    try:
        assert not hip.plamo_draft_restore(s, 5, 1)  # more steps than the checkpoint covers
        assert not hip.plamo_draft_restore(s, 2, 1)  # count is not checkpoint + processed
        m.append(5)
        m.append(6)
        assert hip.plamo_draft_restore(s, 2, 1) and m.cache.count == 6
    finally:
        hip.plamo_draft_checkpoint_free(s)
    assert not hip.plamo_draft_restore(None, 0, 0)
    hip.plamo_draft_checkpoint_free(None)
    # A global cache cannot pass its capacity.
    full = OneLayer(capacity=16, sliding=0)
    for i in range(14):
        full.append(i)
    s = hip.plamo_draft_checkpoint(ctypes.byref(full.model), 4)
    try:
        full.cache.count = 16
        assert not hip.plamo_draft_restore(s, 4, 1)
    finally:
        hip.plamo_draft_checkpoint_free(s)


def test_horizon_follows_reference_client_sequence(hip):
    # tests/draft.c:58-93 through its fake peer: the peer returns as many ids
    # as requested (8 when the first id is 43, a confidence stop); the client
    # clamps each request to its horizon and updates it on acceptance.
    class Client:
        def __init__(self):
            self.horizon = 8

        def reset(self):
            self.horizon, self.requested, self.proposed = 8, 0, 0

        def propose(self, first, limit):
            limit = min(limit, self.horizon)
            count = min(limit, 8) if first == 43 else limit
            self.requested, self.proposed = limit, count
            return count

        def accept(self, consumed):
            self.horizon = hip.plamo_hip_draft_next_horizon(self.horizon, self.requested,
                                                            self.proposed, consumed)

    d = Client()
    d.reset()
    assert d.propose(10, 4) == 4
    d.accept(2)
    d.reset()
    assert d.propose(10, 16) == 8
    d.accept(8)
    assert d.propose(10, 16) == 16
    d.accept(3)
    assert d.propose(10, 16) == 8
    d.accept(1)
    n = 2
    while n <= 16:
        assert d.propose(10, 16) == n
        d.accept(n)
        n *= 2
    assert d.propose(43, 16) == 8
    d.accept(8)
    assert d.propose(10, 16) == 8
    d.accept(8)
    d.reset()
    assert d.propose(10, 16) == 8


@pytest.mark.parametrize("case,expected", [
    ((8, 8, 8, 1), 2),     # first-token rejection of a multi-token block
    ((2, 2, 2, 1), 2),
    ((8, 8, 1, 1), 8),     # the draft stopped at once (EOS): not a rejection
    ((8, 8, 8, 5), 8),     # partial acceptance
    ((16, 16, 10, 10), 8),  # a confidence stop short of the request
    ((2, 2, 2, 2), 4),
    ((4, 4, 4, 4), 8),
    ((8, 8, 8, 8), 16),
    ((16, 16, 16, 16), 16),
    ((8, 4, 4, 4), 16),    # a short request fully accepted grows like a full block
])
def test_horizon_cases(hip, case, expected):
    assert hip.plamo_hip_draft_next_horizon(*case) == expected


def test_draft_entry_points_without_gpu(hip, monkeypatch):
    monkeypatch.setenv("PLAMO_SPECULATIVE", "0")
    assert not hip.plamo_draft_open()
    monkeypatch.delenv("PLAMO_SPECULATIVE")
    assert not hip.plamo_draft_open()  # nothing installed
    hip.plamo_draft_close(None)
    ids = (ctypes.c_uint32 * DRAFT_MAX)()
    assert hip.plamo_draft_propose(None, 10, 4, ids) == 0
    assert hip.plamo_draft_accept(None, 1) == 0
    assert hip.plamo_draft_reset(None, b"text", 1) == 0
    assert hip.plamo_hip_rewind(None, None, 1) == 0
    s = plamo_hip.Synthetic(24, 2, 4, 2, 6, 40, 17, window=2, global_capacity=32, pattern=2)
    inst = s.instance()
    try:
        err = ctypes.create_string_buffer(256)
        cfg = plamo_hip.MetalConfig()
        handle = hip.plamo_hip_draft_open(inst.model_ptr, ctypes.byref(cfg), err, 256)
        if handle:
            hip.plamo_draft_close(handle)
            pytest.skip("a GPU is visible")
        assert b"MI355X" in err.value
    finally:
        inst.close()
        s.close()


def test_draft_settings_are_validated(hip, monkeypatch):
    # runtime/worker.c:199-210: a malformed setting refuses the proposer
    # before any device work.
    s = plamo_hip.Synthetic(24, 2, 4, 2, 6, 40, 17, window=2, global_capacity=32, pattern=2)
    inst = s.instance()
    try:
        cfg = plamo_hip.MetalConfig()
        for name, value in (("PLAMO_DRAFT_MIN_MARGIN", "-1"), ("PLAMO_DRAFT_MIN_MARGIN", "x"),
                            ("PLAMO_DRAFT_MIN_TOKENS", "0"), ("PLAMO_DRAFT_MIN_TOKENS", "17")):
            monkeypatch.setenv(name, value)
            err = ctypes.create_string_buffer(256)
            assert not hip.plamo_hip_draft_open(inst.model_ptr, ctypes.byref(cfg), err, 256)
            assert name.encode() in err.value
            monkeypatch.delenv(name)
    finally:
        inst.close()
        s.close()
