"""Prompt-prefix cache flows on the CPU oracle (runtime/prompt_cache.c,
restated in tests/prompt_cache.py): a restored prefix followed by the suffix
must give bit-identical results to prefilling the whole prompt, and every
miss rule must leave the model untouched."""

import numpy as np

import prompt_cache
from parity import oracle_lib, tiny


def test_restore_then_suffix_is_bitwise_full_prefill():
    s = tiny(h=24, inter=40, dim=6, capacity=64, layers=3, window=32)
    a, b = s.instance(), s.instance()
    try:
        prefix = [3, 1, 4, 1, 5, 9, 2, 6]
        assert oracle_lib.prefill(a, prefix)
        snap = prompt_cache.capture(a, prefix)
        assert snap is not None and snap.tokens == len(prefix)
        ids = prefix + [5, 3, 5, 8, 9, 7]
        a.reset()
        assert prompt_cache.restore(snap, a, ids) == len(prefix)
        assert oracle_lib.prefill(a, ids[len(prefix):])
        assert oracle_lib.prefill(b, ids)
        assert a.logits().tobytes() == b.logits().tobytes()
        assert a.state().tobytes() == b.state().tobytes()
        for i in range(a.model.count):
            n = a.cache(i).count
            assert n == b.cache(i).count
            for which in ("k", "v", "rot"):
                assert a.kv(i, which)[:n].tobytes() == b.kv(i, which)[:n].tobytes()
    finally:
        a.close()
        b.close()
        s.close()


def test_miss_rules_leave_the_model_untouched():
    s = tiny(h=24, inter=40, dim=6, capacity=64, layers=2, window=32)
    a = s.instance()
    try:
        prefix = [3, 1, 4, 1, 5]
        assert prompt_cache.capture(a, prefix) is None  # counts are 0, not the prefix
        assert oracle_lib.prefill(a, prefix)
        snap = prompt_cache.capture(a, prefix)
        assert prompt_cache.capture(a, prefix[:4]) is None  # count != tokens
        assert prompt_cache.capture(a, list(range(65))) is None  # over the prefix limit
        a.reset()
        before = a.snapshot()
        for ids in (prefix, prefix[:3], [9] + prefix[1:] + [2], []):
            assert prompt_cache.restore(snap, a, ids) == 0
        assert prompt_cache.restore(None, a, prefix + [1]) == 0
        after = a.snapshot()
        assert all(x.tobytes() == y.tobytes() for x, y in
                   zip(before["layers"][0][:3], after["layers"][0][:3]))
        assert a.counts() == [0] * a.model.count
    finally:
        a.close()
        s.close()


# The shape of the reference's two translation prefixes (src/prompt.s:64-66
# through runtime/tokenizer.c:178-184): 12 ids, equal but for the language id
# at index 10, both ending in the same id.
TEMPLATE_PREFIXES = ([2, 3, 12, 4, 13, 3, 14, 5, 15, 6, 7, 4],
                     [2, 3, 12, 4, 13, 3, 14, 5, 15, 6, 8, 4])


def test_template_prefixes_agree_at_the_last_row_of_layer_0():
    # The case a backend must not miss: after the engine's prepare order
    # (runtime/engine.c:357-381: prefix 0, then prefix 1, each from a reset),
    # restoring prefix 0 (runtime/prompt_cache.c:62-82) leaves every counter
    # and layer 0's last K and V rows bit-identical; only row 10 differs there.
    # Deeper layers see the differing id through attention and differ in
    # every row from index 10 on.
    s = tiny(h=24, inter=40, dim=6, capacity=64, layers=3, window=32)
    a = s.instance()
    try:
        snaps = []
        for ids in TEMPLATE_PREFIXES:
            a.reset()
            assert oracle_lib.prefill(a, ids)
            snaps.append(prompt_cache.capture(a, ids))
        (w0, s0, k0, v0, r0), (w1, s1, k1, v1, r1) = snaps[0].layers[0], snaps[1].layers[0]
        assert w0 == w1 and s0 == s1
        for x, y in ((k0, k1), (v0, v1)):
            assert x[11].tobytes() == y[11].tobytes()
            assert x[:10].tobytes() == y[:10].tobytes()
            assert x[10].tobytes() != y[10].tobytes()
        for i in range(1, a.model.count):
            ka, kb = snaps[0].layers[i][2], snaps[1].layers[i][2]
            assert ka[:10].tobytes() == kb[:10].tobytes()
            assert all(ka[j].tobytes() != kb[j].tobytes() for j in range(10, 12))
        # Prefix 1 is what the model holds after prepare; restoring prefix 0
        # keeps the counters and layer 0's last rows.
        a.reset()
        assert oracle_lib.prefill(a, TEMPLATE_PREFIXES[1])
        before = [(a.cache(i).count, a.rotation(i).processed_count, a.rotation(i).scale_bits)
                  for i in range(a.model.count)]
        last_k0 = a.kv(0, "k")[11].copy()
        a.reset()
        ids = TEMPLATE_PREFIXES[0] + [9, 1]
        assert prompt_cache.restore(snaps[0], a, ids) == 12
        after = [(a.cache(i).count, a.rotation(i).processed_count, a.rotation(i).scale_bits)
                 for i in range(a.model.count)]
        assert before == after
        assert a.kv(0, "k")[11].tobytes() == last_k0.tobytes()
    finally:
        a.close()
        s.close()
