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
