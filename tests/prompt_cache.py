"""The engine's prompt-prefix cache, restated over plamo_hip.Instance host arrays.

runtime/prompt_cache.c snapshots the K, V and rotated-K rows of a short,
fixed template prefix (at most PLAMO_PROMPT_PREFIX_LIMIT tokens) and copies
them back into a reset model at the start of a request whose ids begin with
that prefix. The backend never sees this code: it only sees host arrays and
counters change between calls, and must upload them before the next step.
These helpers let the tests drive exactly those edits.
"""

import numpy as np

PREFIX_LIMIT = 64  # runtime/prompt_cache.h:8


class Snapshot:
    def __init__(self, ids, layers):
        self.ids = list(ids)
        self.tokens = len(ids)
        self.layers = layers  # per layer: (width, scale_bits, k, v, rot)


def capture(inst, ids):
    """runtime/prompt_cache.c:15-56. None when the model is not exactly the
    prefix (every layer's count and processed count equal to the tokens)."""
    tokens = len(ids)
    if not tokens or tokens > PREFIX_LIMIT or not inst.model.count or inst.model.count > 128:
        return None
    layers = []
    for i in range(inst.model.count):
        c, r = inst.cache(i), inst.rotation(i)
        if not c.width or c.count != tokens or c.capacity < tokens or r.processed_count != tokens:
            return None
        layers.append((c.width, r.scale_bits, inst.kv(i, "k")[:tokens].copy(),
                       inst.kv(i, "v")[:tokens].copy(), inst.kv(i, "rot")[:tokens].copy()))
    return Snapshot(ids, layers)


def restore(snapshot, inst, ids):
    """runtime/prompt_cache.c:58-89: the reused token count, 0 on a miss (a
    missing snapshot, a prompt not longer than the prefix, an id mismatch or a
    changed layer width), in which case nothing is touched."""
    if snapshot is None or len(ids) <= snapshot.tokens or inst.model.count != len(snapshot.layers):
        return 0
    if list(ids[:snapshot.tokens]) != snapshot.ids:
        return 0
    for i, (width, _, _, _, _) in enumerate(snapshot.layers):
        c = inst.cache(i)
        if c.width != width or c.capacity < snapshot.tokens:
            return 0
    t = snapshot.tokens
    for i, (_, scale, k, v, rot) in enumerate(snapshot.layers):
        inst.kv(i, "k")[:t] = k
        inst.kv(i, "v")[:t] = v
        inst.kv(i, "rot")[:t] = rot
        inst.cache(i).count = t
        r = inst.rotation(i)
        r.processed_count = t
        r.scale_bits = scale
    return t


def greedy(inst):
    """Host argmax as runtime/engine.c:517 (first maximal index)."""
    return int(np.argmax(inst.logits()))
