"""Shared helpers of the GPU parity tests: fixtures and the comparison gate.

The gate is the reference's own GPU-vs-CPU check (tests/metal_decode.c:192-216):
over a whole vector, relative L2 error <= 1e-4 and max |delta| <=
1e-5 * (1 + max |reference|); every value finite.
"""

import sys

import numpy as np

import oracle_lib
import plamo_hip

REL_L2 = 1e-4
ABS_SCALE = 1e-5


def gate(actual, expected, name):
    # Copies: a failure report must not touch host arrays freed by the test.
    a = np.array(actual, dtype=np.float64).ravel()
    b = np.array(expected, dtype=np.float64).ravel()
    del actual, expected
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(b)), f"{name}: non-finite values"
    delta = np.abs(a - b)
    norm = float(np.sqrt(np.sum(b * b))) or 1.0
    rel = float(np.sqrt(np.sum(delta * delta))) / norm
    mx = float(delta.max()) if delta.size else 0.0
    mag = float(np.abs(b).max()) if b.size else 0.0
    assert rel <= REL_L2 and mx <= ABS_SCALE * (1 + mag), (
        f"{name}: relative L2 {rel:.3g}, max error {mx:.3g}, magnitude {mag:.3g}")
    return rel, mx


def compare(gpu: "plamo_hip.Instance", cpu: "plamo_hip.Instance", kv=True):
    """State, logits, and every layer's K / V / rotated K rows and counters."""
    gate(gpu.state().copy(), cpu.state().copy(), "state")
    gate(gpu.logits().copy(), cpu.logits().copy(), "logits")
    if not kv:
        return
    for i in range(gpu.model.count):
        ca, cb = gpu.cache(i), cpu.cache(i)
        assert ca.count == cb.count, f"layer {i}: count {ca.count} vs {cb.count}"
        n = ca.count
        for which in ("k", "v", "rot"):
            gate(gpu.kv(i, which)[:n].copy(), cpu.kv(i, which)[:n].copy(), f"layer {i} {which}")
        ra, rb = gpu.rotation(i), cpu.rotation(i)
        assert ra.processed_count == rb.processed_count, f"layer {i}: processed_count"
        assert ra.scale_bits == rb.scale_bits, f"layer {i}: scale_bits"


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def tiny(h=24, inter=40, dim=6, capacity=64, vocab=17, qh=4, kh=2, layers=2, window=2,
         pattern=2, seed=3, **kw):
    """Reference-test style model (tests/metal_decode.c:95-175): layer 0 sliding
    with capacity window+1, layer 1 global."""
    return plamo_hip.Synthetic(h, layers, qh, kh, dim, inter, vocab, window=window,
                               global_capacity=capacity, pattern=pattern, seed=seed, **kw)


__all__ = ["gate", "compare", "say", "tiny", "oracle_lib", "plamo_hip"]
