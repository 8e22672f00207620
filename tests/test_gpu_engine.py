"""The reference engine itself driving the library on the GPU.

tests/engine_link/_build/engine_host is the reference's runtime/engine.c and
runtime/prompt_cache.c, compiled unchanged against include/ and linked with
libplamo_hip.so (tests/engine_link/Makefile; built by __graft_entry__.build()
where the reference checkout exists, and shipped prebuilt). It opens a
real-format checkpoint through plamo_model_open with resident weights and the
GPU backend, prepares the two fixed translation prefixes
(runtime/engine.c:342-388: plamo_metal_prefill, then plamo_prompt_cache_capture
reading the host KV rows), and translates: a direction-1 request restores
prefix 0 from the prompt cache (host KV edits the backend must pick up) and
prefills only the suffix, then decodes with plamo_forward through the
installed hook (runtime/engine.c:514-583).

The toy prefixes have the shape of the reference's template prefixes: 12 ids
that differ only in the language id at index 10 and end in the same id. At
layer 0 a cache row depends only on its token, so after prepare (prefix 0,
then prefix 1) the restore of prefix 0 leaves every counter and the last rows
as they were; only row 10 changes. Direction 1 runs that restore first thing
in a fresh process.

The generated ids must equal the oracle's greedy sequence over the same
checkpoint and prompt ids, and the final logits and state must pass the
reference's GPU gate against the oracle's, with no CPU fallback and no backend
error."""

import json
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

import checkpoint_writer
from parity import gate, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu

HOST = Path(__file__).resolve().parent / "engine_link" / "_build" / "engine_host"


def oracle_greedy(directory, prompt, max_tokens):
    """The oracle's greedy ids, and its logits and state when the loop ends
    (those of the step that produced the last id, as in the engine)."""
    ck = plamo_hip.Checkpoint(directory)
    cpu = ck.instance()
    try:
        assert oracle_lib.prefill(cpu, prompt)
        out = []
        token = int(np.argmax(cpu.logits()))
        while len(out) < max_tokens and token not in (1, 16):
            out.append(token)
            if len(out) == max_tokens:
                break
            assert oracle_lib.forward(cpu, token)
            token = int(np.argmax(cpu.logits()))
        return out, cpu.logits().copy(), cpu.state().copy()
    finally:
        cpu.close()
        ck.close()


@pytest.mark.skipif(not HOST.exists(), reason="engine_host was not built (needs the reference "
                    "checkout at build time)")
def test_reference_engine_translates_on_gpu(tmp_path):
    # Sliding windows of 16 rows hold the 12-id prefixes (a snapshot needs
    # every layer's capacity, runtime/prompt_cache.c:23-25).
    syn = plamo_hip.Synthetic(512, 4, 8, 2, 64, 1024, 1000, window=16, global_capacity=256,
                              pattern=2, seed=31)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    (directory / "tokenizer.jsonl").write_text("1000\n")
    env = dict(os.environ, PLAMO_MODEL_DIR=str(directory),
               LD_LIBRARY_PATH=str(plamo_hip.LIB_PATH.parent))
    dump = tmp_path / "final.f32"
    for direction, text, max_tokens in ((1, "The engine is unchanged.", 1),
                                        (1, "The engine is unchanged.", 12),
                                        (2, "Same engine, other prefix.", 12),
                                        (0, "raw text, no prefix", 12)):
        say(f"engine_host translate direction {direction}, {max_tokens} tokens")
        r = subprocess.run([str(HOST), "translate", str(direction), str(max_tokens), text],
                           capture_output=True, text=True, timeout=120,
                           env=dict(env, ENGINE_HOST_DUMP=str(dump)))
        assert r.returncode == 0, r.stderr
        out = json.loads(r.stdout)
        assert out["backend"] == "metal" and out["memory_mode"] == "resident"
        assert out["cpu_fallbacks"] == 0 and out["errors"] == 0, out
        # Both fixed prefixes were captured at prepare (12 toy-prefix ids each).
        assert out["prefix_tokens"] == [12, 12]
        assert out["cached_prompt_tokens"] == (12 if direction else 0)
        expected, logits, state = oracle_greedy(directory, out["prompt"], max_tokens)
        final = np.fromfile(dump, dtype=np.float32)
        assert final.size == logits.size + state.size
        gate(final[:logits.size], logits, f"direction {direction} final logits")
        gate(final[logits.size:], state, f"direction {direction} final state")
        assert out["generated"] == expected, (out, expected)
        assert out["completion_tokens"] == len(expected)
