"""A real-format checkpoint through the HIP backend.

A synthetic model is written as a Hugging Face style checkpoint (config.json
plus BF16 safetensors shards, tests/checkpoint_writer.py), opened by the C
binder (include/plamo_checkpoint.h), its shard mappings made resident by
plamo_metal_open(), then prefilled and decoded on the GPU against the oracle
over the same checkpoint, with the reference's gate (tests/metal_decode.c:
192-216) on state, logits and every layer's K / V / rotated K rows. The shape
takes the fused decode paths (head dim 64, group 4); two of the four layers
are global (YaRN) and the sliding window of 8 rows overflows during decode.
"""

import numpy as np
import pytest

import checkpoint_writer
from parity import compare, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu


def test_checkpoint_decode_matches_oracle(tmp_path):
    syn = plamo_hip.Synthetic(512, 4, 8, 2, 64, 1024, 1000, window=8, global_capacity=256,
                              pattern=2, seed=23)
    try:
        directory = checkpoint_writer.write(tmp_path / "ck", syn, shards=3)
    finally:
        syn.close()
    ck = plamo_hip.Checkpoint(directory)
    gpu, cpu = ck.instance(pinned=True), ck.instance()
    be = plamo_hip.Backend(ck)
    try:
        prompt = [17, 230, 5, 999, 42, 7, 300]
        say("prefill")
        assert be.prefill(gpu, prompt) == 1
        assert oracle_lib.prefill(cpu, prompt)
        compare(gpu, cpu)
        token = int(np.argmax(cpu.logits()))
        for step in range(5):
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
        ck.close()
