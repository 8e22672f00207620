"""Writes a Hugging Face style PLaMo-3 checkpoint directory (config.json plus
BF16 safetensors shards) from a Synthetic model, for the checkpoint-loader
tests.

Tensor names and shapes follow the reference's schema (tools/weight_schema.py:
15-44); the config keys are those of tools/profiles/*/config.json. The file
format is safetensors: an 8-byte little-endian header length, a JSON header
of {"dtype", "shape", "data_offsets"} per tensor (plus "__metadata__"), padded
with spaces, then the raw tensor bytes.
"""

from __future__ import annotations

import ctypes
import json
import struct
from pathlib import Path

import numpy as np

import plamo_hip


def weights(syn: "plamo_hip.Synthetic") -> list[tuple[str, np.ndarray]]:
    """(name, BF16 bits) of every tensor of the synthetic model, in the
    reference's schema order, read through one instance's descriptors."""
    inst = syn.instance()
    try:
        m = inst.model
        h, v = m.hidden, m.vocab

        def arr(ptr, *shape):
            flat = np.ctypeslib.as_array(ctypes.cast(ptr, plamo_hip.u16p),
                                         shape=(int(np.prod(shape)),))
            return flat.reshape(shape).copy()

        out = [("model.embed_tokens.weight", arr(m.embedding, v, h)),
               ("model.norm.weight", arr(m.norm, h))]
        if not syn.config.tied:
            out.append(("lm_head.weight", arr(m.head, v, h)))
        for i in range(m.count):
            layer = m.layers[i].contents
            mixer = layer.mixer.contents
            q = mixer.qkv.contents
            mlp = layer.mlp.contents
            d, qh, kh, inter = q.dim, q.qh, q.kh, mlp.intermediate
            p = f"model.layers.layers.{i}."
            out += [
                (p + "mixer.qkv_proj.weight", arr(q.weight, (qh + 2 * kh) * d, h)),
                (p + "mixer.o_proj.weight", arr(mixer.weight, h, qh * d)),
                (p + "mixer.q_norm.weight", arr(q.qn, d)),
                (p + "mixer.k_norm.weight", arr(q.kn, d)),
                (p + "mlp.gate_up_proj.weight", arr(mlp.gu, 2 * inter, h)),
                (p + "mlp.down_proj.weight", arr(mlp.down, h, inter)),
                (p + "pre_mixer_norm.weight", arr(layer.pre, h)),
                (p + "post_mixer_norm.weight", arr(layer.post, h)),
                (p + "pre_mlp_norm.weight", arr(mlp.pre, h)),
                (p + "post_mlp_norm.weight", arr(mlp.post, h)),
            ]
        return out
    finally:
        inst.close()


def safetensors_header(tensors, metadata=None, dtype="BF16") -> bytes:
    """The length prefix and the padded JSON header of a safetensors file
    holding `tensors` in order."""
    header, offset = {}, 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, a in tensors:
        size = a.size * a.itemsize
        header[name] = {"dtype": dtype, "shape": list(a.shape),
                        "data_offsets": [offset, offset + size]}
        offset += size
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)
    return struct.pack("<Q", len(text)) + text


def safetensors_bytes(tensors, metadata=None, dtype="BF16") -> bytes:
    return safetensors_header(tensors, metadata, dtype) + b"".join(
        np.ascontiguousarray(a).tobytes() for _, a in tensors)


def config(syn: "plamo_hip.Synthetic", max_positions: int | None = None) -> dict:
    c = syn.config
    return {
        "architectures": ["Plamo3ForCausalLM"],
        "bos_token_id": 1,
        "dtype": "bfloat16",
        "head_dim": c.dim,
        "hidden_size": c.hidden,
        "image_feature_size": None,
        "intermediate_size": c.intermediate,
        "max_position_embeddings": max_positions or c.global_capacity,
        "model_type": "plamo3",
        "num_attention_heads": c.qh,
        "num_hidden_layers": c.layers,
        "num_key_value_heads": c.kh,
        "rms_norm_eps": 1e-06,
        "rope_scaling_factor": c.yarn_factor,
        "scale_embedding": False,
        "sliding_window_pattern": c.pattern,
        "tie_word_embeddings": bool(c.tied),
        "vocab_size": c.vocab,
        "window_size": c.window,
        "rope_parameters": {
            "full_attention": {"rope_type": "yarn", "rope_theta": c.global_theta,
                               "factor": c.yarn_factor,
                               "original_max_position_embeddings": int(c.yarn_original),
                               "beta_fast": c.yarn_beta_fast, "beta_slow": c.yarn_beta_slow,
                               "truncate": False},
            "sliding_attention": {"rope_type": "default", "rope_theta": c.local_theta},
        },
    }


def write(directory: Path, syn: "plamo_hip.Synthetic", shards: int = 2,
          max_positions: int | None = None) -> Path:
    """A checkpoint of `syn` split into `shards` files (round-robin over the
    schema order, so every shard holds some of every layer's tensors)."""
    directory.mkdir(parents=True, exist_ok=True)
    (directory / "config.json").write_text(json.dumps(config(syn, max_positions), indent=2))
    tensors = weights(syn)
    for s in range(shards):
        part = tensors[s::shards]
        # Streamed tensor by tensor: no whole-file buffer (a 0.8B-profile
        # checkpoint is 1.7 GB).
        with open(directory / f"model-{s + 1:05d}-of-{shards:05d}.safetensors", "wb") as f:
            f.write(safetensors_header(part, metadata={"format": "pt"}))
            for _, a in part:
                f.write(memoryview(np.ascontiguousarray(a)).cast("B"))
    return directory
