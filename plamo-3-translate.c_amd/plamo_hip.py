"""ctypes bindings of libplamo_hip.so, the MI355X token-loop backend.

The library's C ABI is the reference's GPU-backend boundary
(runtime/metal.h:48-88, runtime/compute.h:8-14, runtime/model.h:7-86); this
module mirrors those structs field by field so Python tests and the benchmark
drive exactly the entry points a C engine would. Nothing here computes: every
call lands in the HIP library, and loading fails loudly when it is not built.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import (
    POINTER,
    Structure,
    c_char,
    c_char_p,
    c_double,
    c_float,
    c_int,
    c_int64,
    c_size_t,
    c_uint,
    c_uint16,
    c_uint32,
    c_uint64,
    c_void_p,
)
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().with_name("libplamo_hip.so")

f32p = POINTER(c_float)
u16p = POINTER(c_uint16)


class Qkv(Structure):
    _fields_ = [("input", f32p), ("weight", u16p), ("qn", u16p), ("kn", u16p), ("out", f32p),
                ("hidden", c_uint64), ("qh", c_uint64), ("kh", c_uint64), ("dim", c_uint64)]


class Cache(Structure):
    _fields_ = [("k", f32p), ("v", f32p), ("capacity", c_uint64), ("count", c_uint64),
                ("width", c_uint64), ("sliding", c_uint64)]


class Rotation(Structure):
    _fields_ = [("cache", POINTER(Cache)), ("out", f32p), ("freq", f32p), ("cos", f32p),
                ("sin", f32p), ("heads", c_uint64), ("dim", c_uint64),
                ("processed_count", c_uint64), ("scale_bits", c_uint64)]


class Gqa(Structure):
    _fields_ = [("q", f32p), ("k", f32p), ("v", f32p), ("out", f32p), ("scores", f32p),
                ("tokens", c_uint64), ("dim", c_uint64), ("qh", c_uint64), ("kh", c_uint64)]


class Mixer(Structure):
    _fields_ = [("qkv", POINTER(Qkv)), ("cache", POINTER(Cache)), ("rotation", POINTER(Rotation)),
                ("gqa", POINTER(Gqa)), ("weight", u16p), ("out", f32p), ("hidden", c_uint64)]


class Mlp(Structure):
    _fields_ = [("state", f32p), ("pre", u16p), ("post", u16p), ("gu", u16p), ("down", u16p),
                ("normalized", f32p), ("branch", f32p), ("scratch", f32p),
                ("hidden", c_uint64), ("intermediate", c_uint64)]


class Layer(Structure):
    _fields_ = [("state", f32p), ("pre", u16p), ("post", u16p), ("normalized", f32p),
                ("branch", f32p), ("mixer", POINTER(Mixer)), ("mlp", POINTER(Mlp)),
                ("hidden", c_uint64)]


class Model(Structure):
    _fields_ = [("embedding", u16p), ("vocab", c_uint64), ("hidden", c_uint64), ("state", f32p),
                ("layers", POINTER(POINTER(Layer))), ("count", c_uint64), ("scales", f32p),
                ("norm", u16p), ("normalized", f32p), ("head", u16p), ("logits", f32p)]


class Mapping(Structure):
    _fields_ = [("base", c_void_p), ("bytes", c_uint64)]


class Matmul(Structure):
    _fields_ = [("weights", u16p), ("input", f32p), ("output", f32p), ("rows", c_uint64),
                ("columns", c_uint64), ("tokens", c_uint64), ("input_stride", c_uint64),
                ("output_stride", c_uint64)]


class WeightCacheInfo(Structure):
    _fields_ = [(name, c_uint64) for name in (
        "budget_bytes", "max_budget_bytes", "cached_bytes", "staging_bytes", "hits", "hit_bytes",
        "misses", "resizes", "storage_bytes")]


class MetalConfig(Structure):
    _fields_ = [("memory", c_int), ("precision", c_int), ("packing", c_int),
                ("working_weight_bytes", c_uint64), ("maps", POINTER(Mapping)),
                ("fds", POINTER(c_int64)), ("count", c_size_t), ("schema", c_void_p),
                ("reserve", c_uint64), ("available", c_void_p), ("disk_cache_path", c_char_p),
                ("revision", c_char_p), ("prefer_texture_weights", c_uint)]


class MetalInfo(Structure):
    _fields_ = [("device", c_char * 128), ("precision", c_char * 16),
                ("weight_storage", c_char * 24), ("note", c_char * 256),
                ("cache", WeightCacheInfo)] + [(name, c_uint64) for name in (
                    "dispatches", "command_buffers", "fused_mlps", "fused_decodes",
                    "fused_prefills", "cpu_fallbacks", "errors", "allocated_bytes",
                    "recommended_working_set_bytes", "packed_weight_bytes", "weight_heap_bytes",
                    "private_weight_bytes", "disk_cache_hits", "disk_cache_weight_bytes",
                    "disk_cache_storage_bytes", "disk_cache_mapped_bytes",
                    "disk_cache_mapping_bytes", "verification_batches", "verified_tokens",
                    "committed_tokens")] + [("residency_sets", c_uint), ("gpu_seconds", c_double)]


class SyntheticConfig(Structure):
    _fields_ = [(name, c_uint64) for name in (
        "hidden", "layers", "qh", "kh", "dim", "intermediate", "vocab", "window",
        "global_capacity", "pattern", "seed")] + [
        ("weight_std", c_double), ("embedding_std", c_double), ("tied", c_int),
        ("local_theta", c_double), ("global_theta", c_double), ("yarn_factor", c_double),
        ("yarn_original", c_double), ("yarn_beta_fast", c_double), ("yarn_beta_slow", c_double)]


class SafetensorsView(Structure):
    _fields_ = [("header", c_void_p), ("header_size", c_uint64), ("data", c_void_p),
                ("data_size", c_uint64)]


class Number(Structure):
    _fields_ = [("next", c_void_p), ("value", c_uint64)]


class JsonToken(Structure):
    _fields_ = [("next", c_void_p), ("start", c_void_p), ("length", c_uint64),
                ("value", c_uint64)]


class TensorField(Structure):
    _fields_ = [("next", c_void_p), ("offset", c_uint64), ("bytes", c_uint64), ("rank", c_uint64),
                ("dims", c_uint64 * 4)]


class Tensor(Structure):
    _fields_ = [("data", c_void_p), ("bytes", c_uint64), ("rank", c_uint64),
                ("dims", c_uint64 * 4), ("reserved", c_uint64)]


class WeightSpec(Structure):
    _fields_ = [("name", c_char_p), ("rank", c_uint64), ("shape", POINTER(c_uint64)),
                ("slot", POINTER(c_void_p))]


class CheckpointConfig(Structure):
    _fields_ = [(name, c_uint64) for name in (
        "hidden", "layers", "qh", "kh", "dim", "intermediate", "vocab", "window", "pattern",
        "max_positions")] + [
        ("tied", c_int), ("local_theta", c_double), ("global_yarn", c_int),
        ("global_theta", c_double), ("factor", c_double), ("original", c_double),
        ("beta_fast", c_double), ("beta_slow", c_double)]


class CpuPath(Structure):
    _fields_ = [("forward", ctypes.CFUNCTYPE(c_int, POINTER(Model), c_uint64)),
                ("prefill", ctypes.CFUNCTYPE(c_int, POINTER(Model), POINTER(c_uint32), c_uint64,
                                              f32p))]


class DraftStats(Structure):
    """struct plamo_hip_draft_stats (include/plamo_draft.h)."""
    _fields_ = [(name, c_uint64) for name in (
        "proposals", "proposed_tokens", "accepted_tokens", "draft_steps", "device_rewinds",
        "host_restores")] + [("horizon", c_uint)]


class DecodeResult(Structure):
    """struct plamo_hip_decode_result (include/plamo_draft.h)."""
    _fields_ = [(name, c_uint64) for name in (
        "completion_tokens", "decode_steps", "speculative_batches", "speculative_tokens",
        "proposed_tokens", "accepted_tokens")] + [
        ("draft_seconds", c_double), ("decode_seconds", c_double), ("finish", c_uint)]


TOKEN_FN = ctypes.CFUNCTYPE(c_int, c_uint32, c_void_p)
TOKENIZE_FN = ctypes.CFUNCTYPE(c_uint64, c_void_p, c_char_p, c_uint, POINTER(POINTER(c_uint32)))
DRAFT_MAX = 16  # runtime/draft.h:5


# Symbols each public header declares (checked by the ABI tests).
EXPORTS = {
    "plamo_model.h": ["plamo_prefill", "plamo_forward", "plamo_argmax"],
    "plamo_compute.h": ["plamo_compute_context", "plamo_matvec_kernel", "plamo_matmul_kernel",
                        "plamo_mlp_kernel", "plamo_forward_kernel", "plamo_prefill_kernel",
                        "plamo_weight_provider", "plamo_weight_context",
                        "plamo_weight_chunk_bytes", "plamo_register_cpu_path"],
    "plamo_backend.h": ["plamo_metal_open", "plamo_metal_close", "plamo_metal_maintain",
                        "plamo_metal_get_info", "plamo_metal_preload", "plamo_metal_warm_cache",
                        "plamo_metal_prepare_model", "plamo_metal_forward",
                        "plamo_metal_prefill", "plamo_metal_verify", "plamo_metal_commit",
                        "plamo_metal_linear", "plamo_metal_mlp", "plamo_hip_linear_static"],
    "plamo_diag.h": ["plamo_hip_time_kernel", "plamo_hip_debug_waits"],
    "plamo_draft.h": ["plamo_draft_open", "plamo_draft_close", "plamo_draft_reset",
                      "plamo_draft_propose", "plamo_draft_accept", "plamo_draft_checkpoint",
                      "plamo_draft_restore", "plamo_draft_checkpoint_free",
                      "plamo_hip_draft_open", "plamo_hip_draft_install",
                      "plamo_hip_draft_set_tokenizer", "plamo_hip_draft_reset_ids",
                      "plamo_hip_draft_get_stats", "plamo_hip_draft_next_horizon",
                      "plamo_hip_decode", "plamo_hip_rewind", "plamo_hip_invalidate"],
    "plamo_synthetic.h": ["plamo_synthetic_defaults", "plamo_synthetic_build",
                          "plamo_synthetic_free", "plamo_synthetic_weights",
                          "plamo_synthetic_frequencies", "plamo_synthetic_instantiate",
                          "plamo_synthetic_release", "plamo_synthetic_model",
                          "plamo_synthetic_fill_kv"],
}

# enum plamo_hip_kernel (include/plamo_diag.h)
KERNEL_QKV, KERNEL_O, KERNEL_GATE_UP, KERNEL_DOWN, KERNEL_HEAD, KERNEL_ATTENTION = range(6)

_lib = None


def load() -> ctypes.CDLL:
    """Loads the in-tree HIP library; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    M = POINTER(Model)
    sig = {
        "plamo_metal_open": (c_void_p, [POINTER(MetalConfig), c_char_p, c_size_t]),
        "plamo_metal_close": (None, [c_void_p]),
        "plamo_metal_maintain": (None, [c_void_p]),
        "plamo_metal_get_info": (None, [c_void_p, POINTER(MetalInfo)]),
        "plamo_metal_preload": (c_int, [c_void_p, c_void_p, c_uint64]),
        "plamo_metal_warm_cache": (c_int, [c_void_p]),
        "plamo_metal_prepare_model": (c_int, [c_void_p, M]),
        "plamo_metal_forward": (c_int, [c_void_p, M, c_uint64]),
        "plamo_metal_prefill": (c_int, [c_void_p, M, POINTER(c_uint32), c_uint64, f32p]),
        "plamo_metal_verify": (c_int, [c_void_p, M, POINTER(c_uint32), c_uint64,
                                       POINTER(c_uint32)]),
        "plamo_metal_commit": (c_int, [c_void_p, M, c_uint64]),
        "plamo_metal_linear": (c_int, [c_void_p, POINTER(Matmul)]),
        "plamo_hip_linear_static": (c_int, [c_void_p, POINTER(Matmul)]),
        "plamo_metal_mlp": (c_int, [c_void_p, POINTER(Mlp), f32p, c_uint64]),
        "plamo_forward": (c_int, [M, c_uint64]),
        "plamo_prefill": (c_int, [M, POINTER(c_uint32), c_uint64, f32p]),
        "plamo_argmax": (c_uint64, [f32p, c_uint64]),
        "plamo_register_cpu_path": (None, [POINTER(CpuPath)]),
        "plamo_hip_time_kernel": (c_int, [c_void_p, M, c_uint64, c_int, c_int,
                                          POINTER(c_double), POINTER(c_double)]),
        "plamo_draft_open": (c_void_p, []),
        "plamo_draft_close": (None, [c_void_p]),
        "plamo_draft_reset": (c_int, [c_void_p, c_char_p, c_uint]),
        "plamo_draft_propose": (c_uint, [c_void_p, c_uint32, c_uint, POINTER(c_uint32)]),
        "plamo_draft_accept": (c_int, [c_void_p, c_uint]),
        "plamo_draft_checkpoint": (c_void_p, [M, c_uint]),
        "plamo_draft_restore": (c_int, [c_void_p, c_uint, c_uint]),
        "plamo_draft_checkpoint_free": (None, [c_void_p]),
        "plamo_hip_draft_open": (c_void_p, [M, POINTER(MetalConfig), c_char_p, c_size_t]),
        "plamo_hip_draft_install": (None, [c_void_p]),
        "plamo_hip_draft_set_tokenizer": (None, [c_void_p, TOKENIZE_FN, c_void_p]),
        "plamo_hip_draft_reset_ids": (c_int, [c_void_p, POINTER(c_uint32), c_uint64]),
        "plamo_hip_draft_get_stats": (None, [c_void_p, POINTER(DraftStats)]),
        "plamo_hip_draft_next_horizon": (c_uint, [c_uint, c_uint, c_uint, c_uint]),
        "plamo_hip_decode": (c_int, [c_void_p, M, POINTER(c_void_p), POINTER(c_uint32), c_uint64,
                                     c_uint, c_uint, TOKEN_FN, c_void_p, POINTER(DecodeResult),
                                     c_char_p, c_size_t]),
        "plamo_hip_rewind": (c_int, [c_void_p, M, c_uint64]),
        "plamo_hip_invalidate": (None, [c_void_p]),
        "plamo_hip_debug_waits": (None, [c_void_p, c_uint32, c_uint32]),
        "plamo_synthetic_defaults": (None, [POINTER(SyntheticConfig)] + [c_uint64] * 7),
        "plamo_synthetic_build": (c_void_p, [POINTER(SyntheticConfig), c_uint, c_char_p,
                                             c_size_t]),
        "plamo_synthetic_free": (None, [c_void_p]),
        "plamo_synthetic_weights": (POINTER(Mapping), [c_void_p]),
        "plamo_synthetic_frequencies": (f32p, [c_void_p, c_uint64]),
        "plamo_synthetic_instantiate": (c_void_p, [c_void_p, c_int, c_char_p, c_size_t]),
        "plamo_synthetic_release": (None, [c_void_p]),
        "plamo_synthetic_model": (M, [c_void_p]),
        "plamo_synthetic_fill_kv": (c_int, [c_void_p, c_uint64, c_uint64]),
        "plamo_safetensors_view": (c_int, [c_void_p, c_uint64, POINTER(SafetensorsView)]),
        "plamo_parse_u64": (c_int, [c_void_p, c_void_p, POINTER(Number)]),
        "plamo_json_next": (c_int, [c_void_p, c_void_p, POINTER(JsonToken)]),
        "plamo_tensor_descriptor": (c_int, [c_void_p, c_void_p, c_uint64, POINTER(TensorField)]),
        "plamo_find_tensor": (c_int, [c_void_p, c_uint64, c_char_p, POINTER(Tensor)]),
        "plamo_resolve_weight": (c_void_p, [POINTER(Mapping), c_uint64, c_char_p, c_uint64,
                                            POINTER(c_uint64)]),
        "plamo_bind_weights": (c_int, [POINTER(Mapping), c_uint64, POINTER(WeightSpec)]),
        "plamo_checkpoint_open": (c_void_p, [c_char_p, c_uint64, c_char_p, c_size_t]),
        "plamo_checkpoint_close": (None, [c_void_p]),
        "plamo_checkpoint_config": (POINTER(CheckpointConfig), [c_void_p]),
        "plamo_checkpoint_mappings": (POINTER(Mapping), [c_void_p, POINTER(c_size_t)]),
        "plamo_checkpoint_schema": (POINTER(WeightSpec), [c_void_p]),
        "plamo_checkpoint_instantiate": (c_void_p, [c_void_p, c_int, c_char_p, c_size_t]),
        "plamo_model_set_directory": (c_int, [c_char_p]),
        "plamo_model_open": (c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def hook_address(name: str) -> int:
    """Current value of a hook global (0 when unset)."""
    return c_void_p.in_dll(load(), name).value or 0


# BASELINE.json configurations (hidden, layers, qh, kh, dim, intermediate, vocab).
CONFIGS = {
    "c1": dict(hidden=2048, layers=1, qh=16, kh=4, dim=128, intermediate=8192, vocab=16),
    "c2": dict(hidden=2048, layers=16, qh=16, kh=4, dim=128, intermediate=8192, vocab=100000),
    "c3": dict(hidden=2560, layers=24, qh=16, kh=4, dim=128, intermediate=10240, vocab=100000),
    "c4": dict(hidden=4096, layers=32, qh=32, kh=8, dim=128, intermediate=16384, vocab=100000),
    "c5": dict(hidden=6144, layers=60, qh=48, kh=8, dim=128, intermediate=24576, vocab=100000,
               tied=1),
}


def weight_bytes_per_step(cfg: dict) -> int:
    """BF16 bytes a decode step streams: every layer projection plus the head."""
    h, d, qh, kh, inter = cfg["hidden"], cfg["dim"], cfg["qh"], cfg["kh"], cfg["intermediate"]
    per_layer = ((qh + 2 * kh) * d * h + h * qh * d + 2 * inter * h + h * inter) * 2
    return per_layer * cfg["layers"] + cfg["vocab"] * h * 2


class Synthetic:
    """Seeded synthetic model: shared BF16 weights plus any number of instances."""

    def __init__(self, hidden, layers, qh, kh, dim, intermediate, vocab, *, window=2048,
                 global_capacity=8192, pattern=8, seed=1, tied=0, weight_std=0.02,
                 embedding_std=0.02, threads=None):
        lib = load()
        cfg = SyntheticConfig()
        lib.plamo_synthetic_defaults(ctypes.byref(cfg), hidden, layers, qh, kh, dim, intermediate,
                                     vocab)
        cfg.window = window
        cfg.global_capacity = global_capacity
        cfg.pattern = pattern
        cfg.seed = seed
        cfg.tied = tied
        cfg.weight_std = weight_std
        cfg.embedding_std = embedding_std
        self.config = cfg
        err = ctypes.create_string_buffer(256)
        threads = threads or min(16, os.cpu_count() or 1)
        self.handle = lib.plamo_synthetic_build(ctypes.byref(cfg), threads, err, 256)
        if not self.handle:
            raise RuntimeError(err.value.decode())
        self.mapping = lib.plamo_synthetic_weights(self.handle).contents
        self.mappings = [self.mapping]

    def _instantiate(self, pinned: bool, err) -> int:
        return load().plamo_synthetic_instantiate(self.handle, int(pinned), err, len(err))

    def instance(self, pinned=False) -> "Instance":
        return Instance(self, pinned)

    def close(self):
        if self.handle:
            load().plamo_synthetic_free(self.handle)
            self.handle = None


class Checkpoint:
    """A checkpoint directory (config.json + *.safetensors shards) opened by the
    C binder (include/plamo_checkpoint.h); instances share its mapped weights."""

    def __init__(self, directory, global_capacity: int = 0):
        lib = load()
        err = ctypes.create_string_buffer(512)
        self.handle = lib.plamo_checkpoint_open(str(directory).encode(), global_capacity, err, 512)
        if not self.handle:
            raise RuntimeError(err.value.decode())
        self.config = lib.plamo_checkpoint_config(self.handle).contents
        count = c_size_t(0)
        maps = lib.plamo_checkpoint_mappings(self.handle, ctypes.byref(count))
        self.mappings = [maps[i] for i in range(count.value)]

    def schema(self):
        """[(name, shape)] in binding order."""
        out, spec = [], load().plamo_checkpoint_schema(self.handle)
        i = 0
        while spec[i].name:
            out.append((spec[i].name.decode(), [spec[i].shape[k] for k in range(spec[i].rank)]))
            i += 1
        return out

    def _instantiate(self, pinned: bool, err) -> int:
        return load().plamo_checkpoint_instantiate(self.handle, int(pinned), err, len(err))

    def instance(self, pinned=False) -> "Instance":
        return Instance(self, pinned)

    def close(self):
        if self.handle:
            load().plamo_checkpoint_close(self.handle)
            self.handle = None


class Instance:
    """A model instance (descriptors, KV caches, outputs) over shared weights
    (a Synthetic model's or a Checkpoint's)."""

    def __init__(self, synthetic, pinned: bool):
        lib = load()
        err = ctypes.create_string_buffer(256)
        self.synthetic = synthetic
        self.handle = synthetic._instantiate(pinned, err)
        if not self.handle:
            raise RuntimeError(err.value.decode())
        self.model_ptr = lib.plamo_synthetic_model(self.handle)
        self.model = self.model_ptr.contents

    # numpy views of host arrays -------------------------------------------------
    def layer(self, i) -> Layer:
        return self.model.layers[i].contents

    def cache(self, i) -> Cache:
        return self.layer(i).mixer.contents.cache.contents

    def rotation(self, i) -> Rotation:
        return self.layer(i).mixer.contents.rotation.contents

    def state(self):
        return np.ctypeslib.as_array(self.model.state, shape=(self.model.hidden,))

    def normalized(self):
        return np.ctypeslib.as_array(self.model.normalized, shape=(self.model.hidden,))

    def logits(self):
        return np.ctypeslib.as_array(self.model.logits, shape=(self.model.vocab,))

    def kv(self, i, which: str):
        c = self.cache(i)
        ptr = {"k": c.k, "v": c.v, "rot": self.rotation(i).out}[which]
        return np.ctypeslib.as_array(ptr, shape=(c.capacity, c.width))

    def counts(self):
        return [self.cache(i).count for i in range(self.model.count)]

    def reset(self):
        """runtime/engine.c:46-55"""
        for i in range(self.model.count):
            self.cache(i).count = 0
            r = self.rotation(i)
            r.processed_count = 0
            r.scale_bits = 0
            self.layer(i).mixer.contents.gqa.contents.tokens = 0

    def snapshot(self):
        """Copies every host array that a step may change, plus the counters."""
        snap = {"state": self.state().copy(), "normalized": self.normalized().copy(),
                "logits": self.logits().copy(), "layers": []}
        for i in range(self.model.count):
            c, r = self.cache(i), self.rotation(i)
            snap["layers"].append((self.kv(i, "k").copy(), self.kv(i, "v").copy(),
                                   self.kv(i, "rot").copy(), c.count, r.processed_count,
                                   r.scale_bits))
        return snap

    def restore(self, snap):
        self.state()[:] = snap["state"]
        self.normalized()[:] = snap["normalized"]
        self.logits()[:] = snap["logits"]
        for i, (k, v, rot, count, processed, scale) in enumerate(snap["layers"]):
            self.kv(i, "k")[:] = k
            self.kv(i, "v")[:] = v
            self.kv(i, "rot")[:] = rot
            self.cache(i).count = count
            self.rotation(i).processed_count = processed
            self.rotation(i).scale_bits = scale

    def fill_kv(self, rows, seed):
        if not load().plamo_synthetic_fill_kv(self.handle, rows, seed):
            raise ValueError("rows exceed a cache capacity")

    def close(self):
        if self.handle:
            load().plamo_synthetic_release(self.handle)
            self.handle = None


class Backend:
    """plamo_metal_* handle (runtime/metal.h:48-88) opened over a synthetic model."""

    def __init__(self, synthetic=None, memory: int = 0):
        """synthetic: a Synthetic model or a Checkpoint (its weight mappings are
        made resident), or None."""
        lib = load()
        self.lib = lib
        cfg = MetalConfig()
        cfg.memory = memory
        self._maps = None
        if synthetic is not None:
            maps = synthetic.mappings
            self._maps = (Mapping * len(maps))(*maps)
            cfg.maps = self._maps
            cfg.count = len(maps)
        err = ctypes.create_string_buffer(1024)
        self.handle = lib.plamo_metal_open(ctypes.byref(cfg), err, 1024)
        if not self.handle:
            raise RuntimeError(err.value.decode())

    def info(self) -> MetalInfo:
        out = MetalInfo()
        self.lib.plamo_metal_get_info(self.handle, ctypes.byref(out))
        return out

    def forward(self, inst: Instance, token: int) -> int:
        return self.lib.plamo_metal_forward(self.handle, inst.model_ptr, token)

    def prefill(self, inst: Instance, ids, states=None) -> int:
        arr = (c_uint32 * len(ids))(*ids)
        ptr = states.ctypes.data_as(f32p) if states is not None else None
        return self.lib.plamo_metal_prefill(self.handle, inst.model_ptr, arr, len(ids), ptr)

    def verify(self, inst: Instance, ids):
        arr = (c_uint32 * len(ids))(*ids)
        nxt = (c_uint32 * max(1, len(ids)))()
        r = self.lib.plamo_metal_verify(self.handle, inst.model_ptr, arr, len(ids), nxt)
        return r, list(nxt)[: len(ids)]

    def commit(self, inst: Instance, index: int) -> int:
        return self.lib.plamo_metal_commit(self.handle, inst.model_ptr, index)

    def prepare(self, inst: Instance) -> int:
        return self.lib.plamo_metal_prepare_model(self.handle, inst.model_ptr)

    def preload(self, ptr, nbytes) -> int:
        return self.lib.plamo_metal_preload(self.handle, ptr, nbytes)

    def linear(self, weights_ptr, x: np.ndarray, rows: int) -> tuple[int, np.ndarray]:
        tokens, cols = x.shape
        y = np.zeros((tokens, rows), dtype=np.float32)
        mm = Matmul(ctypes.cast(weights_ptr, u16p), x.ctypes.data_as(f32p), y.ctypes.data_as(f32p),
                    rows, cols, tokens, cols, rows)
        return self.lib.plamo_metal_linear(self.handle, ctypes.byref(mm)), y

    def maintain(self):
        """Waits for the backend's stream (runtime/metal.h:51)."""
        self.lib.plamo_metal_maintain(self.handle)

    def invalidate(self):
        """Every layer's host rows are uploaded by the next call."""
        self.lib.plamo_hip_invalidate(self.handle)

    def debug_waits(self, extra: int, polls: int):
        """Test hook: the decode attention's O blocks wait for `extra` more KV
        heads than exist, giving up after `polls` polls (0, 0: normal)."""
        self.lib.plamo_hip_debug_waits(self.handle, extra, polls)

    def time_kernel(self, inst: Instance, layer: int, which: int, reps: int):
        """(ms per launch, algorithmic bytes per launch) of one decode kernel."""
        ms, nbytes = c_double(), c_double()
        if not self.lib.plamo_hip_time_kernel(self.handle, inst.model_ptr, layer, which, reps,
                                              ctypes.byref(ms), ctypes.byref(nbytes)):
            raise RuntimeError(self.info().note.decode())
        return ms.value, nbytes.value

    def close(self):
        if self.handle:
            self.lib.plamo_metal_close(self.handle)
            self.handle = None


class Draft:
    """In-process proposer (include/plamo_draft.h) over a synthetic draft model
    instance; the draft backend is its own plamo_metal handle."""

    def __init__(self, synthetic: Synthetic, inst: Instance):
        lib = load()
        self.lib = lib
        self.synthetic = synthetic
        self.inst = inst
        self._maps = (Mapping * 1)(synthetic.mapping)
        cfg = MetalConfig()
        cfg.maps = self._maps
        cfg.count = 1
        err = ctypes.create_string_buffer(1024)
        self.handle = c_void_p(lib.plamo_hip_draft_open(inst.model_ptr, ctypes.byref(cfg), err,
                                                        1024))
        if not self.handle.value:
            raise RuntimeError(err.value.decode())

    def reset_ids(self, ids) -> int:
        arr = (c_uint32 * len(ids))(*ids)
        return self.lib.plamo_hip_draft_reset_ids(self.handle, arr, len(ids))

    def propose(self, first: int, limit: int):
        out = (c_uint32 * DRAFT_MAX)()
        n = self.lib.plamo_draft_propose(self.handle, first, limit, out)
        return list(out)[:n]

    def accept(self, consumed: int) -> int:
        return self.lib.plamo_draft_accept(self.handle, consumed)

    def stats(self) -> DraftStats:
        out = DraftStats()
        self.lib.plamo_hip_draft_get_stats(self.handle, ctypes.byref(out))
        return out

    def release(self):
        """Hands the handle to a caller that takes ownership (plamo_hip_decode)."""
        h, self.handle = self.handle, c_void_p(None)
        return h

    def close(self):
        if self.handle.value:
            self.lib.plamo_draft_close(self.handle)
            self.handle = c_void_p(None)


def decode(backend: Backend, inst: Instance, prompt, max_tokens: int, draft: Draft | None = None,
           block: int = 0, cancel_after: int | None = None):
    """plamo_hip_decode over a prefilled instance: (tokens, DecodeResult, draft
    still open). The draft, if any, is closed by the library when it fails."""
    lib = load()
    tokens = []

    def on_token(token_id, _ctx):
        tokens.append(int(token_id))
        return 0 if cancel_after is not None and len(tokens) >= cancel_after else 1

    cb = TOKEN_FN(on_token)
    handle = c_void_p(draft.handle.value if draft is not None else None)
    arr = (c_uint32 * max(1, len(prompt)))(*prompt)
    result = DecodeResult()
    err = ctypes.create_string_buffer(256)
    ok = lib.plamo_hip_decode(backend.handle, inst.model_ptr, ctypes.byref(handle), arr,
                              len(prompt), max_tokens, block, cb, None, ctypes.byref(result),
                              err, 256)
    if draft is not None and not handle.value:
        draft.handle = c_void_p(None)  # closed by the library
    if not ok:
        raise RuntimeError(err.value.decode())
    return tokens, result, handle.value is not None
