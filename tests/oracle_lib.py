"""Loader of the CPU oracle (oracle/build/liboracle.so) for tests and the CPU baseline.

Test infrastructure only: the oracle is the checker, never the thing measured
on the GPU path.
"""

from __future__ import annotations

import ctypes
import subprocess
import sys
from ctypes import POINTER, c_double, c_float, c_int, c_uint, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle" / "build" / "liboracle.so"
sys.path.insert(0, str(ROOT / "plamo-3-translate.c_amd"))

import plamo_hip  # noqa: E402

f32p = POINTER(c_float)
u16p = POINTER(c_uint16)
_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not ORACLE.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    lib = ctypes.CDLL(str(ORACLE))
    M = POINTER(plamo_hip.Model)
    sig = {
        "oracle_bf16": (c_float, [c_uint16]),
        "oracle_to_bf16": (c_uint16, [c_float]),
        "oracle_exp": (c_float, [c_float]),
        "oracle_softmax": (None, [f32p, c_uint64]),
        "oracle_swiglu": (None, [f32p, f32p, c_uint64]),
        "oracle_matvec": (None, [u16p, f32p, f32p, c_uint64, c_uint64]),
        "oracle_matmul": (None, [POINTER(plamo_hip.Matmul)]),
        "oracle_matmul_blocked": (None, [POINTER(plamo_hip.Matmul)]),
        "oracle_set_threads": (None, [c_uint]),
        "oracle_threads": (c_uint, []),
        "oracle_rmsnorm": (None, [f32p, u16p, f32p, c_uint64, c_float, c_float]),
        "oracle_residual": (None, [f32p, f32p, c_uint64]),
        "oracle_attention_head": (None, [f32p, f32p, f32p, f32p, f32p, c_uint64, c_uint64,
                                         c_uint64]),
        "oracle_gqa": (None, [POINTER(plamo_hip.Gqa)]),
        "oracle_rope_copy": (None, [f32p, f32p, f32p, f32p, c_uint64, c_uint64]),
        "oracle_sincos": (None, [c_double, f32p]),
        "oracle_rope_table": (None, [f32p, c_uint64, c_uint64, f32p, f32p, c_float]),
        "oracle_rope_frequencies": (None, [c_double, c_uint64, c_int, c_double, c_double, c_double,
                                           c_double, f32p]),
        "oracle_rope_concentration": (c_float, [c_int, c_double]),
        "oracle_cache_append": (c_int, [POINTER(plamo_hip.Cache), f32p, f32p]),
        "oracle_cache_rope_cached": (None, [POINTER(plamo_hip.Rotation), c_float]),
        "oracle_qk_norm": (None, [f32p, u16p, u16p, c_uint64, c_uint64, c_uint64]),
        "oracle_qkv": (None, [POINTER(plamo_hip.Qkv)]),
        "oracle_mixer": (c_int, [POINTER(plamo_hip.Mixer), c_float]),
        "oracle_mlp": (None, [u16p, u16p, f32p, f32p, f32p, c_uint64, c_uint64]),
        "oracle_mlp_branch": (None, [POINTER(plamo_hip.Mlp)]),
        "oracle_layer": (c_int, [POINTER(plamo_hip.Layer), c_float]),
        "oracle_embedding": (c_int, [u16p, c_uint64, c_uint64, c_uint64, f32p]),
        "oracle_forward": (c_int, [M, c_uint64]),
        "oracle_forward_hidden": (c_int, [M, c_uint64]),
        "oracle_prefill": (c_int, [M, POINTER(c_uint32), c_uint64, f32p]),
        "oracle_argmax": (c_uint64, [f32p, c_uint64]),
        "oracle_fnv1a": (c_uint64, [c_void_p, c_uint64, c_uint64]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def forward(inst: "plamo_hip.Instance", token: int) -> int:
    return load().oracle_forward(inst.model_ptr, token)


def prefill(inst: "plamo_hip.Instance", ids, states=None) -> int:
    arr = (c_uint32 * len(ids))(*ids)
    ptr = states.ctypes.data_as(f32p) if states is not None else None
    return load().oracle_prefill(inst.model_ptr, arr, len(ids), ptr)
