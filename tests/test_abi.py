"""CPU checks of the drop-in boundary: layouts, exports, and behaviour without a GPU.

Layout sizes and offsets are the reference's own assertions
(runtime/model.h:76-86, runtime/parallel.h:11); the exported names are the
entry points each header in include/ declares.
"""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle_lib
import plamo_hip

ROOT = Path(__file__).resolve().parents[1]


def test_descriptor_layouts_match_reference_asserts():
    sizes = {plamo_hip.Model: 88, plamo_hip.Qkv: 72, plamo_hip.Cache: 48, plamo_hip.Rotation: 72,
             plamo_hip.Gqa: 72, plamo_hip.Mixer: 56, plamo_hip.Mlp: 80, plamo_hip.Layer: 64,
             plamo_hip.Matmul: 64}
    for struct, size in sizes.items():
        assert ctypes.sizeof(struct) == size, struct.__name__
    assert plamo_hip.Layer.mixer.offset == 40
    assert plamo_hip.Cache.count.offset == 24
    assert plamo_hip.Rotation.processed_count.offset == 56


def test_header_declarations_are_exported(hip):
    # Every function/global a public header declares is exported by the library.
    declared = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        declared |= set(re.findall(r"\b(plamo_[a-z0-9_]+)\s*\(", text))
        declared |= set(re.findall(r"\(\*(plamo_[a-z0-9_]+)\)", text))
        declared |= set(re.findall(r"extern [a-z_ 0-9*]+\b(plamo_[a-z0-9_]+);", text))
        # Function-pointer typedefs name types, not symbols.
        declared -= set(re.findall(r"typedef [^;(]+\(\*(plamo_[a-z0-9_]+)\)", text))
    declared.discard("plamo_reset_request")  # the engine defines it (runtime/engine.c:46)
    for name in declared:
        assert hasattr(hip, name), name
    listed = {n for names in plamo_hip.EXPORTS.values() for n in names}
    assert listed <= declared | {"plamo_compute_context", "plamo_weight_context",
                                 "plamo_weight_chunk_bytes"}


def test_open_without_gpu_fails_cleanly(hip):
    err = ctypes.create_string_buffer(256)
    cfg = plamo_hip.MetalConfig()
    handle = hip.plamo_metal_open(ctypes.byref(cfg), err, 256)
    if handle:  # a GPU is visible: this case is for GPU-less hosts
        hip.plamo_metal_close(handle)
        pytest.skip("a GPU is visible")
    assert b"MI355X" in err.value
    assert plamo_hip.hook_address("plamo_forward_kernel") == 0


def test_trampolines_fall_through_to_registered_cpu_path(hip, oracle):
    # src/forward.s:9-31: no hook installed -> the platform CPU path runs.
    s = plamo_hip.Synthetic(24, 2, 4, 2, 6, 40, 17, window=2, global_capacity=32, pattern=2)
    a, b = s.instance(), s.instance()
    try:
        assert hip.plamo_forward(a.model_ptr, 3) == 0  # nothing registered
        fwd = plamo_hip.CpuPath._fields_[0][1](lambda m, t: oracle.oracle_forward(m, t))
        pre = plamo_hip.CpuPath._fields_[1][1](
            lambda m, ids, n, st: oracle.oracle_prefill(m, ids, n, st))
        path = plamo_hip.CpuPath(fwd, pre)
        hip.plamo_register_cpu_path(ctypes.byref(path))
        ids = (ctypes.c_uint32 * 2)(4, 7)
        states = np.zeros((2, 24), np.float32)
        assert hip.plamo_prefill(a.model_ptr, ids, 2, states.ctypes.data_as(plamo_hip.f32p)) == 1
        assert hip.plamo_forward(a.model_ptr, 3) == 1
        assert oracle_lib.prefill(b, [4, 7]) and oracle_lib.forward(b, 3)
        assert a.logits().tobytes() == b.logits().tobytes()
        assert hip.plamo_prefill(a.model_ptr, ids, 0, None) == 0
        hip.plamo_register_cpu_path(None)
        assert hip.plamo_forward(a.model_ptr, 3) == 0
    finally:
        hip.plamo_register_cpu_path(None)
        a.close()
        b.close()
        s.close()


def test_synthetic_layout_and_determinism(hip):
    cfg = dict(hidden=64, layers=9, qh=4, kh=2, dim=16, intermediate=96, vocab=50)
    s1 = plamo_hip.Synthetic(**cfg, threads=1, seed=9)
    s4 = plamo_hip.Synthetic(**cfg, threads=4, seed=9)
    try:
        w1 = np.ctypeslib.as_array(ctypes.cast(s1.mapping.base, plamo_hip.u16p),
                                   shape=(s1.mapping.bytes // 2,))
        w4 = np.ctypeslib.as_array(ctypes.cast(s4.mapping.base, plamo_hip.u16p),
                                   shape=(s4.mapping.bytes // 2,))
        assert w1.tobytes() == w4.tobytes()
        inst = s1.instance()
        m = inst.model
        for i in range(9):
            c = inst.cache(i)
            glob = (i + 1) % 8 == 0
            assert c.sliding == (not glob)
            assert c.capacity == (8192 if glob else 2049)
            assert c.width == 2 * 16
            scale = np.float32(m.scales[i]).view(np.uint32)
            assert scale == (np.float32(1 + 0.1 * np.log(256)).view(np.uint32) if glob else
                             np.float32(1).view(np.uint32))
        # Shared workspace, as tools/model_layout.py:183-196 lays it out.
        l0, l1 = inst.layer(0), inst.layer(1)
        assert ctypes.addressof(l0.normalized.contents) == ctypes.addressof(l1.normalized.contents)
        assert ctypes.addressof(l0.state.contents) == ctypes.addressof(m.state.contents)
        inst.close()
    finally:
        s1.close()
        s4.close()


def test_synthetic_weight_statistics(hip):
    s = plamo_hip.Synthetic(256, 1, 2, 1, 128, 1024, 64, seed=2)
    try:
        w = np.ctypeslib.as_array(ctypes.cast(s.mapping.base, plamo_hip.u16p),
                                  shape=(s.mapping.bytes // 2,))
        vals = (w.astype(np.uint32) << 16).view(np.float32)
        nz = vals[vals != 0]
        assert abs(float(nz.std()) - 0.02) < 0.001 and abs(float(nz.mean())) < 0.001
    finally:
        s.close()
