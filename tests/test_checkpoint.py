"""The checkpoint binder (include/plamo_checkpoint.h) on the CPU.

The primitives are checked against the reference's own known-answer tests
(tests/load.c, tests/find.c) and against the grammar their assembly encodes
(src/json.s, src/tensor.s, src/find.s, src/resolve.s, src/bind.s). The
end-to-end test writes a checkpoint from a synthetic model, opens it through
the binder, and requires the oracle's results over it to be bit-identical to
the oracle's results over the synthetic model itself: the same bytes must
reach the same descriptor slots, which a wrong name, shape, order or layer
assignment would break.
"""

import ctypes
import json
import struct
import subprocess
import sys

import numpy as np
import pytest

import checkpoint_writer
import plamo_hip
from parity import oracle_lib, tiny


def mem(data: bytes):
    """A C buffer holding `data` and its address (kept alive by the caller)."""
    b = ctypes.create_string_buffer(data, len(data))
    return b, ctypes.addressof(b)


# ---------------------------------------------------------------- tests/load.c

def test_envelope_reference_vectors(hip):
    file = bytearray(20)
    file[0] = 8
    file[8:16] = b"{}      "
    b, a = mem(bytes(file))
    v = plamo_hip.SafetensorsView()
    assert hip.plamo_safetensors_view(a, 20, ctypes.byref(v))
    assert v.header_size == 8 and v.data_size == 4 and v.data == a + 16
    file[0] = 255
    b, a = mem(bytes(file))
    assert not hip.plamo_safetensors_view(a, 20, ctypes.byref(v))
    assert not v.header and not v.data
    assert not hip.plamo_safetensors_view(a, 7, ctypes.byref(v))


def test_envelope_rules(hip):
    v = plamo_hip.SafetensorsView()

    def view(header: bytes, tail=b"xxxx"):
        data = struct.pack("<Q", len(header)) + header + tail
        b, a = mem(data)
        return hip.plamo_safetensors_view(a, len(data), ctypes.byref(v))

    assert view(b"{}")
    assert not view(b"{} \t")      # only spaces may follow the closing brace
    assert not view(b"[]")
    assert not view(b"{ ")          # only spaces after '{'
    assert not view(b"{")           # shorter than 2
    assert view(b'{"a":1}   ')


def test_parse_u64_reference_vectors(hip):
    cases = ["0", "123,", "18446744073709551615", "18446744073709551616", "01", "-1", ""]
    values = [0, 123, 2**64 - 1]
    for i, text in enumerate(cases):
        raw = text.encode()
        b, a = mem(raw + b"\0")
        n = plamo_hip.Number()
        ok = hip.plamo_parse_u64(a, a + len(raw), ctypes.byref(n))
        assert bool(ok) == (i < 3), text
        if ok:
            assert n.value == values[i]
        else:
            assert not n.next and n.value == 0
    b, a = mem(b"123,")
    n = plamo_hip.Number()
    assert hip.plamo_parse_u64(a, a + 4, ctypes.byref(n)) and n.next == a + 3


# ---------------------------------------------------------------- src/json.s

def tokens(hip, text: bytes):
    b, a = mem(text)
    p, end, out = a, a + len(text), []
    while True:
        t = plamo_hip.JsonToken()
        code = hip.plamo_json_next(p, end, ctypes.byref(t))
        if code in (0, -1):
            out.append(code)
            return out
        body = ctypes.string_at(t.start, t.length).decode("latin-1")
        out.append((code, body, t.value))
        p = t.next


def test_lexer(hip):
    assert tokens(hip, b' { "a" : [1 ,23] }\n') == [
        (ord("{"), "{", 0), (256, "a", 0), (ord(":"), ":", 0), (ord("["), "[", 0),
        (257, "1", 1), (ord(","), ",", 0), (257, "23", 23), (ord("]"), "]", 0),
        (ord("}"), "}", 0), 0]
    # Escapes stay raw; every JSON escape is accepted, others are not.
    escaped = rb'"x\"y\\\/\b\f\n\r\t\u00aFz"'
    assert tokens(hip, escaped)[0] == (256, escaped[1:-1].decode(), 0)
    for bad in (rb'"\x"', rb'"\u12g4"', rb'"abc', b'"a\x01b"', b"12a", b"-3", b"1.5", b"true"):
        assert tokens(hip, bad)[-1] == -1, bad
    assert tokens(hip, b"7}") == [(257, "7", 7), (ord("}"), "}", 0), 0]
    assert tokens(hip, "\"é\"".encode())[0][0] == 256  # raw UTF-8 bytes are kept


# ---------------------------------------------------------------- src/tensor.s

def descriptor(hip, text: str, data_bytes=100):
    raw = text.encode()
    b, a = mem(raw)
    f = plamo_hip.TensorField()
    ok = hip.plamo_tensor_descriptor(a, a + len(raw), data_bytes, ctypes.byref(f))
    return ok, f, a


def test_tensor_descriptor_rules(hip):
    ok, f, a = descriptor(hip, '{"shape":[2,3],"data_offsets":[10,22],"dtype":"BF16"} ,')
    assert ok and f.rank == 2 and list(f.dims[:2]) == [2, 3] and f.offset == 10 and f.bytes == 12
    assert f.next == a + len('{"shape":[2,3],"data_offsets":[10,22],"dtype":"BF16"}')
    ok, f, _ = descriptor(hip, '{"dtype":"BF16","shape":[],"data_offsets":[0,2]}')
    assert ok and f.rank == 0 and f.bytes == 2
    ok, f, _ = descriptor(hip, '{"dtype":"BF16","shape":[1,1,1,2],"data_offsets":[0,4]}')
    assert ok and f.rank == 4
    rejected = [
        '{"dtype":"F32","shape":[1],"data_offsets":[0,4]}',           # not BF16
        '{"dtype":"BF16","shape":[1,1,1,1,1],"data_offsets":[0,2]}',  # rank 5
        '{"dtype":"BF16","shape":[2],"data_offsets":[0,2]}',          # bytes != 2 * elements
        '{"dtype":"BF16","shape":[1],"data_offsets":[4,2]}',          # end < begin
        '{"dtype":"BF16","shape":[1],"data_offsets":[100,102]}',      # past the data
        '{"dtype":"BF16","shape":[1]}',                               # missing field
        '{"dtype":"BF16","dtype":"BF16","shape":[1],"data_offsets":[0,2]}',  # duplicate
        '{"dtype":"BF16","shape":[1],"data_offsets":[0,2],"x":1}',   # unknown key
        '{"dtyp\\u0065":"BF16","shape":[1],"data_offsets":[0,2]}',   # escaped key
        '{"dtype":"BF16","shape":[4294967296,4294967296],"data_offsets":[0,2]}',  # overflow
        '{"dtype":"BF16","shape":[1,],"data_offsets":[0,2]}',        # trailing comma
    ]
    for text in rejected:
        ok, f, _ = descriptor(hip, text)
        assert not ok and f.next is None and f.bytes == 0, text


# ---------------------------------------------------------------- tests/find.c

def test_find_reference_vectors(hip):
    h = (b'{"__metadata__":{"format":"pt"},"a":{"dtype":"BF16","shape":[1],"data_offsets":[0,2]},'
         b'"b":{"dtype":"BF16","shape":[2],"data_offsets":[2,6]}}')
    file = struct.pack("<Q", len(h)) + h + struct.pack("<3H", 0x3F80, 0x4000, 0x4040)
    b, a = mem(file)
    t = plamo_hip.Tensor()
    n = len(file)
    assert hip.plamo_find_tensor(a, n, b"b", ctypes.byref(t))
    assert t.bytes == 4 and t.rank == 1 and t.dims[0] == 2
    assert ctypes.cast(t.data, plamo_hip.u16p)[0] == 0x4000
    assert hip.plamo_find_tensor(a, n, b"a", ctypes.byref(t))
    assert ctypes.cast(t.data, plamo_hip.u16p)[0] == 0x3F80
    assert not hip.plamo_find_tensor(a, n, b"ab", ctypes.byref(t)) and not t.data
    assert not hip.plamo_find_tensor(a, n - 1, b"b", ctypes.byref(t)) and not t.data
    # The metadata key is never a tensor; an empty header has none.
    assert not hip.plamo_find_tensor(a, n, b"__metadata__", ctypes.byref(t))
    empty = struct.pack("<Q", 2) + b"{}"
    b2, a2 = mem(empty)
    assert not hip.plamo_find_tensor(a2, len(empty), b"a", ctypes.byref(t))


# ---------------------------------------------------------------- resolve / bind

def shards(hip, *files):
    keep = [mem(f) for f in files]
    maps = (plamo_hip.Mapping * len(files))(*[plamo_hip.Mapping(a, len(f))
                                               for (b, a), f in zip(keep, files)])
    return keep, maps


def test_resolve_and_bind(hip):
    one = checkpoint_writer.safetensors_bytes(
        [("x", np.array([[1, 2, 3]], np.uint16)), ("y", np.array([7], np.uint16))])
    two = checkpoint_writer.safetensors_bytes(
        [("x", np.array([9], np.uint16)), ("z", np.array([[5, 6]], np.uint16))])
    keep, maps = shards(hip, one, two)
    dims = (ctypes.c_uint64 * 4)

    def resolve(name, shape):
        return hip.plamo_resolve_weight(maps, 2, name, len(shape), dims(*shape))

    assert ctypes.cast(resolve(b"x", [1, 3]), plamo_hip.u16p)[2] == 3  # first shard decides
    assert resolve(b"x", [1]) is None                                  # ... even when wrong
    assert ctypes.cast(resolve(b"z", [1, 2]), plamo_hip.u16p)[1] == 6  # found in the second
    assert resolve(b"z", [2, 1]) is None and resolve(b"w", [1]) is None
    assert hip.plamo_resolve_weight(maps, 2, b"y", 5, dims(1, 1, 1, 1)) is None  # rank > 4

    slots = (ctypes.c_void_p * 3)()
    shapes = [dims(1, 3), dims(1), dims(1, 2)]
    spec = (plamo_hip.WeightSpec * 4)(
        plamo_hip.WeightSpec(b"x", 2, shapes[0], ctypes.pointer(ctypes.c_void_p.from_buffer(slots, 0))),
        plamo_hip.WeightSpec(b"y", 1, shapes[1], ctypes.pointer(ctypes.c_void_p.from_buffer(slots, 8))),
        plamo_hip.WeightSpec(b"z", 2, shapes[2], ctypes.pointer(ctypes.c_void_p.from_buffer(slots, 16))),
        plamo_hip.WeightSpec(None, 0, None, None))
    assert hip.plamo_bind_weights(maps, 2, spec)
    assert all(slots[i] for i in range(3))
    shapes[2][1] = 3  # z no longer matches: nothing stays bound
    assert not hip.plamo_bind_weights(maps, 2, spec)
    assert not any(slots[i] for i in range(3))


# ---------------------------------------------------------------- checkpoints

def compare_bitwise(a, b):
    assert a.logits().tobytes() == b.logits().tobytes()
    assert a.state().tobytes() == b.state().tobytes()
    for i in range(a.model.count):
        n = a.cache(i).count
        assert n == b.cache(i).count
        for which in ("k", "v", "rot"):
            assert a.kv(i, which)[:n].tobytes() == b.kv(i, which)[:n].tobytes()


@pytest.mark.parametrize("tied", [0, 1])
def test_checkpoint_matches_synthetic_bitwise(tmp_path, tied):
    syn = tiny(layers=4, pattern=2, window=3, capacity=48, tied=tied, seed=11)
    d = checkpoint_writer.write(tmp_path / "ck", syn, shards=3)
    ck = plamo_hip.Checkpoint(d)
    a, b = syn.instance(), ck.instance()
    try:
        c = ck.config
        assert (c.hidden, c.layers, c.qh, c.kh, c.dim, c.intermediate, c.vocab, c.tied) == (
            24, 4, 4, 2, 6, 40, 17, tied)
        names = [n for n, _ in ck.schema()]
        expected = [n for n, _ in checkpoint_writer.weights(syn)]
        assert names == expected  # tools/weight_schema.py order
        assert len(ck.mappings) == 3
        # Same RoPE tables, concentrations and capacities as the synthetic layout.
        for i in range(4):
            assert a.cache(i).capacity == b.cache(i).capacity
            assert a.cache(i).sliding == b.cache(i).sliding
            fa = np.ctypeslib.as_array(a.rotation(i).freq, shape=(3,))
            fb = np.ctypeslib.as_array(b.rotation(i).freq, shape=(3,))
            assert fa.tobytes() == fb.tobytes()
            assert a.model.scales[i] == b.model.scales[i]
        prompt = [3, 1, 4, 1, 5, 9, 2]
        assert oracle_lib.prefill(a, prompt) and oracle_lib.prefill(b, prompt)
        compare_bitwise(a, b)
        token = int(np.argmax(a.logits()))
        for _ in range(4):  # past the 4-row sliding window: shifts and rebuilt rotations
            assert oracle_lib.forward(a, token) and oracle_lib.forward(b, token)
            compare_bitwise(a, b)
            token = int(np.argmax(a.logits()))
    finally:
        a.close()
        b.close()
        ck.close()
        syn.close()


def test_checkpoint_errors(tmp_path):
    syn = tiny(layers=2, seed=5)
    try:
        good = checkpoint_writer.write(tmp_path / "good", syn, shards=2)
        plamo_hip.Checkpoint(good).close()

        def broken(name, edit):
            d = checkpoint_writer.write(tmp_path / name, syn, shards=2)
            edit(d)
            with pytest.raises(RuntimeError) as e:
                plamo_hip.Checkpoint(d)
            return str(e.value)

        def drop_key(d):
            c = json.loads((d / "config.json").read_text())
            del c["head_dim"]
            (d / "config.json").write_text(json.dumps(c))
        assert "head_dim" in broken("nokey", drop_key)

        def drop_tensor(d):
            kept = [(n, w) for n, w in checkpoint_writer.weights(syn)
                    if n != "model.layers.layers.1.mlp.down_proj.weight"]
            for s in range(2):
                (d / f"model-{s + 1:05d}-of-00002.safetensors").write_bytes(
                    checkpoint_writer.safetensors_bytes(kept[s::2]))
        assert "model.layers.layers.1.mlp.down_proj.weight" in broken("notensor", drop_tensor)

        def reshape(d):
            c = json.loads((d / "config.json").read_text())
            c["intermediate_size"] = 48  # gate/up and down no longer match
            (d / "config.json").write_text(json.dumps(c))
        assert "mlp" in broken("shape", reshape)

        def wrong_dtype(d):
            for f in d.glob("*.safetensors"):
                f.write_bytes(f.read_bytes().replace(b'"BF16"', b'"BF32"'))
        broken("dtype", wrong_dtype)

        def no_shards(d):
            for f in d.glob("*.safetensors"):
                f.unlink()
        assert "no .safetensors" in broken("empty", no_shards)
        with pytest.raises(RuntimeError):
            plamo_hip.Checkpoint(tmp_path / "absent")
    finally:
        syn.close()


def test_model_open_globals(tmp_path):
    """The engine's entry (runtime/model.h:88-101): plamo_model_open() fills
    plamo_model and the weight tables from $PLAMO_MODEL_DIR, once per process."""
    syn = tiny(layers=2, seed=9)
    try:
        d = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    script = f"""
import ctypes, sys
sys.path.insert(0, {str(plamo_hip.LIB_PATH.parent)!r})
import plamo_hip
lib = plamo_hip.load()
assert lib.plamo_model_open() == 1 and lib.plamo_model_open() == 1
m = plamo_hip.Model.in_dll(lib, "plamo_model")
count = ctypes.c_uint64.in_dll(lib, "plamo_weight_mapping_count").value
schema = (plamo_hip.WeightSpec * 4).in_dll(lib, "plamo_weight_schema")
print(m.hidden, m.vocab, m.count, count, schema[0].name.decode(), schema[3].name.decode())
"""
    env = dict(__import__("os").environ, PLAMO_MODEL_DIR=str(d))
    out = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["24", "17", "2", "2", "model.embed_tokens.weight",
                                  "model.layers.layers.0.mixer.qkv_proj.weight"]
