"""The drop-in claim at the source level, on the CPU: the reference's
runtime/engine.c and runtime/prompt_cache.c compile with -Werror against
include/ (through tests/engine_link/shim, the four forwarding headers a
maintainer adds) and link against libplamo_hip.so with -Wl,--no-undefined.
Only the tokenizer (AArch64 assembly in the reference) and the Darwin-only
memory/thread modules are stood in for (tests/engine_link/host_stubs.c); the
draft interface, the model globals and the GPU backend come from the library.

The linked engine then runs what needs no GPU: tokenizer-only requests, and a
GPU open that fails with the backend's message (runtime/engine.c:180-182). The
model globals that runtime/model.h:88-101 declares (profile strings, patch
table) are checked through the library as well.

Skipped where the reference checkout is absent (it is read in place, never
copied)."""

import ctypes
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

import checkpoint_writer
import plamo_hip
from parity import tiny

ROOT = Path(__file__).resolve().parents[1]
HERE = ROOT / "tests" / "engine_link"
REF = Path("/root/reference/runtime")

needs_reference = pytest.mark.skipif(
    not (REF / "engine.c").exists() or shutil.which("gcc") is None or shutil.which("make") is None,
    reason="the reference checkout (runtime/engine.c) or gcc/make is not available")


@pytest.fixture(scope="module")
def engine_host(tmp_path_factory):
    out = tmp_path_factory.mktemp("engine_build")
    r = subprocess.run(["make", "-C", str(HERE), f"REF={REF}", f"OUT={out}", "-B"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return out / "engine_host"


def run(binary, *args, env_extra=None, timeout=60):
    env = dict(os.environ, LD_LIBRARY_PATH=str(plamo_hip.LIB_PATH.parent), **(env_extra or {}))
    return subprocess.run([str(binary), *args], capture_output=True, text=True, env=env,
                          timeout=timeout)


@needs_reference
def test_engine_compiles_against_include(engine_host):
    # The shim headers, not the reference's model.h/compute.h/metal.h/draft.h,
    # are the ones the engine sees.
    r = subprocess.run(["gcc", "-std=gnu11", "-fsyntax-only", "-H", f"-I{HERE / 'shim'}", "-I-",
                        f"-I{ROOT / 'include'}", f"-I{REF}", str(REF / "engine.c")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    included = [line.split()[-1] for line in r.stderr.splitlines() if line.startswith(".")]
    names = {Path(p).name for p in included}
    assert {"plamo_model.h", "plamo_backend.h", "plamo_draft.h", "plamo_parallel.h"} <= names
    for p in included:
        if Path(p).parent == REF:
            assert Path(p).name not in {"model.h", "compute.h", "metal.h", "draft.h"}, p
    assert engine_host.exists()


@needs_reference
def test_tokenizer_only_engine_runs(engine_host, tmp_path):
    (tmp_path / "tokenizer.jsonl").write_text("300\n")
    r = run(engine_host, "tokenize", "1", "hi", env_extra={"PLAMO_MODEL_DIR": str(tmp_path)})
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert out["memory_mode"] == "tokenizer"
    # direction 1: prefix 0, the bytes, the end marker (host_stubs.c). The two
    # prefixes have the template's shape: 12 ids, equal but for index 10.
    prefix0 = [20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 29, 23]
    assert out["ids"] == prefix0 + [32 + ord("h") % 268, 32 + ord("i") % 268, 17]
    r = run(engine_host, "tokenize", "2", "hi", env_extra={"PLAMO_MODEL_DIR": str(tmp_path)})
    assert r.returncode == 0, r.stderr
    ids = json.loads(r.stdout)["ids"]
    assert ids[:10] == prefix0[:10] and ids[10] != prefix0[10] and ids[11] == prefix0[11]
    # No directory: the engine's own error names the profile (runtime/engine.c:40-44).
    r = run(engine_host, "tokenize", "0", "hi", env_extra={"PLAMO_MODEL_DIR": ""})
    assert r.returncode == 1
    assert "plamo-3-translate-custom" in r.stderr and "--model custom" in r.stderr


@needs_reference
def test_engine_reports_backend_open_failure(engine_host, tmp_path):
    err = ctypes.create_string_buffer(256)
    handle = plamo_hip.load().plamo_metal_open(ctypes.byref(plamo_hip.MetalConfig()), err, 256)
    if handle:
        plamo_hip.load().plamo_metal_close(handle)
        pytest.skip("a GPU is visible: this case is for GPU-less hosts")
    syn = tiny(vocab=300)
    try:
        d = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    (d / "tokenizer.jsonl").write_text("300\n")
    r = run(engine_host, "translate", "1", "4", "hi", env_extra={"PLAMO_MODEL_DIR": str(d)})
    assert r.returncode == 1
    assert "MI355X" in r.stderr, r.stderr


def child(script: str, env_extra=None):
    """Runs `script` in a fresh interpreter (the model globals are per process)."""
    head = (f"import ctypes, sys\nsys.path.insert(0, {str(plamo_hip.LIB_PATH.parent)!r})\n"
            "import plamo_hip\nlib = plamo_hip.load()\n")
    env = dict(os.environ, **(env_extra or {}))
    r = subprocess.run([sys.executable, "-c", head + script], env=env, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout.split()


def test_profile_strings(tmp_path):
    """runtime/model.h:91-92: the vocabulary path and the profile name, which
    the engine keys behaviour on (runtime/engine.c:146-149, 322-324)."""
    syn = tiny(vocab=300)
    try:
        d = checkpoint_writer.write(tmp_path / "ck", syn, shards=1)
    finally:
        syn.close()
    # A config with the shape of tools/profiles/8b/config.json.
    cfg = json.loads((d / "config.json").read_text())
    cfg.update(hidden_size=4096, num_hidden_layers=32, num_attention_heads=32,
               num_key_value_heads=4, intermediate_size=16384, head_dim=128,
               tie_word_embeddings=False)
    eight = tmp_path / "8b"
    eight.mkdir()
    (eight / "config.json").write_text(json.dumps(cfg))
    script = """
for name in ("plamo_vocab_path", "plamo_model_name", "plamo_model_repository",
             "plamo_model_revision"):
    print(repr(ctypes.string_at(ctypes.addressof(ctypes.c_char.in_dll(lib, name))).decode()))
"""
    out = child(script, {"PLAMO_MODEL_DIR": str(d)})
    assert out == [repr(f"{d}/tokenizer.jsonl"), repr("plamo-3-translate-custom"), "''", "''"]
    out = child(f"assert lib.plamo_model_set_directory({str(eight).encode()!r}) == 1\n" + script,
                {"PLAMO_MODEL_DIR": ""})
    assert out == [repr(f"{eight}/tokenizer.jsonl"), repr("plamo-3-translate-8b"),
                   repr("pfnet/plamo-3-translate-8b"),
                   repr("19ecab3fb31424ee937b7503730318b50e55771c")]


def test_model_patch_table(tmp_path):
    """src/model_init.s:1-25 and runtime/engine.c:69-74: after the engine moves
    the weights and rebases the schema slots, plamo_model_patch() carries every
    slot into its descriptor field; a NULL slot stores nothing and returns 0."""
    syn = tiny(layers=3, vocab=300)
    try:
        d = checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    script = """
assert lib.plamo_model_open() == 1
P = ctypes.c_void_p
table = (ctypes.c_uint64 * 512).in_dll(lib, "plamo_model_patches")
pairs = []
while table[2 * len(pairs)]:
    pairs.append((table[2 * len(pairs)], table[2 * len(pairs) + 1]))
schema = (plamo_hip.WeightSpec * 64).in_dll(lib, "plamo_weight_schema")
entries = 0
while schema[entries].name:
    entries += 1
print(len(pairs), entries)
# Bound now: every descriptor field already holds its slot's pointer.
assert all(P.from_address(dst).value == P.from_address(src).value for dst, src in pairs)
m = plamo_hip.Model.in_dll(lib, "plamo_model")
fields = {P.from_address(dst).value for dst, _ in pairs}
q = m.layers[2].contents.mixer.contents.qkv.contents
assert ctypes.cast(m.embedding, P).value in fields and ctypes.cast(q.weight, P).value in fields
# Move every weight by 64 bytes, as a rebase onto copies would.
slots = sorted({src for _, src in pairs})
saved = {s: P.from_address(s).value for s in slots}
for s in slots:
    P.from_address(s).value = saved[s] + 64
assert lib.plamo_model_patch(table) == 1
assert all(P.from_address(dst).value == P.from_address(src).value for dst, src in pairs)
assert ctypes.cast(m.embedding, P).value == saved[pairs[0][1]] + 64
# A NULL slot: nothing is stored.
before = [P.from_address(dst).value for dst, _ in pairs]
P.from_address(slots[-1]).value = None
for s in slots[:-1]:
    P.from_address(s).value = saved[s]
assert lib.plamo_model_patch(table) == 0
assert [P.from_address(dst).value for dst, _ in pairs] == before
print("ok")
"""
    out = child(script, {"PLAMO_MODEL_DIR": str(d)})
    # Untied: embedding, norm, head and ten tensors per layer, one field each.
    assert out == [str(3 + 10 * 3), str(3 + 10 * 3), "ok"]
