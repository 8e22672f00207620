"""Robustness of the checkpoint parsers on malformed input, on the CPU.

The safetensors primitives (plamo_safetensors_view, plamo_find_tensor,
plamo_json_next, plamo_tensor_descriptor, plamo_parse_u64) and the
config.json reader behind plamo_checkpoint_open() are built for the host with
AddressSanitizer and UBSan (gcc, no GPU code) and fed mutated files: byte
substitutions biased to JSON punctuation and digits, deletions, truncations
and header lengths at the edges. A sanitizer finding aborts the harness; the
test checks the exit status and that valid files still parse (the seeds).
"""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

import checkpoint_writer
import plamo_hip

ROOT = Path(__file__).resolve().parents[1]
HERE = ROOT / "tests" / "parser_fuzz"
CSRC = ROOT / "plamo-3-translate.c_amd" / "csrc"

needs_gcc = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is not available")


def build(out: Path, main: str) -> Path:
    exe = out / Path(main).stem
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
           "-D__HIP_PLATFORM_AMD__", "-o", str(exe), str(HERE / main), str(HERE / "host_alloc.c"),
           str(CSRC / "checkpoint.c"), str(CSRC / "synthetic.c"), "-lm", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if r.returncode != 0 and "sanitizer" in r.stderr.lower():
        pytest.skip("the host compiler has no sanitizer runtime")
    assert r.returncode == 0, r.stderr
    return exe


@needs_gcc
def test_safetensors_primitives_under_sanitizers(tmp_path):
    exe = build(tmp_path, "safetensors_fuzz.c")
    r = subprocess.run([str(exe), "150000"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert r.stdout.startswith("done 150000 iterations")


@needs_gcc
def test_config_reader_under_sanitizers(tmp_path):
    exe = build(tmp_path, "config_fuzz.c")
    syn = plamo_hip.Synthetic(64, 2, 4, 2, 16, 96, 50, window=4, global_capacity=32, pattern=2,
                              seed=5)
    try:
        checkpoint_writer.write(tmp_path / "ck", syn, shards=2)
    finally:
        syn.close()
    before = (tmp_path / "ck" / "config.json").read_bytes()
    r = subprocess.run([str(exe), str(tmp_path / "ck"), "4000"], capture_output=True, text=True,
                       timeout=600, env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1"))
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert r.stdout.startswith("done 4000 iterations")
    assert (tmp_path / "ck" / "config.json").read_bytes() == before


@needs_gcc
def test_host_lifecycle_under_sanitizers(tmp_path):
    # Synthetic build, page-locked instances, the prefix capture/restore copies
    # and the per-layer host-mirror rows of 69-, 116- and 443-token prompts
    # (sliding layers overflowing), release and free, with the arrays' page
    # tails poisoned past each cache's capacity.
    exe = build(tmp_path, "lifecycle_asan.c")
    r = subprocess.run([str(exe), "3"], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1"))
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert r.stdout.startswith("done 3 cycles")
