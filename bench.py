#!/usr/bin/env python3
"""Benchmark of the MI355X token-loop backend on BASELINE.json's headline config.

Workload (configs[3], "8B-class headline"): hidden 4096, 32 layers, 32 query /
8 KV heads of 128, MLP 16384, vocab 100000, seeded synthetic BF16 weights
~N(0, 0.02) (16.4 GB streamed per decode step, all resident in HBM). Each
request restores a 12-token prefix KV from a snapshot (the engine's prompt
cache, runtime/prompt_cache.c:62-82), prefills the rest of the prompt, then
decodes greedily with the host argmax between steps, exactly the engine's
loop (runtime/engine.c:516-592). A "step" is one decode token:
plamo_metal_forward() + plamo_argmax().

Reported on one JSON line: decode tok/s (value), the step's share of the HBM
roofline (weight bytes per step / step time / 8 TB/s), TTFT at 81/128/455
tokens, the dominant kernel's roofline measured with HIP events on the
backend stream, and the C oracle's decode rate on the host cores (a
reported baseline: the reference's own CPU path is AArch64/Darwin assembly).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "plamo-3-translate.c_amd"))

import plamo_hip  # noqa: E402

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
# The prompt GEMM runs exact FP32 products as three BF16 passes on the
# 2.5 PFLOP/s BF16 matrix cores: its own ceiling is a third of that.
SPLIT_BF16_CEILING_TFLOPS = round(2500.0 / 3, 1)
PREFIX = 12                   # fixed translation-template prefix (runtime/engine.c:358-381)


def log(*args):
    print("[bench]", *args, file=sys.stderr, flush=True)


def capture(inst: plamo_hip.Instance, rows: int):
    """runtime/prompt_cache.c:15-56: K, V and rotated K of the prefix rows."""
    snap = []
    for i in range(inst.model.count):
        snap.append((inst.kv(i, "k")[:rows].copy(), inst.kv(i, "v")[:rows].copy(),
                     inst.kv(i, "rot")[:rows].copy(), inst.rotation(i).scale_bits))
    return snap


def restore(inst: plamo_hip.Instance, snap, rows: int):
    """runtime/engine.c:46-55 request reset, then runtime/prompt_cache.c:62-82."""
    inst.reset()
    for i, (k, v, rot, scale) in enumerate(snap):
        inst.kv(i, "k")[:rows] = k
        inst.kv(i, "v")[:rows] = v
        inst.kv(i, "rot")[:rows] = rot
        inst.cache(i).count = rows
        inst.rotation(i).processed_count = rows
        inst.rotation(i).scale_bits = scale


def prefill_flop(cfg: dict, prefix: int, tokens: int) -> float:
    """Linear-layer FLOP of a prompt (2 per weight per token; the last layer's
    O/MLP and the head run for the final row only) plus attention FLOP."""
    h, d, qh, kh, inter, L = (cfg[k] for k in ("hidden", "dim", "qh", "kh", "intermediate",
                                                 "layers"))
    qkv = (qh + 2 * kh) * d * h
    rest = h * qh * d + 3 * inter * h
    linear = 2.0 * (qkv * tokens * L + rest * (tokens * (L - 1) + 1) + cfg["vocab"] * h)
    keys = sum(prefix + t + 1 for t in range(tokens))
    attention = 4.0 * qh * d * keys * L
    return linear + attention


def cpu_baseline(inst: plamo_hip.Instance, token: int, seconds: float, cfg: dict):
    """Oracle decode steps on the host cores, continuing the GPU's sequence on
    the same (coherent) host arrays."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib  # the checker's CPU path; test infrastructure, not the product

    lib = oracle_lib.load()
    threads = max(1, min(16, os.cpu_count() or 1))
    lib.oracle_set_threads(threads)
    steps, start = 0, time.perf_counter()
    while True:
        if not lib.oracle_forward(inst.model_ptr, token):
            raise RuntimeError("oracle decode failed")
        token = int(lib.oracle_argmax(inst.model.logits, inst.model.vocab))
        steps += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds or steps >= 64:
            break
    return {"value": steps / elapsed, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} greedy decode steps of the {cfg['name']} model by the scalar C "
                      f"oracle (gcc -O2 -ffp-contract=off, row-split over {threads} threads as "
                      f"runtime/parallel.c:35-48), continuing the GPU run's sequence; "
                      f"{elapsed:.1f} s"}


def copy_calibration(nbytes: int, reps: int = 5):
    """Device-to-device copies of a known size through the HIP runtime the
    library links (reads nbytes, writes nbytes per dispatch)."""
    hip = ctypes.CDLL("libamdhip64.so.7")  # the soname libplamo_hip.so links
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(src), ctypes.c_size_t(nbytes)) or \
            hip.hipMalloc(ctypes.byref(dst), ctypes.c_size_t(nbytes)):
        raise RuntimeError("hipMalloc failed")
    try:
        hip.hipMemset(src, 0, ctypes.c_size_t(nbytes))
        hip.hipDeviceSynchronize()
        start = time.perf_counter()
        for _ in range(reps):
            if hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3):  # hipMemcpyDeviceToDevice
                raise RuntimeError("hipMemcpy failed")
        hip.hipDeviceSynchronize()
        elapsed = time.perf_counter() - start
        log(f"copy calibration: {reps} x {nbytes >> 20} MiB device copies, "
            f"{2 * nbytes * reps / elapsed / 1e9:.0f} GB/s read+write (host-timed)")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)


def measured_traffic():
    """HBM bytes per launch of the gate/up GEMV from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    path = ROOT / "profiles" / "gate_up_gemv_c4_hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c4", choices=sorted(plamo_hip.CONFIGS))
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ttft-sizes", default="81,128,455",
                    help="comma-separated prompt lengths for TTFT ('' skips)")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run device-to-device copies of MIB MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} is not supported; shard design is in DESIGN.md)",
              file=sys.stderr)
        return 2
    cfg = dict(plamo_hip.CONFIGS[args.config])
    cfg["name"] = args.config
    tied = cfg.pop("tied", 0)
    shape = {k: cfg[k] for k in ("hidden", "layers", "qh", "kh", "dim", "intermediate", "vocab")}
    t0 = time.perf_counter()
    syn = plamo_hip.Synthetic(**shape, tied=tied, seed=20261201, threads=min(16, os.cpu_count() or 1))
    log(f"synthetic {args.config} weights: {syn.mapping.bytes / 1e9:.2f} GB in "
        f"{time.perf_counter() - t0:.1f} s")
    inst = syn.instance(pinned=True)
    t0 = time.perf_counter()
    be = plamo_hip.Backend(syn)
    log(f"weights resident in HBM in {time.perf_counter() - t0:.1f} s on "
        f"{be.info().device.decode()}")
    lib = plamo_hip.load()
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg["vocab"], size=455).astype(np.uint32).tolist()
    assert be.prefill(inst, prompt[:PREFIX]) == 1
    snap = capture(inst, PREFIX)

    # TTFT: restore the prefix snapshot, prefill the body, logits on the host.
    ttft = {}
    for n in [int(x) for x in args.ttft_sizes.split(",") if x]:
        times = []
        for _ in range(4):
            start = time.perf_counter()
            restore(inst, snap, PREFIX)
            if be.prefill(inst, prompt[PREFIX:n]) != 1:
                raise RuntimeError(be.info().note.decode())
            times.append(time.perf_counter() - start)
        ttft[n] = float(np.median(times[1:])) * 1e3
        log(f"TTFT {n} tokens: {ttft[n]:.2f} ms (runs {[round(t * 1e3, 2) for t in times]})")

    # Decode: prompt of args.prompt tokens, then greedy steps.
    restore(inst, snap, PREFIX)
    assert be.prefill(inst, prompt[PREFIX:args.prompt]) == 1
    logits_ptr, vocab = inst.model.logits, inst.model.vocab
    token = int(lib.plamo_argmax(logits_ptr, vocab))
    for _ in range(args.warmup):
        assert be.forward(inst, token) == 1
        token = int(lib.plamo_argmax(logits_ptr, vocab))
    info0 = be.info()
    be.maintain()
    start = time.perf_counter()
    for _ in range(args.steps):
        if be.forward(inst, token) != 1:
            raise RuntimeError(be.info().note.decode())
        token = int(lib.plamo_argmax(logits_ptr, vocab))
    be.maintain()
    elapsed = time.perf_counter() - start
    info1 = be.info()
    ms_step = elapsed / args.steps * 1e3
    gpu_ms_step = (info1.gpu_seconds - info0.gpu_seconds) / args.steps * 1e3
    step_bytes = plamo_hip.weight_bytes_per_step(plamo_hip.CONFIGS[args.config])
    log(f"decode: {ms_step:.3f} ms/step wall, {gpu_ms_step:.3f} ms/step GPU, "
        f"{step_bytes / ms_step / 1e6:.0f} GB/s of weights")
    assert info1.errors == 0 and info1.cpu_fallbacks == 0, info1.note.decode()

    # Per-kernel HIP-event timings on the backend stream (layer 0 + head).
    kernels = {}
    names = {plamo_hip.KERNEL_QKV: "qkv_gemv", plamo_hip.KERNEL_O: "o_gemv",
             plamo_hip.KERNEL_GATE_UP: "gate_up_swiglu_gemv", plamo_hip.KERNEL_DOWN: "down_gemv",
             plamo_hip.KERNEL_HEAD: "head_gemv", plamo_hip.KERNEL_ATTENTION: "decode_attention"}
    for which, name in names.items():
        ms, nbytes = be.time_kernel(inst, 0, which, args.kernel_reps)
        kernels[name] = {"us": round(ms * 1e3, 2), "bytes": int(nbytes),
                         "GBps": round(nbytes / ms / 1e6, 1)}
        log(f"kernel {name}: {ms * 1e3:.2f} us, {nbytes / ms / 1e6:.0f} GB/s")
    dom = kernels["gate_up_swiglu_gemv"]

    if args.copy_calibration:
        copy_calibration(args.copy_calibration << 20)
    ttft_flop = prefill_flop(plamo_hip.CONFIGS[args.config], PREFIX, 128 - PREFIX)
    traffic = measured_traffic()
    result = {
        "metric": "decode tok/s + % HBM roofline (8B-class, bs=1); prefill TTFT @128 tok",
        "value": round(args.steps / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded BF16 weights ~N(0,0.02), uniform random prompt ids)",
        "config": {"workload": f"{args.config}: greedy decode, batch 1, after a "
                               f"{args.prompt}-token prompt with a {PREFIX}-token prefix KV "
                               f"restored", "hidden": cfg["hidden"], "layers": cfg["layers"],
                   "heads": f"{cfg['qh']}/{cfg['kh']}x{cfg['dim']}",
                   "intermediate": cfg["intermediate"], "vocab": cfg["vocab"]},
        "hbm_roofline_step": {"bytes_per_step": step_bytes,
                              "achieved_GBps": round(step_bytes / ms_step / 1e6, 1),
                              "peak_GBps": HBM_PEAK_GBPS,
                              "frac": round(step_bytes / ms_step / 1e6 / HBM_PEAK_GBPS, 4),
                              "gpu_ms_per_step": round(gpu_ms_step, 4)},
        "ttft_ms": {str(k): round(v, 3) for k, v in ttft.items()},
        "prefill_roofline_128": ({"flop": ttft_flop,
                                  "achieved_TFLOPs": round(ttft_flop / ttft[128] / 1e9, 2),
                                  "peak_TFLOPs": FP32_MFMA_PEAK_TFLOPS,
                                  "frac": round(ttft_flop / ttft[128] / 1e9 /
                                                FP32_MFMA_PEAK_TFLOPS, 4),
                                  "split_bf16_ceiling_TFLOPs": SPLIT_BF16_CEILING_TFLOPS,
                                  "frac_of_split_bf16": round(ttft_flop / ttft[128] / 1e9 /
                                                              SPLIT_BF16_CEILING_TFLOPS, 4)}
                                 if 128 in ttft else None),
        "roofline": {"bound": "hbm", "kernel": "gemv_regp_kernel<8,2,SWIGLU> (gate/up + SwiGLU)",
                     "achieved": dom["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBPS, 4), "traffic": traffic},
        "kernels": kernels,
    }
    if not args.no_cpu:
        log("CPU baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(inst, token, args.cpu_seconds, cfg)
        log(f"CPU baseline: {result['cpu_baseline']['value']:.3f} tok/s")
    be.close()
    inst.close()
    syn.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
