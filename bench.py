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
    """runtime/engine.c:46-55 request reset, then runtime/prompt_cache.c:62-82.
    The arrays' numpy views are made once per instance (they never move), so
    the timed restore is the copies and counter stores the C engine makes,
    without the cost of building 3 x layers ctypes views per call."""
    views = getattr(inst, "_restore_views", None)
    if views is None:
        views = [(inst.kv(i, "k"), inst.kv(i, "v"), inst.kv(i, "rot"), inst.cache(i),
                  inst.rotation(i)) for i in range(inst.model.count)]
        inst._restore_views = views
    inst.reset()
    for (k, v, rot, scale), (vk, vv, vr, cache, rotation) in zip(snap, views):
        vk[:rows] = k
        vv[:rows] = v
        vr[:rows] = rot
        cache.count = rows
        rotation.processed_count = rows
        rotation.scale_bits = scale


def prefill_flop_parts(cfg: dict, prefix: int, tokens: int) -> tuple[float, float]:
    """(linear, attention) FLOP of a prompt: 2 per weight per token for the
    projections (the last layer's O/MLP and the head run for the final row
    only), 4 * dim per visible key per query head for Q K^T and P V."""
    h, d, qh, kh, inter, L = (cfg[k] for k in ("hidden", "dim", "qh", "kh", "intermediate",
                                                 "layers"))
    qkv = (qh + 2 * kh) * d * h
    rest = h * qh * d + 3 * inter * h
    linear = 2.0 * (qkv * tokens * L + rest * (tokens * (L - 1) + 1) + cfg["vocab"] * h)
    keys = sum(prefix + t + 1 for t in range(tokens))
    attention = 4.0 * qh * d * keys * L
    return linear, attention


def prefill_flop(cfg: dict, prefix: int, tokens: int) -> float:
    return sum(prefill_flop_parts(cfg, prefix, tokens))


def prefill_roofline(cfg: dict, prefix: int, tokens: int, ttft_ms: float) -> dict:
    """The prefill against the ceilings of the instructions it runs: the
    projections on the BF16 matrix cores with three products per FP32 input
    (2.5 PFLOP/s / 3), attention on the FP32 matrix cores (157.3 TFLOP/s),
    and the weights crossing HBM once (8 TB/s) as a floor."""
    linear, attention = prefill_flop_parts(cfg, prefix, tokens)
    mfma_ms = (linear / (SPLIT_BF16_CEILING_TFLOPS * 1e12) +
               attention / (FP32_MFMA_PEAK_TFLOPS * 1e12)) * 1e3
    hbm_ms = plamo_hip.weight_bytes_per_step(cfg) / (HBM_PEAK_GBPS * 1e9) * 1e3
    bound_ms = max(mfma_ms, hbm_ms)
    flop = linear + attention
    return {"tokens_after_prefix": tokens, "flop": flop, "linear_flop": linear,
            "attention_flop": attention, "achieved_TFLOPs": round(flop / ttft_ms / 1e9, 2),
            "mfma_bound_ms": round(mfma_ms, 3), "hbm_bound_ms": round(hbm_ms, 3),
            "bound": "mfma" if mfma_ms >= hbm_ms else "hbm",
            "frac": round(bound_ms / ttft_ms, 4),
            "note": "frac = max(linear / 833.3 TFLOP/s (split BF16) + attention / 157.3 TFLOP/s "
                    "(FP32 MFMA), weights / 8 TB/s) / TTFT"}


def host_threads() -> tuple[int, int]:
    """(threads the CPU baseline uses, nproc). The threads are this process's
    CPU share: its affinity set, capped by OMP_NUM_THREADS when the host sets
    it (a shared GPU box allots each GPU a slice of its cores)."""
    nproc = os.cpu_count() or 1
    share = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        share = min(share, int(cap))
    return max(1, share), nproc


def smaller_config_baseline(lib, name: str, threads: int) -> dict:
    """C2 / C3 on the C oracle: decode s/step and the 128-token prefill, at N
    threads and at 1 thread, rows split over threads as
    runtime/parallel.c:35-48. The whole 128-token
    prompt is prefilled at N threads; at 1 thread its first two layers are,
    scaled by the layer count. Decode steps follow the prompt greedily: three
    at N threads, one at 1 thread."""
    c = dict(plamo_hip.CONFIGS[name])
    syn = plamo_hip.Synthetic(**c, seed=20261202, threads=threads)
    inst = syn.instance()
    try:
        prompt = np.random.default_rng(11).integers(0, c["vocab"], size=128).astype(np.uint32)
        ids = (ctypes.c_uint32 * 128)(*prompt.tolist())

        def prefill(n_threads, layers):
            inst.reset()
            view = plamo_hip.Model.from_buffer_copy(inst.model)
            view.count = layers
            lib.oracle_set_threads(n_threads)
            start = time.perf_counter()
            if not lib.oracle_prefill(ctypes.byref(view), ids, 128, None):
                raise RuntimeError(f"{name}: oracle prefill failed")
            return time.perf_counter() - start

        L = c["layers"]
        p_1 = prefill(1, 2) * L / 2
        p_n = prefill(threads, L)
        token = int(lib.oracle_argmax(inst.model.logits, inst.model.vocab))
        step = {}
        for n_threads, count in ((threads, 3), (1, 1)):
            lib.oracle_set_threads(n_threads)
            start = time.perf_counter()
            for _ in range(count):
                if not lib.oracle_forward(inst.model_ptr, token):
                    raise RuntimeError(f"{name}: oracle decode failed")
                token = int(lib.oracle_argmax(inst.model.logits, inst.model.vocab))
            step[str(n_threads)] = round((time.perf_counter() - start) / count, 4)
        return {"decode_s_per_step": step,
                "prefill_128_s": {str(threads): round(p_n, 3), "1": round(p_1, 2)},
                "sample": f"128-token prompt: all {L} layers at {threads} threads, 2 of {L} at "
                          f"1 thread scaled; decode: 3 steps at {threads} threads, 1 at 1 "
                          f"thread"}
    finally:
        inst.close()
        syn.close()


def cpu_baseline(inst: plamo_hip.Instance, token: int, seconds: float, cfg: dict, prompt,
                 snap) -> dict:
    """The C oracle on the host cores (rows split as runtime/parallel.c:35-48), on bounded
    samples of the same workloads: decode steps of the model continuing the
    GPU's sequence on the same host arrays at N threads and at 1 thread, the
    C1 layer step at both, and the 128-token prompt's prefill
    (12-token prefix restored, 116 tokens) over the first layers of the model
    at N threads and over its first layer at 1 thread, scaled to every layer.
    Rows are split over threads in groups of 24 as runtime/parallel.c:35-48;
    the prefill runs its projections token-blocked as the reference's prompt
    path does (src/batch.s, src/matmul8x3.s)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib  # the checker's CPU path; test infrastructure, not the product

    lib = oracle_lib.load()
    threads, nproc = host_threads()
    model = inst.model_ptr

    def decode(n_threads, budget, max_steps):
        nonlocal token
        lib.oracle_set_threads(n_threads)
        steps, start = 0, time.perf_counter()
        while True:
            if not lib.oracle_forward(model, token):
                raise RuntimeError("oracle decode failed")
            token = int(lib.oracle_argmax(inst.model.logits, inst.model.vocab))
            steps += 1
            elapsed = time.perf_counter() - start
            if elapsed >= budget or steps >= max_steps:
                return steps, elapsed

    steps_n, t_n = decode(threads, seconds * 0.3, 64)
    steps_1, t_1 = decode(1, seconds * 0.2, 64)

    # C1: one layer (hidden 2048, 16/4 heads of 128, MLP 8192), 512 rows of
    # pre-filled KV; one decode step of the layer stack.
    c1 = dict(plamo_hip.CONFIGS["c1"])
    syn1 = plamo_hip.Synthetic(**c1, embedding_std=1.0, seed=101)
    layer_ms = {}
    try:
        for n_threads in (threads, 1):
            one = syn1.instance()
            one.fill_kv(512, 7)
            lib.oracle_set_threads(n_threads)
            assert lib.oracle_forward(one.model_ptr, 3)  # rebuilds the rotations
            times = []
            for step in range(5):
                start = time.perf_counter()
                assert lib.oracle_forward(one.model_ptr, step % c1["vocab"])
                times.append(time.perf_counter() - start)
            layer_ms[str(n_threads)] = round(float(np.median(times)) * 1e3, 3)
            one.close()
    finally:
        syn1.close()

    # Prefill of the 116-token body over the first `layers` layers (a model
    # descriptor with a shorter layer list over the same arrays), scaled.
    def prefill(n_threads, layers):
        restore(inst, snap, PREFIX)
        view = plamo_hip.Model.from_buffer_copy(inst.model)
        view.count = layers
        ids = (ctypes.c_uint32 * (128 - PREFIX))(*prompt[PREFIX:128])
        lib.oracle_set_threads(n_threads)
        start = time.perf_counter()
        if not lib.oracle_prefill(ctypes.byref(view), ids, 128 - PREFIX, None):
            raise RuntimeError("oracle prefill failed")
        return time.perf_counter() - start

    L = cfg["layers"]
    sample_n = min(L, 4)
    p_n = prefill(threads, sample_n)
    p_1 = prefill(1, 1)
    smaller = {name: smaller_config_baseline(lib, name, threads)
               for name in ("c2", "c3") if name != cfg["name"]}
    return {"value": steps_n / t_n, "unit": "tok/s", "cores": threads, "kind": "port",
            "nproc": nproc,
            "one_thread_tok_s": steps_1 / t_1,
            "c1_layer_step_ms": layer_ms,
            **{f"{name}": v for name, v in smaller.items()},
            "prefill_128_s": {str(threads): round(p_n * L / sample_n, 2),
                              "1": round(p_1 * L, 2),
                              "measured": f"{sample_n} of {L} layers at {threads} threads "
                                          f"({p_n:.2f} s), 1 of {L} at 1 thread "
                                          f"({p_1:.2f} s), scaled by layer count"},
            "sample": f"{cfg['name']} decode: {steps_n} greedy steps at {threads} threads "
                      f"({t_n:.1f} s) and {steps_1} at 1 thread ({t_1:.1f} s), continuing "
                      f"the GPU run's sequence; C1 layer step: median of 5; prefill: the "
                      f"116-token body of the 128-token prompt after the restored prefix. "
                      f"Scalar C oracle (gcc -O2 -ffp-contract=off; prompt projections "
                      f"token-blocked with AVX2 fused multiply-adds, same bits), rows split "
                      f"over threads as runtime/parallel.c:35-48; {threads} threads = this "
                      f"process's CPU share of the {nproc}-CPU host"}


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


def verify_sweep(args) -> dict:
    """The target's batched candidate verification alone (plamo_metal_verify,
    runtime/metal_model.m:829-830 semantics) on the C5 model (tied head) after
    a 455-token prompt: the median time of one verify of T candidates for
    each T in --verify-tokens, beside the decode step of the same model. One
    to five candidates stream the projections through the token GEMV, more
    through the matrix-core skinny GEMM."""
    tcfg = dict(plamo_hip.CONFIGS["c5"])
    tied = tcfg.pop("tied", 0)
    threads = host_threads()[0]
    target = plamo_hip.Synthetic(**tcfg, tied=tied, seed=20261201, threads=threads)
    inst = target.instance(pinned=True)
    be = plamo_hip.Backend(target)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, tcfg["vocab"], size=455).astype(np.uint32).tolist()
    if be.prefill(inst, prompt) != 1:
        raise RuntimeError(be.info().note.decode())
    verify_ms = {}
    for n in [int(x) for x in args.verify_tokens.split(",") if x]:
        times = []
        for _ in range(5):
            start = time.perf_counter()
            ok, _ = be.verify(inst, prompt[:n])
            times.append((time.perf_counter() - start) * 1e3)
            if ok != 1:
                raise RuntimeError(be.info().note.decode())
        verify_ms[str(n)] = round(float(np.median(times[1:])), 3)
        log(f"verify({n}) {verify_ms[str(n)]:.3f} ms (runs {[round(t, 2) for t in times]})")
    token = int(np.argmax(inst.logits()))
    steps = []
    for _ in range(6):
        start = time.perf_counter()
        if be.forward(inst, token) != 1:
            raise RuntimeError(be.info().note.decode())
        steps.append((time.perf_counter() - start) * 1e3)
        token = int(np.argmax(inst.logits()))
    info = be.info()
    assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    be.close()
    inst.close()
    target.close()
    return {"metric": "batched verify latency (31B-class target)", "unit": "ms",
            "higher_is_better": False, "n_gpus": 1, "dtype": "fp32",
            "data": "synthetic (seeded BF16 weights ~N(0,0.02); uniform random prompt ids)",
            "config": {"workload": "c5 target (tied head), 455-token prompt, one verify of "
                                   "T candidates per call"},
            "verify_ms": verify_ms,
            "decode_step_ms": round(float(np.median(steps[1:])), 3)}


def embed_draft(target: "plamo_hip.Instance", draft: "plamo_hip.Instance", mix: float) -> int:
    """The draft-weight policy of the speculative line: the target contains
    the draft, and its own layers past the draft's are mixed in at `mix`.
    Both models are tied (head = embedding) and share the layer layout rules
    (sliding/global pattern, RoPE tables, attention scales). Before the
    target's weights are uploaded:
      - the embedding (= head) is the draft's in the first `hd` columns and
        zero in the others;
      - the first draft.count layers are the draft's layers and zero
        elsewhere: the draft's query heads of KV group g become target query
        heads tg*g.. (the target's group is larger), its KV heads the
        target's first KV heads, its O, gate/up and down blocks the matching
        sub-blocks; q/k norms are copied;
      - every RMSNorm weight over the hidden dims is rescaled in the draft's
        dims so that (w + offset) / rms over the wider vector equals the
        draft's when the other dims are zero:
        w_t = (w_d + offset) * sqrt(hd / ht) - offset (offsets: 1 pre-norms and
        the final norm, 0.2 post-mixer, 0.0894 post-MLP; src/layer.s:51,
        src/model.s:111);
      - the target's later layers keep their own random weights, and their two
        post-norms (which set the size of what a layer adds to the residual
        stream, whatever its weights) are scaled to `mix` times their own:
        w = mix * (w + offset) - offset.
    With mix 0 the target computes the draft's function exactly (up to the
    rounding of the rescaled norms); with mix 1 its later layers are ordinary
    random layers. Returns the bytes written."""
    tm, dm = target.model, draft.model
    ht, hd, V = tm.hidden, dm.hidden, tm.vocab
    assert dm.vocab == V and dm.count <= tm.count and hd <= ht

    def view(ptr, *shape):
        n = int(np.prod(shape))
        return np.ctypeslib.as_array(ctypes.cast(ptr, plamo_hip.u16p), shape=(n,)).reshape(shape)

    def f32(bits):
        return (bits.astype(np.uint32) << 16).view(np.float32)

    def bf16(x):
        # Round to nearest even (finite inputs).
        b = np.ascontiguousarray(x, np.float32).view(np.uint32)
        return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)

    ratio = np.float32(np.sqrt(hd / ht))
    written = 0

    def put(dst, src):
        nonlocal written
        dst[...] = src
        written += dst.nbytes

    def norm(dst_ptr, src_ptr, offset):
        dst, src = view(dst_ptr, ht), view(src_ptr, hd)
        put(dst[:hd], bf16((f32(src) + np.float32(offset)) * ratio - np.float32(offset)))
        put(dst[hd:], bf16(np.full(ht - hd, -offset, np.float32)))

    emb = view(tm.embedding, V, ht)
    put(emb[:, :hd], view(dm.embedding, V, hd))
    put(emb[:, hd:], 0)
    norm(tm.norm, dm.norm, 1.0)
    for i in range(tm.count):
        tl = tm.layers[i].contents
        tx, tp = tl.mixer.contents, tl.mlp.contents
        tq = tx.qkv.contents
        if i >= dm.count:
            for ptr, offset in ((tl.post, 0.2), (tp.post, 0.08944271909999159)):
                w = view(ptr, ht)
                put(w, bf16(np.float32(mix) * (f32(w) + np.float32(offset)) - np.float32(offset)))
            continue
        dl = dm.layers[i].contents
        dx, dp = dl.mixer.contents, dl.mlp.contents
        dq = dx.qkv.contents
        d, tg, dg = tq.dim, tq.qh // tq.kh, dq.qh // dq.kh
        assert dq.dim == d and dq.kh <= tq.kh and dg <= tg
        norm(tl.pre, dl.pre, 1.0)
        norm(tl.post, dl.post, 0.2)
        norm(tp.pre, dp.pre, 1.0)
        norm(tp.post, dp.post, 0.08944271909999159)
        put(view(tq.qn, d), view(dq.qn, d))
        put(view(tq.kn, d), view(dq.kn, d))
        tw = view(tq.weight, tq.qh + 2 * tq.kh, d, ht)
        dw = view(dq.weight, dq.qh + 2 * dq.kh, d, hd)
        to = view(tx.weight, ht, tq.qh, d)
        do = view(dx.weight, hd, dq.qh, d)
        put(tw, 0)
        put(to, 0)
        for g in range(dq.kh):
            for r in range(dg):
                put(tw[tg * g + r, :, :hd], dw[dg * g + r])
                put(to[:hd, tg * g + r, :], do[:, dg * g + r, :])
            put(tw[tq.qh + g, :, :hd], dw[dq.qh + g])
            put(tw[tq.qh + tq.kh + g, :, :hd], dw[dq.qh + dq.kh + g])
        ti, di = tp.intermediate, dp.intermediate
        tgu, dgu = view(tp.gu, 2 * ti, ht), view(dp.gu, 2 * di, hd)
        tdn = view(tp.down, ht, ti)
        put(tgu, 0)
        put(tdn, 0)
        put(tgu[:di, :hd], dgu[:di])
        put(tgu[ti:ti + di, :hd], dgu[di:])
        put(tdn[:hd, :di], view(dp.down, hd, di))
    return written


def speculative(args) -> dict:
    """the 31B-class model (C5, tied embedding/head) with
    the 0.8B-class model (C2 shape) as the in-process draft, 4 draft tokens
    per verify (a 5-token batched verify), a 455-token prompt and 128 greedy
    tokens through the engine's decode loop (runtime/engine.c:514-566,
    plamo_hip_decode). Speculation must leave the tokens unchanged.

    Draft-weight policy: with unrelated random weights a draft is never right
    (acceptance 0), so by default the draft is embedded in the target
    (embed_draft) and the target's own later layers are mixed in at
    --draft-mix. Random-weight models fall into short greedy cycles (the line
    reports how many distinct tokens the target produced), which is what makes
    the acceptance high when the two models share the cycle; the acceptance is
    a property of this synthetic pair, and the per-round component times and
    the rate projected at other acceptances are reported beside it."""
    tcfg = dict(plamo_hip.CONFIGS["c5"])
    tied = tcfg.pop("tied", 0)
    dcfg = dict(plamo_hip.CONFIGS["c2"])
    threads = host_threads()[0]
    mix = args.draft_mix
    t0 = time.perf_counter()
    target = plamo_hip.Synthetic(**tcfg, tied=tied, seed=20261201, threads=threads)
    if mix is None:
        source = plamo_hip.Synthetic(**dcfg, seed=20261202, threads=threads)
    else:
        source = plamo_hip.Synthetic(**dcfg, tied=1, seed=20261202, threads=threads)
    log(f"synthetic c5 ({target.mapping.bytes / 1e9:.1f} GB) and c2 draft "
        f"({source.mapping.bytes / 1e9:.1f} GB) in {time.perf_counter() - t0:.1f} s")
    inst, d_inst = target.instance(pinned=True), source.instance(pinned=True)
    if mix is not None:
        t0 = time.perf_counter()
        written = embed_draft(inst, d_inst, mix)
        log(f"draft embedded in the target ({written / 1e9:.2f} GB written, later layers "
            f"mixed in at {mix}) in {time.perf_counter() - t0:.1f} s")
    be = plamo_hip.Backend(target)
    draft = plamo_hip.Draft(source, d_inst)
    block, max_tokens = 5, 128
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, tcfg["vocab"], size=455).astype(np.uint32).tolist()

    def run(with_draft, n):
        inst.reset()
        if be.prefill(inst, prompt) != 1:
            raise RuntimeError(be.info().note.decode())
        return plamo_hip.decode(be, inst, prompt, n, draft=draft if with_draft else None,
                                block=block)

    run(False, 4)  # graph capture and workspace growth
    run(True, 8)
    plain, r0, _ = run(False, max_tokens)
    before = draft.stats()
    spec, r, alive = run(True, max_tokens)
    if not alive:
        raise RuntimeError("the draft failed during the run")
    after = draft.stats()
    plain_tps = r0.completion_tokens / r0.decode_seconds
    spec_tps = r.completion_tokens / r.decode_seconds
    log(f"plain {plain_tps:.2f} tok/s ({r0.decode_seconds / r0.decode_steps * 1e3:.3f} ms/step); "
        f"speculative {spec_tps:.2f} tok/s, {r.accepted_tokens}/{r.proposed_tokens} accepted in "
        f"{r.speculative_batches} verifies")

    # Component times: a 5-token verify of the target, a draft step, a commit.
    inst.reset()
    assert be.prefill(inst, prompt) == 1
    verify_ms = []
    for _ in range(6):
        start = time.perf_counter()
        ok, _ = be.verify(inst, plain[:block])
        verify_ms.append((time.perf_counter() - start) * 1e3)
        assert ok == 1
    start = time.perf_counter()
    assert be.commit(inst, 0) == 1
    commit_ms = (time.perf_counter() - start) * 1e3
    assert draft.reset_ids(prompt) == 1
    draft_ms = []
    for _ in range(6):
        start = time.perf_counter()
        ids = draft.propose(plain[0], block)
        draft_ms.append((time.perf_counter() - start) * 1e3 / max(1, len(ids) - 1))
        assert ids and draft.accept(1)
    step_ms = r0.decode_seconds / r0.decode_steps
    t_verify, t_draft = float(np.median(verify_ms[1:])), float(np.median(draft_ms[1:]))
    log(f"verify({block}) {t_verify:.3f} ms, draft step {t_draft:.3f} ms, commit {commit_ms:.3f} ms")
    projected = {}
    for alpha in (0.5, 0.7, 0.9):
        tokens = sum(alpha ** i for i in range(block))  # 1 + expected accepted drafts
        cost = (block - 1) * t_draft + t_verify + tokens * commit_ms
        projected[str(alpha)] = round(tokens / cost * 1e3, 2)
    info = be.info()
    assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
    result = {
        "metric": "speculative decode tok/s + acceptance (31B-class target, 0.8B-class draft)",
        "value": round(spec_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "fp32",
        "data": ("synthetic (seeded BF16 weights ~N(0,0.02); target and draft unrelated; "
                 "uniform random prompt ids)" if mix is None else
                 "synthetic (seeded BF16 weights ~N(0,0.02); the tied c2-shape draft is the "
                 "target's first 16 layers, the target's other 44 layers are its own, mixed "
                 f"into the residual stream at {mix:g}; uniform random prompt ids)"),
        "draft_policy": ("independent" if mix is None else
                         f"embedded draft, later target layers mixed in at {mix:g}"),
        "config": {"workload": "c5 target (tied head) + c2-shape draft in process; 455-token "
                               "prompt, 128 greedy tokens, 4 draft tokens per verify",
                   "block": block, "max_tokens": max_tokens},
        "tokens_identical_to_plain": spec == plain,
        "distinct_tokens": len(set(plain)),
        "completion_tokens": r.completion_tokens,
        "acceptance": round(r.accepted_tokens / max(1, r.proposed_tokens), 4),
        "verifies": r.speculative_batches,
        "draft_device_rewinds": after.device_rewinds - before.device_rewinds,
        "draft_host_restores": after.host_restores - before.host_restores,
        "draft_seconds": round(r.draft_seconds, 4),
        "plain_tok_s": round(plain_tps, 2),
        "components_ms": {"target_decode_step": round(step_ms * 1e3, 3),
                          "verify_5": round(t_verify, 3), "draft_step": round(t_draft, 3),
                          "commit": round(commit_ms, 3)},
        "projected_tok_s_at_acceptance": projected,
    }
    draft.close()
    be.close()
    for x in (inst, d_inst):
        x.close()
    target.close()
    source.close()
    return result


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c4", choices=sorted(plamo_hip.CONFIGS))
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ttft-sizes", default="81,128,455",
                    help="comma-separated prompt lengths for TTFT ('' skips)")
    ap.add_argument("--kernel-reps", type=int, default=50)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run device-to-device copies of MIB MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--speculative", action="store_true",
                    help="measure BASELINE configs[4] (C5 target, 0.8B-class draft) instead")
    ap.add_argument("--verify", action="store_true",
                    help="time the C5 target's batched verify alone, per candidate count")
    ap.add_argument("--verify-tokens", default="1,2,3,4,5,6,8,16")
    ap.add_argument("--draft-mix", type=float, default=0.3,
                    help="--speculative: the draft is the target's first layers, and the "
                         "target's later layers add this fraction of their usual share to the "
                         "residual stream; negative: independent draft and target weights")
    ap.add_argument("--prefill-only", action="store_true",
                    help="measure TTFT for --ttft-sizes only (one JSON line, no decode)")
    ap.add_argument("--ttft-runs", type=int, default=12)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} is not supported)",
              file=sys.stderr)
        return 2
    if args.speculative:
        if args.draft_mix is not None and args.draft_mix < 0:
            args.draft_mix = None
        print(json.dumps(speculative(args)), flush=True)
        return 0
    if args.verify:
        print(json.dumps(verify_sweep(args)), flush=True)
        return 0
    cfg = dict(plamo_hip.CONFIGS[args.config])
    cfg["name"] = args.config
    tied = cfg.pop("tied", 0)
    shape = {k: cfg[k] for k in ("hidden", "layers", "qh", "kh", "dim", "intermediate", "vocab")}
    t0 = time.perf_counter()
    syn = plamo_hip.Synthetic(**shape, tied=tied, seed=20261201, threads=host_threads()[0])
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
    # Median of the last 8 of 12 runs: the first runs after loading 16 GB of
    # weights can be slowed by host-side work (page handling of the pinned
    # arrays the restore and its upload touch).
    ttft = {}
    for n in [int(x) for x in args.ttft_sizes.split(",") if x]:
        times = []
        for _ in range(args.ttft_runs):
            start = time.perf_counter()
            restore(inst, snap, PREFIX)
            if be.prefill(inst, prompt[PREFIX:n]) != 1:
                raise RuntimeError(be.info().note.decode())
            times.append(time.perf_counter() - start)
        ttft[n] = float(np.median(times[min(4, len(times) - 1):])) * 1e3
        log(f"TTFT {n} tokens: {ttft[n]:.2f} ms (runs {[round(t * 1e3, 2) for t in times]})")
    if args.prefill_only:
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
        be.close()
        inst.close()
        syn.close()
        print(json.dumps({
            "metric": "prefill TTFT (12-token prefix restored)", "unit": "ms",
            "higher_is_better": False, "n_gpus": 1, "dtype": "fp32",
            "data": "synthetic (seeded BF16 weights ~N(0,0.02), uniform random prompt ids)",
            "config": {"workload": f"{args.config}: prompt body after a {PREFIX}-token prefix"},
            "ttft_ms": {str(k): round(v, 3) for k, v in ttft.items()},
            "prefill_roofline": {str(n): prefill_roofline(plamo_hip.CONFIGS[args.config], PREFIX,
                                                          n - PREFIX, ttft[n]) for n in ttft}}),
            flush=True)
        return 0

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

    # Per-kernel HIP-event timings on the backend stream (layer 1, whose QKV
    # prologue adds the previous layer's MLP branch as every layer past the
    # first does, and the head).
    kernels = {}
    timed_layer = 1 if inst.model.count > 1 else 0
    names = {plamo_hip.KERNEL_QKV: "qkv_gemv", plamo_hip.KERNEL_O: "o_gemv",
             plamo_hip.KERNEL_GATE_UP: "gate_up_swiglu_gemv", plamo_hip.KERNEL_DOWN: "down_gemv",
             plamo_hip.KERNEL_HEAD: "head_gemv", plamo_hip.KERNEL_ATTENTION: "decode_attention"}
    for which, name in names.items():
        ms, nbytes = be.time_kernel(inst, timed_layer, which, args.kernel_reps)
        kernels[name] = {"us": round(ms * 1e3, 2), "bytes": int(nbytes),
                         "GBps": round(nbytes / ms / 1e6, 1)}
        log(f"kernel {name}: {ms * 1e3:.2f} us, {nbytes / ms / 1e6:.0f} GB/s")
    dom = kernels["gate_up_swiglu_gemv"]

    if args.copy_calibration:
        copy_calibration(args.copy_calibration << 20)
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
        "prefill_roofline": {str(n): prefill_roofline(plamo_hip.CONFIGS[args.config], PREFIX,
                                                      n - PREFIX, ttft[n]) for n in ttft},
        "roofline": {"bound": "hbm", "kernel": "gemv_regp_kernel<8,2,SWIGLU> (gate/up + SwiGLU)",
                     "achieved": dom["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBPS, 4), "traffic": traffic},
        "kernels": kernels,
    }
    if not args.no_cpu:
        log("CPU baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(inst, token, args.cpu_seconds, cfg, prompt, snap)
        cb = result["cpu_baseline"]
        log(f"CPU baseline: {cb['value']:.3f} tok/s at {cb['cores']} threads, "
            f"{cb['one_thread_tok_s']:.3f} at 1; C1 layer {cb['c1_layer_step_ms']} ms; "
            f"prefill 128 {cb['prefill_128_s']}")
    be.close()
    inst.close()
    syn.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
