"""GPU parity: the HIP backend through its C ABI against the CPU oracle.

Restates the reference's GPU-vs-CPU suite (tests/metal_decode.c) with the same
gate (relative L2 <= 1e-4, max |delta| <= 1e-5 * (1 + max |ref|)) on the
reference's fixture shapes — odd widths (hidden 7, head_dim 6), a sliding
layer with capacity 3 so the window shifts every step, growth past 128 rows,
existing prefixes, stale rotations, request resets — plus verify/commit, the
granular projection/MLP entry points and the decline/failure contract.
Every GPU call checks that no CPU fallback or error was counted.
"""

import ctypes

import numpy as np
import pytest

import prompt_cache
from parity import compare, gate, oracle_lib, plamo_hip, say, tiny

pytestmark = pytest.mark.gpu


def clean(backend):
    info = backend.info()
    assert info.errors == 0, info.note.decode()
    assert info.cpu_fallbacks == 0


SHAPES = [  # (hidden, intermediate, head_dim, global capacity) of tests/metal_decode.c:760-785
    (7, 11, 6, 4100),
    (128, 257, 128, 19),
    (128, 4097, 128, 19),
    (16, 300, 6, 264),
]


@pytest.mark.parametrize("pinned", [False, True])
@pytest.mark.parametrize("h,inter,dim,capacity", SHAPES)
def test_decode_steps(h, inter, dim, capacity, pinned):
    # pinned: host arrays the decode graph writes in place (shift and stale
    # steps still take the eager path with host mirror copies).
    say(f"decode h={h} I={inter} dim={dim} cap={capacity} pinned={pinned}")
    s = tiny(h=h, inter=inter, dim=dim, capacity=capacity)
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        steps = min(capacity, 140)
        for step in range(steps):
            if step == 17:  # stale rotations on both sides (tests/metal_decode.c:700-703)
                for inst in (a, b):
                    for i in range(2):
                        inst.rotation(i).processed_count = 0
            tok = (step * 7 + 2) % 17
            assert oracle_lib.forward(b, tok)
            assert be.forward(a, tok) == 1
            compare(a, b)
        clean(be)
        info = be.info()
        assert info.fused_decodes == steps and info.command_buffers == steps
        # A full global cache is a failure without changes (tests/metal_decode.c:720-730).
        if a.cache(1).count == capacity:
            snap = a.snapshot()
            assert be.forward(a, 3) == -1
            assert a.snapshot()["state"].tobytes() == snap["state"].tobytes()
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


# tests/metal_decode.c:239-240 (4096 only after a 2-token prefix, :249-250).
PROMPTS = [1, 2, 3, 4, 7, 8, 9, 17, 31, 32, 33, 116, 128, 129, 255, 256, 257, 443, 511, 512, 513,
           4096]


# (256, 384): every projection past 16 tokens takes the matrix-core GEMM on
# BF16 planes written by its producer (the norms, the prompt attention, and
# the gate/up GEMM's SwiGLU epilogue for down), over one and several 64-token
# tiles and K splits.
@pytest.mark.parametrize("h,inter,dim,capacity",
                         [(7, 11, 6, 4100), (128, 257, 128, 600), (256, 384, 128, 600)])
def test_prefill_then_decode(h, inter, dim, capacity):
    s = tiny(h=h, inter=inter, dim=dim, capacity=capacity)
    a, b = s.instance(), s.instance()
    be = plamo_hip.Backend(s)
    try:
        for prefix in (0, 2, 6):
            for n in PROMPTS:
                if n + prefix >= capacity or (n == 4096 and prefix != 2):
                    continue
                for final_only in (0, 1):
                    say(f"prefill h={h} prefix={prefix} n={n} final_only={final_only}")
                    a.reset()
                    b.reset()
                    for j in range(prefix):
                        assert oracle_lib.forward(a, j % 17)
                        assert oracle_lib.forward(b, j % 17)
                    for i in range(2):  # rebuild stale prefix rotations
                        a.rotation(i).processed_count = 0
                    ids = [(j * 7 + 3) % 17 for j in range(n)]
                    actual = np.zeros((n, h), np.float32)
                    expected = np.zeros((n, h), np.float32)
                    assert be.prefill(a, ids, None if final_only else actual) == 1
                    assert oracle_lib.prefill(b, ids, expected)
                    if not final_only:
                        gate(actual, expected, "all prompt states")
                    compare(a, b)
                    assert be.forward(a, 7) == 1
                    assert oracle_lib.forward(b, 7)
                    compare(a, b)
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_verify_and_commit(pinned):
    # tests/metal_decode.c:309-365. pinned: commit writes the accepted rows
    # into the host arrays from the device (no proposal copy at verify).
    s = tiny(h=128, inter=257, dim=128, capacity=40)
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        ids = [(i * 7 + 3) % 17 for i in range(16)]
        for count in (1, 2, 3, 4, 6, 8, 12, 16):
            say(f"verify count={count}")
            b.reset()
            assert oracle_lib.prefill(b, [2, 5])
            states, logits, gold = [], [], []
            for i in range(count):
                assert oracle_lib.forward(b, ids[i])
                states.append(b.state().copy())
                logits.append(b.logits().copy())
                gold.append(int(np.argmax(b.logits())))
            a.reset()
            assert be.prefill(a, [2, 5]) == 1
            before = a.snapshot()
            r, nxt = be.verify(a, ids[:count])
            assert r == 1
            after = a.snapshot()
            assert after["state"].tobytes() == before["state"].tobytes()
            assert after["logits"].tobytes() == before["logits"].tobytes()
            for la, lb in zip(after["layers"], before["layers"]):
                assert all(x.tobytes() == y.tobytes() for x, y in zip(la[:3], lb[:3]))
                assert la[3:] == lb[3:]
            assert be.commit(a, 1) == 0  # out of order
            for i in range(count):
                lg = logits[i]
                top2 = np.sort(lg)[-2:]
                if top2[1] - top2[0] >= 1e-3:
                    assert nxt[i] == gold[i], f"candidate {i}"
                assert be.commit(a, i) == 1
                gate(a.state().copy(), states[i], "verified state")
                gate(a.logits().copy(), logits[i], "verified logits")
            compare(a, b)
            assert be.commit(a, count) == 0
            if count >= 4:
                b.reset()
                assert oracle_lib.prefill(b, [2, 5])
                for i in range(3):
                    assert oracle_lib.forward(b, ids[i])
                assert oracle_lib.forward(b, 12)
                a.reset()
                assert be.prefill(a, [2, 5]) == 1
                assert be.verify(a, ids[:count])[0] == 1
                for i in range(3):
                    assert be.commit(a, i) == 1
                assert be.forward(a, 12) == 1
                assert be.commit(a, 3) == 0
                compare(a, b)
        clean(be)
        assert be.info().verification_batches > 0
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_verify_through_sliding_window(pinned):
    # Candidates past a full sliding window: commit rebases the window on the device.
    s = tiny(h=24, inter=40, dim=6, capacity=64)
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        ids = [4, 9, 1, 16, 2]
        a.reset()
        b.reset()
        assert be.prefill(a, [3, 8, 11]) == 1
        assert oracle_lib.prefill(b, [3, 8, 11])
        assert be.verify(a, ids)[0] == 1
        for i, t in enumerate(ids):
            assert oracle_lib.forward(b, t)
            assert be.commit(a, i) == 1
            compare(a, b)
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


def test_host_edits_are_uploaded():
    # Prefix restore (runtime/prompt_cache.c:62-82), draft restore
    # (runtime/draft.c:256-296: processed_count = 0) and CPU steps between GPU calls.
    s = tiny(h=128, inter=257, dim=128, capacity=100)
    a, b = s.instance(), s.instance()
    be = plamo_hip.Backend(s)
    try:
        prefix = [1, 4, 9, 16, 3, 8, 2, 11, 5, 7, 10, 6]
        assert oracle_lib.prefill(b, prefix)
        snap = b.snapshot()
        for request in range(3):
            say(f"prefix restore request {request}")
            a.reset()
            b.reset()
            a.restore(snap)
            b.restore(snap)
            body = [(request * 5 + j) % 17 for j in range(9 + request)]
            assert be.prefill(a, body) == 1
            assert oracle_lib.prefill(b, body)
            compare(a, b)
            for t in (3, 14):
                assert be.forward(a, t) == 1
                assert oracle_lib.forward(b, t)
                compare(a, b)
            # A CPU step between GPU steps writes the host KV directly.
            assert oracle_lib.forward(a, 5) and oracle_lib.forward(b, 5)
            assert be.forward(a, 6) == 1 and oracle_lib.forward(b, 6)
            compare(a, b)
            # An edit of the last V row alone (counts and K rows unchanged).
            for inst in (a, b):
                i = 1
                inst.kv(i, "v")[inst.cache(i).count - 1] *= 0.5
            assert be.forward(a, 2) == 1 and oracle_lib.forward(b, 2)
            compare(a, b)
            # An edit of an earlier row at unchanged counters: announced.
            for inst in (a, b):
                inst.kv(1, "v")[0] += 1.0
            be.invalidate()
            assert be.forward(a, 4) == 1 and oracle_lib.forward(b, 4)
            compare(a, b)
            # Draft-style restore: rows kept, rotations marked stale.
            for inst in (a, b):
                for i in range(2):
                    inst.cache(i).count -= 2
                    inst.rotation(i).processed_count = 0
                    inst.rotation(i).scale_bits = 0
            assert be.forward(a, 9) == 1 and oracle_lib.forward(b, 9)
            compare(a, b)
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_prompt_prefix_cache_flows(pinned):
    # The engine's request pattern (runtime/engine.c:337-381 prepare,
    # 451-481 translate): two template prefixes prefilled on the GPU and
    # captured at startup; each request resets the model, restores its
    # direction's prefix (runtime/prompt_cache.c, restated in
    # tests/prompt_cache.py), prefills the suffix and decodes greedily.
    # Requests alternate directions, include a miss (ids that do not start
    # with the prefix: full prefill) and a direction without a prefix. Every
    # request is checked against the oracle running the whole prompt from a
    # reset model. (A sliding window larger than the prefixes: the reference
    # captures only when every layer holds exactly the prefix rows.)
    s = tiny(h=128, inter=257, dim=128, capacity=300, window=48)
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        prefixes = [[1, 4, 9, 16, 3, 8, 2, 11, 5, 7, 10, 6], [2, 13, 5, 8, 1, 14, 9, 3, 12]]
        snaps = []
        for ids in prefixes:
            a.reset()
            assert be.prefill(a, ids) == 1
            snaps.append(prompt_cache.capture(a, ids))
            assert snaps[-1] is not None
        a.reset()
        requests = [(1, 9), (2, 14), (1, 23), (0, 11), (2, 6), (1, -1)]
        for n, (direction, extra) in enumerate(requests):
            if extra < 0:  # a miss: same length as a hit, wrong first id
                ids = [15] + prefixes[0][1:] + [4, 4, 7]
            else:
                base = prefixes[direction - 1] if direction else []
                ids = base + [(n * 7 + j * 3) % 17 for j in range(extra)]
            say(f"prefix request {n}: direction {direction}, {len(ids)} ids")
            a.reset()
            b.reset()
            cached = prompt_cache.restore(snaps[direction - 1], a, ids) if direction else 0
            expect = len(prefixes[direction - 1]) if direction and extra >= 0 else 0
            assert cached == expect
            assert be.prefill(a, ids[cached:]) == 1
            assert oracle_lib.prefill(b, ids)
            compare(a, b)
            for step in range(4):
                token = prompt_cache.greedy(b)
                assert be.forward(a, token) == 1
                assert oracle_lib.forward(b, token)
                compare(a, b)
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_template_prefix_restore_after_prepare(pinned):
    # The engine's prepare order with prefixes of the template's shape
    # (tests/test_prompt_cache.py: 12 ids, equal but for index 10, same last
    # id). After prepare the device holds prefix 1; a request in the other
    # direction restores prefix 0 with every counter and layer 0's last rows
    # unchanged, so only a full upload of the restored rows gives layer 0 the
    # right language row. Then the other direction, and the first again.
    from test_prompt_cache import TEMPLATE_PREFIXES
    s = tiny(h=128, inter=257, dim=128, capacity=300, window=48, layers=3)
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        snaps = []
        for ids in TEMPLATE_PREFIXES:
            a.reset()
            assert be.prefill(a, ids) == 1
            snaps.append(prompt_cache.capture(a, ids))
            assert snaps[-1] is not None
        a.reset()
        for n, direction in enumerate((0, 1, 0)):
            ids = list(TEMPLATE_PREFIXES[direction]) + [(n * 5 + j * 3) % 17 for j in range(7)]
            say(f"template prefix {direction} restored, request {n}")
            a.reset()
            b.reset()
            assert prompt_cache.restore(snaps[direction], a, ids) == 12
            assert be.prefill(a, ids[12:]) == 1
            assert oracle_lib.prefill(b, ids)
            compare(a, b)
            for step in range(2):
                token = prompt_cache.greedy(b)
                assert be.forward(a, token) == 1
                assert oracle_lib.forward(b, token)
                compare(a, b)
        clean(be)
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


def test_decline_and_failure_contract():
    s = tiny(h=24, inter=40, dim=6, capacity=64)
    a = s.instance()
    try:
        be = plamo_hip.Backend(s, memory=2)  # PLAMO_METAL_STREAM: nothing resident
        snap = a.snapshot()
        assert be.forward(a, 2) == 0
        assert be.prefill(a, [2, 5, 9]) == 0
        assert a.snapshot()["state"].tobytes() == snap["state"].tobytes()
        be.close()
        be = plamo_hip.Backend(None)  # no mappings: projections not resident
        assert be.forward(a, 2) == 0 and a.counts() == [0, 0]
        states = np.zeros((3, 24), np.float32)
        assert be.prefill(a, [2, 5, 9], states) == 0 and not states.any()
        assert be.prefill(a, [2, 5, 17], states) == -1  # id out of range
        assert be.forward(a, 17) == -1
        assert a.counts() == [0, 0] and not states.any()
        assert be.preload(s.mapping.base, s.mapping.bytes) == 1
        assert be.forward(a, 2) == 1 and a.counts() == [1, 1]
        r, _ = be.verify(a, [])
        assert r == 0
        be.close()
    finally:
        a.close()
        s.close()


@pytest.mark.parametrize("pinned", [False, True])
def test_device_wait_failure_is_reported(pinned):
    # runtime/metal.h:63-67: a step that fails after partial writes returns -1
    # (not retried) and counts an error. The host raises the target of the
    # decode attention's bounded wait past the KV heads and shortens it, so the
    # output-projection blocks give up and every kernel still exits.
    say(f"bounded wait gives up, pinned={pinned}")
    s = plamo_hip.Synthetic(512, 2, 16, 4, 128, 1024, 300, window=8, global_capacity=64,
                            pattern=2, seed=21)  # attention width 2048: the fused kernel
    a, b = s.instance(pinned=pinned), s.instance()
    be = plamo_hip.Backend(s)
    try:
        assert be.prefill(a, [3, 9, 27]) == 1 and oracle_lib.prefill(b, [3, 9, 27])
        assert be.forward(a, 5) == 1 and oracle_lib.forward(b, 5)
        compare(a, b)
        clean(be)
        be.debug_waits(1, 256)
        assert be.forward(a, 6) == -1
        info = be.info()
        assert info.errors == 1 and b"wait" in info.note
        be.debug_waits(0, 0)
        # The request is abandoned; the next one starts from a reset model.
        a.reset()
        b.reset()
        assert be.prefill(a, [4, 8]) == 1 and oracle_lib.prefill(b, [4, 8])
        for t in (6, 1):
            assert be.forward(a, t) == 1 and oracle_lib.forward(b, t)
            compare(a, b)
        assert be.info().errors == 1
    finally:
        be.close()
        a.close()
        b.close()
        s.close()


def test_hooks_and_trampolines(hip):
    s = tiny(h=24, inter=40, dim=6, capacity=64)
    a, b = s.instance(), s.instance()
    try:
        assert plamo_hip.hook_address("plamo_forward_kernel") == 0
        be = plamo_hip.Backend(s)
        assert plamo_hip.hook_address("plamo_forward_kernel") != 0
        assert plamo_hip.hook_address("plamo_compute_context") == be.handle
        ids = (ctypes.c_uint32 * 3)(2, 5, 9)
        assert hip.plamo_prefill(a.model_ptr, ids, 3, None) == 1
        assert oracle_lib.prefill(b, [2, 5, 9])
        assert hip.plamo_forward(a.model_ptr, 4) == 1 and oracle_lib.forward(b, 4)
        compare(a, b)
        assert hip.plamo_forward(a.model_ptr, 99) == 0  # failed hook is not retried
        info = be.info()
        assert info.fused_prefills == 1 and info.fused_decodes == 1
        be.close()
        assert plamo_hip.hook_address("plamo_forward_kernel") == 0
        assert plamo_hip.hook_address("plamo_compute_context") == 0
    finally:
        a.close()
        b.close()
        s.close()


def test_compute_hooks_through_their_pointers(oracle):
    # The reference's CPU layer calls the void matvec / matmul hooks and the
    # 1/0 mlp hook through the pointers of runtime/compute.h:8-14 with
    # plamo_compute_context as the last argument. Call them the same way.
    s = tiny(h=128, inter=257, dim=128, capacity=64)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        ctx = ctypes.c_void_p(plamo_hip.hook_address("plamo_compute_context"))
        assert ctx.value == be.handle
        matvec_t = ctypes.CFUNCTYPE(None, plamo_hip.u16p, plamo_hip.f32p, plamo_hip.f32p,
                                    ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p)
        matmul_t = ctypes.CFUNCTYPE(None, ctypes.POINTER(plamo_hip.Matmul), ctypes.c_void_p)
        mlp_t = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(plamo_hip.Mlp), plamo_hip.f32p,
                                 ctypes.c_uint64, ctypes.c_void_p)
        matvec = matvec_t(plamo_hip.hook_address("plamo_matvec_kernel"))
        matmul = matmul_t(plamo_hip.hook_address("plamo_matmul_kernel"))
        mlp_hook = mlp_t(plamo_hip.hook_address("plamo_mlp_kernel"))
        layer = a.layer(0)
        q = layer.mixer.contents.qkv.contents
        rows, cols = (q.qh + 2 * q.kh) * q.dim, q.hidden
        rng = np.random.default_rng(4)
        x = rng.standard_normal(cols).astype(np.float32)
        y, ref = np.full(rows, np.nan, np.float32), np.zeros(rows, np.float32)
        matvec(q.weight, x.ctypes.data_as(plamo_hip.f32p), y.ctypes.data_as(plamo_hip.f32p),
               rows, cols, ctx)
        oracle.oracle_matvec(q.weight, x.ctypes.data_as(plamo_hip.f32p),
                             ref.ctypes.data_as(plamo_hip.f32p), ctypes.c_uint64(rows),
                             ctypes.c_uint64(cols))
        gate(y, ref, "matvec hook")
        for tokens in (2, 24):
            x = rng.standard_normal((tokens, cols + 3)).astype(np.float32)
            y = np.full((tokens, rows + 5), np.nan, np.float32)
            ref = np.zeros_like(y)
            for out, call in ((y, lambda mm: matmul(ctypes.byref(mm), ctx)),
                              (ref, lambda mm: oracle.oracle_matmul(ctypes.byref(mm)))):
                call(plamo_hip.Matmul(q.weight, x.ctypes.data_as(plamo_hip.f32p),
                                      out.ctypes.data_as(plamo_hip.f32p), rows, cols, tokens,
                                      cols + 3, rows + 5))
            gate(y[:, :rows], ref[:, :rows], f"matmul hook tokens={tokens}")
            assert np.isnan(y[:, rows:]).all()  # the row padding is untouched
        mlp = layer.mlp.contents
        st = rng.standard_normal((3, 128)).astype(np.float32)
        ref = st.copy()
        assert mlp_hook(ctypes.byref(mlp), st.ctypes.data_as(plamo_hip.f32p), 3, ctx) == 1
        for t in range(3):
            row = ref[t].copy()
            m2 = plamo_hip.Mlp(row.ctypes.data_as(plamo_hip.f32p), mlp.pre, mlp.post, mlp.gu,
                               mlp.down, mlp.normalized, mlp.branch, mlp.scratch, 128,
                               mlp.intermediate)
            oracle.oracle_mlp_branch(ctypes.byref(m2))
            ref[t] = row
        gate(st, ref, "mlp hook")
        clean(be)
    finally:
        be.close()
        a.close()
        s.close()


def test_linear_and_mlp_entry_points(oracle):
    s = tiny(h=128, inter=257, dim=128, capacity=64)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        layer = a.layer(0)
        q = layer.mixer.contents.qkv.contents
        rows, cols = (q.qh + 2 * q.kh) * q.dim, q.hidden
        rng = np.random.default_rng(1)
        for tokens in (1, 3, 37):
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            r, y = be.linear(q.weight, x, rows)
            assert r == 1
            ref = np.zeros((tokens, rows), np.float32)
            mm = plamo_hip.Matmul(q.weight, x.ctypes.data_as(plamo_hip.f32p),
                                  ref.ctypes.data_as(plamo_hip.f32p), rows, cols, tokens, cols,
                                  rows)
            oracle.oracle_matmul(ctypes.byref(mm))
            gate(y, ref, f"linear tokens={tokens}")
        mlp = layer.mlp.contents
        for tokens in (1, 5):
            st = rng.standard_normal((tokens, 128)).astype(np.float32)
            ref = st.copy()
            assert be.lib.plamo_metal_mlp(be.handle, ctypes.byref(mlp),
                                          st.ctypes.data_as(plamo_hip.f32p), tokens) == 1
            for t in range(tokens):
                row = ref[t].copy()
                m2 = plamo_hip.Mlp(row.ctypes.data_as(plamo_hip.f32p), mlp.pre, mlp.post, mlp.gu,
                                   mlp.down, mlp.normalized, mlp.branch, mlp.scratch, 128,
                                   mlp.intermediate)
                oracle.oracle_mlp_branch(ctypes.byref(m2))
                ref[t] = row
            gate(st, ref, f"mlp tokens={tokens}")
        clean(be)
    finally:
        be.close()
        a.close()
        s.close()
