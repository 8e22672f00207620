"""Pins the CPU oracle (oracle/plamo_oracle.c) before it is trusted as the checker.

Every test restates a known answer the reference itself relies on — its
golden data (src/rope_constants.s), its known-answer C tests (tests/*.c), or a
closed form the mathematics fixes — and each is chosen so that a plausible
slip (dropped term, wrong index or sign, wrong reduction order) fails it:

  exp / softmax / SwiGLU      tests/activation.c:7-26 (libm bound, closed forms)
  sincos                      tests/trig.c:9-18 (libm bound, same angle stream)
  RoPE frequencies            src/rope_constants.s (bit-exact golden tables)
  RoPE table                  tests/rope_table.c:10-23 (libm bound)
  matvec reduction order      tests/matvec_reference.s:8-31 (a cancellation case
                              whose value depends on the 4-lane tree)
  matvec values               float64 product with the FP32 summation bound
  matmul == matvec            tests/matmul.c:36-69 (bit-exact invariant)
  RMSNorm, QKV, MLP           tests/qkv.c, tests/model.c (float64 closed forms)
  attention / GQA             tests/attention.c:13-70
  cache append / rotation     tests/cache_reference.s semantics, incremental ==
                              full rotation (bit-exact)
  mixer/layer/forward/prefill tests/mixer.c:65-140 (symmetric closed forms)
  prefill == sequential       tests/prefill.c (bit-exact invariant)
  argmax, FNV-1a              src/token.s:37-63, published FNV-1a vectors
"""

import ctypes
import json
import math
from ctypes import POINTER, c_float, c_uint16, c_uint32
from pathlib import Path

import numpy as np
import pytest

import oracle_lib
import plamo_hip

GOLDEN = Path(__file__).resolve().parent / "golden" / "rope_constants.json"
f32p = POINTER(c_float)
u16p = POINTER(c_uint16)


def fp(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def u16(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint16))


def P(a):
    return a.ctypes.data_as(f32p if a.dtype == np.float32 else u16p)


def bf(bits):
    return float((np.asarray([bits], np.uint32) << 16).view(np.float32)[0])


def test_exp_against_libm(oracle):
    # tests/activation.c:7-13: relative error <= 5e-6 on [-86, 87].
    for i in range(-8600, 8701, 7):
        x = np.float32(i / 100.0)
        a = oracle.oracle_exp(float(x))
        assert abs(a / math.exp(float(x)) - 1) <= 5e-6, x
    assert oracle.oracle_exp(0.0) == 1.0
    assert oracle.oracle_exp(-87.5) == 0.0
    assert math.isinf(oracle.oracle_exp(88.5))
    assert oracle.oracle_exp(float("nan")) == 0.0


def test_exp_polynomial_terms(oracle):
    """The reference's exponential (src/activation.s, tests/activation_reference.s:
    8-50) reduces x = n ln2 + r, |r| <= ln2/2, and evaluates a degree-7
    polynomial. Its worst relative error over [-86, 87] is 3.0e-7 (FP32
    rounding); a dropped r^6 term would add up to 1.7e-6, so 4e-7 pins it. The
    r^7 term is worth at most 8.4e-8 relative at |r| = ln2/2, within the
    rounding of a single value, but not on average: at inputs with r in
    [0.30, 0.345] the signed error a/exp(x) - 1 averages zero, and without the
    r^7 term it would average about -5e-8 (that term's mean over the range)."""
    worst = 0.0
    for i in range(-860000, 870001, 97):
        x = float(np.float32(i / 10000.0))
        worst = max(worst, abs(oracle.oracle_exp(x) / math.exp(x) - 1))
    assert worst <= 4e-7
    ln2 = math.log(2.0)
    signed = []
    for k in range(-120, 121):
        for j in range(40):
            x = float(np.float32(k * ln2 + 0.30 + 0.045 * j / 40))
            r = x - round(x / ln2) * ln2
            if 0.30 <= r <= 0.345 and -86 < x < 87:
                signed.append(oracle.oracle_exp(x) / math.exp(x) - 1)
    assert len(signed) > 5000
    assert abs(float(np.mean(signed))) < 2e-8


def test_softmax_and_swiglu(oracle):
    # tests/activation.c:14-26
    x = fp([1000, 1001, 999, -1000])
    oracle.oracle_softmax(P(x), 4)
    s = math.exp(0) + math.exp(1) + math.exp(-1)
    assert abs(x[0] - 1 / s) <= 1e-6 and abs(x[1] - math.e / s) <= 1e-6
    assert abs(x[2] - math.exp(-1) / s) <= 1e-6 and x[3] == 0
    h = fp([-100, -2, 0, 2, 100, 1, 2, 3, 4, 5])
    out = fp(np.zeros(5))
    oracle.oracle_swiglu(P(h), P(out), 5)
    for i in range(5):
        g, u = float(h[i]), float(h[i + 5])
        assert abs(out[i] - g / (1 + math.exp(-g)) * u) <= 1e-5


def test_sincos_against_libm(oracle):
    # tests/trig.c:9-18, same angle stream (|angle| up to 2^22).
    out = fp([0, 0])
    rng = 7
    worst = 0.0
    for _ in range(20000):
        rng = (rng * 6364136223846793005 + 1) % 2**64
        a = ((rng >> 20) - (1 << 43)) / 2097152.0
        oracle.oracle_sincos(a, P(out))
        worst = max(worst, abs(out[0] - math.sin(a)), abs(out[1] - math.cos(a)))
    assert worst <= 2e-7
    oracle.oracle_sincos(0.0, P(out))
    assert out[0] == 0 and out[1] == 1


def test_rope_frequencies_match_golden_tables(oracle):
    # src/rope_constants.s, generated by tools/rope_constants.py:21-70.
    g = json.loads(GOLDEN.read_text())["tables"]
    local = fp(np.zeros(64))
    oracle.oracle_rope_frequencies(10000.0, 64, 0, 0, 0, 0, 0, P(local))
    assert local.view(np.uint32).tolist() == g["plamo_rope_local"]["bits"]
    glob = fp(np.zeros(64))
    oracle.oracle_rope_frequencies(1e6, 64, 1, 256.0, 4096.0, 32.0, 1.0, P(glob))
    assert glob.view(np.uint32).tolist() == g["plamo_rope_global"]["bits"]
    conc = np.float32(oracle.oracle_rope_concentration(1, 256.0))
    assert [int(conc.view(np.uint32))] == g["plamo_rope_global_scale"]["bits"]
    assert oracle.oracle_rope_concentration(0, 0.0) == 1.0


def test_synthetic_builder_frequencies_match_golden(hip):
    # The product's own frequency generator (plamo_synthetic.c) is pinned the same way.
    g = json.loads(GOLDEN.read_text())["tables"]
    s = plamo_hip.Synthetic(256, 8, 2, 1, 128, 64, 32)
    try:
        local = np.ctypeslib.as_array(hip.plamo_synthetic_frequencies(s.handle, 0), shape=(64,))
        glob = np.ctypeslib.as_array(hip.plamo_synthetic_frequencies(s.handle, 7), shape=(64,))
        assert local.view(np.uint32).tolist() == g["plamo_rope_local"]["bits"]
        assert glob.view(np.uint32).tolist() == g["plamo_rope_global"]["bits"]
    finally:
        s.close()


def test_rope_table_against_libm(oracle):
    # tests/rope_table.c:10-23
    g = json.loads(GOLDEN.read_text())["tables"]
    for name, scale in (("plamo_rope_local", 1.0),
                        ("plamo_rope_global", g["plamo_rope_global_scale"]["values"][0])):
        f = fp(g[name]["values"])
        c, s = fp(np.zeros(64)), fp(np.zeros(64))
        for pos in (0, 1, 2048, 4096, 262143):
            oracle.oracle_rope_table(P(f), pos, 64, P(c), P(s), scale)
            a = (np.float32(pos) * f).astype(np.float64)
            assert np.max(np.abs(c - np.cos(a) * scale)) <= 4e-7
            assert np.max(np.abs(s - np.sin(a) * scale)) <= 4e-7
        assert np.all(f[1:] < f[:-1]) and np.all(f > 0)


def test_matvec_reduction_tree(oracle):
    # tests/matvec_reference.s: lanes k mod 4, then (a0+a1)+(a2+a3), then an
    # FMA tail. With x = [1e8, 1, -1e8, 1] the tree gives 0 (1e8+1 and -1e8+1
    # both round back), a sequential sum would give 1.
    w = u16([0x3F80] * 5)
    x = fp([1e8, 1, -1e8, 1, 1])
    y = fp([0])
    oracle.oracle_matvec(P(w), P(x), P(y), 1, 4)
    assert y[0] == 0.0
    oracle.oracle_matvec(P(w), P(x), P(y), 1, 5)
    assert y[0] == 1.0  # tail element is fused onto the reduced sum


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 2), (5, 3), (7, 4), (9, 11), (31, 64),
                                       (64, 257), (24, 4096)])
def test_matvec_values(oracle, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    w = u16(rng.integers(0, 65536, size=rows * cols) & 0xBFFF)  # finite BF16
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(rows, cols)
    x = fp(rng.standard_normal(cols))
    y = fp(np.zeros(rows))
    oracle.oracle_matvec(P(w), P(x), P(y), rows, cols)
    exact = wf @ x.astype(np.float64)
    bound = (cols + 2) * 2.0 ** -24 * (np.abs(wf) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y - exact) <= bound)


def test_matmul_is_matvec_per_token(oracle):
    # tests/matmul.c:36-69 and src/matmul.s:1-4: bit-identical to matvec.
    rng = np.random.default_rng(3)
    rows, cols, tokens = 17, 37, 5
    w = u16(rng.integers(0, 65536, size=rows * cols) & 0xBFFF)
    x = fp(rng.standard_normal((tokens, cols + 3)))
    y = fp(np.zeros((tokens, rows + 2)))
    mm = plamo_hip.Matmul(P(w), P(x), P(y), rows, cols, tokens, cols + 3, rows + 2)
    oracle.oracle_matmul(ctypes.byref(mm))
    for t in range(tokens):
        yt = fp(np.zeros(rows))
        xt = fp(x[t, :cols])
        oracle.oracle_matvec(P(w), P(xt), P(yt), rows, cols)
        assert y[t, :rows].tobytes() == yt.tobytes()


@pytest.mark.parametrize("threads", [1, 4])
def test_blocked_matmul_is_matvec_per_token(oracle, threads):
    # The prefill's token-blocked products against the per-token definition,
    # bit for bit: ragged token counts around the 4-token and 64-token blocks,
    # widths with a sequential tail, shapes large enough for the row-split pool.
    rng = np.random.default_rng(5)
    oracle.oracle_set_threads(threads)
    try:
        for rows, cols, tokens in ((17, 37, 5), (300, 1027, 2), (300, 1027, 65), (96, 4099, 130),
                                   (1000, 512, 63)):
            w = u16(rng.integers(0, 65536, size=rows * cols) & 0xBFFF)
            x = fp(rng.standard_normal((tokens, cols + 3)))
            y = fp(np.zeros((tokens, rows + 2)))
            ref = fp(np.zeros((tokens, rows + 2)))
            args = (P(w), P(x))
            mm = plamo_hip.Matmul(*args, P(y), rows, cols, tokens, cols + 3, rows + 2)
            oracle.oracle_matmul_blocked(ctypes.byref(mm))
            mr = plamo_hip.Matmul(*args, P(ref), rows, cols, tokens, cols + 3, rows + 2)
            oracle.oracle_matmul(ctypes.byref(mr))
            assert y.tobytes() == ref.tobytes(), (rows, cols, tokens)
    finally:
        oracle.oracle_set_threads(1)


def test_rmsnorm_closed_form(oracle):
    x = fp([0.5, -1.25, 3.0, 2.0, -0.75])
    w = u16([0x3F00, 0xBF00, 0, 0x3F80, 0x4000])
    y = fp(np.zeros(5))
    oracle.oracle_rmsnorm(P(x), P(w), P(y), 5, 1e-6, 0.2)
    xd = x.astype(np.float64)
    inv = 1 / math.sqrt(np.mean(xd * xd) + 1e-6)
    ref = xd * inv * (np.array([bf(v) for v in w]) + np.float64(np.float32(0.2)))
    assert np.max(np.abs(y - ref)) <= 2e-6
    oracle.oracle_rmsnorm(P(x), P(w), P(x), 5, 1e-6, 0.2)  # in place
    assert x.tobytes() == y.tobytes()


def test_qkv_head_norm(oracle):
    # tests/qkv.c:17-47
    H, QH, KH, D = 5, 4, 2, 3
    R = (QH + 2 * KH) * D
    vals = [0xBF80, 0, 0x3F00, 0x3F80]
    w = u16([vals[(i + i // 7) % 4] for i in range(R * H)])
    qn, kn = u16([0x3F00, 0xBF00, 0]), u16([0, 0x3F80, 0xBF00])
    inp = fp([(i - 2) * 0.2 for i in range(H)])
    out = fp(np.zeros(R))
    d = plamo_hip.Qkv(P(inp), P(w), P(qn), P(kn), P(out), H, QH, KH, D)
    oracle.oracle_qkv(ctypes.byref(d))
    wf = np.array([bf(v) for v in w]).reshape(R, H)
    ref = wf @ inp.astype(np.float64)
    for head in range(QH + KH):
        seg = ref[head * D:(head + 1) * D]
        nw = qn if head < QH else kn
        ref[head * D:(head + 1) * D] = seg / math.sqrt(np.mean(seg * seg) + 1e-6) * (
            1 + np.array([bf(v) for v in nw]))
    assert np.max(np.abs(out - ref)) <= 2e-6


def test_mlp_and_branch(oracle):
    # tests/model.c:22-97
    H, I = 5, 7
    vals = [0xBF80, 0xBF00, 0, 0x3F00, 0x3F80]
    gu = u16([vals[(i * 7 + i // 5) % 5] for i in range(2 * I * H)])
    down = u16([vals[(i * 3 + i // 7) % 5] for i in range(H * I)])
    inp = fp([(i - 2) * 0.125 for i in range(H)])
    out, scratch = fp(np.zeros(H)), fp(np.zeros(2 * I))
    guf = np.array([bf(v) for v in gu]).reshape(2 * I, H)
    df = np.array([bf(v) for v in down]).reshape(H, I)

    def mlp64(x):
        g, u = guf[:I] @ x, guf[I:] @ x
        return df @ (g / (1 + np.exp(-g)) * u)

    oracle.oracle_mlp(P(gu), P(down), P(inp), P(out), P(scratch), H, I)
    assert np.max(np.abs(out - mlp64(inp.astype(np.float64)))) <= 1e-5
    pre, post = u16(vals), u16(vals[::-1])
    state = fp([(i - 2) * 0.3 for i in range(H)])
    s64 = state.astype(np.float64)
    n = s64 / math.sqrt(np.mean(s64 * s64) + 1e-6) * (1 + np.array([bf(v) for v in pre]))
    br = mlp64(n)
    ref = s64 + br / math.sqrt(np.mean(br * br) + 1e-6) * (
        np.array([bf(v) for v in post]) + 1 / 5 ** 1.5)
    norm, branch = fp(np.zeros(H)), fp(np.zeros(H))
    b = plamo_hip.Mlp(P(state), P(pre), P(post), P(gu), P(down), P(norm), P(branch), P(scratch),
                      H, I)
    oracle.oracle_mlp_branch(ctypes.byref(b))
    assert np.max(np.abs(state - ref)) <= 2e-5


def test_attention_and_gqa(oracle):
    # tests/attention.c:13-70
    D, N, S = 5, 4, 15
    q = fp([(j - 2) * 0.3 for j in range(D)])
    k = fp([((i * 7) % 19 - 9) * 0.1 for i in range(N * S)])
    v = fp([((i * 3) % 17 - 8) * 0.2 for i in range(N * S)])
    out, scores = fp(np.zeros(D)), fp(np.zeros(N))
    kq = k.ctypes.data + D * 4
    vq = v.ctypes.data + D * 4
    oracle.oracle_attention_head(P(q), ctypes.cast(kq, f32p), ctypes.cast(vq, f32p), P(out),
                                 P(scores), N, D, S)
    kk = k.astype(np.float64).reshape(N, S)[:, D:2 * D]
    vv = v.astype(np.float64).reshape(N, S)[:, D:2 * D]
    p = np.exp(kk @ q.astype(np.float64) / math.sqrt(D))
    assert np.max(np.abs(out - (p / p.sum()) @ vv)) <= 2e-6
    oracle.oracle_attention_head(P(q), ctypes.cast(k.ctypes.data + (S + D) * 4, f32p),
                                 ctypes.cast(v.ctypes.data + (S + D) * 4, f32p), P(out),
                                 P(scores), 1, D, S)
    assert out.tobytes() == v[S + D:S + 2 * D].tobytes()
    QH, KH, GD, GN = 6, 2, 4, 3
    gq = fp([(i % 7 - 3) * 0.2 for i in range(QH * GD)])
    gk = fp([(i % 11 - 5) * 0.3 for i in range(GN * KH * GD)])
    gv = fp([(i % 13 - 6) * 0.1 for i in range(GN * KH * GD)])
    go, gs = fp(np.zeros(QH * GD)), fp(np.zeros(GN))
    g = plamo_hip.Gqa(P(gq), P(gk), P(gv), P(go), P(gs), GN, GD, QH, KH)
    oracle.oracle_gqa(ctypes.byref(g))
    K = gk.astype(np.float64).reshape(GN, KH, GD)
    V = gv.astype(np.float64).reshape(GN, KH, GD)
    for h in range(QH):
        kv = h // (QH // KH)
        p = np.exp(K[:, kv] @ gq[h * GD:(h + 1) * GD].astype(np.float64) / math.sqrt(GD))
        assert np.max(np.abs(go[h * GD:(h + 1) * GD] - (p / p.sum()) @ V[:, kv])) <= 2e-6


def test_cache_append_semantics(oracle):
    # tests/cache_reference.s:8-56
    width = 3
    k, v = fp(np.zeros(2 * width)), fp(np.zeros(2 * width))
    c = plamo_hip.Cache(P(k), P(v), 2, 0, width, 1)
    rows = [fp([r, r + 0.5, r + 0.25]) for r in range(1, 4)]
    for r in rows:
        assert oracle.oracle_cache_append(ctypes.byref(c), P(r), P(r * 2))
    # Sliding: the oldest row was dropped and the rest moved up by one row.
    assert c.count == 2
    assert k.tolist() == rows[1].tolist() + rows[2].tolist()
    assert v.tolist() == (rows[1] * 2).tolist() + (rows[2] * 2).tolist()
    c.sliding = 0
    before = k.copy()
    assert not oracle.oracle_cache_append(ctypes.byref(c), P(rows[0]), P(rows[0]))
    assert c.count == 2 and k.tobytes() == before.tobytes()
    c.count = 3
    assert not oracle.oracle_cache_append(ctypes.byref(c), P(rows[0]), P(rows[0]))


def test_rotation_cache_incremental_equals_full(oracle):
    # src/cache_rope.s:11-75: reusing rows only when exactly one was appended
    # at the same concentration must give the full recomputation's bits.
    heads, dim, cap = 2, 8, 6
    width = heads * dim
    rng = np.random.default_rng(5)
    k, v = fp(np.zeros(cap * width)), fp(np.zeros(cap * width))
    freq = fp([1.0, 0.3, 0.05, 0.001])
    outs = []
    for mode in range(2):
        c = plamo_hip.Cache(P(k), P(v), cap, 0, width, 0)
        rot = fp(np.zeros(cap * width))
        cs, sn = fp(np.zeros(dim // 2)), fp(np.zeros(dim // 2))
        r = plamo_hip.Rotation(ctypes.pointer(c), P(rot), P(freq), P(cs), P(sn), heads, dim, 0, 0)
        rng = np.random.default_rng(5)
        for step in range(cap):
            row = fp(rng.standard_normal(width))
            oracle.oracle_cache_append(ctypes.byref(c), P(row), P(row))
            if mode == 1:
                r.processed_count = 0  # force full recomputation every step
            oracle.oracle_cache_rope_cached(ctypes.byref(r), 1.25)
            assert r.processed_count == c.count
            assert r.scale_bits == int(np.float32(1.25).view(np.uint32))
        outs.append(rot.copy())
        # The scratch holds the table of row count-1 (used to rotate Q).
        a = (np.float32(cap - 1) * freq).astype(np.float64)
        assert np.max(np.abs(cs - np.cos(a) * 1.25)) <= 4e-7
    assert outs[0].tobytes() == outs[1].tobytes()
    # Closed form of one rotated row: split-half rotation at its row position.
    kk = k.reshape(cap, heads, dim).astype(np.float64)
    rr = outs[0].reshape(cap, heads, dim)
    for row in range(cap):
        a = row * freq.astype(np.float64)
        c_, s_ = np.cos(a) * 1.25, np.sin(a) * 1.25
        x0, x1 = kk[row, :, :dim // 2], kk[row, :, dim // 2:]
        assert np.max(np.abs(rr[row, :, :dim // 2] - (x0 * c_ - x1 * s_))) <= 1e-5
        assert np.max(np.abs(rr[row, :, dim // 2:] - (x1 * c_ + x0 * s_))) <= 1e-5


class TinyModel:
    """The hand-built model of tests/mixer.c:65-140 (H=2, QH=2, KH=1, D=2)."""

    def __init__(self):
        self.keep = []
        self.input = fp([2, 3])
        self.qkvout, self.k, self.v, self.rk = fp(np.zeros(8)), *(fp(np.zeros(4)) for _ in range(3))
        self.freq, self.cos, self.sin = fp([1]), fp([0]), fp([0])
        self.a, self.scores, self.out = fp(np.zeros(4)), fp(np.zeros(2)), fp(np.zeros(2))
        w = np.zeros(16, np.uint16)
        for r in range(8):
            w[r * 2 + r % 2] = 0x3F80
        self.w, self.norm = u16(w), u16([0, 0])
        self.ow = u16([0x3F80, 0, 0x3F80, 0, 0, 0x3F80, 0, 0x3F80])
        self.q = plamo_hip.Qkv(P(self.input), P(self.w), P(self.norm), P(self.norm), P(self.qkvout),
                               2, 2, 1, 2)
        self.c = plamo_hip.Cache(P(self.k), P(self.v), 2, 0, 2, 0)
        self.r = plamo_hip.Rotation(ctypes.pointer(self.c), P(self.rk), P(self.freq), P(self.cos),
                                    P(self.sin), 1, 2, 0, 0)
        self.g = plamo_hip.Gqa(None, None, None, P(self.a), P(self.scores), 0, 2, 2, 1)
        self.m = plamo_hip.Mixer(ctypes.pointer(self.q), ctypes.pointer(self.c),
                                 ctypes.pointer(self.r), ctypes.pointer(self.g), P(self.ow),
                                 P(self.out), 2)


def test_mixer_layer_forward_prefill_closed_forms(oracle):
    t = TinyModel()
    # V projection is the identity; O sums duplicated V heads.
    assert oracle.oracle_mixer(ctypes.byref(t.m), 1.0) and t.c.count == 1
    assert t.out.tolist() == [4.0, 6.0]
    assert oracle.oracle_mixer(ctypes.byref(t.m), 1.0) and t.c.count == 2
    assert np.max(np.abs(t.out - [4, 6])) <= 1e-6
    assert not oracle.oracle_mixer(ctypes.byref(t.m), 1.0) and t.c.count == 2
    state = fp([2, 2])
    normalized, mout, mn, mb, ms = fp([0, 0]), fp([0, 0]), fp([0, 0]), fp([0, 0]), fp(np.zeros(4))
    gu = u16([0x3F80, 0, 0, 0x3F80, 0x3F80, 0, 0, 0x3F80])
    down = u16([0x3F80, 0, 0, 0x3F80])
    mlp = plamo_hip.Mlp(P(state), P(t.norm), P(t.norm), P(gu), P(down), P(mn), P(mb), P(ms), 2, 2)
    layer = plamo_hip.Layer(P(state), P(t.norm), P(t.norm), P(normalized), P(mout),
                            ctypes.pointer(t.m), ctypes.pointer(mlp), 2)
    t.c.count = 0
    assert oracle.oracle_layer(ctypes.byref(layer), 1.0) and t.c.count == 1
    pre = 2 / math.sqrt(4 + 1e-6)
    mix = 2 * pre
    after = 2 + mix / math.sqrt(mix * mix + 1e-6) * 0.2
    mp = after / math.sqrt(after * after + 1e-6)
    ml = mp / (1 + math.exp(-mp)) * mp
    expected = after + ml / math.sqrt(ml * ml + 1e-6) / 5 ** 1.5
    assert np.max(np.abs(state - expected)) <= 2e-6
    t.c.count = t.c.capacity
    old = float(state[0])
    assert not oracle.oracle_layer(ctypes.byref(layer), 1.0) and state[0] == old
    emb = u16([0x4000, 0x4000, 0x3F80, 0x3F80])
    head = u16([0x3F80, 0, 0, 0x3F80])
    final, logits, scales = fp([0, 0]), fp([0, 0]), fp([1])
    layers = (POINTER(plamo_hip.Layer) * 1)(ctypes.pointer(layer))
    model = plamo_hip.Model(P(emb), 2, 2, P(state), layers, 1, P(scales), P(t.norm), P(final),
                            P(head), P(logits))
    mp_ = ctypes.pointer(model)
    t.c.count = 0
    assert oracle.oracle_forward(mp_, 0) and t.c.count == 1
    expected_logit = expected / math.sqrt(expected * expected + 1e-6)
    assert np.max(np.abs(logits - expected_logit)) <= 2e-6
    prev = float(state[0])
    assert not oracle.oracle_forward(mp_, 2) and state[0] == prev and t.c.count == 1
    t.c.count = 0
    logits[0], final[0] = 123, 456
    assert oracle.oracle_forward_hidden(mp_, 0) and t.c.count == 1
    assert logits[0] == 123 and final[0] == 456
    t.c.count = 0
    ids = (c_uint32 * 2)(0, 0)
    states = fp(np.zeros(4))
    assert oracle.oracle_prefill(mp_, ids, 2, P(states)) and t.c.count == 2
    assert np.max(np.abs(logits - expected_logit)) <= 2e-6
    # Layer-major prefill equals token-major forward on distinct inputs.
    emb[2], emb[3] = 0x3F80, 0x4040
    t.c.count = 0
    assert oracle.oracle_forward_hidden(mp_, 0) and oracle.oracle_forward(mp_, 1)
    seq_logits, seq_state = logits.copy(), state.copy()
    t.c.count = 0
    ids = (c_uint32 * 2)(0, 1)
    assert oracle.oracle_prefill(mp_, ids, 2, P(states))
    assert np.max(np.abs(logits - seq_logits)) <= 1e-6
    assert np.max(np.abs(state - seq_state)) <= 1e-6


def test_prefill_bitwise_equals_sequential_forward(oracle, hip):
    # tests/prefill.c: layer-major prefill == token-major decode, bit for bit,
    # including a sliding layer (capacity 3) that shifts during the prompt.
    s = plamo_hip.Synthetic(24, 3, 4, 2, 6, 40, 19, window=2, global_capacity=64, pattern=3,
                            seed=11)
    a, b = s.instance(), s.instance()
    try:
        ids = [3, 7, 1, 18, 0, 5, 9]
        for t in ids:
            assert oracle_lib.forward(a, t)
        states = fp(np.zeros((len(ids), 24)))
        assert oracle_lib.prefill(b, ids, states)
        assert a.logits().tobytes() == b.logits().tobytes()
        assert a.state().tobytes() == b.state().tobytes()
        assert states[-1].tobytes() == b.state().tobytes()
        for i in range(3):
            assert a.counts() == b.counts()
            n = a.cache(i).count
            for which in ("k", "v", "rot"):
                assert a.kv(i, which)[:n].tobytes() == b.kv(i, which)[:n].tobytes()
        assert a.cache(0).count == 3  # window 2 -> capacity 3, shifted
    finally:
        a.close()
        b.close()
        s.close()


def test_long_prefill_bitwise_equals_sequential_forward(oracle, hip):
    # The same invariant past one 64-token block of the blocked products, with
    # widths whose projections run on the row-split pool (4 threads).
    s = plamo_hip.Synthetic(256, 2, 8, 2, 32, 1000, 300, window=40, global_capacity=128,
                            pattern=2, seed=12)
    a, b = s.instance(), s.instance()
    oracle.oracle_set_threads(4)
    try:
        ids = [(7 * j + 3) % 300 for j in range(70)]
        for t in ids:
            assert oracle_lib.forward(a, t)
        states = fp(np.zeros((len(ids), 256)))
        assert oracle_lib.prefill(b, ids, states)
        assert a.logits().tobytes() == b.logits().tobytes()
        assert a.state().tobytes() == b.state().tobytes()
        for i in range(2):
            assert a.counts() == b.counts()
            n = a.cache(i).count
            for which in ("k", "v", "rot"):
                assert a.kv(i, which)[:n].tobytes() == b.kv(i, which)[:n].tobytes()
        assert a.cache(0).count == 41  # window 40 -> capacity 41, shifted
    finally:
        oracle.oracle_set_threads(1)
        a.close()
        b.close()
        s.close()


def test_argmax_and_hashes(oracle, hip):
    for lib, fn in ((oracle, "oracle_argmax"), (hip, "plamo_argmax")):
        argmax = getattr(lib, fn)
        x = fp([1, 3, 3, 2])
        assert argmax(P(x), 4) == 1
        x = fp([float("-inf"), -5])
        assert argmax(P(x), 2) == 1
        x = fp([1, float("nan"), 9])
        assert argmax(P(x), 3) == 2**64 - 1
        assert argmax(P(x), 0) == 2**64 - 1
    # The library's vectorized argmax against the oracle's sequential scan:
    # ties (first index wins, also 0.0 after -0.0), NaN anywhere, ragged tails.
    rng = np.random.default_rng(5)
    cases = []
    for n in list(range(1, 70)) + [100000]:
        x = fp(rng.integers(-4, 5, size=n))  # many ties
        cases.append(x)
        y = fp(rng.standard_normal(n))
        cases.append(y)
        if n > 2:
            z = y.copy()
            z[rng.integers(0, n)] = np.nan
            cases.append(z)
    cases.append(fp([-0.0, 0.0, -1.0]))
    cases.append(fp([0.0, -0.0]))
    cases.append(fp([float("-inf")] * 33))
    for x in cases:
        assert hip.plamo_argmax(P(x), x.size) == oracle.oracle_argmax(P(x), x.size), x[:8]
    # FNV-1a 64 published vectors (runtime/engine.c:30-38).
    basis = 0xCBF29CE484222325
    assert oracle.oracle_fnv1a(None, 0, basis) == basis
    assert oracle.oracle_fnv1a(ctypes.c_char_p(b"a"), 1, basis) == 0xAF63DC4C8601EC8C
    assert oracle.oracle_fnv1a(ctypes.c_char_p(b"foobar"), 6, basis) == 0x85944171F73967E8


ARGMAX_CHECK = r"""
import sys
import numpy as np
sys.path[:0] = sys.argv[1:3]
import oracle_lib, plamo_hip
from ctypes import POINTER, c_float
hip, oracle = plamo_hip.load(), oracle_lib.load()
P = lambda a: a.ctypes.data_as(POINTER(c_float))
rng = np.random.default_rng(11)
cases = [np.array([-0.0, 0.0, -1.0], np.float32), np.array([float("-inf")] * 97, np.float32)]
for n in list(range(1, 140)) + [1000, 100000]:
    x = rng.integers(-3, 4, size=n).astype(np.float32)
    cases.append(x)
    y = rng.standard_normal(n).astype(np.float32)
    cases.append(y)
    if n > 2:
        z = y.copy()
        z[rng.integers(0, n)] = np.nan
        cases.append(z)
        w = x.copy()
        w[-1] = w.max() + 1
        cases.append(w)
for x in cases:
    assert hip.plamo_argmax(P(x), x.size) == oracle.oracle_argmax(P(x), x.size), (x.size, x[:8])
print("ok", len(cases))
"""


@pytest.mark.parametrize("isa", ["sse2", "avx2", "avx512"])
def test_argmax_every_vector_width(oracle, hip, isa):
    # plamo_argmax picks its vector width once per process (PLAMO_ARGMAX_ISA
    # caps it): each width against the oracle's sequential scan, in a process
    # of its own. Where the CPU lacks a width the next narrower one runs.
    import subprocess
    import sys
    here = Path(__file__).resolve().parent
    env = dict(__import__("os").environ, PLAMO_ARGMAX_ISA=isa)
    r = subprocess.run([sys.executable, "-c", ARGMAX_CHECK, str(here),
                        str(here.parent / "plamo-3-translate.c_amd")],
                       capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
