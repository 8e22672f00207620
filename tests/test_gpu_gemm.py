"""GPU parity of the prompt GEMM through plamo_metal_linear
(runtime/metal.m:239-385): the split-BF16 matrix-core path (one and two
32-row tiles per wave, several M tiles, N not a multiple of the tile, split-K
with the last-block reduction), for at most 16 tokens the weight-streaming
skinny path (one and two 16-row tiles per block, ragged last tiles, every
token count up to 16; K = 256 and 384 are not whole 512-column chunks, and
6..16 tokens take it for any K), and for 1..5 tokens over whole chunks the
vector-ALU token GEMV (short last
sub-steps, K slices, ragged last units, SwiGLU fused through
plamo_metal_mlp) against the oracle's matmul (src/matmul.s, bit-identical to
per-token matvec) and MLP branch, with the reference's GPU gate.

The three-term split of each FP32 input is exact, so the products carry no
input rounding at all; a float64 product bounds that: a split that dropped its
third term would leave a relative error near 1e-5, far above the 3e-6 allowed
here for FP32 accumulation over 4096 terms.
"""

import numpy as np
import pytest

from parity import gate, oracle_lib, plamo_hip, say

pytestmark = pytest.mark.gpu


def reference(oracle, weights, x, rows):
    ref = np.zeros((x.shape[0], rows), np.float32)
    mm = plamo_hip.Matmul(weights, x.ctypes.data_as(plamo_hip.f32p),
                          ref.ctypes.data_as(plamo_hip.f32p), rows, x.shape[1], x.shape[0],
                          x.shape[1], rows)
    oracle.oracle_matmul(plamo_hip.ctypes.byref(mm))
    return ref


def weights_f64(ptr, rows, cols):
    w = np.ctypeslib.as_array(plamo_hip.ctypes.cast(ptr, plamo_hip.u16p), shape=(rows * cols,))
    return (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(rows, cols)


@pytest.mark.parametrize("tokens", [1, 2, 5, 16, 17, 31, 33, 64, 65, 130])
def test_split_bf16_gemm(oracle, tokens):
    # hidden 256, MLP 4096, vocab 300: down is N=256 x K=4096 (split-K),
    # gate/up N=8192 x K=256, head N=300 (ragged last tile) x K=256.
    s = plamo_hip.Synthetic(256, 1, 2, 1, 128, 4096, 300, window=4, global_capacity=64,
                            pattern=1, seed=11)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        mlp = a.layer(0).mlp.contents
        cases = [("down", mlp.down, 256, 4096), ("gate_up", mlp.gu, 8192, 256),
                 ("head", a.model.head, 300, 256)]
        rng = np.random.default_rng(tokens)
        for name, ptr, rows, cols in cases:
            say(f"gemm {name} tokens={tokens} rows={rows} cols={cols}")
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            x[0, :8] *= 1e3   # wide dynamic range within a row
            x[-1, 8:16] *= 1e-3
            r, y = be.linear(ptr, x, rows)
            assert r == 1
            gate(y, reference(oracle, ptr, x, rows), f"{name} tokens={tokens}")
            exact = x.astype(np.float64) @ weights_f64(ptr, rows, cols).T
            err = np.sqrt(np.sum((y - exact) ** 2) / np.sum(exact ** 2))
            assert err <= 3e-6, f"{name}: relative L2 {err:.3g} against the float64 product"
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()


@pytest.mark.parametrize("hidden", [192, 320])
def test_split_bf16_gemm_stage_counts(oracle, hidden):
    # The matrix-core GEMM runs its 32-column K stages in unrolled rounds of
    # three steps and the last K % 96 / 32 steps after them: hidden 192 is
    # six stages (two whole rounds), 320 is ten (three rounds and one more);
    # down (K 512, split in four) has four stages per split.
    s = plamo_hip.Synthetic(hidden, 1, hidden // 64, 1, 64, 512, 300, window=4,
                            global_capacity=64, pattern=1, seed=12)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        mlp = a.layer(0).mlp.contents
        cases = [("gate_up", mlp.gu, 1024, hidden), ("head", a.model.head, 300, hidden),
                 ("down", mlp.down, hidden, 512)]
        rng = np.random.default_rng(hidden)
        for tokens in (40, 130):
            for name, ptr, rows, cols in cases:
                say(f"gemm stages {name} hidden={hidden} tokens={tokens}")
                x = rng.standard_normal((tokens, cols)).astype(np.float32)
                r, y = be.linear(ptr, x, rows)
                assert r == 1
                gate(y, reference(oracle, ptr, x, rows), f"{name} hidden={hidden} tokens={tokens}")
                exact = x.astype(np.float64) @ weights_f64(ptr, rows, cols).T
                err = np.sqrt(np.sum((y - exact) ** 2) / np.sum(exact ** 2))
                assert err <= 3e-6, f"{name}: relative L2 {err:.3g} against the float64 product"
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()


@pytest.mark.parametrize("tokens", [130, 200])
def test_split_bf16_gemm_192_row_tiles(oracle, tokens):
    # Past 128 tokens a projection whose 256-row tiles leave CUs idle takes
    # 192-row tiles: gate/up of MLP 768 as a plain linear is 1536 rows, 6
    # tiles of 256 or 8 of 192 per 64 tokens.
    s = plamo_hip.Synthetic(256, 1, 2, 1, 128, 768, 300, window=4, global_capacity=64,
                            pattern=1, seed=13)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        ptr, rows, cols = a.layer(0).mlp.contents.gu, 1536, 256
        say(f"gemm 192-row tiles tokens={tokens}")
        x = np.random.default_rng(tokens).standard_normal((tokens, cols)).astype(np.float32)
        r, y = be.linear(ptr, x, rows)
        assert r == 1
        gate(y, reference(oracle, ptr, x, rows), f"192-row tiles tokens={tokens}")
        exact = x.astype(np.float64) @ weights_f64(ptr, rows, cols).T
        err = np.sqrt(np.sum((y - exact) ** 2) / np.sum(exact ** 2))
        assert err <= 3e-6, f"relative L2 {err:.3g} against the float64 product"
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()


@pytest.mark.parametrize("tokens", [1, 3, 5, 8, 13, 16])
def test_skinny_gemm_two_row_tiles(oracle, tokens):
    # gate/up of MLP 8200 is N=16400 (two 16-row tiles per block, the last
    # block half full) x K=384; down is N=384 x K=8200 is not a multiple of
    # 128 columns and takes the tiled path.
    s = plamo_hip.Synthetic(384, 1, 3, 1, 128, 8200, 40, window=4, global_capacity=64,
                            pattern=1, seed=5)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        mlp = a.layer(0).mlp.contents
        rng = np.random.default_rng(100 + tokens)
        for name, ptr, rows, cols in [("gate_up", mlp.gu, 16400, 384),
                                      ("down", mlp.down, 384, 8200)]:
            say(f"skinny {name} tokens={tokens}")
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            r, y = be.linear(ptr, x, rows)
            assert r == 1
            gate(y, reference(oracle, ptr, x, rows), f"{name} tokens={tokens}")
            exact = x.astype(np.float64) @ weights_f64(ptr, rows, cols).T
            err = np.sqrt(np.sum((y - exact) ** 2) / np.sum(exact ** 2))
            assert err <= 3e-6, f"{name}: relative L2 {err:.3g} against the float64 product"
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()


@pytest.mark.parametrize("tokens", [2, 3, 4, 5, 6, 8])
def test_token_gemv(oracle, tokens):
    # The vector-ALU token GEMV (1..5 tokens, K a multiple of 512). Hidden
    # 2560 is five 512-column chunks, so two-chunk sub-steps end short. The
    # MLP's 10240 columns split into K slices that the last block of each row
    # group adds. The 1002-row head ends in a quarter-full eight-row unit.
    # Six and eight tokens run the same shapes through the skinny GEMM.
    s = plamo_hip.Synthetic(2560, 1, 4, 1, 128, 10240, 1002, window=4, global_capacity=64,
                            pattern=1, seed=31)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        mlp = a.layer(0).mlp.contents
        q = a.layer(0).mixer.contents.qkv.contents
        cases = [("qkv", q.weight, (q.qh + 2 * q.kh) * q.dim, 2560),
                 ("gate_up", mlp.gu, 20480, 2560), ("down", mlp.down, 2560, 10240),
                 ("head", a.model.head, 1002, 2560)]
        rng = np.random.default_rng(300 + tokens)
        for name, ptr, rows, cols in cases:
            say(f"token gemv {name} tokens={tokens} rows={rows} cols={cols}")
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            x[0, :8] *= 1e3
            x[-1, 8:16] *= 1e-3
            r, y = be.linear(ptr, x, rows)
            assert r == 1
            gate(y, reference(oracle, ptr, x, rows), f"{name} tokens={tokens}")
            exact = x.astype(np.float64) @ weights_f64(ptr, rows, cols).T
            err = np.sqrt(np.sum((y - exact) ** 2) / np.sum(exact ** 2))
            assert err <= 3e-6, f"{name}: relative L2 {err:.3g} against the float64 product"
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()


@pytest.mark.parametrize("tokens", [1, 2, 4, 5, 6, 9])
def test_mlp_fused_swiglu(oracle, tokens):
    # plamo_metal_mlp over 1..5 tokens takes the token GEMV with SwiGLU in its
    # epilogue (gate rows 4j .. 4j + 3 and up rows 8192 + 4j .. 8192 + 4j + 3
    # per unit; at five tokens the gate/up K of 4096 splits in two, so the
    # activation runs after the slice merge); six and nine tokens take the
    # matrix-core GEMMs and the separate SwiGLU launch. Each row is checked
    # against the oracle's MLP branch.
    s = plamo_hip.Synthetic(4096, 1, 4, 1, 128, 8192, 40, window=4, global_capacity=64,
                            pattern=1, seed=37)
    a = s.instance()
    be = plamo_hip.Backend(s)
    try:
        mlp = a.layer(0).mlp.contents
        rng = np.random.default_rng(400 + tokens)
        st = rng.standard_normal((tokens, 4096)).astype(np.float32)
        ref = st.copy()
        say(f"mlp tokens={tokens}")
        assert be.lib.plamo_metal_mlp(be.handle, plamo_hip.ctypes.byref(mlp),
                                      st.ctypes.data_as(plamo_hip.f32p), tokens) == 1
        for t in range(tokens):
            row = ref[t].copy()
            m2 = plamo_hip.Mlp(row.ctypes.data_as(plamo_hip.f32p), mlp.pre, mlp.post, mlp.gu,
                               mlp.down, mlp.normalized, mlp.branch, mlp.scratch, 4096,
                               mlp.intermediate)
            oracle.oracle_mlp_branch(plamo_hip.ctypes.byref(m2))
            ref[t] = row
        gate(st, ref, f"mlp tokens={tokens}")
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0
    finally:
        be.close()
        a.close()
        s.close()
