"""GPU parity of the prompt GEMM through plamo_metal_linear
(runtime/metal.m:239-385): the split-BF16 matrix-core path (one and two
32-row tiles per wave, several M tiles, N not a multiple of the tile, split-K
with the last-block reduction) and, for at most 16 tokens, the weight-streaming
skinny path (one and two 16-row tiles per block, ragged last tiles, every
token count up to 16) against the oracle's matmul (src/matmul.s,
bit-identical to per-token matvec), with the reference's GPU gate.

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
