"""plamo_hip_linear_static, the projection entry point that allocates nothing
(its GEMM scratch is a static device array), against plamo_metal_linear on
the same resident weights: several calls in a row on one backend, each
smaller than the one before, must give the allocating entry point's bits.
The buffers are the test's own device memory (hipMalloc through the HIP
runtime the library links); the entry point takes device pointers."""

import ctypes

import numpy as np
import pytest

from parity import plamo_hip, say

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2  # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


class DeviceArray:
    """FP32 device buffer owned by the test."""

    def __init__(self, hip, floats):
        self.hip, self.floats = hip, floats
        self.ptr = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(floats * 4)) == 0

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        assert a.size <= self.floats
        assert self.hip.hipMemcpy(self.ptr, a.ctypes.data_as(ctypes.c_void_p),
                                  ctypes.c_size_t(a.nbytes), H2D) == 0

    def download(self, floats):
        out = np.empty(floats, np.float32)
        assert self.hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                                  ctypes.c_size_t(floats * 4), D2H) == 0
        return out

    def f32p(self):
        return ctypes.cast(self.ptr, plamo_hip.f32p)

    def free(self):
        if self.ptr:
            self.hip.hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()


def test_static_linear_matches_allocating_linear():
    lib = plamo_hip.load()
    hip = ctypes.CDLL("libamdhip64.so.7")  # the soname libplamo_hip.so links
    # One layer at the C4 hidden width: the QKV projection is 6144 x 4096.
    s = plamo_hip.Synthetic(4096, 1, 32, 8, 128, 1024, 64, window=8, global_capacity=64,
                            pattern=1, seed=31)
    inst = s.instance()
    be = plamo_hip.Backend(s)
    buffers = []
    try:
        q = inst.layer(0).mixer.contents.qkv.contents
        rows, cols = (q.qh + 2 * q.kh) * q.dim, q.hidden
        xs, ys = cols + 4, rows + 4  # strided device rows
        rng = np.random.default_rng(8)
        # 40 tokens: split-BF16 GEMM with split-K partials and counters in the
        # static scratch; 3: the token GEMV over K slices; 1: the decode GEMV.
        for tokens in (40, 3, 1):
            say(f"static linear: {tokens} tokens x {cols} columns -> {rows} rows")
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            r, expected = be.linear(q.weight, x, rows)
            assert r == 1
            dx, dy = DeviceArray(hip, tokens * xs), DeviceArray(hip, tokens * ys)
            buffers += [dx, dy]
            padded = np.zeros((tokens, xs), np.float32)
            padded[:, :cols] = x
            dx.upload(padded)
            dy.upload(np.full(tokens * ys, np.nan, np.float32))
            mm = plamo_hip.Matmul(q.weight, dx.f32p(), dy.f32p(), rows, cols, tokens, xs, ys)
            assert lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm)) == 1, \
                be.info().note.decode()
            got = dy.download(tokens * ys).reshape(tokens, ys)
            assert got[:, :rows].tobytes() == expected.tobytes(), f"{tokens} tokens"
            if tokens > 1:  # the row padding of each output row is untouched
                assert np.isnan(got[:, rows:]).all()
        info = be.info()
        assert info.errors == 0 and info.cpu_fallbacks == 0, info.note.decode()
        # A prompt whose input planes exceed the static scratch is refused
        # before anything is launched.
        big = 1400
        dx, dy = DeviceArray(hip, big * cols), DeviceArray(hip, big * rows)
        buffers += [dx, dy]
        mm = plamo_hip.Matmul(q.weight, dx.f32p(), dy.f32p(), rows, cols, big, cols, rows)
        assert lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm)) == 0
        assert b"static scratch" in be.info().note
        # Weights that are not resident are refused.
        stray = np.zeros(rows * cols, np.uint16)
        mm = plamo_hip.Matmul(stray.ctypes.data_as(plamo_hip.u16p), dx.f32p(), dy.f32p(), rows,
                              cols, 2, cols, rows)
        assert lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm)) == 0
        assert b"not resident" in be.info().note
        # Host memory (what plamo_metal_linear takes) is refused before any
        # launch, as input and as output; so are strides that reach past the
        # end of a device buffer.
        host = np.zeros(2 * cols, np.float32)
        hp = host.ctypes.data_as(plamo_hip.f32p)
        small_x, small_y = DeviceArray(hip, 2 * cols), DeviceArray(hip, 2 * rows)
        buffers += [small_x, small_y]
        for x_, y_, xs_, ys_ in ((hp, small_y.f32p(), cols, rows),
                                 (small_x.f32p(), hp, cols, rows),
                                 (small_x.f32p(), small_y.f32p(), cols + 1, rows),
                                 (small_x.f32p(), small_y.f32p(), cols, rows + 1)):
            mm = plamo_hip.Matmul(q.weight, x_, y_, rows, cols, 2, xs_, ys_)
            assert lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm)) == 0
            assert b"device memory" in be.info().note
        mm = plamo_hip.Matmul(q.weight, small_x.f32p(), small_y.f32p(), rows, cols, 2, cols, rows)
        assert lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm)) == 1
    finally:
        for b in buffers:
            b.free()
        be.close()
        inst.close()
        s.close()


def test_static_linear_calls_from_two_backends():
    # Two backend instances of one process (a target and a draft) call the
    # entry point from two threads at once. One call at a time owns the GPU's
    # static scratch: every call either matches plamo_metal_linear bit for bit
    # or is refused with a note; none sees the other's partial tiles.
    import threading
    lib = plamo_hip.load()
    hip = ctypes.CDLL("libamdhip64.so.7")
    s = plamo_hip.Synthetic(4096, 1, 32, 8, 128, 1024, 64, window=8, global_capacity=64,
                            pattern=1, seed=37)
    inst = s.instance()
    backends = [plamo_hip.Backend(s), plamo_hip.Backend(s)]
    buffers = []
    try:
        q = inst.layer(0).mixer.contents.qkv.contents
        rows, cols, tokens = (q.qh + 2 * q.kh) * q.dim, q.hidden, 200
        rng = np.random.default_rng(5)
        jobs = []
        for be in backends:
            x = rng.standard_normal((tokens, cols)).astype(np.float32)
            r, expected = be.linear(q.weight, x, rows)
            assert r == 1
            dx, dy = DeviceArray(hip, tokens * cols), DeviceArray(hip, tokens * rows)
            buffers += [dx, dy]
            dx.upload(x)
            jobs.append((be, plamo_hip.Matmul(q.weight, dx.f32p(), dy.f32p(), rows, cols, tokens,
                                              cols, rows), dy, expected))
        outcomes = {"done": 0, "refused": 0}
        for round_ in range(6):
            results = [None, None]

            def call(j):
                be, mm, _, _ = jobs[j]
                results[j] = lib.plamo_hip_linear_static(be.handle, ctypes.byref(mm))

            threads = [threading.Thread(target=call, args=(j,)) for j in range(2)]
            for t in threads:
                t.start()
            for t in threads:
                t.join()
            for j, (be, _, dy, expected) in enumerate(jobs):
                if results[j] == 1:
                    got = dy.download(tokens * rows).reshape(tokens, rows)
                    assert got.tobytes() == expected.tobytes(), f"round {round_} backend {j}"
                    outcomes["done"] += 1
                else:
                    assert b"in use by another call" in be.info().note
                    outcomes["refused"] += 1
                dy.upload(np.full(tokens * rows, np.nan, np.float32))
        say(f"static linear from two threads: {outcomes}")
        assert outcomes["done"] >= 6
    finally:
        for b in buffers:
            b.free()
        for be in backends:
            be.close()
        inst.close()
        s.close()
