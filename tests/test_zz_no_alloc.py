"""cc_topk_noalloc, the allocation-free top-k (include/ccdecode.h), against
the entry point it varies, cc_op_topk (topkRows, web/model/kernels.js:2129-2144),
through the C ABI: the same ids and value bits on two calls in a row, the
second smaller, for greedy (M = 1) and top-M; and a refusal past its scratch.

The device buffers come from the HIP runtime the library itself links
(libamdhip64.so.7, already loaded with it), through ctypes: the entry point
takes device pointers the caller owns."""
import ctypes as C

import numpy as np
import pytest

from chattorrent_amd import configs

pytestmark = pytest.mark.gpu


class _Hip:
    def __init__(self):
        self.h = C.CDLL("libamdhip64.so.7")
        self.h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.h.hipFree.argtypes = [C.c_void_p]
        self.h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.h.hipDeviceSynchronize.argtypes = []
        self.h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.h.hipStreamDestroy.argtypes = [C.c_void_p]
        self.h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p,
                                               C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.h.hipGraphDestroy.argtypes = [C.c_void_p]
        self.bufs = []

    def check(self, e):
        assert e == 0, f"HIP error {e}"

    def alloc(self, nbytes):
        p = C.c_void_p()
        self.check(self.h.hipMalloc(C.byref(p), nbytes))
        self.bufs.append(p)
        return p

    def upload(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        self.check(self.h.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, 1))   # host to device
        return p

    def download(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self.check(self.h.hipMemcpy(out.ctypes.data_as(C.c_void_p), p, out.nbytes, 2))   # device to host
        return out

    def free(self):
        for p in self.bufs:
            self.h.hipFree(p)
        self.bufs = []


@pytest.fixture(scope="module")
def ctx(gpu):
    from chattorrent_amd.ccdecode import Context
    c = Context(configs.with_layers(configs.SMOLLM2, 1), n_max=256, t_max=8, slots=1)
    yield c
    c.close()


def _bind(lib):
    lib.cc_topk_noalloc.restype = C.c_int32
    lib.cc_topk_noalloc.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                    C.c_void_p, C.c_void_p]


def _noalloc(c, hip, logits, M, stream=None):
    lib = c.lib
    _bind(lib)
    rows, V = logits.shape
    dl = hip.upload(logits.astype(np.float32))
    dv = hip.alloc(rows * M * 4)
    di = hip.alloc(rows * M * 4)
    st = lib.cc_topk_noalloc(c.h, dl, rows, V, M, dv, di, stream)
    assert st == 0, lib.cc_last_error(c.h).decode()
    if stream is None:
        hip.check(hip.h.hipDeviceSynchronize())
    else:
        hip.check(hip.h.hipStreamSynchronize(stream))
    return hip.download(dv, (rows, M), np.float32), hip.download(di, (rows, M), np.uint32)


@pytest.mark.parametrize("M", [1, 7, 256])
def test_noalloc_topk_equals_op_topk_twice(ctx, M):
    """Two calls in a row (the second with fewer rows and a shorter
    vocabulary, so the shared scratch holds the first call's keys when the
    second starts), each equal to cc_op_topk on the same logits bit for bit.
    Rows carry ties so the lower-id rule is exercised."""
    hip = _Hip()
    try:
        rng = np.random.default_rng(40 + M)
        for rows, V in ((12, 151936), (3, 49152)):
            logits = rng.standard_normal((rows, V)).astype(np.float32)
            logits[:, V // 3] = logits[:, V // 5] = 9.0      # a tie at the top
            vals, ids = _noalloc(ctx, hip, logits, M)
            want_v, want_i = ctx.op_topk(logits, M)
            assert np.array_equal(ids, want_i), (rows, V, M)
            assert np.array_equal(vals.view(np.uint32), want_v.view(np.uint32)), (rows, V, M)
            assert ids[0, 0] == min(V // 3, V // 5)
    finally:
        hip.free()


def test_noalloc_topk_refuses_past_its_scratch(ctx):
    """A call whose staged keys exceed the static scratch is refused with
    CC_EARG and a message; nothing is launched."""
    hip = _Hip()
    try:
        lib = ctx.lib
        _bind(lib)
        rows, V, M = 64, 262144, 256            # 64 * 64 * 256 keys in the first stage alone
        dl, dv, di = hip.alloc(4), hip.alloc(4), hip.alloc(4)
        st = lib.cc_topk_noalloc(ctx.h, dl, rows, V, M, dv, di, None)
        assert st == 5, st                      # CC_EARG
        assert "scratch" in lib.cc_last_error(ctx.h).decode()
    finally:
        hip.free()


def test_noalloc_topk_on_the_callers_stream(ctx):
    """The call runs on a stream the caller created and synchronises, not the
    context's: twice, the second smaller, each equal to cc_op_topk bitwise."""
    hip = _Hip()
    st = C.c_void_p()
    hip.check(hip.h.hipStreamCreate(C.byref(st)))
    try:
        rng = np.random.default_rng(77)
        for rows, V, M in ((9, 151936, 4), (2, 49152, 1)):
            logits = rng.standard_normal((rows, V)).astype(np.float32)
            vals, ids = _noalloc(ctx, hip, logits, M, stream=st)
            want_v, want_i = ctx.op_topk(logits, M)
            assert np.array_equal(ids, want_i), (rows, V, M)
            assert np.array_equal(vals.view(np.uint32), want_v.view(np.uint32)), (rows, V, M)
    finally:
        hip.check(hip.h.hipStreamDestroy(st))
        hip.free()


def test_noalloc_topk_under_graph_capture(ctx):
    """Captured once into a HIP graph on the caller's stream (relaxed capture
    mode) and replayed four times over fresh logits copied in eagerly between
    the replays: every replay equals cc_op_topk on that replay's logits. The
    call records kernels only, no memset nodes, and allocates nothing, so it
    can sit inside a caller's graph."""
    hip = _Hip()
    lib = ctx.lib
    _bind(lib)
    st = C.c_void_p()
    hip.check(hip.h.hipStreamCreate(C.byref(st)))
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        rows, V, M = 5, 151936, 3
        rng = np.random.default_rng(91)
        dl = hip.alloc(rows * V * 4)
        dv = hip.alloc(rows * M * 4)
        di = hip.alloc(rows * M * 4)
        hip.check(hip.h.hipStreamBeginCapture(st, 2))          # hipStreamCaptureModeRelaxed
        code = lib.cc_topk_noalloc(ctx.h, dl, rows, V, M, dv, di, st)
        hip.check(hip.h.hipStreamEndCapture(st, C.byref(graph)))
        assert code == 0, lib.cc_last_error(ctx.h).decode()
        hip.check(hip.h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0))
        for rep in range(4):
            logits = rng.standard_normal((rows, V)).astype(np.float32)
            logits[rep % rows, 7 + rep] = logits[rep % rows, 3 * rep + 11] = 12.0   # a tie at the top
            hip.check(hip.h.hipMemcpy(dl, logits.ctypes.data_as(C.c_void_p), logits.nbytes, 1))
            hip.check(hip.h.hipGraphLaunch(exe, st))
            hip.check(hip.h.hipStreamSynchronize(st))
            vals = hip.download(dv, (rows, M), np.float32)
            ids = hip.download(di, (rows, M), np.uint32)
            want_v, want_i = ctx.op_topk(logits, M)          # eager work between the replays
            assert np.array_equal(ids, want_i), rep
            assert np.array_equal(vals.view(np.uint32), want_v.view(np.uint32)), rep
    finally:
        if exe.value:
            hip.h.hipGraphExecDestroy(exe)
        if graph.value:
            hip.h.hipGraphDestroy(graph)
        hip.check(hip.h.hipStreamDestroy(st))
        hip.free()
