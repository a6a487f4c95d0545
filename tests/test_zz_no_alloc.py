"""exn_mm_noalloc: exn_mm's products with no device allocation (the bf16 staging of fp32
rows in the library's static per-device scratch array), against exn_mm itself on the
same inputs -- bit for bit: the same kernels on the same operands.  Two calls in a row,
the second smaller, so that the second reads none of the first's stale staging; and the call
captured in a HIP graph on the context's stream, replayed.  Needs an MI355X."""
import ctypes
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = X.Context(0)
    yield c
    c.close()


def _mm(ctx, name, w, x, xdt, n, ydt):
    yt = np.float32 if ydt == X.DT_F32 else np.uint16
    y = X.DevBuf(ctx, (n, w.rows), yt)
    X.call(name, ctx.h, w.h, x.h, xdt, y.h, ydt, n)
    return y.get()


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
def test_noalloc_equals_mm_twice(ctx, resident):
    N, K = 4096, 4096
    say("exn_mm_noalloc vs exn_mm", N, K, "resident" if resident else "q8_0")
    w = X.Weight.synth(ctx, 9, 400, N, K)
    if resident:
        w.resident()
    rng = np.random.default_rng(12)
    for n, ydt in ((3000, X.DT_F32), (700, X.DT_BF16)):          # the second call smaller
        x = X.DevBuf.of(ctx, rng.normal(0, 1, (n, K)).astype(np.float32))
        got = _mm(ctx, "exn_mm_noalloc", w, x, X.DT_F32, n, ydt)
        want = _mm(ctx, "exn_mm", w, x, X.DT_F32, n, ydt)
        say("n %d: equal %s" % (n, np.array_equal(got, want)))
        assert np.array_equal(got, want)
    # bf16 rows and the n <= 4 GEMV need no staging; the same results too
    xb = X.DevBuf.of(ctx, xo.bf16_bits(rng.normal(0, 1, (50, K)).astype(np.float32)))
    assert np.array_equal(_mm(ctx, "exn_mm_noalloc", w, xb, X.DT_BF16, 50, X.DT_F32),
                          _mm(ctx, "exn_mm", w, xb, X.DT_BF16, 50, X.DT_F32))
    x4 = X.DevBuf.of(ctx, rng.normal(0, 1, (4, K)).astype(np.float32))
    assert np.array_equal(_mm(ctx, "exn_mm_noalloc", w, x4, X.DT_F32, 4, X.DT_F32),
                          _mm(ctx, "exn_mm", w, x4, X.DT_F32, 4, X.DT_F32))
    w.free()


def test_noalloc_f32_matrix_and_limit(ctx):
    rng = np.random.default_rng(13)
    wf = rng.normal(0, 0.05, (256, 512)).astype(np.float32)
    w = X.Weight.f32(ctx, wf)
    x = X.DevBuf.of(ctx, rng.normal(0, 1, (40, 512)).astype(np.float32))
    assert np.array_equal(_mm(ctx, "exn_mm_noalloc", w, x, X.DT_F32, 40, X.DT_F32),
                          _mm(ctx, "exn_mm", w, x, X.DT_F32, 40, X.DT_F32))
    w.free()
    # fp32 rows whose bf16 copy would pass the 64 MiB scratch: refused before any launch
    w = X.Weight.synth(ctx, 9, 401, 64, 12288)
    big = (64 << 20) // (2 * 12288) + 1
    x = X.DevBuf(ctx, (big, 12288), np.float32)
    y = X.DevBuf(ctx, (big, 64), np.float32)
    with pytest.raises(X.ExnError) as e:
        X.call("exn_mm_noalloc", ctx.h, w.h, x.h, X.DT_F32, y.h, X.DT_F32, big)
    assert e.value.code == X.EINVAL and "scratch" in str(e.value)
    w.free()


def test_noalloc_under_graph_capture(ctx):
    """After one call on the device (which takes the scratch address and sets the kernels'
    attributes), exn_mm_noalloc captures into a HIP graph on the context's stream: the graph
    replayed three times, with the program's own eager work and a synchronisation between the
    replays, gives exn_mm's output bit for bit every time."""
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    for f in ("hipStreamCreate", "hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate",
              "hipGraphLaunch", "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy",
              "hipStreamDestroy"):
        getattr(hip, f).restype = ctypes.c_int
    s = vp()
    assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    N, K, n = 4096, 4096, 1024
    w = X.Weight.synth(ctx, 9, 402, N, K)
    rng = np.random.default_rng(14)
    x = X.DevBuf.of(ctx, rng.normal(0, 1, (n, K)).astype(np.float32))
    y = X.DevBuf(ctx, (n, N), np.uint16)
    g, ge = vp(), vp()
    try:
        X.call("exn_set_stream", ctx.h, s)
        want = _mm(ctx, "exn_mm", w, x, X.DT_F32, n, X.DT_BF16)
        assert np.array_equal(_mm(ctx, "exn_mm_noalloc", w, x, X.DT_F32, n, X.DT_BF16), want)   # the warm call
        assert hip.hipStreamBeginCapture(s, 0) == 0            # hipStreamCaptureModeGlobal
        X.call("exn_mm_noalloc", ctx.h, w.h, x.h, X.DT_F32, y.h, X.DT_BF16, n)
        assert hip.hipStreamEndCapture(s, ctypes.byref(g)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0) == 0
        for r in range(3):
            y.upload(np.zeros((n, N), np.uint16))              # eager work between the replays
            assert hip.hipGraphLaunch(ge, s) == 0
            assert hip.hipStreamSynchronize(s) == 0
            got = y.get()
            say("replay %d: equal %s" % (r, np.array_equal(got, want)))
            assert np.array_equal(got, want)
    finally:
        if ge.value:
            hip.hipGraphExecDestroy(ge)
        if g.value:
            hip.hipGraphDestroy(g)
        X.call("exn_set_stream", ctx.h, None)
        hip.hipStreamSynchronize(s)
        hip.hipStreamDestroy(s)
        w.free()
