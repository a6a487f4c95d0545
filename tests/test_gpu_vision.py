"""The vision tower on the GPU through the C ABI: its kernels against float64
brute force, and whole encodes against the oracle (oracle/exn_vision_oracle.py,
itself pinned against inspect/ref_vision.py's own outputs).  The tower runs in
fp32 as the reference does, so the bar is float32 arithmetic in another summation
order: the kernels within 2e-5 of float64 relative to the operands' scale, a
whole 27-block encode within relative L2 1e-4 of the oracle.  Needs an MI355X."""
import math
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo
from oracle import exn_vision_oracle as vo

pytestmark = pytest.mark.gpu
SEED = 21
QSCALE = 1.4426950408889634 / math.sqrt(72)


def say(*a):
    print("[gpu]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = X.Context(0)
    yield c
    c.close()


_KEEP = []


def dev(ctx, a):
    b = X.DevBuf.of(ctx, np.ascontiguousarray(a))
    _KEEP.append(b)
    return b


def gelu_tanh64(x):
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def gelu_erf64(x):
    from scipy.special import erf
    return 0.5 * x * (1 + erf(x / math.sqrt(2)))


GEMM_CASES = [  # M, N, K, act, residual
    (64, 1152, 1152, 0, False),        # one row of 64 x 64 tiles
    (2048, 4304, 1152, 1, False),      # an N tail (4304 = 67 x 64 + 16), GELU tanh
    (256, 1152, 4304, 0, True),        # K not a multiple of 32 (the ffn_down shape), residual
    (100, 200, 68, 2, True),           # M, N, K tails everywhere, GELU erf
    (16, 4096, 4608, 0, False),        # a merger's fc2 for one merge row of a small picture
]


@pytest.mark.parametrize("case", GEMM_CASES)
def test_vis_gemm_against_float64(ctx, case):
    m, n, k, act, res = case
    say("vis_gemm", case)
    x = xo.normal(1, 7001, m * k).reshape(m, k)
    w = (xo.normal(1, 7002, n * k).reshape(n, k) / np.float32(math.sqrt(k))).astype(np.float32)
    b = xo.normal(1, 7003, n) * np.float32(0.1)
    r = xo.normal(1, 7004, m * n).reshape(m, n) if res else None
    dx, dw, db = dev(ctx, x), dev(ctx, w), dev(ctx, b)
    dy = dev(ctx, r) if res else X.DevBuf(ctx, (m, n), np.float32)
    _KEEP.append(dy)
    X.call("exn_vis_gemm", ctx.h, dx.h, dw.h, db.h, dy.h if res else None, dy.h, m, n, k, act)
    got = dy.get()
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    if res:
        want = want + r
    if act == 1:
        want = gelu_tanh64(want)
    elif act == 2:
        want = gelu_erf64(want)
    scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T + 1.0
    err = np.abs(got - want) / scale
    assert err.max() < 2e-5, err.max()


@pytest.mark.parametrize("n,heads", [(260, 2), (64, 1), (4096, 16)])
def test_vis_attend_against_float64(ctx, n, heads):
    """Every patch over every patch, tails of the 128-query and 64-key tiles (n = 260),
    and the 1024 x 1024 picture's 4096 patches (three heads checked)."""
    say("vis_attend", n, heads)
    q = xo.normal(2, 7010, heads * n * 72).reshape(heads, n, 72) * np.float32(2.0)
    k = xo.normal(2, 7011, heads * n * 72).reshape(heads, n, 72) * np.float32(2.0)
    v = xo.normal(2, 7012, heads * n * 72).reshape(heads, n, 72)
    vt = np.ascontiguousarray(v.transpose(0, 2, 1))
    dq = dev(ctx, (q * np.float32(QSCALE)).astype(np.float32))
    dk, dvt = dev(ctx, k), dev(ctx, vt)
    da = X.DevBuf(ctx, (n, heads * 72), np.float32)
    _KEEP.append(da)
    X.call("exn_vis_attend", ctx.h, n, heads, dq.h, dk.h, dvt.h, da.h)
    got = da.get().reshape(n, heads, 72)
    for h in sorted({0, heads // 2, heads - 1}):
        s = q[h].astype(np.float64) @ k[h].astype(np.float64).T / math.sqrt(72)
        assert s.max() - s.min() > 20          # a sharp softmax: the running max moves
        p = np.exp(s - s.max(1, keepdims=True))
        want = (p / p.sum(1, keepdims=True)) @ v[h].astype(np.float64)
        assert np.abs(got[:, h] - want).max() < 2e-5


def test_vis_ln_against_float64(ctx):
    for rows, width in ((37, 1152), (9, 4608), (3, 144)):
        x = xo.normal(3, 7020, rows * width).reshape(rows, width) * np.float32(3.0) + np.float32(1.5)
        w = np.float32(1) + np.float32(0.1) * xo.normal(3, 7021, width)
        b = np.float32(0.02) * xo.normal(3, 7022, width)
        dx, dw, db = dev(ctx, x), dev(ctx, w), dev(ctx, b)
        dy = X.DevBuf(ctx, (rows, width), np.float32)
        _KEEP.append(dy)
        X.call("exn_vis_ln", ctx.h, rows, width, dx.h, dw.h, db.h, dy.h)
        x64 = x.astype(np.float64)
        m = x64.mean(1, keepdims=True)
        want = (x64 - m) / np.sqrt(((x64 - m) ** 2).mean(1, keepdims=True) + 1e-6) * w + b
        assert np.abs(dy.get() - want).max() < 1e-5


@pytest.fixture(scope="module")
def tower(ctx):
    say("vision synth", SEED)
    v = X.load_vision(seed=SEED, ctx=ctx)
    yield v
    v.destroy()


@pytest.fixture(scope="module")
def owt():
    return vo.SynthVision(SEED)


@pytest.mark.parametrize("hw", [(128, 128), (96, 224), (512, 512), (1024, 1024)])
def test_encode_against_oracle(tower, owt, hw):
    """The whole tower (27 blocks, the three deepstack mergers, the merger) on
    synthetic fp16-valued weights: a 4 x 4 grid of merge blocks, a 3 x 7 one (the
    table resampled to a wide grid), the 1024 patches of a 512 x 512 picture and the
    4096 of the timed 1024 x 1024 one."""
    h, w = hw
    say("vision encode", h, w)
    px = vo.synth_picture(SEED + h + w, h, w)
    tower.trace(True)
    merged, deep, m = X.vision_encode(tower, px, h, w)
    n = 4 * m
    embed, blk0 = tower.traced(0, n), tower.traced(1, n)
    tower.trace(False)
    want = vo.encode(px, owt)
    assert xo.rel_l2(embed, want["embed"]) < 1e-6
    assert xo.rel_l2(blk0, want["blk0"]) < 1e-5
    e_m = xo.rel_l2(merged, want["merged"])
    e_d = [xo.rel_l2(deep[j], want["ds"][j]) for j in range(3)]
    say("merged", e_m, "deepstack", e_d)
    assert e_m < 1e-4 and max(e_d) < 1e-4
    assert np.isfinite(merged).all() and np.isfinite(deep).all()


def test_encode_reads_a_table_of_another_side_and_f16_tensors(ctx, owt):
    """exn_vision_set: the position table of a 36 x 36 grid (F32), the matrices as the fp16
    bit patterns an mmproj-f16 file holds, except the blocks' attn_out matrices as bf16 bit
    patterns (their values rounded to bf16 on both sides), 1-D tensors as F32: the encode
    matches the oracle run on the same values."""
    s36 = vo.VShape(side=36)
    wt = vo.SynthVision(SEED, s36)
    wt.cache = {k: a for k, a in owt.cache.items() if k != "v.position_embd.weight"}   # the same tensors
    v = X.Vision(ctx)
    try:
        for name, shape in vo.vision_expected(s36):
            a = wt(name)
            if name.endswith("attn_out.weight"):
                b = xo.bf16_bits(a)
                wt.cache[name] = xo.bf16_to_f32(b).reshape(a.shape)     # the oracle reads the same values
                v.set(name, X.BF16, b, shape)
            elif a.ndim > 1 and name != "v.position_embd.weight":
                v.set(name, X.F16, a.astype(np.float16).view(np.uint16), shape)
            else:
                v.set(name, X.F32, a, shape)
        v.check()
        h, w = 64, 160
        px = vo.synth_picture(SEED + 5, h, w)
        merged, deep, m = X.vision_encode(v, px, h, w)
        want = vo.encode(px, wt, s36)
        assert xo.rel_l2(merged, want["merged"]) < 1e-4
        assert xo.rel_l2(deep[2], want["ds"][2]) < 1e-4
    finally:
        v.destroy()


def test_release_frees_scratch_and_keeps_weights(tower):
    """vision-release (src/cuda-vision.lisp:103-107): the scratch freed, the weights kept; the
    next encode makes its buffers again and gives the same rows bit for bit."""
    px = vo.synth_picture(SEED + 3, 128, 128)
    a, da, m = X.vision_encode(tower, px, 128, 128)
    w, s = tower.memory()
    assert s > 0
    tower.release()
    assert tower.memory() == (w, 0)
    b, db, _ = X.vision_encode(tower, px, 128, 128)
    assert np.array_equal(a, b) and np.array_equal(da, db) and 0 < tower.memory()[1] <= s


def test_vision_errors(ctx, tower):
    v = X.Vision(ctx)
    try:
        with pytest.raises(X.ExnError) as e:
            v.check()
        assert e.value.code == X.ESTATE and "v.patch_embd.weight" in str(e.value)
        with pytest.raises(X.ExnError) as e:
            v.set("v.blk.0.ln1.weight", X.F32, np.zeros(1000, np.float32), (1000,))
        assert e.value.code == X.EINVAL
        with pytest.raises(X.ExnError) as e:
            v.set("v.position_embd.weight", X.F32, np.zeros(10 * 1152, np.float32), (10, 1152))
        assert e.value.code == X.EINVAL                      # not a square table
        with pytest.raises(X.ExnError) as e:
            v.set("v.no_such.weight", X.F32, np.zeros(4, np.float32), (4,))
        assert e.value.code == X.EINVAL
    finally:
        v.destroy()
    with pytest.raises(X.ExnError) as e:
        X.vision_encode(tower, np.zeros((48, 64, 4), np.float32), 48, 64)
    assert e.value.code == X.EINVAL                          # 48 is not a multiple of 32
    wb, sb = tower.memory()
    assert wb > 2.2e9
