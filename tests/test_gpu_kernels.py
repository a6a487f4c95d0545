"""The HIP kernels against the oracle, through the C ABI (libexn-hip.so).
Integer and byte work bit-exact; floating point to the tolerance written in
each test.  Needs an MI355X."""
import ctypes
import math
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


_KEEP = []


@pytest.fixture(autouse=True)
def _keep_alive():
    """Device buffers made inline for a call stay alive until the test ends
    (a temporary's exn_free would otherwise run before the kernel does)."""
    yield
    _KEEP.clear()


def dev(ctx, a):
    b = X.DevBuf.of(ctx, np.ascontiguousarray(a))
    _KEEP.append(b)
    return b


def bf16(a):
    return xo.bf16_bits(np.asarray(a, np.float32))


def from_bf16(b):
    return xo.bf16_to_f32(b)


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def from_f16(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


# --- Q8_0: generator, repack, dequant (bit-exact) -------------------------------------

def test_synth_q8_bit_exact(ctx):
    say("synth q8 96x4096 seed 5 tensor 17")
    w = X.Weight.synth(ctx, 5, 17, 96, 4096)
    f = X.DevBuf(ctx, (96, 4096), np.float32)
    b = X.DevBuf(ctx, (96, 4096), np.uint16)
    X.call("exn_dequant", ctx.h, w.h, f.h, b.h)
    qs, d = xo.q8_0_synth(5, 17, 96, 4096)
    want = xo.dequant_q8_0(qs, d)
    got = f.get()
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    assert (b.get() == xo.bf16_bits(want)).all()


def test_repack_dequant_exhaustive(ctx):
    """Every fp16 scale (subnormals, zero, +-inf, NaN included) times every int8
    value through GGUF block_q8_0 records: the device's fp32 equals fp32(d) * q
    bit for bit (NaN where the product is NaN), its bf16 the RNE rounding."""
    say("repack exhaustive 4096 x 4096")
    d = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    nb = d.size * 8
    blocks = np.empty((nb, 34), np.uint8)
    blocks[:, 0:2] = np.repeat(d, 8).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = np.tile(q.view(np.uint8).reshape(8, 32), (d.size, 1))
    rows, cols = 4096, 4096
    w = X.Weight.q8_0(ctx, blocks.reshape(-1), rows, cols)
    f = X.DevBuf(ctx, (rows, cols), np.float32)
    b = X.DevBuf(ctx, (rows, cols), np.uint16)
    X.call("exn_dequant", ctx.h, w.h, f.h, b.h)
    with np.errstate(invalid="ignore"):
        want = xo.dequant_q8_0_blocks(blocks.reshape(-1)).reshape(rows, cols)
    got = f.get()
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()
    gb = b.get()
    wb = xo.bf16_bits(want)
    assert (gb[~nan] == wb[~nan]).all()


# --- the products -----------------------------------------------------------------------

GEMM_CASES = [  # (M, N, K): ragged, the block shapes, proj_out's N = 64, img_in's K = 64, down's K = 12288;
    # from 512 rows the Q8_0 products take 512 x 128 tiles: ragged rows and a last half chunk of 128 rows
    (77, 96, 128), (256, 512, 4096), (300, 4096, 4096), (257, 64, 4096), (130, 4096, 12288), (64, 4096, 64),
    (4352, 12288, 4096), (1100, 640, 4096), (513, 128, 128)]


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
@pytest.mark.parametrize("M,N,K", GEMM_CASES)
def test_gemm_q8_bf16(ctx, M, N, K, resident):
    """Q8_0 dequantised inside the product, or streamed from the resident bf16
    expansion (exn_weight_resident) by the LDS-DMA kernel: the same bf16 operands."""
    say("gemm q8", M, N, K, "resident bf16" if resident else "q8_0")
    rng = np.random.default_rng(M + N + K)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    xb = bf16(x)
    w = X.Weight.synth(ctx, 3, 200, N, K)
    if resident:
        w.resident()
    qs, d = xo.q8_0_synth(3, 200, N, K)
    wf = xo.dequant_q8_0(qs, d)
    dx = dev(ctx, xb)
    y = X.DevBuf(ctx, (M, N), np.float32)
    X.call("exn_mm", ctx.h, w.h, dx.h, X.DT_BF16, y.h, X.DT_F32, M)
    got = y.get()
    # same bf16 operands, fp32 sums: only the summation order differs
    rows = slice(None) if M <= 512 else np.r_[0:64, M - 64:M]
    want_b = from_bf16(xb[rows]).astype(np.float64) @ from_bf16(bf16(wf)).astype(np.float64).T
    assert xo.rel_l2(got[rows], want_b) < 2e-6
    # against the fp32 oracle product: the bf16 rounding of the operands only
    want = x[rows] @ wf.T
    assert xo.rel_l2(got[rows], want) < 1e-2


FEW_ROWS = [(20, 1024, 4096), (24, 1024, 4096), (64, 1024, 4096), (128, 1024, 4096), (129, 1024, 4096),
            (200, 1024, 4096), (256, 1024, 4096), (37, 512, 256), (256, 256, 12288), (200, 1024, 512),
            (256, 384, 512), (200, 384, 1024)]


@pytest.mark.parametrize("M,N,K", FEW_ROWS)
def test_few_row_products(ctx, M, N, K):
    """Products of at most 256 rows: the few-row kernel (128-row tiles up to 128 rows, 256-row
    tiles above where K is under 768: 512 here) and, from 129 rows with K of 768 or more, the
    tall kernel's 256 x 128 tiles (N 384: the last tile half of a 256-row chunk of the tiled
    operand); K of one group of 4 steps up to the down product's 12288:
    fp32 out, the gated residual and SwiGLU, from Q8_0 and from the resident bf16 expansion --
    the same bits from either, the same bits on a second call, and within 2e-6 of float64 on the
    same bf16 operands."""
    say("few-row products", M, N, K)
    rng = np.random.default_rng(M)
    xb = bf16(rng.normal(0, 1, (M, K)).astype(np.float32))
    w = X.Weight.synth(ctx, 5, 210, N, K)
    wf = xo.dequant_q8_0(*xo.q8_0_synth(5, 210, N, K))
    prod = from_bf16(xb).astype(np.float64) @ from_bf16(bf16(wf)).T.astype(np.float64)
    dx = dev(ctx, xb)
    outs = []
    for resident in (False, True, True):
        w.resident(resident)
        y = X.DevBuf(ctx, (M, N), np.float32)
        X.call("exn_mm", ctx.h, w.h, dx.h, X.DT_BF16, y.h, X.DT_F32, M)
        outs.append(y.get())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
    assert xo.rel_l2(outs[0], prod) < 2e-6
    # the gated residual, rows below p taking the second gate row
    resid = rng.normal(0, 1, (M, N)).astype(np.float32)
    gate = rng.normal(0, 0.5, (2, 4 * N)).astype(np.float32)
    n0, p = 3, 11
    got = []
    for resident in (False, True):
        w.resident(resident)
        r = dev(ctx, resid)
        X.call("exn_mm_gate_add", ctx.h, w.h, dx.h, M, r.h, n0, p, 4 * N, dev(ctx, gate).h)
        got.append(r.get())
    rows = np.where(n0 + np.arange(M) < p, 1, 0)
    want = resid + np.tanh(gate[rows, :N].astype(np.float64)) * prod
    assert np.array_equal(got[0], got[1]) and xo.rel_l2(got[0] - resid, want - resid) < 1e-5
    w.free()
    # SwiGLU on a paired gate_up matrix
    ws = X.Weight.synth(ctx, 5, 211, N, K)
    ws.pairs()
    wsf = xo.dequant_q8_0(*xo.q8_0_synth(5, 211, N, K))
    gu = from_bf16(xb).astype(np.float64) @ from_bf16(bf16(wsf)).T.astype(np.float64)
    F = N // 2
    ffs = []
    for resident in (False, True):
        ws.resident(resident)
        ff = X.DevBuf(ctx, (M, F), np.uint16)
        X.call("exn_mm_swiglu", ctx.h, ws.h, dx.h, ff.h, M)
        ffs.append(ff.get())
    assert np.array_equal(ffs[0], ffs[1])
    want = gu[:, :F] / (1 + np.exp(-gu[:, :F])) * gu[:, F:]
    assert xo.rel_l2(from_bf16(ffs[0]), want) < 4e-3
    ws.free()


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
def test_gemm_bf16_out_and_f32_in(ctx, resident):
    say("gemm f32 in, bf16 out; gemv n <= 4")
    rng = np.random.default_rng(1)
    M, N, K = 40, 256, 4096
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    w = X.Weight.synth(ctx, 4, 201, N, K)
    if resident:
        w.resident()
    wf = xo.dequant_q8_0(*xo.q8_0_synth(4, 201, N, K))
    dx = dev(ctx, x)
    y = X.DevBuf(ctx, (M, N), np.uint16)
    X.call("exn_mm", ctx.h, w.h, dx.h, X.DT_F32, y.h, X.DT_BF16, M)
    want = from_bf16(bf16(x)).astype(np.float64) @ from_bf16(bf16(wf)).T.astype(np.float64)
    assert xo.rel_l2(from_bf16(y.get()), want) < 4e-3
    # n <= 4, fp32 activations: the GEMV in fp32 (the timestep path)
    for m in (1, 2, 4):
        yg = X.DevBuf(ctx, (m, N), np.float32)
        X.call("exn_mm", ctx.h, w.h, dev(ctx, x[:m]).h, X.DT_F32, yg.h, X.DT_F32, m)
        assert xo.rel_l2(yg.get(), x[:m].astype(np.float64) @ wf.T.astype(np.float64)) < 1e-6


def test_gemm_weight_f32_branch(ctx):
    """A non-Q8_0 matrix (src/cuda-dit.lisp:77-80): F32 kept as fp32 rows and multiplied in fp32,
    as d41_mm_f32 (:127-130) -- against the float64 product of the unrounded operands, and
    visibly apart from a product of bf16-rounded weights; BF16 rows on the bf16 MFMA."""
    say("gemm f32 weight (fp32 product), bf16 weight")
    rng = np.random.default_rng(2)
    for M, N, K in ((100, 192, 256), (300, 4096, 4096)):
        wf = rng.normal(0, 0.05, (N, K)).astype(np.float32)      # not on the bf16 grid
        x = rng.normal(0, 1, (M, K)).astype(np.float32)
        w = X.Weight.f32(ctx, wf)
        y = X.DevBuf(ctx, (M, N), np.float32)
        X.call("exn_mm", ctx.h, w.h, dev(ctx, x).h, X.DT_F32, y.h, X.DT_F32, M)
        want = x.astype(np.float64) @ wf.T.astype(np.float64)
        e = xo.rel_l2(y.get(), want)
        e_b = xo.rel_l2(y.get(), x.astype(np.float64) @ from_bf16(bf16(wf)).T.astype(np.float64))
        say("f32 weight %dx%dx%d: rel-L2 %.2e to the fp32 product, %.2e to the bf16-weight product" % (M, N, K, e, e_b))
        # fp32 sums over K terms: rounding grows about as sqrt(K) x 2^-24 (4096: 4e-6)
        assert e < 4e-6 and e_b > 1e-4
        yg = X.DevBuf(ctx, (2, N), np.float32)
        X.call("exn_mm", ctx.h, w.h, dev(ctx, x[:2]).h, X.DT_F32, yg.h, X.DT_F32, 2)
        assert xo.rel_l2(yg.get(), want[:2]) < 4e-6
        # an fp32 matrix multiplies fp32 rows into fp32 rows only
        with pytest.raises(X.ExnError) as err:
            X.call("exn_mm", ctx.h, w.h, dev(ctx, bf16(x)).h, X.DT_BF16, y.h, X.DT_F32, M)
        assert err.value.code == X.EINVAL
        w.free()
    # a BF16 matrix: bf16 operands on the MFMA product
    M, N, K = 100, 192, 256
    wb = bf16(rng.normal(0, 0.05, (N, K)).astype(np.float32))
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    wbh = X.Weight.bf16(ctx, wb)
    y = X.DevBuf(ctx, (M, N), np.float32)
    X.call("exn_mm", ctx.h, wbh.h, dev(ctx, bf16(x)).h, X.DT_BF16, y.h, X.DT_F32, M)
    want = from_bf16(bf16(x)).astype(np.float64) @ from_bf16(wb).T.astype(np.float64)
    assert xo.rel_l2(y.get(), want) < 2e-6


# the block products of the cached 1024^2 pass's neighbour, the uncached pass: 4352 rows (4096 image +
# 256 text) through each block matrix with the Q8_0 dequantised inside the product
CFG1 = {"out": (4096, 4096), "gate_up": (2 * 12288, 4096), "down": (4096, 12288)}


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
@pytest.mark.parametrize("which", list(CFG1))
def test_block_products_at_4352_rows(ctx, which, resident):
    """to_out (+ gated residual), gate_up (+ SwiGLU) and down (+ gated residual) at M = 4352 from
    Q8_0 weights (the dequantisation inside the product) and from the resident bf16 expansion:
    sampled rows against float64 on the same bf16 operands and against the fp32 oracle."""
    N, K = CFG1[which]
    M = 4352
    say("block product", which, M, N, K, "resident" if resident else "q8_0")
    rng = np.random.default_rng(N + K)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    xb = bf16(x)
    seed, tid = 11, 300 + N // 4096 + K // 4096
    w = X.Weight.synth(ctx, seed, tid, N, K)
    if resident:
        w.resident()
    wf = xo.dequant_q8_0(*xo.q8_0_synth(seed, tid, N, K))
    rows = np.r_[0:64, 2000:2064, M - 64:M]
    xr = from_bf16(xb[rows]).astype(np.float64)
    prod = xr @ from_bf16(bf16(wf)).T.astype(np.float64)
    prod32 = x[rows] @ wf.T
    if which == "gate_up":
        w.pairs()
        F = N // 2
        ff = X.DevBuf(ctx, (M, F), np.uint16)
        X.call("exn_mm_swiglu", ctx.h, w.h, dev(ctx, xb).h, ff.h, M)
        got = from_bf16(ff.get()[rows])
        want = prod[:, :F] / (1 + np.exp(-prod[:, :F])) * prod[:, F:]
        e, e32 = xo.rel_l2(got, want), xo.rel_l2(got, xo.silu(prod32[:, :F]) * prod32[:, F:])
        say("swiglu rows rel-L2 %.2e (bf16 operands), %.2e (fp32 oracle)" % (e, e32))
        assert e < 4e-3 and e32 < 2e-2
    else:
        n0, p = 0, 256                          # the uncached pass: rows below 256 take the prompt's gate
        resid = rng.normal(0, 1, (M, N)).astype(np.float32)
        gate = rng.normal(0, 0.5, (2, 4 * N)).astype(np.float32)
        r = dev(ctx, resid)
        X.call("exn_mm_gate_add", ctx.h, w.h, dev(ctx, xb).h, M, r.h, n0, p, 4 * N, dev(ctx, gate).h)
        g = np.tanh(gate[np.where(rows < p, 1, 0), :N].astype(np.float64))
        got = r.get()[rows] - resid[rows]
        e, e32 = xo.rel_l2(got, g * prod), xo.rel_l2(got, g * prod32)
        say("gated residual rows rel-L2 %.2e (bf16 operands), %.2e (fp32 oracle)" % (e, e32))
        assert e < 1e-5 and e32 < 1e-2
    w.free()


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
def test_mm_gate_add(ctx, resident):
    """x += tanh(gate[row]) * (X W^T), rows below p taking the second gate row."""
    say("mm gate_add")
    rng = np.random.default_rng(3)
    M, N, K, n0, p = 200, 4096, 4096, 30, 100
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    resid = rng.normal(0, 1, (M, N)).astype(np.float32)
    gate = rng.normal(0, 0.5, (2, 4 * N)).astype(np.float32)
    w = X.Weight.synth(ctx, 6, 202, N, K)
    if resident:
        w.resident()
    wf = xo.dequant_q8_0(*xo.q8_0_synth(6, 202, N, K))
    r = dev(ctx, resid)
    g = dev(ctx, gate)
    X.call("exn_mm_gate_add", ctx.h, w.h, dev(ctx, bf16(x)).h, M, r.h, n0, p, 4 * N, g.h)
    h = from_bf16(bf16(x)).astype(np.float64) @ from_bf16(bf16(wf)).T.astype(np.float64)
    rows = np.where(n0 + np.arange(M) < p, 1, 0)
    want = resid + np.tanh(gate[rows, :N].astype(np.float64)) * h
    assert xo.rel_l2(r.get() - resid, want - resid) < 1e-5


@pytest.mark.parametrize("resident", [False, True], ids=["q8_0", "resident_bf16"])
def test_mm_swiglu(ctx, resident):
    say("mm swiglu")
    rng = np.random.default_rng(4)
    M, F, K = 150, 512, 4096
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    w = X.Weight.synth(ctx, 7, 203, 2 * F, K)
    if resident:           # expanded before the interleave: exn_weight_pairs re-expands it
        w.resident()
    w.pairs()
    wf = xo.dequant_q8_0(*xo.q8_0_synth(7, 203, 2 * F, K))
    ff = X.DevBuf(ctx, (M, F), np.uint16)
    X.call("exn_mm_swiglu", ctx.h, w.h, dev(ctx, bf16(x)).h, ff.h, M)
    gu = from_bf16(bf16(x)).astype(np.float64) @ from_bf16(bf16(wf)).T.astype(np.float64)
    want = gu[:, :F] / (1 + np.exp(-gu[:, :F])) * gu[:, F:]
    assert xo.rel_l2(from_bf16(ff.get()), want) < 4e-3
    assert xo.rel_l2(from_bf16(ff.get()), xo.silu((x @ wf.T)[:, :F]) * (x @ wf.T)[:, F:]) < 2e-2


# --- bandwidth kernels -------------------------------------------------------------------

def test_ln_mod(ctx):
    """inspect/metal-kernels-test.lisp:91-102's case: width 4096, n 9, n0 3, p 6, inputs x50."""
    say("ln_mod")
    rng = np.random.default_rng(7)
    n, n0, p = 9, 3, 6
    x = rng.uniform(-50, 50, (n, 4096)).astype(np.float32)
    mod = rng.uniform(-1, 1, (2, 4096)).astype(np.float32)
    rows = np.where(n0 + np.arange(n) < p, 1, 0)
    want = xo.layernorm(x.astype(np.float64)) * (1 + mod[rows])
    out = X.DevBuf(ctx, (n, 4096), np.float32)
    X.call("exn_ln_mod", ctx.h, n, n0, p, 4096, dev(ctx, x).h, 4096, dev(ctx, mod).h, out.h, X.DT_F32)
    assert np.abs(out.get() - want).max() / np.abs(want).max() < 1e-5
    outb = X.DevBuf(ctx, (n, 4096), np.uint16)
    X.call("exn_ln_mod", ctx.h, n, n0, p, 4096, dev(ctx, x).h, 4096, dev(ctx, mod).h, outb.h, X.DT_BF16)
    assert np.abs(from_bf16(outb.get()) - want).max() / np.abs(want).max() < 4e-3
    # the final norm: one scale row for all rows (mstride 0, p 0), rows LDX apart
    xs = rng.normal(0, 3, (5, 2 * 4096)).astype(np.float32)
    sc = rng.normal(0, 1, 4096).astype(np.float32)
    o2 = X.DevBuf(ctx, (5, 4096), np.float32)
    X.call("exn_ln_mod", ctx.h, 5, 0, 0, 0, dev(ctx, xs).h, 2 * 4096, dev(ctx, sc).h, o2.h, X.DT_F32)
    w2 = xo.layernorm(xs[:, :4096].astype(np.float64)) * (1 + sc)
    assert np.abs(o2.get() - w2).max() / np.abs(w2).max() < 1e-5


def test_rms(ctx):
    """inspect/metal-kernels-test.lisp:104-111's case: width 3072, n 5, inputs x100."""
    say("rms")
    rng = np.random.default_rng(8)
    x = rng.uniform(-100, 100, (5, 3072)).astype(np.float32)
    w = rng.uniform(-1, 1, 3072).astype(np.float32)
    want = xo.rmsnorm(x.astype(np.float64), w)
    y = X.DevBuf(ctx, (5, 3072), np.float32)
    X.call("exn_rms", ctx.h, 5, 3072, 1e-6, dev(ctx, x).h, dev(ctx, w).h, y.h, X.DT_F32)
    assert np.abs(y.get() - want).max() / np.abs(want).max() < 1e-5


def test_gate_add_swiglu_gelu_silu_euler(ctx):
    say("gate_add swiglu gelu silu euler")
    rng = np.random.default_rng(9)
    n, W, n0, p = 37, 4096, 5, 20
    x = rng.normal(0, 1, (n, W)).astype(np.float32)
    h = rng.normal(0, 1, (n, W)).astype(np.float32)
    gate = rng.normal(0, 1, (2, 4 * W)).astype(np.float32)
    dx = dev(ctx, x)
    X.call("exn_gate_add", ctx.h, n * W, W, n0, p, 4 * W, dx.h, dev(ctx, h).h, dev(ctx, gate).h)
    rows = np.where(n0 + np.arange(n) < p, 1, 0)
    want = x + np.tanh(gate[rows, :W]) * h
    assert np.abs(dx.get() - want).max() < 1e-5
    # swiglu (bf16 in and out)
    f = 12288
    gu = rng.normal(0, 2, (7, 2 * f)).astype(np.float32)
    gub = bf16(gu)
    o = X.DevBuf(ctx, (7, f), np.uint16)
    X.call("exn_swiglu", ctx.h, 7, f, dev(ctx, gub).h, o.h)
    g64 = from_bf16(gub).astype(np.float64)
    wsw = g64[:, :f] / (1 + np.exp(-g64[:, :f])) * g64[:, f:]
    assert np.abs(from_bf16(o.get()) - wsw).max() / np.abs(wsw).max() < 4e-3
    # gelu, silu (fp32 in place)
    v = np.linspace(-10, 10, 5001).astype(np.float32)
    dv = dev(ctx, v)
    X.call("exn_gelu_tanh", ctx.h, v.size, dv.h)
    assert np.abs(dv.get() - xo.gelu_tanh(v.astype(np.float64))).max() < 2e-6
    dv = dev(ctx, v)
    X.call("exn_silu", ctx.h, v.size, dv.h)
    assert np.abs(dv.get() - xo.silu(v.astype(np.float64))).max() < 2e-6
    # euler: z + ds * v, two single-float roundings (src/generate.lisp:135)
    z = rng.normal(0, 1, 1000).astype(np.float32)
    vv = rng.normal(0, 1, 1000).astype(np.float32)
    ds = np.float32(0.414568 - 0.704534)
    dz = dev(ctx, z)
    X.call("exn_euler", ctx.h, 1000, dz.h, dev(ctx, vv).h, ds)
    assert (dz.get() == z + ds * vv).all()


def _qkv_case(ctx, n, row0, lcap, seed):
    rng = np.random.default_rng(seed)
    qkv = rng.normal(0, 3, (n, 3 * 4096)).astype(np.float32)
    qkvb = f16(qkv)
    wq = (1 + 0.1 * rng.normal(0, 1, 128)).astype(np.float32)
    wk = (1 + 0.1 * rng.normal(0, 1, 128)).astype(np.float32)
    pos = rng.integers(-32, 300, (row0 + n, 3)).astype(np.float32)
    cos, sin = xo.rope_tables(pos)
    cs = np.stack([cos, sin], -1).reshape(row0 + n, 128).astype(np.float32)
    q = X.DevBuf(ctx, (32, n, 128), np.uint16)
    k = X.DevBuf(ctx, (32, lcap, 128), np.uint16)
    vt = X.DevBuf(ctx, (32, 128, lcap), np.uint16)
    X.call("exn_qkv_prep", ctx.h, dev(ctx, qkvb).h, n, dev(ctx, wq).h, dev(ctx, wk).h, dev(ctx, cs).h, q.h, k.h,
           vt.h, row0, lcap)
    f = from_f16(qkvb).reshape(n, 3, 32, 128).astype(np.float64)
    c, s = cos[row0:], sin[row0:]
    wantq = xo.rope(xo.rmsnorm(f[:, 0], wq), c, s) * (math.log2(math.e) / math.sqrt(128))
    wantk = xo.rope(xo.rmsnorm(f[:, 1], wk), c, s)
    return q.get(), k.get(), vt.get(), wantq, wantk, f[:, 2]


def test_qkv_prep(ctx):
    """x_qk_norm_rope's computation (src/cuda/dit.cu:43-58), its outputs rounded to
    halves as the Metal twin's are (bound 2e-3 there, inspect/metal-kernels-test.lisp:
    113-128), and v transposed."""
    say("qkv_prep n 70 row0 33 lcap 128")
    n, row0, lcap = 70, 33, 128
    gq, gk, gvt, wq, wk, wv = _qkv_case(ctx, n, row0, lcap, 11)
    gotq = from_f16(gq).transpose(1, 0, 2)
    gotk = from_f16(gk[:, row0:row0 + n]).transpose(1, 0, 2)
    assert np.abs(gotq - wq).max() / np.abs(wq).max() < 2e-3
    assert np.abs(gotk - wk).max() / np.abs(wk).max() < 2e-3
    gotv = from_f16(gvt[:, :, vt_pos(np.arange(row0, row0 + n))]).transpose(2, 0, 1)
    assert (gotv == wv).all()                                   # v only moves: bit-exact
    assert sorted(vt_pos(np.arange(lcap))) == list(range(lcap))  # a permutation inside each 16 keys


@pytest.mark.parametrize("resident", [True, False], ids=["resident_bf16", "q8_0"])
@pytest.mark.parametrize("n,row0,lcap", [(300, 37, 384), (512, 256, 832), (257, 0, 320)])
def test_mm_qkv_fused(ctx, n, row0, lcap, resident):
    """exn_mm_qkv: the QKV product with x_qk_norm_rope and the K/V^T stores in its epilogue,
    against the unfused pair (exn_mm to fp16 rows, then exn_qkv_prep) on the same operands --
    V^T bit-exact (the same fp32 sums, rounded once), q and k within fp16 rounding -- and
    against float64 on three heads.  row0 37: V^T key by key; 256: 16 keys at once; n 257:
    a last tile of one row.  K rows and V^T columns outside row0 .. row0+n-1 stay as they were.
    From the resident bf16 expansion or from Q8_0 dequantised in the product."""
    say("mm_qkv n", n, "row0", row0, "lcap", lcap, "resident" if resident else "q8_0")
    rng = np.random.default_rng(n + row0)
    w = X.Weight.synth(ctx, 9, 400, 3 * 4096, 4096).resident(resident)
    x = rng.normal(0, 1, (n, 4096)).astype(np.float32)
    xb = bf16(x)
    wq = (1 + 0.1 * rng.normal(0, 1, 128)).astype(np.float32)
    wk = (1 + 0.1 * rng.normal(0, 1, 128)).astype(np.float32)
    pos = rng.integers(-32, 300, (row0 + n, 3)).astype(np.float32)
    cos, sin = xo.rope_tables(pos)
    cs = np.stack([cos, sin], -1).reshape(row0 + n, 128).astype(np.float32)
    dx, dwq, dwk, dcs = dev(ctx, xb), dev(ctx, wq), dev(ctx, wk), dev(ctx, cs)
    SENT = 0x7BFF
    outs = []
    for fused in (True, False):
        q = X.DevBuf.of(ctx, np.full((32, n, 128), SENT, np.uint16))
        k = X.DevBuf.of(ctx, np.full((32, lcap, 128), SENT, np.uint16))
        vt = X.DevBuf.of(ctx, np.full((32, 128, lcap), SENT, np.uint16))
        if fused:
            X.call("exn_mm_qkv", ctx.h, w.h, dx.h, n, dwq.h, dwk.h, dcs.h, q.h, k.h, vt.h, row0, lcap)
        else:
            qkv = X.DevBuf(ctx, (n, 3 * 4096), np.uint16)
            X.call("exn_mm", ctx.h, w.h, dx.h, X.DT_BF16, qkv.h, 2, n)
            X.call("exn_qkv_prep", ctx.h, qkv.h, n, dwq.h, dwk.h, dcs.h, q.h, k.h, vt.h, row0, lcap)
        outs.append((q.get(), k.get(), vt.get()))
    (fq, fk, fvt), (uq, uk, uvt) = outs
    cols = vt_pos(np.arange(row0, row0 + n))
    outside = np.setdiff1d(np.arange(lcap), cols)
    assert (fk[:, :row0] == SENT).all() and (fk[:, row0 + n:] == SENT).all()
    assert (fvt[:, :, outside] == SENT).all()
    assert np.array_equal(fvt[:, :, cols], uvt[:, :, cols])
    for a, b in ((fq, uq), (fk[:, row0:row0 + n], uk[:, row0:row0 + n])):
        fa, fb = from_f16(a), from_f16(b)
        assert np.abs(fa - fb).max() <= 2e-3 * np.abs(fb).max()
    # float64 on heads 0, 17, 31 of q, k and v: bf16 operands, the oracle's norm and rotation
    wf = xo.dequant_q8_0(*xo.q8_0_synth(9, 400, 3 * 4096, 4096))
    wb = from_bf16(bf16(wf)).astype(np.float64)
    xf = from_bf16(xb).astype(np.float64)
    c, sn = cos[row0:], sin[row0:]
    for hh in (0, 17, 31):
        y = [xf @ wb[part * 4096 + hh * 128:part * 4096 + hh * 128 + 128].T for part in range(3)]
        wantq = xo.rope(xo.rmsnorm(y[0][:, None], wq), c, sn)[:, 0] * (math.log2(math.e) / math.sqrt(128))
        wantk = xo.rope(xo.rmsnorm(y[1][:, None], wk), c, sn)[:, 0]
        gq = from_f16(fq[hh]).astype(np.float64)
        gk = from_f16(fk[hh, row0:row0 + n]).astype(np.float64)
        gv = from_f16(fvt[hh][:, cols]).T.astype(np.float64)
        assert np.abs(gq - wantq).max() <= 2e-3 * np.abs(wantq).max()
        assert np.abs(gk - wantk).max() <= 2e-3 * np.abs(wantk).max()
        assert np.abs(gv - y[2]).max() <= 2 ** -10 * np.abs(y[2]).max() + 1e-3


def vt_pos(k):
    """V^T's column of key k (exn_qkv_prep's layout): bits 2 and 3 swapped."""
    k = np.asarray(k)
    return k ^ ((((k >> 2) ^ (k >> 3)) & 1) * 12)


def _attend_case(ctx, n, q0, p, l, b0, b1, seed, heads_checked=(0, 7, 31), prescaled=False):
    """prescaled: q is stored times log2(e)/sqrt(128), as exn_qkv_prep leaves it for the
    DiT, and the kernel's own scale is 1."""
    rng = np.random.default_rng(seed)
    lcap = (l + 63) // 64 * 64
    q = rng.uniform(-2, 2, (n, 32, 128)).astype(np.float32)
    k = rng.uniform(-2, 2, (l, 32, 128)).astype(np.float32)
    v = rng.uniform(-1, 1, (l, 32, 128)).astype(np.float32)
    scale = 1 / math.sqrt(128)
    kscale = scale * math.log2(math.e)
    if prescaled:
        q = q * np.float32(kscale)
        scale, kscale = 1 / math.log2(math.e), 1.0
    qb, kb, vb = f16(q), f16(k), f16(v)
    qh = np.ascontiguousarray(qb.transpose(1, 0, 2))                         # [32][n][128]
    kh = np.zeros((32, lcap, 128), np.uint16)
    kh[:, :l] = kb.transpose(1, 0, 2)
    vth = np.zeros((32, 128, lcap), np.uint16)
    vth[:, :, vt_pos(np.arange(l))] = vb.transpose(1, 2, 0)
    out = X.DevBuf(ctx, (n, 4096), np.uint16)
    X.call("exn_attend", ctx.h, dev(ctx, qh).h, dev(ctx, kh).h, dev(ctx, vth).h, out.h, n, q0, p, l, lcap, b0, b1,
           kscale)
    got = from_bf16(out.get()).reshape(n, 32, 128)
    qf, kf, vf = (from_f16(a).astype(np.float64) for a in (qb, kb, vb))
    want = np.zeros((n, len(heads_checked), 128))
    for t in range(n):
        lim = int(xo.xa_lim(q0 + t, p, l, b0, b1))
        for j, h in enumerate(heads_checked):
            s = kf[:lim + 1, h] @ qf[t, h] * scale
            e = np.exp(s - s.max())
            want[t, j] = e @ vf[:lim + 1, h] / e.sum()
    return got[:, list(heads_checked)], want


@pytest.mark.parametrize("n,q0,p,l,b0,b1", [(77, 0, 20, 77, 20, 20), (70, 33, 33, 103, 33, 33),
                                            (90, 0, 40, 90, 12, 30)])
def test_attention_mask_cases(ctx, n, q0, p, l, b0, b1):
    """The three mask cases of inspect/metal-kernels-test.lisp:144-146, float64
    brute force on the same fp16 inputs; the bound is the Metal test's 3e-3 for
    P in halves, plus the output's rounding to bf16 (2^-9 of |out| <= 1)."""
    say("attend", n, q0, p, l, b0, b1)
    got, want = _attend_case(ctx, n, q0, p, l, b0, b1, n + l)
    assert np.abs(got - want).max() < 3e-3 + 2 ** -9
    assert xo.rel_l2(got, want) < 3e-3


def test_attention_longer(ctx):
    """Image queries after a cached prompt over several key tiles, every head."""
    say("attend 300 queries over 556 keys")
    got, want = _attend_case(ctx, 300, 256, 256, 556, 0, 0, 5, heads_checked=tuple(range(0, 32, 3)))
    assert xo.rel_l2(got, want) < 3e-3


@pytest.mark.parametrize("n,q0,p,l,b0,b1", [(300, 256, 256, 556, 0, 0), (90, 0, 40, 90, 12, 30),
                                            (200, 0, 72, 200, 0, 0), (64, 64, 64, 128, 0, 0)])
def test_attention_prescaled(ctx, n, q0, p, l, b0, b1):
    """The DiT's call: q already in log2 units (times log2(e)/sqrt(128)) and scale 1, the
    path where each tile's product starts from minus the running max.  Tile counts odd
    and even, one and several."""
    say("attend prescaled", n, q0, p, l, b0, b1)
    got, want = _attend_case(ctx, n, q0, p, l, b0, b1, 7 + n, prescaled=True)
    assert np.abs(got - want).max() < 3e-3 + 2 ** -9
    assert xo.rel_l2(got, want) < 3e-3


# --- the int8 products (src/cuda-dit.lisp:110-126) ------------------------------------------

def test_quant_q8_bit_exact(ctx):
    """exn_quant_q8 against the oracle's quant_q8_0, code for code and scale for scale: rows at
    magnitudes 1e-3 .. 1e3, a zero block, a block whose x / d lands half-way (away from zero),
    from fp32 rows and from bf16 rows, with a row stride past K."""
    rng = np.random.default_rng(21)
    n, K, ld = 300, 4096, 4096 + 64
    x = (rng.normal(0, 1, (n, ld)) * rng.uniform(1e-3, 1e3, (n, 1))).astype(np.float32)
    x[5, 64:96] = 0
    x[7, :32] = 0
    x[7, :5] = [0.5, 2.5, -1.5, 126.5, 127.0]
    for dt in (X.DT_F32, X.DT_BF16):
        xin = x if dt == X.DT_F32 else bf16(x)
        want = x[:, :K] if dt == X.DT_F32 else from_bf16(bf16(x))[:, :K]
        q = X.DevBuf(ctx, (n, K), np.int8)
        dd = X.DevBuf(ctx, (n, K // 32), np.uint16)
        X.call("exn_quant_q8", ctx.h, dev(ctx, xin).h, dt, ld, n, K, q.h, dd.h)
        wq, wd = xo.quant_q8_0(want)
        gq, gd = q.get(), dd.get()
        say("quant_q8 from %s: codes equal %s, scales equal %s" % ("fp32" if dt == X.DT_F32 else "bf16",
                                                                 np.array_equal(gq, wq), np.array_equal(gd, wd.view(np.uint16))))
        assert np.array_equal(gq, wq) and np.array_equal(gd, wd.view(np.uint16))
        if dt == X.DT_F32:
            assert list(gq[7, :5]) == [1, 3, -2, 127, 127] and not gq[5, 64:96].any() and gd[5, 2] == 0


# K = 96 (3 blocks) takes the product without the DMA path (K not a multiple of 64)
W8A8_CASES = [(64, 256, 4096), (300, 4096, 4096), (77, 12288, 4096), (128, 4096, 12288), (40, 4096, 64),
              (50, 256, 96)]


@pytest.mark.parametrize("M,N,K", W8A8_CASES)
def test_mm_w8a8_bit_exact(ctx, M, N, K):
    """exn_mm_w8a8 on exn_quant_q8's codes against the oracle's linear_w8a8, bit for bit (the
    same exact integer block sums, float32 scale products and single-rounding fused
    multiply-adds in the same order): partial tiles in M and N, K of 2 to 384 blocks, through
    the DMA path and (K = 96) the direct one; fp16 out equal to the fp32 result rounded."""
    say("mm_w8a8", M, N, K)
    rng = np.random.default_rng(M + N + K)
    x = (rng.normal(0, 1, (M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    seed, tid = 12, 400 + N // 64 + K // 64
    w = X.Weight.synth(ctx, seed, tid, N, K)
    qs, d = xo.q8_0_synth(seed, tid, N, K)
    q = X.DevBuf(ctx, (M, K), np.int8)
    dd = X.DevBuf(ctx, (M, K // 32), np.uint16)
    X.call("exn_quant_q8", ctx.h, dev(ctx, x).h, X.DT_F32, K, M, K, q.h, dd.h)
    y = X.DevBuf(ctx, (M, N), np.float32)
    X.call("exn_mm_w8a8", ctx.h, w.h, q.h, dd.h, M, y.h, X.DT_F32)
    got, want = y.get(), xo.linear_w8a8(x, qs, d)
    say("bit-exact %s, rel-L2 %.2e; against the unquantised product %.2e" %
        (np.array_equal(got, want), xo.rel_l2(got, want), xo.rel_l2(got, x @ xo.dequant_q8_0(qs, d).T)))
    assert np.array_equal(got, want)
    y16 = X.DevBuf(ctx, (M, N), np.uint16)
    X.call("exn_mm_w8a8", ctx.h, w.h, q.h, dd.h, M, y16.h, X.DT_F16)
    assert np.array_equal(y16.get(), want.astype(np.float16).view(np.uint16))


def test_allocation_failure_is_a_status(ctx):
    """exn_alloc of an absurd size (1 PiB) returns EXN_ENOMEM with a message naming the size,
    raises nothing, and leaves the context usable: a buffer, an upload and a product after it."""
    h = ctypes.c_void_p()
    code = X.lib().exn_alloc(ctx.h, ctypes.c_size_t(1 << 50), ctypes.byref(h))
    msg = X.lib().exn_last_error().decode()
    say("exn_alloc(1 PiB): status %d, %s" % (code, msg))
    assert code == X.ENOMEM and "hipMalloc" in msg and str(1 << 50) in msg and not h.value
    rng = np.random.default_rng(21)
    w = X.Weight.synth(ctx, 9, 403, 256, 512)
    x = dev(ctx, rng.normal(0, 1, (64, 512)).astype(np.float32))
    y = X.DevBuf(ctx, (64, 256), np.float32)
    X.call("exn_mm", ctx.h, w.h, x.h, X.DT_F32, y.h, X.DT_F32, 64)
    want = x.get() @ xo.dequant_q8_0(*xo.q8_0_synth(9, 403, 256, 512)).T
    assert xo.rel_l2(y.get(), want) < 1e-2
    w.free()
