"""The oracle pinned: against the reference's own numpy DiT (golden vectors
from inspect/ref_dit.py), against its C twin, against numpy's and torch's
IEEE conversions, and against closed forms, invariants and float64 brute
force.  CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import exn_oracle as xo

TINY = xo.Shape(width=256, layers=2, head_dim=128, ffn=512, latent=64, context=256, freq=256)


def _c():
    lib = xo.clib()
    if lib is None:
        pytest.fail("oracle/liboracle.so is not built (make -C oracle)")
    return lib


# --- the Q8_0 codec and the conversions ---------------------------------------------

def test_f16_to_f32_exhaustive():
    lib = _c()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.exo_f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    w = want[::7]
    same = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
    assert same.all()


def test_f16_rne_against_numpy():
    lib = _c()
    rng = np.random.default_rng(1)
    # every fp16 rounding boundary (the midpoints), one fp32 ulp either side, plus random values
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    pts = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf)),
                          np.abs(rng.normal(0, 2e-4, 20000)).astype(np.float32),
                          rng.uniform(-7e4, 7e4, 2000).astype(np.float32),
                          np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24], np.float32)])
    pts = pts[::3].astype(np.float32)
    got = np.array([lib.exo_f16_rne(float(x)) for x in pts], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = pts.astype(np.float16).view(np.uint16)
    assert (got == want).all(), pts[got != want][:5]


def test_bf16_rne_three_ways():
    lib = _c()
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.normal(0, 1, 50000), rng.normal(0, 1e-30, 1000), rng.normal(0, 1e30, 1000),
                        [0.0, -0.0, np.inf, -np.inf, 3.4e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]]).astype(np.float32)
    a = xo.bf16_bits(x)
    b = np.empty_like(a)
    lib.exo_bf16_rne_n(xo._ptr(x), xo._ptr(b), x.size)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (a == b).all() and (a == t).all()


def test_dequant_exhaustive_closed_form():
    """fp32(d) * q for every finite fp16 d and every int8 q, -128 and 0 included:
    the numpy and C dequant both equal the float64 product (exact in fp32)."""
    lib = _c()
    d = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    d = d[np.isfinite(d.view(np.float16))]
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    nb = d.size * 8                               # 8 blocks of 32 q values per d
    blocks = np.empty((nb, 34), np.uint8)
    blocks[:, 0:2] = np.repeat(d, 8).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = np.tile(q.view(np.uint8).reshape(8, 32), (d.size, 1))
    got = xo.dequant_q8_0_blocks(blocks)
    want = (np.repeat(d.view(np.float16).astype(np.float64), 256) * np.tile(q.astype(np.float64), d.size))
    assert (want.astype(np.float32) == want).all()          # exactness of the product itself
    assert (got == want.astype(np.float32)).all()
    gc = np.empty(nb * 32, np.float32)
    lib.exo_dequant_q8_0_blocks(xo._ptr(blocks), nb, xo._ptr(gc))
    assert (gc.view(np.uint32) == got.view(np.uint32)).all()


def test_generator_numpy_equals_c():
    lib = _c()
    for seed, tid, rows, cols in [(0, 0, 3, 64), (7, 42, 17, 96), (2 ** 40 + 5, 265, 5, 4096)]:
        qs, d = xo.q8_0_synth(seed, tid, rows, cols)
        qc = np.empty((rows, cols), np.int8)
        dc = np.empty((rows, cols // 32), np.uint16)
        lib.exo_q8_0_synth(seed, tid, rows, cols, xo._ptr(qc), xo._ptr(dc))
        assert (qs == qc).all() and (d.view(np.uint16) == dc).all()
        bl = np.empty(rows * cols // 32 * 34, np.uint8)
        lib.exo_q8_0_synth_blocks(seed, tid, rows, cols, xo._ptr(bl))
        assert (bl == xo.q8_0_to_blocks(qs, d)).all()
        z = xo.normal(seed, tid, 1000)
        zc = np.empty(1000, np.float32)
        lib.exo_normal(seed, tid, 1000, xo._ptr(zc))
        assert (z.view(np.uint32) == zc.view(np.uint32)).all()


def test_generator_distribution():
    qs, d = xo.q8_0_synth(5, 3, 256, 4096)
    assert qs.min() == -127 and qs.max() == 127
    assert abs(qs.astype(np.float64).mean()) < 0.2
    dd = d.astype(np.float64)
    assert (dd >= 0).all()
    # |N(0, 2e-4)|: E|z| = sigma sqrt(2/pi) for a normal; Irwin-Hall of 4 gives 1.5% more
    assert abs(dd.mean() / (2e-4 * math.sqrt(2 / math.pi)) - 1) < 0.04
    assert (dd < 6.103515625e-05).mean() > 0.1                # fp16 subnormal scales occur
    z = xo.normal(1, 2, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


# --- forward against the reference's own numpy DiT ------------------------------------

@pytest.mark.parametrize("case", [0, 1, 2])
def test_forward_matches_ref_dit_vectors(golden, case):
    seed, p, h, w, sigma = golden["c%d_meta" % case]
    seed, p, h, w = int(seed), int(p), int(h), int(w)
    wt = xo.SynthWeights(seed, TINY, gain=4.0)
    ctx, lat = xo.synth_inputs(seed, p, h, w, TINY)
    assert (ctx == golden["c%d_ctx" % case]).all() and (lat == golden["c%d_latent" % case]).all()
    wsum = np.array([float(np.sum(wt(n), dtype=np.float64)) for n, _ in xo.dit_expected(TINY)])
    assert (wsum == golden["c%d_wsum" % case]).all()
    dump = {}
    v = xo.forward(wt, ctx, lat, float(sigma), TINY, dump=dump)
    assert xo.rel_l2(dump["txt"], golden["c%d_txt" % case]) < 1e-6
    assert xo.rel_l2(dump["blk"][0], golden["c%d_blk0" % case]) < 1e-6
    assert xo.rel_l2(v, golden["c%d_v" % case]) < 1e-5
    # the fixture is sensitive: block 0 moves x by far more than the tolerance
    x_in = np.concatenate([dump["txt"], xo.linear(xo.tokens(lat), wt("img_in.weight"))])
    assert xo.rel_l2(golden["c%d_blk0" % case], x_in) > 1e-2


# --- the pieces: closed forms, invariants, brute force --------------------------------

def test_layernorm_rmsnorm():
    rng = np.random.default_rng(3)
    x = (rng.normal(0, 1, (9, 4096)) * 50 + 3).astype(np.float32)
    y = xo.layernorm(x).astype(np.float64)
    assert np.abs(y.mean(-1)).max() < 1e-5 and np.abs(y.var(-1) - 1).max() < 1e-5
    w = rng.normal(0, 1, 4096).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.abs(xo.rmsnorm(x, w) - want).max() / np.abs(want).max() < 1e-5


def test_activations_closed_forms():
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    g = np.array([0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))) for v in x.astype(float)])
    assert np.abs(xo.gelu_tanh(x) - g).max() < 1e-5
    s = np.array([v / (1 + math.exp(-v)) for v in x.astype(float)])
    assert np.abs(xo.silu(x) - s).max() < 1e-5
    # gelu's tanh form stays within 1e-3 of the erf form
    e = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(float)])
    assert np.abs(xo.gelu_tanh(x) - e).max() < 1e-3


def test_timestep_embedding():
    e0 = xo.timestep_embedding(0.0)
    assert (e0[:128] == 1).all() and (e0[128:] == 0).all()
    for t in (1.0, 500.0, 978.453):
        f = [math.exp(-math.log(1e4) * j / 128) for j in range(128)]      # host.lisp:9-15, in double
        want = np.array([math.cos(t * fj) for fj in f] + [math.sin(t * fj) for fj in f])
        assert np.abs(xo.timestep_embedding(t) - want).max() < 2e-4


def test_positions_plain_and_edit():
    pos = xo.positions(3, 3, 4)
    assert pos.shape == (15, 3)
    assert (pos[:3] == np.array([[0, 0, 0], [1, 1, 1], [2, 2, 2]])).all()
    assert (pos[3:, 0] == 3).all()
    assert sorted(set(pos[3:, 1])) == [-2, -1, 0] and sorted(set(pos[3:, 2])) == [-2, -1, 0, 1]
    assert (pos[3:, 1] == np.repeat([-2, -1, 0], 4)).all() and (pos[3:, 2] == np.tile([-2, -1, 0, 1], 3)).all()
    # edit: 2 text rows, a 2x3 picture, 4 text rows after, then the 3x4 image (p = 2 + 6 + 4)
    e = xo.positions(12, 3, 4, ref=(2, 2, 3))
    assert e.shape == (24, 3)
    assert (e[:2] == [[0, 0, 0], [1, 1, 1]]).all()
    assert (e[2:8, 0] == 2).all() and (e[2:8, 1] == np.repeat([-1, 0], 3)).all() and (e[2:8, 2] == np.tile([-2, -1, 0], 2)).all()
    assert (e[8:12] == np.repeat((2 + 3 + np.arange(4))[:, None], 3, 1)).all()
    assert (e[12:, 0] == 2 + 3 + 4).all()
    assert (e[12:, 1:] == pos[3:, 1:]).all()
    # a reference picture of zero rows is the plain case
    assert (xo.positions(5, 3, 4, ref=(5, 0, 0)) == xo.positions(5, 3, 4)).all()


def test_rope_invariants():
    rng = np.random.default_rng(4)
    pos = rng.integers(-40, 300, (20, 3)).astype(np.float32)
    cos, sin = xo.rope_tables(pos)
    assert cos.shape == (20, 64)
    x = rng.normal(0, 1, (20, 2, 128)).astype(np.float32)
    r = xo.rope(x, cos, sin)
    pair = lambda a: a[..., 0::2] ** 2 + a[..., 1::2] ** 2
    assert np.abs(pair(r) - pair(x)).max() < 1e-4
    c0, s0 = xo.rope_tables(np.zeros((1, 3), np.float32))
    assert (xo.rope(x[:1], c0, s0) == x[:1]).all()
    # relative positions: <rope(q, i), rope(k, j)> depends on i - j per axis only
    q, k = x[0:1], x[1:2]
    d = np.array([[5, -3, 7]], np.float32)
    for base in ([0, 0, 0], [11, 20, -9]):
        bq = np.array([base], np.float32)
        cq, sq = xo.rope_tables(bq + d)
        ck, sk = xo.rope_tables(bq)
        dot = float(np.sum(xo.rope(q, cq, sq) * xo.rope(k, ck, sk)))
        if base == [0, 0, 0]:
            ref = dot
    assert abs(dot - ref) < 1e-3
    # the angle of pair i of axis a is pos_a / theta^(2i/d_a); first pair of each axis turns by pos itself
    cos1, sin1 = xo.rope_tables(np.array([[1.0, 2.0, 3.0]], np.float32))
    assert abs(cos1[0, 0] - math.cos(1)) < 1e-7 and abs(cos1[0, 8] - math.cos(2)) < 1e-7
    assert abs(cos1[0, 36] - math.cos(3)) < 1e-7


def test_xa_lim_mask():
    # src/cuda/dit.cu:60-66 -- image rows see all keys, the reference block itself whole, the rest causal
    p, l, b0, b1 = 40, 90, 12, 30
    g = np.arange(90)
    lim = xo.xa_lim(g, p, l, b0, b1)
    assert (lim[:12] == g[:12]).all() and (lim[12:30] == 29).all() and (lim[30:40] == g[30:40]).all()
    assert (lim[40:] == 89).all()
    assert (np.diff(lim) >= 0).all()


def _attention_brute(q, k, v, q0, p, b0, b1):
    n, H, hd = q.shape
    l = k.shape[0]
    out = np.zeros((n, H, hd))
    for t in range(n):
        g = q0 + t
        lim = l - 1 if g >= p else (b1 - 1 if b0 <= g < b1 else g)
        for h in range(H):
            s = np.array([float(np.dot(q[t, h].astype(np.float64), k[j, h].astype(np.float64))) for j in range(lim + 1)])
            s /= math.sqrt(hd)
            e = np.exp(s - s.max())
            out[t, h] = (e[:, None] * v[:lim + 1, h].astype(np.float64)).sum(0) / e.sum()
    return out


# the three mask cases of inspect/metal-kernels-test.lisp:144-146: (n, q0, p, l, b0, b1)
MASK_CASES = [(77, 0, 20, 77, 20, 20), (70, 33, 33, 103, 33, 33), (90, 0, 40, 90, 12, 30)]


@pytest.mark.parametrize("n,q0,p,l,b0,b1", MASK_CASES)
def test_attention_brute_force(n, q0, p, l, b0, b1):
    rng = np.random.default_rng(n)
    q = rng.uniform(-2, 2, (n, 2, 128)).astype(np.float32)
    k = rng.uniform(-2, 2, (l, 2, 128)).astype(np.float32)
    v = rng.uniform(-1, 1, (l, 2, 128)).astype(np.float32)
    got = xo.attention(q, k, v, q0, p, b0, b1)
    want = _attention_brute(q, k, v, q0, p, b0, b1)
    assert np.abs(got - want).max() < 1e-5


def test_attention_invariants():
    rng = np.random.default_rng(5)
    n, l, p = 30, 50, 20
    q = rng.normal(0, 2, (n, 2, 128)).astype(np.float32)
    k = rng.normal(0, 2, (l, 2, 128)).astype(np.float32)
    v = np.broadcast_to(rng.normal(0, 1, (1, 2, 128)), (l, 2, 128)).astype(np.float32)
    out = xo.attention(q, k, v, 20, p)
    assert np.abs(out - v[:n]).max() < 1e-5                   # constant V comes back
    # a prompt query (q0 = 0) does not see keys past itself: changing them changes nothing
    v2 = rng.normal(0, 1, (l, 2, 128)).astype(np.float32)
    a = xo.attention(q[:10], k, v2, 0, p)
    k3, v3 = k.copy(), v2.copy()
    k3[10:] = 0
    v3[10:] = 9
    b = xo.attention(q[:10], k3, v3, 0, p)
    assert np.abs(a - b).max() < 1e-6


def test_prefix_cache_matches_uncached():
    """The cached pass (image rows against the kept prompt K/V) gives the
    uncached pass's velocity (src/cuda-dit.lisp:6-9)."""
    wt = xo.SynthWeights(9, TINY, gain=4.0)
    ctx, lat = xo.synth_inputs(9, 6, 3, 4, TINY)
    cache = xo.PrefixCache()
    v1 = xo.forward(wt, ctx, lat, 0.9, TINY, cache=cache, prefix_key="k")
    assert cache.key == "k" and cache.length == 6
    v2 = xo.forward(wt, ctx, lat, 0.9, TINY, cache=cache, prefix_key="k")
    v0 = xo.forward(wt, ctx, lat, 0.9, TINY)
    assert xo.rel_l2(v1, v0) < 1e-6 and xo.rel_l2(v2, v0) < 1e-5
    # another sigma: the kept prompt K/V still serve (they do not depend on t)
    v3 = xo.forward(wt, ctx, lat, 0.5, TINY, cache=cache, prefix_key="k")
    assert xo.rel_l2(v3, xo.forward(wt, ctx, lat, 0.5, TINY)) < 1e-5
    # a changed key or prompt length invalidates the cache
    v4 = xo.forward(wt, ctx[:5], lat, 0.5, TINY, cache=cache, prefix_key="k")
    assert cache.length == 5
    assert xo.rel_l2(v4, xo.forward(wt, ctx[:5], lat, 0.5, TINY)) < 1e-6


def test_edit_mode_cache_and_prefix():
    wt = xo.SynthWeights(10, TINY, gain=4.0)
    ctx, lat, ref = xo.synth_inputs(10, 7, 3, 4, TINY, ref_hw=(2, 3))
    cache = xo.PrefixCache()
    r = (2, ref)
    v1 = xo.forward(wt, ctx, lat, 0.8, TINY, ref=r, cache=cache, prefix_key=("edit", 1))
    assert cache.length == 7 + 6
    v2 = xo.forward(wt, ctx, lat, 0.8, TINY, ref=r, cache=cache, prefix_key=("edit", 1))
    assert xo.rel_l2(v1, v2) < 1e-5
    # the reference picture matters, and so does where it sits
    v3 = xo.forward(wt, ctx, lat, 0.8, TINY, ref=(2, ref * 0.5))
    assert xo.rel_l2(v3, v1) > 1e-3
    v4 = xo.forward(wt, ctx, lat, 0.8, TINY, ref=(4, ref))
    assert xo.rel_l2(v4, v1) > 1e-4


def test_euler_update():
    """z <- z + (s' - s) v with (s' - s) rounded to a single float (src/generate.lisp:135)."""
    wt = xo.SynthWeights(12, TINY, gain=4.0)
    ctx, lat = xo.synth_inputs(12, 4, 2, 3, TINY)
    vs = []
    z = xo.euler(wt, ctx, lat, TINY, sigmas=(1.0, 0.95418, 0.5), on_step=lambda s, v, z: vs.append(v))
    want = lat + np.float32(0.95418 - 1.0) * vs[0]
    want = want + np.float32(0.5 - 0.95418) * vs[1]
    assert (z == want).all()


def test_step_flops_match_the_cost_model():
    """docs/design.md:127-132's cost, as counted for the roofline."""
    c = xo.step_flops(4096, 256, cached=True)
    assert abs(c["gemm"] / 1e12 - 57.175) < 0.01 and abs(c["attention"] / 1e12 - 9.346) < 0.01
    assert abs(c["total"] / 1e12 - 66.525) < 0.01
    u = xo.step_flops(4096, 256, cached=False)
    assert abs(u["total"] / 1e12 - 70.133) < 0.01


# --- the edit assembly pinned by what the mask fixes --------------------------------------

def _kept(wt, ctx, lat, ref):
    """An uncached pass's kept prefix K/V, per layer (keys and values, rows 0..p-1)."""
    cache = xo.PrefixCache()
    xo.forward(wt, ctx, lat, 0.8, TINY, ref=ref, cache=cache, prefix_key="k")
    return cache.kv


def test_edit_with_an_empty_picture_is_the_plain_step():
    """A reference picture of 0 x 0 puts nothing in the prefix: positions, mask and
    rows are the plain step's, so the velocity is the same bits (src/host.lisp:37-50,
    src/cuda-dit.lisp:179-187, src/cuda/dit.cu:60-66 with b0 = b1)."""
    wt = xo.SynthWeights(21, TINY, gain=4.0)
    ctx, lat = xo.synth_inputs(21, 6, 3, 4, TINY)
    empty = np.zeros((64, 0, 0), np.float32)
    plain = xo.forward(wt, ctx, lat, 0.7, TINY)
    for a in (0, 2, 6):
        assert np.array_equal(xo.forward(wt, ctx, lat, 0.7, TINY, ref=(a, empty)), plain)


def test_edit_mask_fixes_what_each_prefix_row_sees():
    """The prefix is [text 0..a-1 | picture a..a+nref-1 | text a+nref..p-1].  The text rows
    are causal and the picture's rows see the whole picture and everything before it
    (xa_lim, src/cuda/dit.cu:60-66), so in the kept K/V of every layer:
      - the picture changes nothing in rows 0..a-1, and changes the text after it (from the
        second layer on, once attention has mixed it in);
      - the text after the picture changes nothing in rows 0..a+nref-1;
      - the picture's first row sees its last one (the block is whole, not causal)."""
    wt = xo.SynthWeights(22, TINY, gain=4.0)
    a, rh, rw = 3, 2, 3
    nref = rh * rw
    ctx, lat, rl = xo.synth_inputs(22, 8, 3, 4, TINY, ref_hw=(rh, rw))
    p = ctx.shape[0] + nref
    base = _kept(wt, ctx, lat, (a, rl))
    other_pic = _kept(wt, ctx, lat, (a, rl * 0.5 + 0.3))
    ctx2 = ctx.copy()
    ctx2[a:] = ctx2[a:] * -1.0 + 0.2
    other_after = _kept(wt, ctx2, lat, (a, rl))
    last = rl.copy()
    last[:, rh - 1, rw - 1] += 3.0
    other_last = _kept(wt, ctx, lat, (a, last))
    for il in range(TINY.layers):
        for kv in range(2):
            b = base[il][kv]
            assert b.shape[0] == p
            assert np.array_equal(other_pic[il][kv][:a], b[:a])
            assert np.array_equal(other_after[il][kv][:a + nref], b[:a + nref])
            assert not np.array_equal(other_after[il][kv][a + nref:], b[a + nref:])
            if il >= 1:
                assert np.abs(other_pic[il][kv][a + nref:] - b[a + nref:]).max() > 1e-4
                assert np.abs(other_last[il][kv][a] - b[a]).max() > 1e-4
    # and the image rows' positions start after the text that follows the picture
    pos = xo.positions(p, 3, 4, (a, rh, rw))
    assert pos[p, 0] == a + max(rh, rw) + (p - a - nref)


# --- the W8A8 product (src/cuda-dit.lisp:110-126) ------------------------------------------

def test_quant_q8_0_closed_forms():
    """Blocks whose quantisation the definition fixes: values on the grid of d come back as
    their integers; a value x with x / d half-way between two integers goes away from zero
    (0.5 -> 1, 2.5 -> 3, -1.5 -> -2, where half-to-even would give 0, 2, -2); the block's
    largest magnitude maps to +-127; an all-zero block gives d = 0 and zeros; d is amax / 127
    rounded to fp16."""
    k = np.arange(-127, 128, 8, dtype=np.float32)                    # 32 integers, 127 among them
    k = np.concatenate([k, np.zeros(32 - k.size, np.float32)])[:32]
    k[0] = -127.0
    half = np.full(32, 0.0, np.float32)
    half[:4] = [0.5, 2.5, -1.5, 126.5]
    half[4] = 127.0                                                  # amax 127 -> d = 1
    x = np.stack([k * np.float32(0.125), half, np.zeros(32, np.float32),
                  np.linspace(-3, 7, 32, dtype=np.float32)])
    q, d = xo.quant_q8_0(x)
    assert np.array_equal(q[0], k.astype(np.int8)) and d[0] == np.float16(0.125)
    assert list(q[1, :5]) == [1, 3, -2, 127, 127] and d[1] == np.float16(1.0)
    assert not q[2].any() and d[2] == 0
    assert q[3].max() == 127 and np.argmax(q[3]) == 31
    assert d[3] == np.float16(np.float32(7) / np.float32(127))


def test_quant_q8_0_error_bound():
    """Every value within half a step of d q (plus the fp16 rounding of d), |q| <= 127."""
    rng = np.random.default_rng(3)
    x = (rng.normal(0, 1, (64, 256)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    q, d = xo.quant_q8_0(x)
    df = np.repeat(d.astype(np.float64), 32, axis=1)
    err = np.abs(x.astype(np.float64) - df * q)
    assert np.abs(q.astype(np.int32)).max() <= 127
    assert (err <= 0.5 * df * (1 + 1e-3) + 127 * df * 2.0 ** -11).all()


def test_linear_w8a8_is_the_product_of_the_dequantised_operands():
    """Per block, dx dw sum(qx qw) is the product of the dequantised operands summed over the
    block, so linear_w8a8 equals (dx qx) (dw qw)^T up to float32 rounding (a wrong block index
    or scale fails at 1e-2), against float64 brute force over the blocks too; and it stays within
    the activations' quantisation error of the unquantised product."""
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (40, 256)).astype(np.float32)
    qs, d = xo.q8_0_synth(2, 7, 48, 256)
    y = xo.linear_w8a8(x, qs, d)
    xq, xd = xo.quant_q8_0(x)
    deq = xo.dequant_q8_0(xq, xd).astype(np.float64) @ xo.dequant_q8_0(qs, d).astype(np.float64).T
    brute = np.zeros((40, 48))
    for b in range(8):
        c = slice(32 * b, 32 * b + 32)
        brute += (xd[:, b:b + 1].astype(np.float64) * d[:, b].astype(np.float64)[None, :]) * \
            (xq[:, c].astype(np.int64) @ qs[:, c].astype(np.int64).T)
    assert xo.rel_l2(y, deq) < 1e-6 and xo.rel_l2(y, brute) < 1e-6
    assert xo.rel_l2(deq, brute) < 1e-12
    e = xo.rel_l2(y, x @ xo.dequant_q8_0(qs, d).T)
    assert 1e-4 < e < 2e-2



def _f32_round(q):
    """The float32 nearest the rational Q, ties to even, by exact comparison."""
    from fractions import Fraction
    f = np.float32(float(q))
    lo, hi = (np.nextafter(f, np.float32(-np.inf)), f) if Fraction(float(f)) > q else (f, np.nextafter(f, np.float32(np.inf)))
    dlo, dhi = q - Fraction(float(lo)), Fraction(float(hi)) - q
    if dlo != dhi:
        return lo if dlo < dhi else hi
    return lo if (int(np.float32(lo).view(np.uint32)) & 1) == 0 else hi


def test_linear_w8a8_accumulates_with_single_rounding_fmas():
    """Each block adds float(isum) * (dx * dw) to the sum with one rounding (a fused multiply-add
    on the rounded scale product): rebuilt here in exact rational arithmetic on a small product,
    every step rounded to float32 where the definition rounds, and equal bit for bit; a product
    then a sum, each rounded, differs somewhere."""
    from fractions import Fraction
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (6, 256)).astype(np.float32)
    qs, d = xo.q8_0_synth(3, 9, 5, 256)
    y = xo.linear_w8a8(x, qs, d)
    xq, xd = xo.quant_q8_0(x)
    acc = [[np.float32(0)] * 5 for _ in range(6)]
    two = [[np.float32(0)] * 5 for _ in range(6)]
    for b in range(8):
        c = slice(32 * b, 32 * b + 32)
        isum = xq[:, c].astype(np.int64) @ qs[:, c].astype(np.int64).T
        for i in range(6):
            for j in range(5):
                sc = np.float32(xd[i, b]) * np.float32(d[j, b])      # float32 product, rounded
                exact = Fraction(int(isum[i, j])) * Fraction(float(sc)) + Fraction(float(acc[i][j]))
                acc[i][j] = _f32_round(exact)
                two[i][j] = np.float32(two[i][j] + np.float32(np.float32(isum[i, j]) * sc))
    want, sep = np.array(acc, np.float32), np.array(two, np.float32)
    assert np.array_equal(y, want)
    assert not np.array_equal(sep, want) and xo.rel_l2(sep, want) < 1e-6


def test_forward_w8a8_routes_q8_0_products_of_16_rows_or_more():
    """The int8 mode changes the velocity by about the activations' quantisation error and
    leaves a pass of fewer than 16 rows (every product through linear) exactly as it was."""
    seed, p, h, w = 3, 8, 4, 4
    wt = xo.SynthWeights(seed, TINY, gain=4.0)
    ctxa, lat = xo.synth_inputs(seed, p, h, w, TINY)
    v = xo.forward(wt, ctxa, lat, 0.7, TINY)
    v8 = xo.forward(wt, ctxa, lat, 0.7, TINY, w8a8=True)
    e = xo.rel_l2(v8, v)
    assert 1e-5 < e < 5e-2
    small = xo.forward(wt, ctxa[:4], lat[:, :2, :2], 0.7, TINY, w8a8=True)
    assert np.array_equal(small, xo.forward(wt, ctxa[:4], lat[:, :2, :2], 0.7, TINY))
