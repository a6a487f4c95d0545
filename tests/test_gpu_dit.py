"""The DiT step on the GPU through the C ABI's backend trio, against the
oracle: per block (relative L2 <= 1e-2, on the block's output and on its
update), per step, the prefix cache, edit mode, and the 8 Euler steps
(<= 2e-2 on the final latent).  Needs an MI355X."""
import os
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print("[gpu]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = X.Context(0)
    yield c
    c.close()


def model(ctx, layers, seed):
    d = X.Dit(ctx, layers)
    d.synth(seed)
    d.check()
    return d


def test_missing_and_misshapen_tensors(ctx):
    say("dit check / set errors")
    d = X.Dit(ctx, 2)
    with pytest.raises(X.ExnError) as e:
        d.check()
    assert e.value.code == X.ESTATE and "missing img_in.weight" in str(e.value)
    with pytest.raises(X.ExnError) as e:
        d.set("transformer_blocks.0.attn.norm_q.weight", X.F32, np.zeros(64, np.float32), (64,))
    assert e.value.code == X.EINVAL and "not (128 1)" in str(e.value)
    with pytest.raises(X.ExnError) as e:
        d.set("transformer_blocks.2.attn.to_q.weight", X.Q8_0, np.zeros(34, np.uint8), (4096, 4096))
    assert e.value.code == X.EINVAL
    with pytest.raises(X.ExnError):
        X.dit_velocity(d, np.zeros((4, 4096), np.float32), 4, np.zeros((64, 2, 2), np.float32), 2, 2, 0.5)
    d.destroy()


def _trace(ctx, d, rows):
    """The residual stream before the first block (slot 0) and after each block."""
    buf = X.DevBuf(ctx, (d.layers + 1, rows, 4096), np.float32)
    X.call("exn_dit_trace", d.h, buf.h, (d.layers + 1) * rows * 4096)
    return buf


def test_one_block_cfg0(ctx):
    """The single-block workload: 1024 image rows (32 x 32) and 64 text rows,
    sigma 0.5, reference dims (width 4096, 32 x 128 heads, SwiGLU 12288)."""
    seed, p, h, w = 0, 64, 32, 32
    say("one block, p", p, "image", h, "x", w)
    d = model(ctx, 1, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    tr = _trace(ctx, d, p + h * w)
    v = X.dit_velocity(d, ctxa, p, lat, h, w, 0.5)
    t = tr.get()
    x_in_gpu, x_gpu = t[0], t[1]
    wt = xo.SynthWeights(seed)
    dump = {}
    v_ref = xo.forward(wt, ctxa, lat, 0.5, dump=dump, layers=1)
    x_in = np.concatenate([dump["txt"], xo.linear(xo.tokens(lat), wt("img_in.weight"))])
    x_ref = dump["blk"][0]
    e_in = xo.rel_l2(x_in_gpu, x_in)                        # txt_in and img_in, fp32 on the device
    e_x, e_v = xo.rel_l2(x_gpu, x_ref), xo.rel_l2(v, v_ref)
    e_dx = xo.rel_l2(x_gpu - x_in_gpu, x_ref - x_in)        # the block's own update
    say("rel-L2: block input %.2e, block output %.2e, block update %.2e, velocity %.2e" % (e_in, e_x, e_dx, e_v))
    assert e_in < 1e-4
    assert e_x < 1e-2 and e_dx < 1e-2 and e_v < 1e-2
    d.destroy()


def test_prefix_cache(ctx):
    """A cached pass gives the uncached pass's velocity (src/cuda-dit.lisp:6-9), bit for bit:
    the image rows are multiplied alike in both passes, and every product's split (the edge
    products' included) follows its own shape, not the picture's."""
    say("prefix cache, 2 blocks")
    d = model(ctx, 2, 3)
    ctxa, lat = xo.synth_inputs(3, 20, 4, 6)
    v0 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9)
    v1 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="a")
    v2 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="a")          # cached
    assert np.array_equal(v1, v0) and np.array_equal(v2, v0)
    v3 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.5, prefix_key="a")          # cached, another t
    v4 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.5)
    assert xo.rel_l2(v3, v4) < 1e-5
    # a changed prompt length invalidates the kept K/V
    v5 = X.dit_velocity(d, ctxa[:17], 17, lat, 4, 6, 0.5, prefix_key="a")
    v6 = X.dit_velocity(d, ctxa[:17], 17, lat, 4, 6, 0.5)
    assert xo.rel_l2(v5, v6) < 1e-6 and xo.rel_l2(v5, v4) > 1e-4
    wt = xo.SynthWeights(3)
    ref = xo.forward(wt, ctxa, lat, 0.5, layers=2)
    assert xo.rel_l2(v4, ref) < 1e-2
    X.dit_release(d)
    v7 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.5, prefix_key="a")          # released: recomputed
    assert xo.rel_l2(v7, v4) < 1e-6
    # a larger image over the kept prompt: the K/V arrays grow and carry the 20 prompt rows over
    _, big = xo.synth_inputs(3, 20, 24, 24)
    v8 = X.dit_velocity(d, ctxa, 20, big, 24, 24, 0.5, prefix_key="a")        # cached, 596 keys
    v9 = X.dit_velocity(d, ctxa, 20, big, 24, 24, 0.5)
    assert np.array_equal(v8, v9)
    d.destroy()


def test_prefix_cache_follows_the_weights_and_the_prompt(ctx):
    """Kept K/V belong to the weights and the prompt they were made from: re-synthesised
    weights under the same key and length recompute them, and generate_latent's default
    key is the prompt's content, so two prompts of one length each get their own."""
    say("prefix cache vs new weights and new prompts, 2 blocks")
    d = model(ctx, 2, 3)
    ctxa, lat = xo.synth_inputs(3, 20, 4, 6)
    X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="a")                # keeps seed 3's K/V
    d.synth(31)
    v1 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="a")
    v0 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9)
    assert xo.rel_l2(v1, v0) < 1e-6
    # the same through exn_dit_set: one layer's to_out scaled
    name = "transformer_blocks.1.attn.to_out.0.weight"
    qs, dd = xo.q8_0_synth(31, xo.tensor_id(name), 4096, 4096)
    X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="b")
    d.set(name, X.Q8_0, xo.q8_0_to_blocks(qs, (dd.astype(np.float32) * 2).astype(np.float16)), (4096, 4096))
    v2 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9, prefix_key="b")
    v3 = X.dit_velocity(d, ctxa, 20, lat, 4, 6, 0.9)
    assert xo.rel_l2(v2, v3) < 1e-6 and xo.rel_l2(v3, v0) > 1e-4
    # two prompts of one length through generate_latent: each as its own uncached run
    ctxb = xo.synth_inputs(35, 20, 4, 6)[0]
    sig = (1.0, 0.95418, 0.5)
    za = X.generate_latent(d, ctxa, 20, lat, 4, 6, sigmas=sig)
    zb = X.generate_latent(d, ctxb, 20, lat, 4, 6, sigmas=sig)
    for c, z in ((ctxa, za), (ctxb, zb)):
        want = lat.copy()
        for s0, s1 in zip(sig[:-1], sig[1:]):
            want = want + np.float32(s1 - s0) * X.dit_velocity(d, c, 20, want, 4, 6, s0)
        assert xo.rel_l2(z, want) < 1e-5
    assert xo.rel_l2(za, zb) > 1e-4
    d.destroy()


@pytest.mark.parametrize("p,h,w", [(20, 4, 6), (256, 32, 32)])
def test_last_block_image_rows_alone(ctx, p, h, w):
    """An uncached pass's last block runs its attention and products on the image rows alone
    (nothing reads the prompt rows past their kept K/V); a pass recording exn_dit_stats takes
    every row.  Both give the same velocity bit for bit, and so does a cached pass over the
    K/V the shortened pass kept."""
    say("last block on the image rows: p", p, "image", h, "x", w)
    d = model(ctx, 3, 5)
    ctxa, lat = xo.synth_inputs(5, p, h, w)
    v_short = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7, prefix_key="k")
    v_cached = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7, prefix_key="k")
    d.stats(True)
    v_full = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7)
    d.stats(False)
    assert np.array_equal(v_short, v_full) and np.array_equal(v_cached, v_full)
    d.destroy()


class _Weights:
    """The oracle's synthetic weights with some matrices replaced."""

    def __init__(self, base, over):
        self.base, self.over = base, over

    def __call__(self, name):
        return self.over[name] if name in self.over else self.base(name)


# matrices the real GGUF stores as F32 or BF16 (src/metal-dit.lisp:4-7), and the other edge ones
EDGE_MATS = ["img_in.weight", "txt_in.in_layer.weight", "txt_in.out_layer.weight", "norm_out.linear.weight",
             "proj_out.weight", "time_text_embed.timestep_embedder.linear_1.weight",
             "time_text_embed.timestep_embedder.linear_2.weight", "modulation.1.weight"]


def test_matrices_of_every_kind(ctx):
    """upload-dit takes F32 and BF16 matrices besides Q8_0 (src/cuda-dit.lisp:77-80,127-130).
    Edge matrices stay as given: F32 multiplied in fp32 (d41_mm_f32) -- the dequantised values
    as F32 give the Q8_0 run's velocity bit for bit, and values off the bf16 grid reach the
    block input at fp32 precision; BF16 on their bf16 values.  Block matrices given as F32 or
    BF16 (or mixed with Q8_0 slots in one fused matrix) run from bf16 rows: the dequantised
    values give the resident run's velocity bit for bit."""
    seed, p, h, w = 13, 16, 8, 8
    say("F32 / BF16 / Q8_0 matrices through exn_dit_set, 2 blocks")
    d = model(ctx, 2, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    wt = xo.SynthWeights(seed)
    dims = dict(xo.dit_expected(xo.Shape(layers=2)))
    v_q8 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6)
    # (a) the edge matrices as F32, exactly the dequantised values
    for name in EDGE_MATS:
        d.set(name, X.F32, wt(name), dims[name])
    v_f32 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6)
    assert np.array_equal(v_f32, v_q8)
    # (b) F32 and BF16 edge matrices off the bf16 grid, against the oracle on those weights
    rng = np.random.default_rng(5)
    over = {n: (wt(n) * (1 + 1e-2 * rng.normal(size=wt(n).shape))).astype(np.float32) for n in EDGE_MATS}
    for kind in (X.F32, X.BF16):
        o = dict(over) if kind == X.F32 else {n: xo.bf16_round(m) for n, m in over.items()}
        for name in EDGE_MATS:
            d.set(name, kind, o[name] if kind == X.F32 else xo.bf16_bits(o[name]), dims[name])
        tr = _trace(ctx, d, p + h * w)
        v = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6)
        X.call("exn_dit_trace", d.h, None, 0)
        dump = {}
        want = xo.forward(_Weights(wt, o), ctxa, lat, 0.6, dump=dump, layers=2)
        x_in = np.concatenate([dump["txt"], xo.linear(xo.tokens(lat), o["img_in.weight"])])
        e_in, e_v = xo.rel_l2(tr.get()[0], x_in), xo.rel_l2(v, want)
        say("edge %s: block input rel-L2 %.2e, velocity %.2e" % ("F32" if kind == X.F32 else "BF16", e_in, e_v))
        assert e_in < 1e-5 and e_v < 1e-2
    # (c) back to Q8_0 edges; block matrices as F32, BF16 and Q8_0 slots of one fused matrix
    d.synth(seed)
    v_res = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6)
    assert np.array_equal(v_res, v_q8)
    X.dit_velocity(d, ctxa, p, lat, h, w, 0.6, prefix_key="k")
    blk = "transformer_blocks.%d."
    d.set(blk % 0 + "attn.to_q.weight", X.F32, wt(blk % 0 + "attn.to_q.weight"), (4096, 4096))
    d.set(blk % 0 + "attn.to_v.weight", X.BF16, xo.bf16_bits(wt(blk % 0 + "attn.to_v.weight")), (4096, 4096))
    n = blk % 0 + "attn.to_k.weight"
    d.set(n, X.Q8_0, xo.q8_0_to_blocks(*xo.q8_0_synth(seed, xo.tensor_id(n), 4096, 4096)), (4096, 4096))
    d.set(blk % 1 + "img_mlp.gate_up.weight", X.BF16, xo.bf16_bits(wt(blk % 1 + "img_mlp.gate_up.weight")),
          (4096, 2 * 12288))
    d.set(blk % 1 + "img_mlp.out.weight", X.F32, wt(blk % 1 + "img_mlp.out.weight"), (12288, 4096))
    d.set(blk % 1 + "attn.to_out.0.weight", X.BF16, xo.bf16_bits(wt(blk % 1 + "attn.to_out.0.weight")), (4096, 4096))
    v_mix = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6, prefix_key="k")    # the sets dropped the kept K/V
    assert np.array_equal(v_mix, v_q8)
    # the dense rows take a later Q8_0 slot's values: to_q scaled by 2 as Q8_0
    n = blk % 0 + "attn.to_q.weight"
    qs, dd = xo.q8_0_synth(seed, xo.tensor_id(n), 4096, 4096)
    d2 = (dd.astype(np.float32) * 2).astype(np.float16)
    d.set(n, X.Q8_0, xo.q8_0_to_blocks(qs, d2), (4096, 4096))
    v_q2 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.6)
    want = xo.forward(_Weights(wt, {n: xo.dequant_q8_0(qs, d2)}), ctxa, lat, 0.6, layers=2)
    e = xo.rel_l2(v_q2, want)
    say("mixed fused matrix after a Q8_0 slot: velocity rel-L2 %.2e" % e)
    assert e < 1e-2 and xo.rel_l2(v_q2, v_q8) > 1e-5
    d.destroy()


def test_edit_mode(ctx):
    """A reference picture in the prefix (src/cuda-dit.lisp:179-192; host.lisp:37-50):
    3 text rows, a 4 x 5 picture, 9 text rows more, a 4 x 6 image."""
    say("edit mode, 2 blocks")
    seed = 4
    d = model(ctx, 2, seed)
    ctxa, lat, rl = xo.synth_inputs(seed, 12, 4, 6, ref_hw=(4, 5))
    v1 = X.dit_velocity(d, ctxa, 12, lat, 4, 6, 0.8, prefix_key="e", ref=(3, rl, 4, 5))
    v2 = X.dit_velocity(d, ctxa, 12, lat, 4, 6, 0.8, prefix_key="e", ref=(3, rl, 4, 5))
    assert xo.rel_l2(v2, v1) < 1e-5
    wt = xo.SynthWeights(seed)
    ref = xo.forward(wt, ctxa, lat, 0.8, ref=(3, rl), layers=2)
    e = xo.rel_l2(v1, ref)
    say("edit velocity rel-L2 %.2e" % e)
    assert e < 1e-2
    d.destroy()


def test_q8_0_and_resident_bf16_agree(ctx):
    """The block matrices from Q8_0 (dequantised inside the products' pipeline) and from their
    resident bf16 expansions (the default) give one velocity, bit for bit: the operands are the
    same bf16 values, bf16(fp32(d) q), and the products take the same MFMAs in the same order
    (the split products' k ranges included)."""
    say("q8_0 vs resident bf16 weights, 2 blocks")
    seed, p, h, w = 8, 40, 16, 16
    d = model(ctx, 2, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    v_bf = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7)
    d.resident(False)
    v_q8 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7)
    d.resident(True)
    v_bf2 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7)
    ref = xo.forward(xo.SynthWeights(seed), ctxa, lat, 0.7, layers=2)
    e, e_ref = xo.rel_l2(v_bf, v_q8), xo.rel_l2(v_bf, ref)
    say("resident vs q8_0 rel-L2 %.2e, vs oracle %.2e" % (e, e_ref))
    assert np.array_equal(v_q8, v_bf) and np.array_equal(v_bf2, v_bf)
    assert e_ref < 1e-2 and xo.rel_l2(v_q8, ref) < 1e-2
    d.destroy()


def test_device_and_host_paths_agree(ctx):
    """exn_dit_velocity (host arrays) and exn_dit_velocity_dev (device arrays) give
    the same velocity; generate's Euler loop on the device gives the host loop's
    latent (z + ds v, two single roundings either way)."""
    say("host and device paths, 2 blocks")
    seed, p, h, w = 5, 24, 8, 8
    d = model(ctx, 2, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    v_host = X.dit_velocity(d, ctxa, p, lat, h, w, 1.0)
    cd, zd = X.DevBuf.of(ctx, ctxa), X.DevBuf.of(ctx, lat)
    vd = X.DevBuf(ctx, (64, h, w), np.float32)
    X.call("exn_dit_velocity_dev", d.h, cd.h, p, zd.h, h, w, 1.0, 0, 0, None, 0, 0, vd.h)
    e = xo.rel_l2(vd.get(), v_host)
    say("velocity host vs device rel-L2 %.2e" % e)
    assert e < 1e-6
    sig = (1.0, 0.978453, 0.95418)
    z = lat.copy()
    for s, s2 in zip(sig[:-1], sig[1:]):
        v = X.dit_velocity(d, ctxa, p, z, h, w, s, prefix_key="k")
        z = z + np.float32(s2 - s) * v
    sg = np.array(sig, np.float64)
    X.call("exn_dit_generate_dev", d.h, cd.h, p, zd.h, h, w, X.ptr(sg), len(sg), 0, None, 0, 0)
    e = xo.rel_l2(zd.get(), z)
    say("two Euler steps, device loop vs host loop rel-L2 %.2e" % e)
    assert e < 1e-6
    d.destroy()


def test_full_depth_steps_against_oracle(ctx):
    """32 blocks, 32 text rows, an 8 x 8 latent: each of the 8 Turbo steps'
    velocity (<= 1e-2) and the final latent after the Euler loop (<= 2e-2),
    against the oracle's results cached in tests/golden/dit_depth32_small.npz."""
    g = np.load(os.path.join(GOLDEN, "dit_depth32_small.npz"))
    seed, p, h, w = (int(v) for v in g["meta"])
    say("32 blocks, 8 steps, p", p, "image", h, "x", w)
    d = model(ctx, 32, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    z = lat.copy()
    sig = xo.TURBO_SIGMAS
    for i, (s, s2) in enumerate(zip(sig[:-1], sig[1:])):
        v = X.dit_velocity(d, ctxa, p, z, h, w, s, prefix_key="prompt")
        e = xo.rel_l2(v, g["v_steps"][i])
        say("step %d velocity rel-L2 %.2e" % (i, e))
        assert e < 1e-2
        z = z + np.float32(s2 - s) * v
    ez = xo.rel_l2(z, g["z_final"])
    say("final latent rel-L2 %.2e" % ez)
    assert ez < 2e-2
    # the same loop on the device (exn_dit_generate_dev) gives the same latent
    zd = X.DevBuf.of(ctx, lat)
    cd = X.DevBuf.of(ctx, ctxa)
    sg = np.array(sig, np.float64)
    X.call("exn_dit_generate_dev", d.h, cd.h, p, zd.h, h, w, X.ptr(sg), len(sg), 0, None, 0, 0)
    assert xo.rel_l2(zd.get(), z) < 1e-5
    d.destroy()


# --- the workloads' full shapes, two blocks deep -------------------------------------------

FULL_CASES = {  # name: (seed, text rows, image h, w, reference picture (a, rh, rw) or None, sigma)
    "cfg2_1024sq": (2, 256, 64, 64, None, 0.978453),
    "cfg3_1536x1024": (6, 256, 96, 64, None, 0.95418),
    "cfg4_edit_1024sq": (7, 512, 64, 64, (8, 64, 64), 0.926626),
}


@pytest.mark.parametrize("case", list(FULL_CASES))
def test_full_shapes_two_blocks(ctx, case):
    """Every kernel at a workload's real sizes (4096 or 6144 image rows; 256 text rows, or
    512 text rows plus a 64 x 64 reference picture = 8704 keys), two blocks deep: the
    uncached pass and then the cached pass against the oracle's velocity (<= 1e-2; the
    oracle's results cached in tests/golden/dit_full_shapes_2blocks.npz as float16), and
    against each other (the kept K/V give the same velocity)."""
    seed, p, h, w, ref, sigma = FULL_CASES[case]
    say(case, "p", p, "image", h, "x", w, "ref", ref)
    want = np.load(os.path.join(GOLDEN, "dit_full_shapes_2blocks.npz"))[case].astype(np.float32)
    d = model(ctx, 2, seed)
    if ref is None:
        ctxa, lat = xo.synth_inputs(seed, p, h, w)
        refarg = None
    else:
        a, rh, rw = ref
        ctxa, lat, rl = xo.synth_inputs(seed, p, h, w, ref_hw=(rh, rw))
        refarg = (a, rl, rh, rw)
    v0 = X.dit_velocity(d, ctxa, p, lat, h, w, sigma, prefix_key="k", ref=refarg)     # uncached, keeps K/V
    v1 = X.dit_velocity(d, ctxa, p, lat, h, w, sigma, prefix_key="k", ref=refarg)     # cached
    e0, e1, e01 = xo.rel_l2(v0, want), xo.rel_l2(v1, want), xo.rel_l2(v1, v0)
    say("velocity rel-L2: uncached %.2e, cached %.2e, cached vs uncached %.2e" % (e0, e1, e01))
    assert e0 < 1e-2 and e1 < 1e-2 and e01 < 1e-5
    d.destroy()


@pytest.mark.parametrize("resident", [True, False], ids=["resident_bf16", "q8_0"])
def test_cfg2_eight_steps_full_depth(ctx, resident):
    """The 1024^2 workload end to end: 32 blocks, 4096 image rows over 256 text rows, the
    first step's velocity (uncached, <= 1e-2) and the final latent after the 8 Turbo steps
    of the device Euler loop (<= 2e-2), against the oracle's run cached as float16 in
    tests/golden/dit_cfg2_8step.npz (about 75 minutes of numpy); from the resident bf16
    expansion and from Q8_0 dequantised in the products."""
    g = np.load(os.path.join(GOLDEN, "dit_cfg2_8step.npz"))
    seed, p, h, w = (int(v) for v in g["meta"])
    say("cfg2: 32 blocks, p", p, "image", h, "x", w, "8 steps, resident", resident)
    d = model(ctx, 32, seed)
    d.resident(resident)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    v0 = X.dit_velocity(d, ctxa, p, lat, h, w, xo.TURBO_SIGMAS[0])
    e0 = xo.rel_l2(v0, g["v_step0"].astype(np.float32))
    zd, cd = X.DevBuf.of(ctx, lat), X.DevBuf.of(ctx, ctxa)
    sg = np.array(xo.TURBO_SIGMAS, np.float64)
    X.call("exn_dit_generate_dev", d.h, cd.h, p, zd.h, h, w, X.ptr(sg), len(sg), 0, None, 0, 0)
    ez = xo.rel_l2(zd.get(), g["z_final"].astype(np.float32))
    say("cfg2: step-0 velocity rel-L2 %.2e, final latent rel-L2 %.2e" % (e0, ez))
    assert e0 < 1e-2 and ez < 2e-2
    d.destroy()


WORKLOADS = {  # name: (seed, text rows, image h, w, reference picture (a, rh, rw) or None, the oracle's run)
    "cfg3_1536x1024": (6, 256, 96, 64, None, "dit_cfg3_8step.npz"),
    "cfg4_edit_1024sq": (7, 512, 64, 64, (8, 64, 64), "dit_cfg4_edit_8step.npz"),
}


@pytest.mark.parametrize("case", list(WORKLOADS))
def test_workloads_eight_steps_full_depth(ctx, case):
    """The 1536 x 1024 workload (6144 image rows over 256 text rows) and the edit workload
    (512 text rows with a 64 x 64 reference picture after the first 8, then a 64 x 64 image:
    8704 keys) end to end, 32 blocks: the first step's velocity (uncached, <= 1e-2) and the
    final latent after the 8 Turbo steps (<= 2e-2) against the oracle's run cached as float16
    in tests/golden (hours of numpy each); the first step again on the kept prefix K/V (one
    velocity, <= 1e-5); the host loop (exn_dit_velocity and the Euler update in numpy) and the
    device loop (exn_dit_generate_dev) give one latent (<= 1e-5), every value finite."""
    seed, p, h, w, ref, fixture = WORKLOADS[case]
    g = np.load(os.path.join(GOLDEN, fixture))
    assert [int(v) for v in g["meta"]] == [seed, p, h, w]
    say(case, "32 blocks, p", p, "image", h, "x", w, "ref", ref, "8 steps")
    d = model(ctx, 32, seed)
    if ref is None:
        ctxa, lat = xo.synth_inputs(seed, p, h, w)
        refarg, rl = None, None
    else:
        a, rh, rw = ref
        ctxa, lat, rl = xo.synth_inputs(seed, p, h, w, ref_hw=(rh, rw))
        refarg = (a, rl, rh, rw)
    sig = xo.TURBO_SIGMAS
    v0 = X.dit_velocity(d, ctxa, p, lat, h, w, sig[0], prefix_key="k", ref=refarg)
    v0c = X.dit_velocity(d, ctxa, p, lat, h, w, sig[0], prefix_key="k", ref=refarg)
    e01 = xo.rel_l2(v0c, v0)
    e0 = xo.rel_l2(v0, g["v_step0"].astype(np.float32))
    say("%s: step 0 against the oracle rel-L2 %.2e, cached vs uncached %.2e" % (case, e0, e01))
    assert np.isfinite(v0).all() and e01 < 1e-5 and e0 < 1e-2
    z = lat.copy()
    for i, (s, s2) in enumerate(zip(sig[:-1], sig[1:])):
        v = v0c if i == 0 else X.dit_velocity(d, ctxa, p, z, h, w, s, prefix_key="k", ref=refarg)
        assert np.isfinite(v).all()
        z = z + np.float32(s2 - s) * v
    zd, cd = X.DevBuf.of(ctx, lat), X.DevBuf.of(ctx, ctxa)
    rd = X.DevBuf.of(ctx, rl) if rl is not None else None
    sg = np.array(sig, np.float64)
    if ref is None:
        X.call("exn_dit_generate_dev", d.h, cd.h, p, zd.h, h, w, X.ptr(sg), len(sg), 0, None, 0, 0)
    else:
        X.call("exn_dit_generate_dev", d.h, cd.h, p, zd.h, h, w, X.ptr(sg), len(sg), ref[0], rd.h, ref[1], ref[2])
    zg = zd.get()
    ez = xo.rel_l2(zg, z)
    eo = xo.rel_l2(zg, g["z_final"].astype(np.float32))
    say("%s: final latent against the oracle rel-L2 %.2e, device loop vs host loop %.2e" % (case, eo, ez))
    assert np.isfinite(zg).all() and ez < 1e-5 and eo < 2e-2
    d.destroy()


def test_w8a8_mode(ctx):
    """The reference's default *int8* products (exn_dit_w8a8; src/cuda-dit.lisp:110-126): 2 blocks,
    40 text rows and a 16 x 16 image (every block product, txt_in, img_in and proj_out of at
    least 16 rows go the int8 way), against the oracle's forward in its int8 mode (<= 1e-2, and
    nearer to it than to the oracle's bf16-free forward); the cached pass equals the uncached
    one bit for bit; switching the mode off gives the bf16 products' velocity back, bit for bit."""
    say("int8 mode, 2 blocks")
    seed, p, h, w = 9, 40, 16, 16
    d = model(ctx, 2, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    v_bf = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7)
    d.w8a8(True)
    v8 = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7, prefix_key="k")
    v8c = X.dit_velocity(d, ctxa, p, lat, h, w, 0.7, prefix_key="k")
    wt = xo.SynthWeights(seed)
    want = xo.forward(wt, ctxa, lat, 0.7, layers=2, w8a8=True)
    plain = xo.forward(wt, ctxa, lat, 0.7, layers=2)
    e, e_plain, e_mode = xo.rel_l2(v8, want), xo.rel_l2(v8, plain), xo.rel_l2(want, plain)
    say("int8 velocity rel-L2: against the int8 oracle %.2e, against the plain oracle %.2e; the oracle's "
        "two modes differ by %.2e; cached vs uncached %.2e" % (e, e_plain, e_mode, xo.rel_l2(v8c, v8)))
    assert e < 1e-2 and e < e_plain
    assert np.array_equal(v8c, v8)
    d.w8a8(False)
    assert np.array_equal(X.dit_velocity(d, ctxa, p, lat, h, w, 0.7), v_bf)
    d.destroy()


def test_stats_count_a_planted_nan_at_its_block(ctx):
    """*dit-trace*'s numbers (exn_dit_stats): with every value finite they are the largest |x| of
    the stream, the attention's output and the MLP's rows after each block (against the trace's
    copy of the stream), and none is counted not finite; a NaN planted in block 1's norm_q
    weights reaches block 1's attention and stream -- counted there, not at block 0 -- and
    every block after it."""
    seed, p, h, w = 17, 24, 8, 8
    say("stats: 3 blocks, a NaN in block 1's norm_q")
    d = model(ctx, 3, seed)
    ctxa, lat = xo.synth_inputs(seed, p, h, w)
    n = p + h * w
    tr = _trace(ctx, d, n)
    d.stats(True)
    X.dit_velocity(d, ctxa, p, lat, h, w, 0.8)
    X.call("exn_dit_trace", d.h, None, 0)
    mx, bad = d.stats_read()
    xs = tr.get()
    say("finite: stream max |x| by block", np.round(mx[:, 0], 2), "att", np.round(mx[1:, 1], 2), "ff", np.round(mx[1:, 2], 2))
    assert (bad == 0).all() and (mx[1:, :3] > 0).all() and mx[0, 3] > 0
    for i in range(4):   # the stream's maximum is the trace's, exactly
        assert mx[i, 0] == np.float32(np.abs(xs[i]).max())
    nq = xo.synth_vector(seed, "transformer_blocks.1.attn.norm_q.weight", 128).astype(np.float32)
    nq[5] = np.nan
    d.set("transformer_blocks.1.attn.norm_q.weight", X.F32, nq, (128,))
    X.dit_velocity(d, ctxa, p, lat, h, w, 0.8)
    mx, bad = d.stats_read()
    say("NaN in block 1: values not finite, rows before, blocks 0..2 (x att ff):", bad[:, :3].tolist())
    assert (bad[0] == 0).all() and (bad[1] == 0).all()
    assert bad[2, 1] > 0 and bad[2, 0] > 0 and bad[3, 0] > 0
    d.stats(False)
    d.destroy()
