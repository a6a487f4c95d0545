"""The VAE decoder and encoder on the GPU through the C ABI, against the oracle
(oracle/exn_vae_oracle.py) and the reference script's own pictures
(tests/golden/ref_vae_tiny.npz).  The picture's bar is the reference's for its
half-precision decoder against the decoder in floats: within 3 of 255
(README.md:130-132), so max |difference| <= 6/255 on -1..1; and relative L2 <=
1e-2.  Needs an MI355X."""
import os
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo
from oracle import exn_vae_oracle as vo

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PICTURE_MAX = 6.0 / 255.0


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
    """A device copy of A kept alive for the module: a temporary freed at once could hand
    its memory to the next upload before the kernel reads it."""
    b = X.DevBuf.of(ctx, np.ascontiguousarray(a))
    _KEEP.append(b)
    return b


def pack_conv(w, kp):
    """(o, i, [1,] k, k) -> bf16 rows of (tap, channel), K padded to kp: the device form."""
    o, i = w.shape[0], w.shape[1]
    k = w.shape[-1]
    rows = w.reshape(o, i, k * k).transpose(0, 2, 1).reshape(o, k * k * i)
    out = np.zeros((o, kp), np.uint16)
    out[:, :rows.shape[1]] = xo.bf16_bits(rows)
    return out


CONV_CASES = [  # (h, w, c, cout, taps, up, out, with res)
    (5, 7, 64, 144, 9, 0, 0, False),
    (16, 16, 144, 288, 9, 0, 0, True),
    (6, 10, 288, 144, 9, 0, 1, False),
    (3, 4, 1152, 1152, 9, 0, 0, True),
    (9, 9, 144, 4, 9, 0, 2, False),
    (8, 6, 576, 576, 9, 1, 0, False),
    (20, 18, 288, 288, 9, 1, 0, False),
    (7, 9, 1152, 3456, 1, 0, 0, False),
    (11, 5, 288, 144, 1, 0, 0, True),
    (4, 4, 64, 64, 1, 0, 1, False),
    (10, 7, 64, 12, 9, 0, 0, True),      # the narrow tile (16 columns) with a residual
    # the encoder's: stride 2 (the input 2h x 2w), the 96- and 192-wide tiles
    (12, 20, 96, 96, 9, 2, 0, False),
    (40, 36, 192, 384, 9, 2, 0, True),
    (7, 5, 768, 768, 9, 2, 0, False),
    (17, 15, 96, 192, 9, 0, 0, True),
    (9, 11, 384, 768, 9, 0, 1, False),
    (13, 7, 96, 192, 1, 0, 0, True),
    (21, 19, 64, 96, 1, 0, 0, False),   # encoder.conv1: a 1 x 1 product over RGBA neighbourhoods
    (6, 6, 768, 128, 9, 0, 1, False),   # the encoder's head: 128 of a 144-wide tile
    # 2^18 pixels: the 128-pixel tiles of 4 waves, two workgroups a CU
    (512, 512, 144, 144, 9, 0, 0, True),
    (512, 512, 96, 96, 9, 0, 1, False),
    (512, 512, 64, 96, 1, 0, 0, False),
]


SPLIT_CASES = [  # split K: fewer tiles than CUs, 3 x 3, no upsampling, fp32 or bf16 out
    (12, 13, 1152, 1152, 9, 0, 0, True),
    (9, 7, 576, 288, 9, 0, 1, True),
    (16, 20, 288, 144, 9, 0, 0, False),
    (4, 4, 1152, 576, 9, 0, 0, True),
    (8, 8, 768, 768, 9, 0, 0, True),     # the 192-wide tile split
]


@pytest.mark.parametrize("case,split", [(c, False) for c in CONV_CASES] + [(c, True) for c in SPLIT_CASES])
def test_conv_against_float64(ctx, case, split):
    """The implicit-GEMM convolution: partial pixel and channel tiles, K not a
    multiple of 64 (144, 288 wide), the upsampling fold, stride 2, the three outputs; with a
    partials buffer, K split over up to 4 workgroups a tile (their sum in order)."""
    h, w, c, cout, taps, up, out, with_res = case
    say("conv", case, "split" if split else "")
    rng = np.random.default_rng(h * 1000 + c + cout)
    hs, ws = (h // 2, w // 2) if up == 1 else (2 * h, 2 * w) if up == 2 else (h, w)
    x = xo.bf16_round(rng.standard_normal((hs, ws, c)).astype(np.float32))
    k = 3 if taps == 9 else 1
    wt = xo.bf16_round((rng.standard_normal((cout, c, 1, k, k)) / np.sqrt(c * taps)).astype(np.float32))
    b = rng.standard_normal(cout).astype(np.float32) * 0.1
    kp = (taps * c + 63) // 64 * 64
    res = rng.standard_normal((h * w, cout)).astype(np.float32) if with_res else None
    xin = np.repeat(np.repeat(x, 2, 0), 2, 1) if up == 1 else x
    if up == 2:
        want = vo.conv3s2(x.astype(np.float64), wt.astype(np.float64), b.astype(np.float64)).reshape(h * w, cout)
    else:
        want = vo.conv(xin.astype(np.float64), wt.astype(np.float64), b.astype(np.float64), k).reshape(h * w, cout)
    if with_res:
        want = want + res
    if out == 2:
        want = np.clip(want, -1, 1)
    y = X.DevBuf(ctx, (h * w, cout), np.uint16 if out == 1 else np.float32)
    rbuf = dev(ctx, res) if with_res else None
    part = X.DevBuf(ctx, (4 * h * w * cout,), np.float32) if split else None
    X.call("exn_vae_conv", ctx.h, taps, up, out, dev(ctx, xo.bf16_bits(x)).h, dev(ctx, pack_conv(wt, kp)).h,
           dev(ctx, b).h, rbuf.h if rbuf else None, y.h, h, w, c, cout, kp, part.h if part else None,
           4 * h * w * cout if part else 0)
    got = y.get()
    if out == 1:
        got = xo.bf16_to_f32(got)
        assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    else:
        assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())


def test_conv_rejects_bad_shapes(ctx):
    with pytest.raises(X.ExnError) as e:
        X.call("exn_vae_conv", ctx.h, 9, 0, 0, dev(ctx, np.zeros(64, np.uint16)).h, dev(ctx, np.zeros(64, np.uint16)).h,
               dev(ctx, np.zeros(4, np.float32)).h, None, dev(ctx, np.zeros(64, np.float32)).h, 1, 1, 40, 4, 384,
               None, 0)
    assert e.value.code == X.EINVAL


@pytest.mark.parametrize("c,silu", [(144, 1), (288, 1), (576, 1), (1152, 1), (1152, 0)])
def test_rms_silu(ctx, c, silu):
    rng = np.random.default_rng(c + silu)
    n = 777
    x = (rng.standard_normal((n, c)) * 3 + 0.5).astype(np.float32)
    x[5] = 0.0                                   # the 1e-12 floor
    g = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    want = vo.rms(x.reshape(1, n, c), g).reshape(n, c)
    if silu:
        want = vo.silu(want)
    y = X.DevBuf(ctx, (n, c), np.uint16)
    X.call("exn_vae_rms_silu", ctx.h, n, c, dev(ctx, x).h, dev(ctx, g).h, y.h, silu)
    got = xo.bf16_to_f32(y.get())
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max()
    assert np.all(got[5] == 0)


@pytest.mark.parametrize("cin,cout,ft", [(1152, 1152, 2), (1152, 576, 2), (576, 288, 1)])
def test_dupup_add(ctx, cin, cout, ft):
    rng = np.random.default_rng(cin + cout)
    h, w = 3, 5
    x = rng.standard_normal((h, w, cin)).astype(np.float32)
    y0 = rng.standard_normal((2 * h, 2 * w, cout)).astype(np.float32)
    y = dev(ctx, y0)
    X.call("exn_vae_dupup_add", ctx.h, cin, cout, ft, h, w, dev(ctx, x).h, y.h)
    assert np.array_equal(y.get(), y0 + vo.dupup(x, cout, ft))


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "ref_vae_tiny.npz"))


@pytest.fixture(scope="module")
def vae(ctx, golden):
    v = X.upload_vae(seed=int(golden["seed"][0]), ctx=ctx)
    yield v
    v.destroy()


@pytest.mark.parametrize("case", [0, 1])
def test_decode_against_reference_script(vae, golden, case):
    """The whole decoder on the synthetic weights, against the pictures the
    reference's inspect/ref_vae.py made from the same weights and latents."""
    z = golden["latent_%d" % case]
    h, w = z.shape[1:]
    want = golden["picture_%d" % case]
    got, ph, pw = X.vae_decode(vae, z, h, w)
    assert (ph, pw) == (16 * h, 16 * w)
    e, m = xo.rel_l2(got, want), float(np.abs(got - want).max())
    say("decode %d x %d: rel-L2 %.2e, max |diff| %.4f (%.2f of 255)" % (h, w, e, m, m * 127.5))
    assert e < 1e-2 and m <= PICTURE_MAX


def test_release_frees_scratch_and_keeps_weights(vae, golden):
    """vae-release (src/cuda-vae.lisp:28-33): the scratch freed, the weights kept; the next
    decode makes its buffers again and gives the same picture bit for bit."""
    z = golden["latent_0"]
    h, w = z.shape[1:]
    a, _, _ = X.vae_decode(vae, z, h, w)
    wb, sb = vae.memory()
    assert sb > 0
    vae.release()
    assert vae.memory() == (wb, 0)
    b, _, _ = X.vae_decode(vae, z, h, w)
    assert np.array_equal(a, b) and 0 < vae.memory()[1] <= sb


def test_decode_square_against_oracle(vae, golden):
    """A 4 x 4 latent (a 64 x 64 picture: every stage with several tiles of
    pixels), against the oracle on the same weights."""
    z = vo.synth_latent(21, 4, 4)
    got, _, _ = X.vae_decode(vae, z, 4, 4)
    want = vo.decode(vo.SynthVae(int(golden["seed"][0])), z)
    e, m = xo.rel_l2(got, want), float(np.abs(got - want).max())
    say("decode 4 x 4: rel-L2 %.2e, max |diff| %.4f (%.2f of 255)" % (e, m, m * 127.5))
    assert e < 1e-2 and m <= PICTURE_MAX
    # a second decode on the same scratch gives the same picture
    again, _, _ = X.vae_decode(vae, z, 4, 4)
    assert np.array_equal(again, got)


def test_vae_set_and_check_errors(ctx):
    v = X.Vae(ctx)
    with pytest.raises(X.ExnError) as e:
        v.check()
    assert e.value.code == X.ESTATE and "missing conv2.weight" in str(e.value)
    with pytest.raises(X.ExnError) as e:
        v.set("decoder.conv1.weight", X.F32, np.zeros(10, np.float32), (1152, 64, 3, 3))
    assert e.value.code == X.EINVAL and "not (1152 64 1 3 3)" in str(e.value)
    with pytest.raises(X.ExnError) as e:
        v.set("decoder.nothing", X.F32, np.zeros(1, np.float32), (1,))
    assert e.value.code == X.EINVAL
    v.set("decoder.head.2.bias", X.BF16, xo.bf16_bits(np.array([0.5, -0.25, 0, 1], np.float32)), (4,))
    v.destroy()


# --- the encoder ----------------------------------------------------------------------

@pytest.mark.parametrize("cin,cout,ft,h,w", [(96, 96, 1, 8, 12), (96, 192, 2, 6, 4), (384, 768, 2, 4, 6),
                                             (192, 384, 2, 10, 2)])
def test_avgdown_add(ctx, cin, cout, ft, h, w):
    """AvgDown3D's shortcut, added: against the oracle's view-and-mean form (fp32 sums of at
    most 8 values in another order: 1e-6)."""
    rng = np.random.default_rng(cin + cout + h)
    x = rng.standard_normal((h, w, cin)).astype(np.float32)
    y0 = rng.standard_normal((h // 2, w // 2, cout)).astype(np.float32)
    yb = X.DevBuf.of(ctx, y0)
    X.call("exn_vae_avgdown_add", ctx.h, cin, cout, ft, h, w, dev(ctx, x).h, yb.h)
    want = y0 + vo.avgdown(x, cout, ft)
    assert np.abs(yb.get() - want).max() <= 1e-6 * max(1.0, np.abs(want).max())


ENC_SEED = 23


@pytest.fixture(scope="module")
def enc_vae(ctx):
    v = X.upload_vae(seed=ENC_SEED, ctx=ctx)
    v.check_encoder()
    yield v
    v.destroy()


# the latent's distance to the oracle: bf16 operands (8 significant bits) in every convolution
# and the attention, through 14 residual blocks; measured 5.4e-3 .. 5.9e-3 (5.0e-3 with the
# blocks identities and centre-tap resamples), bar 1e-2
ENC_REL = 1e-2


@pytest.mark.parametrize("h,w", [(64, 64), (96, 128), (160, 48)])
def test_encode_against_oracle(enc_vae, h, w):
    """vae-encode on synthetic weights: the latent's mean against the oracle's encode of the
    same picture (one and several pixel tiles a stage; a picture taller than wide)."""
    px = vo.synth_picture(ENC_SEED + h, h, w)
    say("encode", h, "x", w)
    got = X.vae_encode(enc_vae, px, h, w)
    want = vo.encode(vo.SynthVae(ENC_SEED), px)
    e = xo.rel_l2(got, want)
    say("encode %d x %d: latent rel-L2 %.2e, |z| %.3f" % (h, w, e, float(np.sqrt((want * want).mean()))))
    assert got.shape == (64, h // 16, w // 16) and np.isfinite(got).all() and e < ENC_REL


def test_release_then_encode(enc_vae):
    """An encode after vae-release makes its buffers again: the same latent bit for bit."""
    px = vo.synth_picture(6, 64, 64)
    a = X.vae_encode(enc_vae, px, 64, 64)
    enc_vae.release()
    assert enc_vae.memory()[1] == 0
    assert np.array_equal(X.vae_encode(enc_vae, px, 64, 64), a)


def test_encode_device_entry_matches_host(ctx, enc_vae):
    """exn_vae_encode_dev on device arrays gives the host entry point's latent bit for bit."""
    h, w = 64, 96
    px = vo.synth_picture(5, h, w)
    want = X.vae_encode(enc_vae, px, h, w)
    pd = X.DevBuf.of(ctx, px)
    zd = X.DevBuf(ctx, (64, h // 16, w // 16), np.float32)
    X.call("exn_vae_encode_dev", enc_vae.h, pd.h, h, w, zd.h)
    assert np.array_equal(zd.get(), want)


def skeleton(wt):
    """Weights that make the encoder's blocks identities: every residual block's second
    convolution zero (a block returns its input or its shortcut), the attention's projection
    zero, and each stride-2 convolution the centre tap of its channel (output pixel (y, x) =
    input pixel (2y + 1, 2x + 1)): {name: array}, set into WT's cache too."""
    out = {}
    for n, shape in vo.vae_encoder_expected():
        if ".residual.6." in n or n.startswith("encoder.middle.1.proj.") or (".resample.1." in n and n.endswith(".bias")):
            out[n] = np.zeros(shape, np.float32)
        elif ".resample.1." in n:
            w = np.zeros(shape, np.float32)
            w[np.arange(shape[0]), np.arange(shape[0]), 1, 1] = 1
            out[n] = w
    wt.cache.update(out)
    return out


def test_encode_skeleton_wiring(ctx):
    """With the blocks identities and the stride-2 convolutions centre taps (the oracle's
    latent then a closed form of the wiring, tests/test_vae_oracle.py), the GPU's encode
    against the oracle's on the same weights: the first convolution, the blocks' output
    sampled by the stride-2 convolution plus AvgDown3D of each stage's input, the last stage's
    input added, the head.  Rounding moves it as far as the full encode (5e-3: the blocks'
    output and the head in bf16); a wiring mistake moves it by its own size, so the bar is the
    full encode's."""
    h, w = 64, 48
    v = X.upload_vae(seed=ENC_SEED, ctx=ctx)
    try:
        wt = vo.SynthVae(ENC_SEED)
        shapes = dict(vo.vae_encoder_expected())
        for n, a in skeleton(wt).items():
            v.set(n, X.F32, a, shapes[n])
        px = vo.synth_picture(41, h, w)
        got = X.vae_encode(v, px, h, w)
        want = vo.encode(wt, px)
        e = xo.rel_l2(got, want)
        say("skeleton encode rel-L2 %.2e" % e)
        assert e < ENC_REL
    finally:
        v.destroy()


def test_encode_rejects(ctx, enc_vae):
    """A picture whose sides are not multiples of 16; a decoder loaded without the encoder's
    tensors (EXN_ESTATE naming the first missing one)."""
    with pytest.raises(X.ExnError) as e:
        X.vae_encode(enc_vae, np.zeros((40, 64, 4), np.float32), 40, 64)
    assert e.value.code == X.EINVAL
    v = X.Vae(ctx)
    try:
        with pytest.raises(X.ExnError) as e:
            X.vae_encode(v, np.zeros((32, 32, 4), np.float32), 32, 32)
        assert e.value.code == X.ESTATE and "encoder.conv1.weight" in str(e.value)
    finally:
        v.destroy()


def test_large_pictures_tiles_agree(ctx, enc_vae):
    """Pictures of 2^18 pixels or more run their 96- and 144-wide convolutions on 128-pixel tiles
    (the norm in the store, the residual, the first convolution's 1 x 1 included): a 32 x 32
    latent's decode and a 512 x 512 picture's encode equal, bit for bit, the same on 256-pixel
    tiles only."""
    z = vo.synth_latent(33, 32, 32)
    px = vo.synth_picture(34, 512, 512)
    a, _, _ = X.vae_decode(enc_vae, z, 32, 32)
    la = X.vae_encode(enc_vae, px, 512, 512)
    X.call("exn_vae_tiles", enc_vae.h, 0)
    try:
        b, _, _ = X.vae_decode(enc_vae, z, 32, 32)
        lb = X.vae_encode(enc_vae, px, 512, 512)
    finally:
        X.call("exn_vae_tiles", enc_vae.h, 1)
    assert np.isfinite(a).all() and np.isfinite(la).all()
    assert np.array_equal(a, b) and np.array_equal(la, lb)
