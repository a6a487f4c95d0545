"""Pins oracle/exn_vae_oracle.py (the VAE decoder's and encoder's CPU restatement):
decode against the reference's own inspect/ref_vae.py (vectors in
tests/golden/ref_vae_tiny.npz, written by make_ref_vae_vectors.py from the same
synthetic weights), and the pieces against float64 brute force, closed forms and
src/cuda/vae.cu's index formulas; the encoder's stride-2 convolution by brute
force, its AvgDown3D against x_avgdown_add's index formula, its stage wiring by a
closed form on identity blocks."""
import os

import numpy as np
import pytest

from oracle import exn_oracle as xo
from oracle import exn_vae_oracle as vo

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "ref_vae_tiny.npz"))


@pytest.fixture(scope="module")
def wt(golden):
    return vo.SynthVae(int(golden["seed"][0]))


@pytest.mark.parametrize("case", [0, 1])
def test_decode_matches_reference_script(golden, wt, case):
    """The whole decoder, 2 x 2 and 2 x 3 latents at full widths, against
    inspect/ref_vae.py run on the same bf16 weights: float32 both, so only the
    summation order differs."""
    z = golden["latent_%d" % case]
    want = golden["picture_%d" % case]
    got = vo.decode(wt, z)
    assert got.shape == want.shape == (16 * z.shape[1], 16 * z.shape[2], 4)
    assert np.abs(got - want).max() < 1e-4
    assert (np.abs(want) >= 1).mean() > 0.05          # the clamp is exercised


def test_synthetic_weights_are_bf16_and_deterministic(wt):
    a = wt("decoder.upsamples.2.upsamples.0.shortcut.weight")
    assert a.shape == (576, 1152, 1, 1, 1)
    assert np.array_equal(xo.bf16_round(a), a)
    b = vo.SynthVae(int(wt.seed))("decoder.upsamples.2.upsamples.0.shortcut.weight")
    assert np.array_equal(a, b)
    g = wt("decoder.head.0.gamma")
    assert g.shape == (144, 1, 1, 1) and abs(float(g.mean()) - 1) < 0.05


def test_schema_follows_the_stages():
    """src/weights.lisp:69-98: a shortcut exactly where a residual block changes
    width, a resample convolution on the four upsampling stages."""
    names = dict(vo.vae_expected())
    shortcuts = sorted(n for n in names if n.endswith("shortcut.weight"))
    assert shortcuts == ["decoder.upsamples.%d.upsamples.0.shortcut.weight" % s for s in (2, 3, 4)]
    assert [s for s in range(5) if "decoder.upsamples.%d.upsamples.3.resample.1.weight" % s in names] == [0, 1, 2, 3]
    assert names["decoder.conv1.weight"] == (1152, 64, 1, 3, 3)
    assert names["decoder.middle.1.to_qkv.weight"] == (3456, 1152, 1, 1)
    assert names["decoder.head.2.weight"] == (4, 144, 1, 3, 3)


def test_conv3_against_direct_sum():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 7, 6)).astype(np.float32)
    w = rng.standard_normal((4, 6, 1, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    got = vo.conv(x, w, b, 3)
    want = np.zeros((5, 7, 4))
    for y in range(5):
        for xx in range(7):
            for o in range(4):
                s = float(b[o])
                for dy in range(3):
                    for dx in range(3):
                        sy, sx = y + dy - 1, xx + dx - 1
                        if 0 <= sy < 5 and 0 <= sx < 7:
                            s += float(np.dot(x[sy, sx].astype(np.float64), w[o, :, 0, dy, dx].astype(np.float64)))
                want[y, xx, o] = s
    assert np.abs(got - want).max() < 1e-4


def test_rms_closed_form():
    """A pixel whose channels are all v (v != 0) normalizes to sign(v) * gamma;
    a zero pixel stays zero (the 1e-12 floor)."""
    x = np.zeros((1, 2, 8), np.float32)
    x[0, 0] = -3.0
    g = np.arange(1, 9, dtype=np.float32).reshape(8, 1, 1, 1)
    y = vo.rms(x, g)
    assert np.allclose(y[0, 0], -np.arange(1, 9), atol=1e-6) and np.all(y[0, 1] == 0)


@pytest.mark.parametrize("cin,cout,ft", [(8, 8, 2), (8, 4, 2), (4, 2, 1), (6, 6, 1)])
def test_dupup_index_formula(cin, cout, ft):
    """src/cuda/vae.cu's x_dupup_add: output channel c of pixel (Y, X) is input
    channel j / rep of pixel (Y/2, X/2), j = ((c ft + ft - 1) 2 + Y%2) 2 + X%2."""
    rng = np.random.default_rng(cin * 10 + cout)
    x = rng.standard_normal((3, 2, cin)).astype(np.float32)
    got = vo.dupup(x, cout, ft)
    rep = cout * ft * 4 // cin
    for yy in range(6):
        for xx in range(4):
            for c in range(cout):
                j = ((c * ft + ft - 1) * 2 + yy % 2) * 2 + xx % 2
                assert got[yy, xx, c] == x[yy // 2, xx // 2, j // rep]


def test_attention_against_float64():
    rng = np.random.default_rng(3)
    c = 16
    t = {"p.norm.gamma": (1 + 0.1 * rng.standard_normal((c, 1, 1))).astype(np.float32),
         "p.to_qkv.weight": (rng.standard_normal((3 * c, c, 1, 1)) / 4).astype(np.float32),
         "p.to_qkv.bias": (0.1 * rng.standard_normal(3 * c)).astype(np.float32),
         "p.proj.weight": (rng.standard_normal((c, c, 1, 1)) / 4).astype(np.float32),
         "p.proj.bias": (0.1 * rng.standard_normal(c)).astype(np.float32)}
    x = rng.standard_normal((3, 5, c)).astype(np.float32)
    got = vo.attention(t.__getitem__, "p", x)
    xd = x.reshape(-1, c).astype(np.float64)
    n = np.sqrt((xd * xd).sum(-1, keepdims=True))
    y = xd / n * np.sqrt(c) * t["p.norm.gamma"].reshape(-1)
    qkv = y @ t["p.to_qkv.weight"][:, :, 0, 0].T.astype(np.float64) + t["p.to_qkv.bias"]
    q, k, v = qkv[:, :c], qkv[:, c:2 * c], qkv[:, 2 * c:]
    s = q @ k.T / np.sqrt(c)
    p = np.exp(s - s.max(-1, keepdims=True))
    a = (p / p.sum(-1, keepdims=True)) @ v
    want = a @ t["p.proj.weight"][:, :, 0, 0].T.astype(np.float64) + t["p.proj.bias"] + xd
    assert np.abs(got.reshape(-1, c) - want).max() < 1e-4


def test_decode_flops_counts_every_product(monkeypatch, golden, wt):
    """decode_flops against the products decode actually takes (convolutions
    counted as they run, the attention's two products added)."""
    count = {"f": 0}
    real = vo.conv

    def counting(x, w, b, k):
        count["f"] += 2 * x.shape[0] * x.shape[1] * w.shape[0] * w.shape[1] * k * k
        return real(x, w, b, k)

    monkeypatch.setattr(vo, "conv", counting)
    z = golden["latent_1"]
    vo.decode(wt, z)
    h, w = z.shape[1:]
    n = h * w
    assert count["f"] + 2 * 2 * n * n * 1152 == vo.decode_flops(h, w)
    assert vo.decode_flops(64, 64) == pytest.approx(17.03e12, rel=1e-3)



# --- the encoder ----------------------------------------------------------------------

def test_encoder_schema_follows_the_stages():
    """src/weights.lisp:100-134: conv1 on RGBA, two residual blocks a stage with a shortcut
    where the width changes, a stride-2 convolution (no frame axis) on the four downsampling
    stages, the middle, the head to 2 x 64 channels and conv1 (1 x 1)."""
    names = dict(vo.vae_encoder_expected())
    assert len(names) == 98
    assert names["encoder.conv1.weight"] == (96, 4, 1, 3, 3)
    shortcuts = sorted(n for n in names if n.endswith("shortcut.weight"))
    assert shortcuts == ["encoder.downsamples.%d.downsamples.0.shortcut.weight" % s for s in (1, 2, 3)]
    assert [s for s in range(5) if "encoder.downsamples.%d.downsamples.2.resample.1.weight" % s in names] == [0, 1, 2, 3]
    assert names["encoder.downsamples.3.downsamples.2.resample.1.weight"] == (768, 768, 3, 3)
    assert names["encoder.middle.1.to_qkv.weight"] == (2304, 768, 1, 1)
    assert names["encoder.head.2.weight"] == (128, 768, 1, 3, 3)
    assert names["conv1.weight"] == (128, 128, 1, 1, 1)
    assert not set(names) & set(dict(vo.vae_expected()))   # no name shared with the decoder


def test_conv3s2_against_direct_sum():
    """The stride-2 convolution against a float64 sum over every output pixel and tap, the
    input padded with zeros below and to the right only (x_conv3s2's bounds: rows 2y .. 2y + 2
    and columns 2x .. 2x + 2 of the input, off it zero)."""
    rng = np.random.default_rng(7)
    h2, w2, c, o = 6, 10, 5, 3
    x = rng.standard_normal((h2, w2, c))
    w = rng.standard_normal((o, c, 3, 3))
    b = rng.standard_normal(o)
    got = vo.conv3s2(x, w, b)
    want = np.zeros((h2 // 2, w2 // 2, o))
    for y in range(h2 // 2):
        for xx in range(w2 // 2):
            for ky in range(3):
                for kx in range(3):
                    sy, sx = 2 * y + ky, 2 * xx + kx
                    if sy < h2 and sx < w2:
                        want[y, xx] += w[:, :, ky, kx] @ x[sy, sx]
            want[y, xx] += b
    assert np.abs(got - want).max() < 1e-4
    # a symmetric padding (rows 2y - 1 .. 2y + 1) gives another answer
    xs = np.pad(x, ((1, 1), (1, 1), (0, 0)))
    sym = sum(xs[ky:ky + h2:2, kx:kx + w2:2] @ w[:, :, ky, kx].T for ky in range(3) for kx in range(3)) + b
    assert np.abs(sym - want).max() > 0.1


def avgdown_index_formula(x, cout, ft, swap_rc=False, pad_last=False, chan_mod=False):
    """src/cuda/vae.cu's x_avgdown_add as a loop: output channel o of pixel (Y, X) sums x at
    channel j / (4 ft), row 2Y + (j / 2) % 2, column 2X + j % 2 for the j = o g .. o g + g - 1
    whose frame (j / 4) % ft is the last, over g = cin ft 4 / cout.  The flags plant mistakes:
    the block's row and column bits exchanged, the real frame first, the channel as j % cin."""
    h, w, cin = x.shape
    g = cin * ft * 4 // cout
    out = np.zeros((h // 2, w // 2, cout))
    for yy in range(h // 2):
        for xx in range(w // 2):
            for o in range(cout):
                s = 0.0
                for k in range(g):
                    j = o * g + k
                    if (j >> 2) % ft != (0 if pad_last else ft - 1):
                        continue
                    r, c = (j >> 1) & 1, j & 1
                    if swap_rc:
                        r, c = c, r
                    s += x[2 * yy + r, 2 * xx + c, j % cin if chan_mod else j // (4 * ft)]
                out[yy, xx, o] = s / g
    return out


# (cin, cout, ft, the planted mistakes the case tells apart)
AVGDOWN_CASES = [(8, 8, 1, ("chan_mod",)), (6, 12, 2, ("pad_last",)), (4, 8, 1, ("swap_rc", "chan_mod")),
                 (4, 16, 2, ("swap_rc", "pad_last")), (12, 12, 2, ("chan_mod",)), (8, 4, 1, ("chan_mod",))]


@pytest.mark.parametrize("cin,cout,ft,mistakes", AVGDOWN_CASES)
def test_avgdown_view_against_index_formula(cin, cout, ft, mistakes):
    """The view-and-mean form of AvgDown3D (the oracle) against x_avgdown_add's index formula,
    and the formula with each planted mistake the case's geometry can show failing it."""
    rng = np.random.default_rng(cin * 10 + cout + ft)
    x = rng.standard_normal((6, 4, cin)).astype(np.float32)
    got = vo.avgdown(x, cout, ft)
    want = avgdown_index_formula(x.astype(np.float64), cout, ft)
    assert np.abs(got - want).max() < 1e-6
    for m in mistakes:
        assert np.abs(avgdown_index_formula(x.astype(np.float64), cout, ft, **{m: True}) - got).max() > 1e-3, m


def test_encode_identity_blocks_closed_form():
    """The stage wiring: with every residual block's second convolution, every stride-2
    convolution and the attention's projection zero, a block returns its input (or its
    shortcut) and the encoder is the first convolution, then per downsampling stage the mean
    of each 2 x 2 block of the stage's input (with temporal downsampling only the odd output
    channels, o // 2's mean: the padding frame comes first), the last stage's input doubled,
    and the head -- computed here by hand from those rules."""
    wt = vo.SynthVae(3)
    for n, shape in vo.vae_encoder_expected():
        if ".residual.6." in n or ".resample.1." in n or n.startswith("encoder.middle.1.proj."):
            wt.cache[n] = np.zeros(shape, np.float32)
    px = vo.synth_picture(9, 32, 48)
    got = vo.encode(wt, px)
    x = vo.conv(px, wt("encoder.conv1.weight"), wt("encoder.conv1.bias"), 3).astype(np.float64)
    for s, (i, o, down, tdown) in enumerate(vo.ENC_STAGES):
        if not down:
            x = 2 * x
            continue
        h, w = x.shape[0] // 2, x.shape[1] // 2
        m = x.reshape(h, 2, w, 2, i).mean(axis=(1, 3))
        if tdown:
            y = np.zeros((h, w, o))
            y[..., 1::2] = m   # odd channel o: channel o // 2 of the stage's input
            x = y
        else:
            x = m
    x = x.astype(np.float32)
    x = vo.silu(vo.rms(x, wt("encoder.head.0.gamma")))
    x = vo.conv(x, wt("encoder.head.2.weight"), wt("encoder.head.2.bias"), 3)
    x = vo.conv(x, wt("conv1.weight"), wt("conv1.bias"), 1)
    want = x[..., :64].transpose(2, 0, 1)
    assert got.shape == (64, 2, 3)
    assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())


def identity_resample(shape):
    """A stride-2 convolution's weights (o, o, 3, 3) taking each channel's centre tap: output
    pixel (y, x) = input pixel (2y + 1, 2x + 1)."""
    w = np.zeros(shape, np.float32)
    o = shape[0]
    w[np.arange(o), np.arange(o), 1, 1] = 1
    return w


def centre_tap_by_hand(wt, px, skip_from_blocks=False):
    """test_encode_identity_blocks_centre_tap_closed_form's latent by the rules alone; with
    SKIP_FROM_BLOCKS the planted mistake of AvgDown3D taken of the blocks' output instead of the
    stage's input."""
    x = vo.conv(px, wt("encoder.conv1.weight"), wt("encoder.conv1.bias"), 3).astype(np.float64)
    for s, (i, o, down, tdown) in enumerate(vo.ENC_STAGES):
        keep = x
        if i != o:   # the first block's shortcut (1 x 1): its second convolution is zero
            p = "encoder.downsamples.%d.downsamples.0.shortcut" % s
            w = wt(p + ".weight").reshape(o, i).astype(np.float64)
            x = x @ w.T + wt(p + ".bias")
        if not down:
            x = x + keep
            continue
        src, c = (x, o) if skip_from_blocks else (keep, i)
        h, w2 = src.shape[0] // 2, src.shape[1] // 2
        g = c * (2 if tdown else 1) * 4 // o
        m = src.reshape(h, 2, w2, 2, c).mean(axis=(1, 3))
        if tdown:   # odd output channel o: input channel o // 2 (g = 4); g = 8: the mean of two
            full = np.zeros((h, w2, c, 2))
            full[..., 1] = m
            skip = full.reshape(h, w2, o, g // 4).mean(-1) if g > 4 else None
            if g == 4:
                skip = np.zeros((h, w2, o))
                skip[..., 1::2] = m
        else:
            skip = m if c == o else m.reshape(h, w2, o, c // o).mean(-1)
        x = x[1::2, 1::2] + skip
    x = x.astype(np.float32)
    x = vo.silu(vo.rms(x, wt("encoder.head.0.gamma")))
    x = vo.conv(x, wt("encoder.head.2.weight"), wt("encoder.head.2.bias"), 3)
    x = vo.conv(x, wt("conv1.weight"), wt("conv1.bias"), 1)
    return x[..., :64].transpose(2, 0, 1)


def test_encode_identity_blocks_centre_tap_closed_form():
    """The wiring with the stride-2 convolutions live: residual blocks their input or their
    shortcut (second convolutions zero), each stride-2 convolution the centre tap of its
    channel, the attention's projection zero.  A downsampling stage's output is then the
    stage's blocks' output at the odd rows and columns (the resample reads the blocks, at 2y +
    1) plus AvgDown3D of the stage's input; computed by hand, and the same by hand with the
    skip taken of the blocks' output instead fails it."""
    wt = vo.SynthVae(5)
    shapes = dict(vo.vae_encoder_expected())
    for n, shape in shapes.items():
        if ".residual.6." in n or n.startswith("encoder.middle.1.proj.") or (".resample.1." in n and n.endswith(".bias")):
            wt.cache[n] = np.zeros(shape, np.float32)
        elif ".resample.1." in n:
            wt.cache[n] = identity_resample(shape)
    px = vo.synth_picture(12, 32, 48)
    got = vo.encode(wt, px)
    want = centre_tap_by_hand(wt, px)
    assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())
    wrong = centre_tap_by_hand(wt, px, skip_from_blocks=True)
    assert np.abs(got - wrong).max() > 1e-2 * np.abs(want).max()


def test_encode_flops_counts_every_product(monkeypatch):
    """encode_flops against the products encode takes (every convolution as it runs, the
    stride-2 ones at their output size, the attention's two added)."""
    count = {"f": 0}
    real_conv, real_s2 = vo.conv, vo.conv3s2

    def counting(x, w, b, k):
        count["f"] += 2 * x.shape[0] * x.shape[1] * w.shape[0] * w.shape[1] * k * k
        return real_conv(x, w, b, k)

    def counting_s2(x, w, b):
        count["f"] += 2 * (x.shape[0] // 2) * (x.shape[1] // 2) * w.shape[0] * w.shape[1] * 9
        return real_s2(x, w, b)

    monkeypatch.setattr(vo, "conv", counting)
    monkeypatch.setattr(vo, "conv3s2", counting_s2)
    vo.encode(vo.SynthVae(4), vo.synth_picture(2, 32, 32))
    n = 2 * 2
    assert count["f"] + 2 * 2 * n * n * 768 == vo.encode_flops(32, 32)
