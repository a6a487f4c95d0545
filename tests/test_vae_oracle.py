"""Pins oracle/exn_vae_oracle.py (the VAE decoder's CPU restatement): decode
against the reference's own inspect/ref_vae.py (vectors in
tests/golden/ref_vae_tiny.npz, written by make_ref_vae_vectors.py from the same
synthetic weights), and the pieces against float64 brute force, closed forms and
src/cuda/vae.cu's index formulas."""
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
