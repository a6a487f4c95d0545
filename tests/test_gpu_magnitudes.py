"""Parity off the unit-scale synthetic data: the 1024^2 workload's shapes, two blocks deep,
with weights that put the activations where real checkpoints put them (the oracle's
MAGNITUDE_CASES), against the oracle's velocity (relative L2 <= 1e-2; cached in
tests/golden/dit_magnitudes_2blocks.npz as float16 by make_dit_vectors.py mag).

txt_in_8e5: txt_in's GELU rows at about 8e5, as the reference records for the real weights
(src/metal-dit.lisp:5-7), so the prompt rows of the residual stream reach about 7e5 while the
image rows sit near 1.  img_in_outliers: eight of the residual stream's 4096 channels 80 times
the rest on every image row, so each LayerNorm's variance is theirs.  Needs an MI355X."""
import os
import sys

import numpy as np
import pytest

import exn_hip as X
from oracle import exn_oracle as xo

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEED, P, H, W, SIGMA = 2, 256, 64, 64, 0.978453


def say(*a):
    print("[gpu]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = X.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("case", list(xo.MAGNITUDE_CASES))
def test_real_checkpoint_magnitudes(ctx, case):
    want = np.load(os.path.join(GOLDEN, "dit_magnitudes_2blocks.npz"))[case].astype(np.float32)
    say(case, ": 2 blocks, p", P, "image", H, "x", W)
    d = X.Dit(ctx, 2)
    d.synth(SEED)
    base = xo.SynthWeights(SEED, cache_bytes=0)
    over = xo.magnitude_overrides(base, case)
    dims = dict(xo.dit_expected(xo.Shape(layers=2)))
    for name, m in over.items():
        d.set(name, X.F32, m, dims[name])   # edge matrices the real file stores as F32: multiplied in fp32
    d.check()
    ctxa, lat = xo.synth_inputs(SEED, P, H, W)
    n = P + H * W
    tr = X.DevBuf(ctx, (3, n, 4096), np.float32)
    X.call("exn_dit_trace", d.h, tr.h, 3 * n * 4096)
    v0 = X.dit_velocity(d, ctxa, P, lat, H, W, SIGMA, prefix_key="k")
    X.call("exn_dit_trace", d.h, None, 0)
    x_in = tr.get()[0]   # the residual stream entering the first block
    if case == "txt_in_8e5":
        top = float(np.abs(x_in[:P]).max())
        say("prompt rows of the block input: max |x| %.3g; image rows %.3g" % (top, float(np.abs(x_in[P:]).max())))
        assert top > 1e5
    else:
        rows = list(xo.MAGNITUDE_CASES[case][1])
        rest = np.delete(x_in[P:], rows, axis=1)
        ratio = float(np.sqrt((x_in[P:, rows] ** 2).mean() / (rest ** 2).mean()))
        say("image rows: outlier channels' rms %.1f x the others'" % ratio)
        assert ratio > 20
    v1 = X.dit_velocity(d, ctxa, P, lat, H, W, SIGMA, prefix_key="k")   # cached: the kept prompt K/V
    d.resident(False)
    v2 = X.dit_velocity(d, ctxa, P, lat, H, W, SIGMA)                     # Q8_0 dequantised in the products
    d.resident(True)
    e0, e01 = xo.rel_l2(v0, want), xo.rel_l2(v1, v0)
    say("%s: velocity against the oracle rel-L2 %.2e, cached vs uncached %.2e" % (case, e0, e01))
    assert np.isfinite(v0).all() and e0 < 1e-2 and e01 < 1e-5
    assert np.array_equal(v2, v0)
    d.destroy()
