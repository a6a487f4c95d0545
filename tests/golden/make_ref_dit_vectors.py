"""Writes tests/golden/ref_dit_tiny.npz: input/output vectors of the
reference's own numpy DiT (inspect/ref_dit.py `forward`, :108-153) at tiny
shapes, so that the oracle's forward composition is pinned against the
reference's and not against a retyping of it.

Run where the reference tree is (it does not travel with the tests):

    python tests/golden/make_ref_dit_vectors.py [/root/reference]

ref_dit.py imports llama.cpp's gguf-py at module level for its GGUF loader
(`Weights`, :23-30).  gguf-py is not installed; forward() takes the weights as
a callable and never touches gguf, so an empty placeholder module is put in
sys.modules for the import and nothing of it is ever called.  The weights are
the oracle's synthetic Q8_0 tensors, dequantised to fp32, handed to forward()
as the callable `wt`, each matrix times a float32 gain of 4 (GAIN) so that
the blocks change x visibly at this width.  The module globals W, HEADS, HD, FFN, LAYERS that
forward reads at call time (:19) are set to a tiny model: width 256, 2 heads
of 128 (HD stays 128 so the 16/56/56 RoPE axes still fit), FFN 512, 2 layers.

Fixture contents per case i: c{i}_meta = [seed, p, h, w, sigma], c{i}_ctx,
c{i}_latent (the inputs, so a test sees the generator unchanged), c{i}_wsum
(float64 sum of every weight tensor in dit_expected order), c{i}_txt,
c{i}_blk0, c{i}_v (forward's dumps and result).
"""
import importlib.util
import os
import sys
import tempfile
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
from oracle import exn_oracle as xo  # noqa: E402

TINY = xo.Shape(width=256, layers=2, head_dim=128, ffn=512, latent=64, context=256, freq=256)
GAIN = 4.0
CASES = [  # seed, p, h, w, sigma
    (7, 8, 4, 4, 0.5),
    (11, 5, 3, 6, 0.978453),
    (3, 1, 2, 5, 1.0),
]


def load_ref_dit(ref_root):
    path = os.path.join(ref_root, "inspect", "ref_dit.py")
    placeholder = types.ModuleType("gguf")
    placeholder.quants = types.ModuleType("gguf.quants")
    sys.modules.setdefault("gguf", placeholder)
    sys.modules.setdefault("gguf.quants", placeholder.quants)
    spec = importlib.util.spec_from_file_location("ref_dit_reference", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.W, mod.HEADS, mod.HD, mod.FFN, mod.LAYERS = (TINY.width, TINY.heads, TINY.head_dim, TINY.ffn, TINY.layers)
    return mod


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_ref_dit(ref_root)
    out = {}
    for i, (seed, p, h, w, sigma) in enumerate(CASES):
        wt = xo.SynthWeights(seed, TINY, gain=GAIN)
        ctx, lat = xo.synth_inputs(seed, p, h, w, TINY)
        with tempfile.TemporaryDirectory() as d:
            v = ref.forward(wt, ctx, lat, sigma, dump=d)
            txt = np.fromfile(os.path.join(d, "txt.f32"), dtype=np.float32).reshape(p, TINY.width)
            blk0 = np.fromfile(os.path.join(d, "blk0.f32"), dtype=np.float32).reshape(p + h * w, TINY.width)
        out["c%d_meta" % i] = np.array([seed, p, h, w, sigma], dtype=np.float64)
        out["c%d_ctx" % i] = ctx
        out["c%d_latent" % i] = lat
        out["c%d_wsum" % i] = np.array([float(np.sum(wt(n), dtype=np.float64)) for n, _ in xo.dit_expected(TINY)])
        out["c%d_txt" % i] = txt
        out["c%d_blk0" % i] = blk0
        out["c%d_v" % i] = v.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "ref_dit_tiny.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_dit_tiny.npz"), sorted(out))


if __name__ == "__main__":
    main()
