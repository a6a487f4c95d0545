"""Writes tests/golden/ref_vision_tiny.npz: the outputs of the reference's own numpy
vision tower (inspect/ref_vision.py `main`, :72-148) on synthetic weights at a
narrow width, the vectors that pin oracle/exn_vision_oracle.py's encode.

Run where the reference tree is (it does not travel with the tests):

    python tests/golden/make_ref_vision_vectors.py [/root/reference]

ref_vision.py imports llama.cpp's gguf-py at module level and reads its weights
through its `Weights` class (:26-33), a GGUF reader.  gguf-py is not installed:
an empty placeholder module stands in for the import and nothing of it is
called, and the module's `Weights` is replaced by the oracle's synthetic
tensors (oracle/exn_vision_oracle.py's SynthVision), handed over by name as
the reader would.  The module globals main() reads at call time (:20-22) are
set to a narrow tower: width 144, 2 heads of 72 (the head dim of the real
one, so the 2-D rotary's 18 + 18 frequencies are unchanged), FFN 160, 4
blocks with the deepstack mergers after blocks 1, 2 and 3, an output width
of 96 and a 6 x 6 position table.  main() is called with the pixels (RGB, H x
W x 3 floats, as its usage line says) in a temporary file and reads its
outputs back from the directory it writes.

Fixture contents per case i: c{i}_meta = [seed, h, w], c{i}_px (the RGBA
picture: the oracle reads channels 0-2, ref_vision.py the same three),
c{i}_wsum (float64 sum of every tensor in vision_expected order),
c{i}_embed, c{i}_blk0, c{i}_merged, c{i}_ds (3 x M x OUT).
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
from oracle import exn_vision_oracle as vo  # noqa: E402

TINY = vo.VShape(width=144, heads=2, ffn=160, depth=4, deepstack=(1, 2, 3), out=96, side=6)
SEED = 13
CASES = [(64, 96), (32, 32), (128, 64)]   # h, w: a wide grid, one merge block, a grid taller than the table


def load_ref_vision(ref_root):
    path = os.path.join(ref_root, "inspect", "ref_vision.py")
    placeholder = types.ModuleType("gguf")
    placeholder.quants = types.ModuleType("gguf.quants")
    sys.modules.setdefault("gguf", placeholder)
    sys.modules.setdefault("gguf.quants", placeholder.quants)
    spec = importlib.util.spec_from_file_location("ref_vision_reference", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.D, mod.HEADS, mod.FF, mod.DEPTH, mod.OUT = TINY.width, TINY.heads, TINY.ffn, TINY.depth, TINY.out
    mod.HD = TINY.head_dim
    mod.DEEPSTACK = TINY.deepstack
    return mod


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_ref_vision(ref_root)
    wt = vo.SynthVision(SEED, TINY)
    ref.Weights = lambda path: wt
    out = {}
    for i, (h, w) in enumerate(CASES):
        px = vo.synth_picture(SEED + i, h, w)
        m = (h // 32) * (w // 32)
        with tempfile.TemporaryDirectory() as d:
            pix = os.path.join(d, "px.f32")
            np.ascontiguousarray(px[..., :3]).tofile(pix)
            argv = sys.argv
            sys.argv = ["ref_vision.py", "synthetic.gguf", pix, str(h), str(w), d]
            try:
                ref.main()
            finally:
                sys.argv = argv
            n = (h // 16) * (w // 16)
            rd = lambda name, rows, cols: np.fromfile(os.path.join(d, name), dtype=np.float32).reshape(rows, cols)
            out["c%d_embed" % i] = rd("embed.f32", n, TINY.width)
            out["c%d_blk0" % i] = rd("blk0.f32", n, TINY.width)
            out["c%d_merged" % i] = rd("merged.f32", m, TINY.out)
            out["c%d_ds" % i] = np.stack([rd("ds%d.f32" % j, m, TINY.out) for j in range(3)])
        out["c%d_meta" % i] = np.array([SEED, h, w], dtype=np.int64)
        out["c%d_px" % i] = px
        out["c%d_wsum" % i] = np.array([float(np.sum(wt(n), dtype=np.float64)) for n, _ in vo.vision_expected(TINY)])
    np.savez_compressed(os.path.join(HERE, "ref_vision_tiny.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_vision_tiny.npz"), sorted(out))


if __name__ == "__main__":
    main()
