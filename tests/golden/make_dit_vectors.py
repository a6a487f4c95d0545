"""Writes the oracle's results for the full-depth GPU parity tests, which the
GPU tests cannot afford to recompute (a 32-block numpy step is
minutes of CPU).  These are the oracle's outputs (oracle/exn_oracle.py,
itself pinned against the reference's ref_dit.py vectors), cached:

    python tests/golden/make_dit_vectors.py small      # dit_depth32_small.npz
    python tests/golden/make_dit_vectors.py cfg2       # dit_cfg2_8step.npz (about 1.5 hours)
    python tests/golden/make_dit_vectors.py full2      # dit_full_shapes_2blocks.npz (a few minutes)
    python tests/golden/make_dit_vectors.py cfg3       # dit_cfg3_8step.npz (hours)
    python tests/golden/make_dit_vectors.py cfg4       # dit_cfg4_edit_8step.npz (hours)
    python tests/golden/make_dit_vectors.py mag        # dit_magnitudes_2blocks.npz (a few minutes)

small: 32 blocks of the real shape, synthetic Q8_0 weights (seed 1), 32 text
rows, an 8 x 8 latent: the velocity of each of the 8 Turbo steps (the first
uncached, the rest on the kept prompt K/V) and the final latent.
cfg2: the 1024^2 workload -- 4096 image rows, 256 text rows, 32 blocks (seed
2) -- through the 8 Euler steps: the first step's velocity and the final
latent, stored as float16 (far below the 2e-2 tolerance).
cfg3: the 1536 x 1024 workload -- 6144 image rows (96 x 64), 256 text rows,
32 blocks (seed 6) -- the same 8 steps and fields as cfg2.
cfg4: the edit workload -- a 64 x 64 image after 512 text rows with a 64 x 64
reference picture after the first 8 of them (8704 keys), 32 blocks (seed 7) --
the same 8 steps (the prefix, text and reference picture, kept after the first).
mag: the 1024^2 workload's shapes, two blocks deep (seed 2, sigma 0.978453), with the
weights of each of the oracle's MAGNITUDE_CASES (activations at real-checkpoint magnitudes):
the velocity, as float16.
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import exn_oracle as xo  # noqa: E402


def run(seed, p, h, w, out, half=False, ref=None):
    sh = xo.Shape()
    wt = xo.SynthWeights(seed, sh, cache_bytes=0, keep_q8=True)
    if ref is None:
        ctx, lat = xo.synth_inputs(seed, p, h, w, sh)
        oref = None
    else:
        a, rh, rw = ref
        ctx, lat, rl = xo.synth_inputs(seed, p, h, w, sh, ref_hw=(rh, rw))
        oref = (a, rl)
    vs = []
    t0 = time.time()

    def on_step(s, v, z):
        vs.append(v)
        print("step sigma %.6f: |v| %.4f, %.0fs" % (s, float(np.sqrt((v * v).mean())), time.time() - t0), flush=True)

    z = xo.euler(wt, ctx, lat, sh, ref=oref, on_step=on_step)
    dt = np.float16 if half else np.float32
    arrays = {"meta": np.array([seed, p, h, w], np.int64), "z_final": z.astype(dt)}
    if ref is not None:
        arrays["ref"] = np.array(ref, np.int64)
    if half:
        arrays["v_step0"] = vs[0].astype(dt)
    else:
        arrays["v_steps"] = np.stack(vs).astype(dt)
    np.savez_compressed(os.path.join(HERE, out), **arrays)
    print("wrote", out)


# the workloads' full shapes, two blocks deep: (seed, text rows, h, w, (a, rh, rw) or None, sigma)
FULL_CASES = {
    "cfg2_1024sq": (2, 256, 64, 64, None, 0.978453),
    "cfg3_1536x1024": (6, 256, 96, 64, None, 0.95418),
    "cfg4_edit_1024sq": (7, 512, 64, 64, (8, 64, 64), 0.926626),
}


def full_shapes(out):
    arrays = {}
    for name, (seed, p, h, w, ref, sigma) in FULL_CASES.items():
        t0 = time.time()
        if ref is None:
            ctx, lat = xo.synth_inputs(seed, p, h, w)
            oref = None
        else:
            a, rh, rw = ref
            ctx, lat, rl = xo.synth_inputs(seed, p, h, w, ref_hw=(rh, rw))
            oref = (a, rl)
        v = xo.forward(xo.SynthWeights(seed, cache_bytes=0), ctx, lat, sigma, ref=oref, layers=2)
        arrays[name] = v.astype(np.float16)
        print("%s: |v| %.4f, %.0fs" % (name, float(np.sqrt((v * v).mean())), time.time() - t0), flush=True)
    np.savez_compressed(os.path.join(HERE, out), **arrays)
    print("wrote", out)


def magnitudes(out):
    seed, p, h, w, _, sigma = FULL_CASES["cfg2_1024sq"]
    ctx, lat = xo.synth_inputs(seed, p, h, w)
    arrays = {}
    for case in xo.MAGNITUDE_CASES:
        t0 = time.time()
        base = xo.SynthWeights(seed, cache_bytes=0)
        wt = xo.Overrides(base, xo.magnitude_overrides(base, case))
        v = xo.forward(wt, ctx, lat, sigma, layers=2)
        arrays[case] = v.astype(np.float16)
        print("%s: |v| %.4f, %.0fs" % (case, float(np.sqrt((v * v).mean())), time.time() - t0), flush=True)
    np.savez_compressed(os.path.join(HERE, out), **arrays)
    print("wrote", out)


if __name__ == "__main__":
    which = sys.argv[1] if len(sys.argv) > 1 else "small"
    if which == "small":
        run(1, 32, 8, 8, "dit_depth32_small.npz")
    elif which == "cfg2":
        run(2, 256, 64, 64, "dit_cfg2_8step.npz", half=True)
    elif which == "full2":
        full_shapes("dit_full_shapes_2blocks.npz")
    elif which == "cfg3":
        run(6, 256, 96, 64, "dit_cfg3_8step.npz", half=True)
    elif which == "cfg4":
        run(7, 512, 64, 64, "dit_cfg4_edit_8step.npz", half=True, ref=(8, 64, 64))
    elif which == "mag":
        magnitudes("dit_magnitudes_2blocks.npz")
