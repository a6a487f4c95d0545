"""Writes tests/golden/ref_vae_tiny.npz: the reference's own decoder in numpy
(inspect/ref_vae.py, run unmodified as `python3 -I ref_vae.py VAE LATENT H W
OUT`) on synthetic bf16 weights and two tiny latents, the vectors that pin
oracle/exn_vae_oracle.py's decode.

    python tests/golden/make_ref_vae_vectors.py [/root/reference]

The weights (oracle/exn_vae_oracle.py's SynthVae, seed 11) are written to a
temporary safetensors file with the shapes src/weights.lisp:69-98 gives; the
fixture keeps only the seed, the latents and the pictures (RGBA, 16H x 16W x 4,
channels last as src/cuda-vae.lisp:94-136 returns them).
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import exn_oracle as xo  # noqa: E402
from oracle import exn_vae_oracle as vo  # noqa: E402

SEED = 11
CASES = ((2, 2), (2, 3))


def write_safetensors(path, wt):
    header, blobs, off = {}, [], 0
    for name, shape in vo.vae_expected():
        b = xo.bf16_bits(wt(name).reshape(-1)).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    script = os.path.join(ref, "inspect", "ref_vae.py")
    wt = vo.SynthVae(SEED)
    arrays = {"seed": np.array([SEED], np.int64)}
    with tempfile.TemporaryDirectory() as tmp:
        st = os.path.join(tmp, "vae.safetensors")
        write_safetensors(st, wt)
        for ci, (h, w) in enumerate(CASES):
            z = vo.synth_latent(SEED + ci, h, w)
            lat, out = os.path.join(tmp, "z.f32"), os.path.join(tmp, "out.f32")
            z.astype(np.float32).tofile(lat)
            subprocess.run([sys.executable, "-I", script, st, lat, str(h), str(w), out], check=True)
            pic = np.fromfile(out, dtype=np.float32).reshape(4, 16 * h, 16 * w).transpose(1, 2, 0)
            arrays["latent_%d" % ci] = z.astype(np.float32)
            arrays["picture_%d" % ci] = np.ascontiguousarray(pic)
            print("case %d: %d x %d latent, picture rms %.4f, clipped %.3f" %
                  (ci, h, w, float(np.sqrt((pic * pic).mean())), float((np.abs(pic) >= 1).mean())), flush=True)
    np.savez_compressed(os.path.join(HERE, "ref_vae_tiny.npz"), **arrays)
    print("wrote ref_vae_tiny.npz")


if __name__ == "__main__":
    main()
