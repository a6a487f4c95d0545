"""exn_vae_oracle -- the CPU restatement of ex-nihilo's VAE decoder, float32 numpy.

TEST INFRASTRUCTURE ONLY.  Tests and the benchmark's checks use this module as
the checker; the product path (libexn-hip.so and the exn_hip host package)
never imports it.

It restates:
  - inspect/ref_vae.py (all of the decoder): conv (3 x 3 'same' and 1 x 1, with
    bias), rms (the channel RMS norm, eps 1e-12, times sqrt(C) and gamma), silu,
    resblock, attention (one head over every pixel), dupup (DupUp3D, frame
    ft - 1), decode (conv2, decoder.conv1, the middle, the five stages, the head,
    the clamp);
  - src/weights.lisp:65-98: the stages and the decoder's tensor names and
    shapes (vae-expected);
  - src/cuda-vae.lisp:94-136: the output as 16H x 16W rows of RGBA (channels
    last), the reference script writing it channel-major.
Activations here are channels last (H, W, C), the layout the GPU decoder uses;
inspect/ref_vae.py keeps them channel-major, which changes no arithmetic.

The synthetic weights (bf16, as the real file ships them) come from the same
counter-based generator as the DiT's (oracle/exn_oracle.py), tensor ids from
VAE_ID0 on.

How it is pinned (tests/test_vae_oracle.py): decode against vectors that the
reference's own inspect/ref_vae.py wrote from the same synthetic weights
(tests/golden/ref_vae_tiny.npz, made by tests/golden/make_ref_vae_vectors.py);
the pieces against float64 brute force and closed forms.
"""
from __future__ import annotations

import numpy as np

from oracle import exn_oracle as xo

# (in, out, spatial up, temporal up), deepest first: src/weights.lisp:65-67, inspect/ref_vae.py:15-16
STAGES = ((1152, 1152, True, True), (1152, 1152, True, True), (1152, 576, True, True),
          (576, 288, True, False), (288, 144, False, False))
Z = 64          # latent channels
OUT = 4         # RGBA
RMS_EPS = 1e-12
VAE_ID0 = 4000  # the generator's tensor ids for the decoder, past the DiT's and its inputs'
INPUT_VAE_LATENT = 4999


def vae_expected(stages=STAGES, z=Z, out=OUT):
    """(name, shape) of every tensor the decoder reads, in src/weights.lisp:69-98's
    order (the video-only time_conv tensors, unused on one frame, left out)."""
    top = stages[0][0]
    r = []

    def conv(name, o, i, k, frames=True):
        r.append((name + ".weight", (o, i, 1, k, k) if frames else (o, i, k, k)))
        r.append((name + ".bias", (o,)))

    def res(p, i, o):
        r.append((p + ".residual.0.gamma", (i, 1, 1, 1)))
        conv(p + ".residual.2", o, i, 3)
        r.append((p + ".residual.3.gamma", (o, 1, 1, 1)))
        conv(p + ".residual.6", o, o, 3)
        if i != o:
            conv(p + ".shortcut", o, i, 1)

    conv("conv2", z, z, 1)
    conv("decoder.conv1", top, z, 3)
    res("decoder.middle.0", top, top)
    r.append(("decoder.middle.1.norm.gamma", (top, 1, 1)))
    conv("decoder.middle.1.to_qkv", 3 * top, top, 1, frames=False)
    conv("decoder.middle.1.proj", top, top, 1, frames=False)
    res("decoder.middle.2", top, top)
    for s, (i, o, up, _tup) in enumerate(stages):
        for j in range(3):
            res("decoder.upsamples.%d.upsamples.%d" % (s, j), i if j == 0 else o, o)
        if up:
            conv("decoder.upsamples.%d.upsamples.3.resample.1" % s, o, o, 3, frames=False)
    r.append(("decoder.head.0.gamma", (stages[-1][1], 1, 1, 1)))
    conv("decoder.head.2", out, stages[-1][1], 3)
    return r


def vae_tensor_id(name, stages=STAGES):
    return VAE_ID0 + [n for n, _ in vae_expected(stages)].index(name)


def synth_scale(name, shape):
    """(base, scale) of a synthetic tensor: value = bf16(base + scale * normal).
    Convolutions at unit gain over their fan-in (the second of a residual
    block and the attention's projection at half, so the residual stream grows
    slowly; the head at 1.2, so that the clamp bites about a tenth of the
    values); biases 0.02 z; norm gammas 1 + 0.1 z."""
    if name.endswith(".gamma"):
        return 1.0, 0.1
    if name.endswith(".bias"):
        return 0.0, 0.02
    fan = int(np.prod(shape[1:]))
    g = 0.5 if (".residual.6." in name or name.startswith("decoder.middle.1.proj")) else 1.0
    if name.startswith("decoder.head.2"):
        g = 1.2
    return 0.0, g / np.sqrt(fan)


def normal_fast(seed, tensor, n):
    """xo.normal through the C twin when it is built (identical output)."""
    lib = xo.clib()
    if lib is None:
        return xo.normal(seed, tensor, n)
    out = np.empty(n, dtype=np.float32)
    lib.exo_normal(seed, tensor, n, xo._ptr(out))
    return out


class SynthVae:
    """wt(name) -> the tensor as float32 in the file's shape, each value a bf16."""

    def __init__(self, seed, stages=STAGES):
        self.seed, self.stages = seed, stages
        self.shapes = dict(vae_expected(stages))
        self.cache = {}

    def __call__(self, name):
        if name not in self.cache:
            shape = self.shapes[name]
            base, scale = synth_scale(name, shape)
            z = normal_fast(self.seed, vae_tensor_id(name, self.stages), int(np.prod(shape)))
            self.cache[name] = xo.bf16_round(np.float32(base) + np.float32(scale) * z).reshape(shape)
        return self.cache[name]


def synth_latent(seed, h, w):
    """The decoder's input, 64 x h x w ~ N(0, 1) (already denormalized)."""
    return xo.normal(seed, INPUT_VAE_LATENT, Z * h * w).reshape(Z, h, w)


# --- the pieces (inspect/ref_vae.py:36-99), channels last ------------------------

def conv(x, w, b, k):
    """x: (H, W, C); w: (O, C, [1,] k, k); 'same' zero padding, stride 1; + b.
    inspect/ref_vae.py:36-47."""
    o, c = w.shape[0], w.shape[1]
    w = w.reshape(o, c, k, k)
    h, wd, _ = x.shape
    if k == 1:
        return (x.reshape(-1, c) @ w[:, :, 0, 0].T).reshape(h, wd, o) + b
    xp = np.pad(x, ((1, 1), (1, 1), (0, 0)))
    out = np.zeros((h * wd, o), dtype=np.float32)
    for dy in range(3):
        for dx in range(3):
            out += xp[dy:dy + h, dx:dx + wd].reshape(-1, c) @ w[:, :, dy, dx].T
    return out.reshape(h, wd, o) + b


def rms(x, gamma):
    """x / max(||x||, 1e-12) * sqrt(C) * gamma over each pixel's channels:
    inspect/ref_vae.py:50-52."""
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    return x / np.maximum(n, np.float32(RMS_EPS)) * np.float32(np.sqrt(x.shape[-1])) * gamma.reshape(-1)


def silu(x):
    return x / (1 + np.exp(-x))


def resblock(wt, p, x):
    """inspect/ref_vae.py:59-65."""
    i = x.shape[-1]
    o = wt(p + ".residual.2.weight").shape[0]
    h = conv(x, wt(p + ".shortcut.weight"), wt(p + ".shortcut.bias"), 1) if i != o else x
    y = conv(silu(rms(x, wt(p + ".residual.0.gamma"))), wt(p + ".residual.2.weight"), wt(p + ".residual.2.bias"), 3)
    y = conv(silu(rms(y, wt(p + ".residual.3.gamma"))), wt(p + ".residual.6.weight"), wt(p + ".residual.6.bias"), 3)
    return y + h


def attention(wt, p, x):
    """One head over every pixel, c wide: inspect/ref_vae.py:68-76."""
    h, w, c = x.shape
    y = rms(x, wt(p + ".norm.gamma"))
    qkv = conv(y, wt(p + ".to_qkv.weight"), wt(p + ".to_qkv.bias"), 1).reshape(h * w, 3 * c)
    q, k, v = qkv[:, :c], qkv[:, c:2 * c], qkv[:, 2 * c:]
    s = q @ k.T / np.float32(np.sqrt(c))
    s = np.exp(s - s.max(-1, keepdims=True))
    a = (s / s.sum(-1, keepdims=True)) @ v
    return conv(a.reshape(h, w, c), wt(p + ".proj.weight"), wt(p + ".proj.bias"), 1) + x


def dupup(x, out_c, ft, fs=2):
    """DupUp3D on the first frame: output channel c of pixel (2y + a, 2x + b) is
    input channel j // rep of pixel (y, x), j = ((c ft + ft - 1) 2 + a) 2 + b,
    rep = out_c ft fs^2 / C.  inspect/ref_vae.py:79-85."""
    h, w, c = x.shape
    rep = out_c * ft * fs * fs // c
    xr = np.repeat(x, rep, axis=-1).reshape(h, w, out_c, ft, fs, fs)[:, :, :, ft - 1]   # h, w, out_c, fs, fs
    return xr.transpose(0, 3, 1, 4, 2).reshape(h * fs, w * fs, out_c)


def up2(x):
    return np.repeat(np.repeat(x, 2, axis=0), 2, axis=1)


def decode(wt, z, stages=STAGES, on_stage=None):
    """z: (64, h, w) float32, denormalized -> (16h, 16w, 4) RGBA in -1..1, channels
    last (src/cuda-vae.lisp:94-136).  inspect/ref_vae.py:88-105."""
    x = np.ascontiguousarray(np.asarray(z, np.float32).transpose(1, 2, 0))
    x = conv(x, wt("conv2.weight"), wt("conv2.bias"), 1)
    x = conv(x, wt("decoder.conv1.weight"), wt("decoder.conv1.bias"), 3)
    x = resblock(wt, "decoder.middle.0", x)
    x = attention(wt, "decoder.middle.1", x)
    x = resblock(wt, "decoder.middle.2", x)
    for s, (i, o, up, tup) in enumerate(stages):
        x0 = x
        for j in range(3):
            x = resblock(wt, "decoder.upsamples.%d.upsamples.%d" % (s, j), x)
        if up:
            p = "decoder.upsamples.%d.upsamples.3.resample.1" % s
            x = conv(up2(x), wt(p + ".weight"), wt(p + ".bias"), 3)
            x = x + dupup(x0, o, 2 if tup else 1)
        if on_stage:
            on_stage(s, x)
    x = silu(rms(x, wt("decoder.head.0.gamma")))
    x = conv(x, wt("decoder.head.2.weight"), wt("decoder.head.2.bias"), 3)
    return np.clip(x, -1, 1).astype(np.float32)


# --- work counts -----------------------------------------------------------------

def decode_flops(h, w, stages=STAGES, z=Z, out=OUT):
    """Algorithmic FLOPs of one decode of an h x w latent: every convolution's
    2 * pixels * cin * cout * taps, and the attention's two products."""
    f = 0
    n = h * w
    top = stages[0][0]
    f += 2 * n * z * z + 2 * n * z * top * 9

    def res(n, i, o):
        return 2 * n * (i * o * 9 + o * o * 9 + (i * o if i != o else 0))

    f += 2 * res(n, top, top)
    f += 2 * n * top * 3 * top + 2 * 2 * n * n * top + 2 * n * top * top
    hh, ww = h, w
    for i, o, up, _ in stages:
        n = hh * ww
        f += res(n, i, o) + 2 * res(n, o, o)
        if up:
            hh, ww = 2 * hh, 2 * ww
            f += 2 * hh * ww * o * o * 9
    f += 2 * hh * ww * stages[-1][1] * out * 9
    return f
