"""exn_vae_oracle -- the CPU restatement of ex-nihilo's VAE decoder and encoder, float32 numpy.

TEST INFRASTRUCTURE ONLY.  Tests and the benchmark's checks use this module as
the expected values; the product path (libexn-hip.so and the exn_hip host package)
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
    last), the reference script writing it channel-major;
  - the encoder, src/cuda-vae.lisp:138-190 with src/weights.lisp:100-134 (its
    stages, names and shapes) and src/cuda/vae.cu's x_conv3s2 and
    x_avgdown_add (the stride-2 convolution, zero-padded below and to the
    right; AvgDown3D on one frame, padded in front with zero frames): conv1 on
    RGBA, per stage two residual blocks then the stride-2 convolution plus
    AvgDown3D of the stage's input (or the input added), the middle, the head
    (norm, SiLU, 3 x 3 to the mean and log-variance, conv1), the mean kept.
Activations here are channels last (H, W, C), the layout the GPU decoder uses;
inspect/ref_vae.py keeps them channel-major, which changes no arithmetic.

The synthetic weights (bf16, as the real file ships them) come from the same
counter-based generator as the DiT's (oracle/exn_oracle.py), tensor ids from
VAE_ID0 on.

How it is pinned (tests/test_vae_oracle.py): decode against vectors that the
reference's own inspect/ref_vae.py wrote from the same synthetic weights
(tests/golden/ref_vae_tiny.npz, made by tests/golden/make_ref_vae_vectors.py);
the pieces against float64 brute force and closed forms.  The encoder shares
conv, rms, silu, resblock and attention with the decoder (pinned there); its own
pieces are pinned by brute force (the stride-2 convolution) and by the index
formula of x_avgdown_add against the view-and-mean form here; its stage wiring
by a closed form on weights that make every block an identity.  Parity
unpinned: the encoder's composition as a whole has no reference vectors (the
reference's inspect/ref_vae.py holds the decoder only, and diffusers is not
installed), so beyond those checks it rests on reading src/cuda-vae.lisp and
src/metal-vae.lisp.
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


# the encoder: (in, out, spatial down, temporal down), the picture's end first
# (src/weights.lisp:100-102)
ENC_STAGES = ((96, 96, True, False), (96, 192, True, True), (192, 384, True, True),
              (384, 768, True, True), (768, 768, False, False))
IN = 4          # RGBA


def vae_encoder_expected(enc_stages=ENC_STAGES, z=Z, inp=IN):
    """(name, shape) of every tensor the encoder reads, in src/weights.lisp:104-134's
    order (the video-only time_conv tensors left out)."""
    top = enc_stages[-1][1]
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

    conv("encoder.conv1", enc_stages[0][0], inp, 3)
    for s, (i, o, down, _td) in enumerate(enc_stages):
        for j in range(2):
            res("encoder.downsamples.%d.downsamples.%d" % (s, j), i if j == 0 else o, o)
        if down:
            conv("encoder.downsamples.%d.downsamples.2.resample.1" % s, o, o, 3, frames=False)
    res("encoder.middle.0", top, top)
    r.append(("encoder.middle.1.norm.gamma", (top, 1, 1)))
    conv("encoder.middle.1.to_qkv", 3 * top, top, 1, frames=False)
    conv("encoder.middle.1.proj", top, top, 1, frames=False)
    res("encoder.middle.2", top, top)
    r.append(("encoder.head.0.gamma", (top, 1, 1, 1)))
    conv("encoder.head.2", 2 * z, top, 3)
    conv("conv1", 2 * z, 2 * z, 1)
    return r


def vae_tensor_id(name, stages=STAGES, enc_stages=ENC_STAGES):
    """The generator's id of a tensor: VAE_ID0 + its index in the decoder's list, then the
    encoder's."""
    names = [n for n, _ in vae_expected(stages)] + [n for n, _ in vae_encoder_expected(enc_stages)]
    return VAE_ID0 + names.index(name)


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
    g = 0.5 if (".residual.6." in name or name.startswith("decoder.middle.1.proj")
                or name.startswith("encoder.middle.1.proj")) else 1.0
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

    def __init__(self, seed, stages=STAGES, enc_stages=ENC_STAGES):
        self.seed, self.stages, self.enc_stages = seed, stages, enc_stages
        self.shapes = dict(vae_expected(stages) + vae_encoder_expected(enc_stages))
        self.cache = {}

    def __call__(self, name):
        if name not in self.cache:
            shape = self.shapes[name]
            base, scale = synth_scale(name, shape)
            z = normal_fast(self.seed, vae_tensor_id(name, self.stages, self.enc_stages), int(np.prod(shape)))
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


# --- the encoder (src/cuda-vae.lisp:138-190), channels last --------------------------

def conv3s2(x, w, b):
    """x: (2H, 2W, C) -> (H, W, O): the 3 x 3 convolution at stride 2, the input padded with one
    row of zeros below and one column to the right (src/cuda/vae.cu's x_conv3s2: output pixel
    (y, x) takes input rows 2y .. 2y + 2 and columns 2x .. 2x + 2); + b."""
    o, c = w.shape[0], w.shape[1]
    w = w.reshape(o, c, 3, 3)
    h2, w2, _ = x.shape
    h, wd = h2 // 2, w2 // 2
    xp = np.pad(x, ((0, 1), (0, 1), (0, 0)))
    out = np.zeros((h * wd, o), dtype=np.float32)
    for dy in range(3):
        for dx in range(3):
            out += xp[dy:dy + 2 * h:2, dx:dx + 2 * wd:2].reshape(-1, c) @ w[:, :, dy, dx].T
    return out.reshape(h, wd, o) + b


def avgdown(x, out_c, ft, fs=2):
    """AvgDown3D on one frame, padded in front to FT frames with zeros: the (C, FT, fs, fs) view
    of each fs x fs block (channel, frame, row, column: frames 0 .. ft-2 zero, the last the
    block) flattened, cut into OUT_C groups of g = C ft fs^2 / OUT_C, each group's mean -- the
    view-and-mean form of AvgDown3D."""
    h, w, c = x.shape
    g = c * ft * fs * fs // out_c
    blocks = x.reshape(h // fs, fs, w // fs, fs, c).transpose(0, 2, 4, 1, 3)   # H', W', C, fs, fs
    full = np.zeros((h // fs, w // fs, c, ft, fs, fs), np.float32)
    full[:, :, :, ft - 1] = blocks
    return full.reshape(h // fs, w // fs, out_c, g).mean(-1, dtype=np.float64).astype(np.float32)


def encode(wt, px, enc_stages=ENC_STAGES, z=Z, on_stage=None):
    """px: (H, W, 4) RGBA in -1..1 (H, W multiples of 16) -> the latent's mean, (64, H/16, W/16)
    float32 channel-major, denormalized (src/cuda-vae.lisp:138-190)."""
    x = conv(np.asarray(px, np.float32), wt("encoder.conv1.weight"), wt("encoder.conv1.bias"), 3)
    for s, (i, o, down, tdown) in enumerate(enc_stages):
        keep = x
        for j in range(2):
            x = resblock(wt, "encoder.downsamples.%d.downsamples.%d" % (s, j), x)
        if down:
            p = "encoder.downsamples.%d.downsamples.2.resample.1" % s
            x = conv3s2(x, wt(p + ".weight"), wt(p + ".bias")) + avgdown(keep, o, 2 if tdown else 1)
        else:
            x = x + keep
        if on_stage:
            on_stage(s, x)
    x = resblock(wt, "encoder.middle.0", x)
    x = attention(wt, "encoder.middle.1", x)
    x = resblock(wt, "encoder.middle.2", x)
    x = silu(rms(x, wt("encoder.head.0.gamma")))
    x = conv(x, wt("encoder.head.2.weight"), wt("encoder.head.2.bias"), 3)
    x = conv(x, wt("conv1.weight"), wt("conv1.bias"), 1)
    return np.ascontiguousarray(x[..., :z].transpose(2, 0, 1)).astype(np.float32)


INPUT_VAE_PICTURE = 4998


def synth_picture(seed, h, w):
    """An encoder input: h x w RGBA, each value 0.5 z clipped to -1 .. 1."""
    return np.clip(np.float32(0.5) * xo.normal(seed, INPUT_VAE_PICTURE, h * w * 4), -1, 1).reshape(h, w, 4)


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


def encode_flops(h, w, enc_stages=ENC_STAGES, z=Z, inp=IN):
    """Algorithmic FLOPs of one encode of an h x w picture: every convolution's
    2 * pixels * cin * cout * taps (the first at its 4 input channels), the attention's two
    products."""
    def res(n, i, o):
        return 2 * n * (i * o * 9 + o * o * 9 + (i * o if i != o else 0))

    f = 2 * h * w * inp * enc_stages[0][0] * 9
    hh, ww = h, w
    for i, o, down, _ in enc_stages:
        n = hh * ww
        f += res(n, i, o) + res(n, o, o)
        if down:
            hh, ww = hh // 2, ww // 2
            f += 2 * hh * ww * o * o * 9
    n, top = hh * ww, enc_stages[-1][1]
    f += 2 * res(n, top, top)
    f += 2 * n * top * 3 * top + 2 * 2 * n * n * top + 2 * n * top * top
    f += 2 * n * top * 2 * z * 9 + 2 * n * 2 * z * 2 * z
    return f
