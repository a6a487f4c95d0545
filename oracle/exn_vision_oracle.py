"""exn_vision_oracle -- the CPU restatement of Qwen3-VL's vision tower as ex-nihilo
runs it for editing, float32 numpy.

TEST INFRASTRUCTURE ONLY.  Tests use this module for the expected values; the product path
(libexn-hip.so and the exn_hip host package) never imports it.

It restates:
  - inspect/ref_vision.py (all of its arithmetic): layernorm (:35-38), gelu_tanh
    (:41-42), gelu_erf (:45-47), merge_order (:50-60), interp_taps (:63-69), the
    patch embedding with the two frames' kernels summed (:80-84), the learned
    positions resampled bilinearly (:86-95), the 2-D rotary (:97-107), the merger
    (:109-118) and the 27 blocks with the deepstack mergers after blocks 8, 16
    and 24 (:120-144);
  - src/host.lisp:103-190 and src/cuda-vision.lisp:34-101: the picture handed
    over as RGBA rows (H x W x 4 floats, -1 .. 1), of which the patches read
    channels 0-2 (vision-patches); the outputs as M = N/4 rows of 4096 in
    merge-block order (merged, then the three deepstack sets).
The synthetic weights (matrices fp16-valued, as mmproj-f16.gguf ships them;
norms and biases fp32) and pictures come from the counter-based generator of
oracle/exn_oracle.py, tensor ids from VISION_ID0 on.

How it is pinned (tests/test_vision_oracle.py): encode against vectors that the
reference's own inspect/ref_vision.py wrote from the same synthetic weights at a
narrow width (tests/golden/ref_vision_tiny.npz, made by
tests/golden/make_ref_vision_vectors.py); merge order, taps and rotary against
closed forms.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from oracle import exn_oracle as xo
from oracle import exn_vae_oracle as vo

PATCH, MERGE = 16, 2          # inspect/ref_vision.py:20; src/host.lisp:112
THETA = 10000.0               # inspect/ref_vision.py:23
EPS = 1e-6                    # inspect/ref_vision.py:35; src/cuda-vision.lisp:70
VISION_ID0 = 6000             # the generator's tensor ids for the tower, past the DiT's and the VAE's
INPUT_VISION_PX = 6999


@dataclass(frozen=True)
class VShape:
    """The tower's dimensions (inspect/ref_vision.py:20-23; src/host.lisp:104-112).
    The tests narrow WIDTH, HEADS, FFN, DEPTH, OUT and the position table's SIDE
    for the golden vectors; the head dim stays 72 (WIDTH / HEADS)."""
    width: int = 1152
    heads: int = 16
    ffn: int = 4304
    depth: int = 27
    deepstack: tuple = (8, 16, 24)
    out: int = 4096
    side: int = 48

    @property
    def head_dim(self):
        return self.width // self.heads


def vision_expected(s: VShape = VShape()):
    """(name, shape) of every tensor the tower reads, as inspect/ref_vision.py
    names them (row-major shapes, a matrix (out, in))."""
    d, f, o = s.width, s.ffn, s.out
    r = [("v.patch_embd.weight", (d, 3, PATCH, PATCH)), ("v.patch_embd.weight.1", (d, 3, PATCH, PATCH)),
         ("v.patch_embd.bias", (d,)), ("v.position_embd.weight", (s.side * s.side, d))]
    for i in range(s.depth):
        p = "v.blk.%d." % i
        r += [(p + "ln1.weight", (d,)), (p + "ln1.bias", (d,)),
              (p + "attn_qkv.weight", (3 * d, d)), (p + "attn_qkv.bias", (3 * d,)),
              (p + "attn_out.weight", (d, d)), (p + "attn_out.bias", (d,)),
              (p + "ln2.weight", (d,)), (p + "ln2.bias", (d,)),
              (p + "ffn_up.weight", (f, d)), (p + "ffn_up.bias", (f,)),
              (p + "ffn_down.weight", (d, f)), (p + "ffn_down.bias", (d,))]
    for i in s.deepstack:
        p = "v.deepstack.%d." % i
        r += [(p + "norm.weight", (4 * d,)), (p + "norm.bias", (4 * d,)),
              (p + "fc1.weight", (4 * d, 4 * d)), (p + "fc1.bias", (4 * d,)),
              (p + "fc2.weight", (o, 4 * d)), (p + "fc2.bias", (o,))]
    r += [("v.post_ln.weight", (d,)), ("v.post_ln.bias", (d,)),
          ("mm.0.weight", (4 * d, 4 * d)), ("mm.0.bias", (4 * d,)),
          ("mm.2.weight", (o, 4 * d)), ("mm.2.bias", (o,))]
    return r


def synth_scale(name, shape):
    """(base, scale, fp16) of a synthetic tensor: value = base + scale * normal,
    rounded to fp16 when FP16.  Matrices (2-D and up) are fp16 at unit gain over
    their fan-in (the residual branches' outputs, attn_out and ffn_down, at half;
    QKV at 2, so that the scores spread to a standard deviation of about 4; the
    two patch kernels at 0.7 each, summing to about unit gain; the position table
    at 1); biases 0.02 z and norm weights 1 + 0.1 z, fp32."""
    if len(shape) == 1:     # a bias, or a LayerNorm's weight
        return (0.0, 0.02, False) if name.endswith(".bias") else (1.0, 0.1, False)
    if name.startswith("v.position_embd"):
        return 0.0, 1.0, True
    fan = int(np.prod(shape[1:]))
    g = 1.0
    if name.startswith("v.patch_embd"):
        g = 0.7
    elif name.endswith("attn_qkv.weight"):
        g = 2.0
    elif name.endswith("attn_out.weight") or name.endswith("ffn_down.weight"):
        g = 0.5
    return 0.0, g / math.sqrt(fan), True


class SynthVision:
    """wt(name) -> the tensor as float32 in its row-major shape."""

    def __init__(self, seed, s: VShape = VShape()):
        self.seed, self.s = seed, s
        self.shapes = dict(vision_expected(s))
        self.ids = {n: VISION_ID0 + i for i, (n, _) in enumerate(vision_expected(s))}
        self.cache = {}

    def __call__(self, name):
        if name not in self.cache:
            shape = self.shapes[name]
            base, scale, f16 = synth_scale(name, shape)
            z = vo.normal_fast(self.seed, self.ids[name], int(np.prod(shape)))
            v = np.float32(base) + np.float32(scale) * z
            if f16:
                v = v.astype(np.float16).astype(np.float32)
            self.cache[name] = v.reshape(shape)
        return self.cache[name]


def synth_picture(seed, h, w):
    """An RGBA picture (h, w, 4) in -1 .. 1: RGB = clip(0.5 z, -1, 1), alpha 1."""
    z = xo.normal(seed, INPUT_VISION_PX, h * w * 4).reshape(h, w, 4)
    px = np.clip(np.float32(0.5) * z, -1.0, 1.0).astype(np.float32)
    px[..., 3] = 1.0
    return px


# --- the pieces -----------------------------------------------------------------------

def layernorm(x, w, b, eps=EPS):
    """inspect/ref_vision.py:35-38."""
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * w + b


def gelu_tanh(x):
    """inspect/ref_vision.py:41-42."""
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def gelu_erf(x):
    """inspect/ref_vision.py:45-47: erf of the float32 x / sqrt 2 in double, the
    sum rounded to float32."""
    try:
        from scipy.special import erf
        e = erf((x / math.sqrt(2)).astype(np.float64))
    except ImportError:
        e = np.vectorize(math.erf)((x / math.sqrt(2)).astype(np.float64))
    return 0.5 * x * (1 + e).astype(np.float32)


def merge_order(gh, gw):
    """(rows, cols) of the patches in merge-block order: block row, block column,
    then the 2 x 2 inside (inspect/ref_vision.py:50-60; src/host.lisp:119-125)."""
    rows, cols = [], []
    for br in range(gh // MERGE):
        for bc in range(gw // MERGE):
            for ir in range(MERGE):
                for ic in range(MERGE):
                    rows.append(br * MERGE + ir)
                    cols.append(bc * MERGE + ic)
    return np.array(rows, dtype=np.int64), np.array(cols, dtype=np.int64)


def interp_taps(index, size, side):
    """Bilinear, corners aligned: 2 taps and weights an index (inspect/ref_vision.py:63-69)."""
    src = index.astype(np.float64) * (side - 1) / max(size - 1, 1)
    fl = np.floor(src)
    taps = np.stack([fl, fl + 1], 1).astype(np.int64)
    w = np.clip(1 - np.abs(src[:, None] - taps), 0, None)
    return np.clip(taps, 0, side - 1), w


def patches(px, rows, cols):
    """(n, 3 * 16 * 16): each patch's (channel, row, column) from the RGBA picture
    (inspect/ref_vision.py:82-83 on RGB; src/host.lisp:127-137 on RGBA)."""
    rgb = px[..., :3]
    return np.stack([rgb[r * PATCH:(r + 1) * PATCH, c * PATCH:(c + 1) * PATCH, :].transpose(2, 0, 1).reshape(-1)
                     for r, c in zip(rows, cols)]).astype(np.float32)


def pos_embed(table, rows, cols, gh, gw, side):
    """The position table resampled to the grid (inspect/ref_vision.py:86-95)."""
    d = table.shape[1]
    ht, hw_ = interp_taps(rows, gh, side)
    wt, ww = interp_taps(cols, gw, side)
    pe = np.zeros((len(rows), d), np.float32)
    for a in range(2):
        for b in range(2):
            pe += (hw_[:, a] * ww[:, b])[:, None].astype(np.float32) * table[ht[:, a] * side + wt[:, b]]
    return pe


def rotary(rows, cols, hd):
    """cos, sin (n, hd): hd/4 frequencies of the row, then of the column, the hd/2
    twice (inspect/ref_vision.py:97-101)."""
    inv = 1.0 / (THETA ** (np.arange(0, hd // 2, 2, dtype=np.float32) / (hd // 2)))
    f = np.concatenate([rows[:, None] * inv, cols[:, None] * inv], 1)
    f = np.concatenate([f, f], 1).astype(np.float32)
    return np.cos(f), np.sin(f)


def rope(t, cos, sin):
    """t: (n, heads, hd) turned by rotate_half (inspect/ref_vision.py:103-106)."""
    half = t.shape[-1] // 2
    rot = np.concatenate([-t[..., half:], t[..., :half]], -1)
    return t * cos[:, None, :] + rot * sin[:, None, :]


def merger(x, wt, s, prefix=None):
    """Four patches' rows to one row of OUT: LayerNorm after the reshape
    (deepstack, PREFIX) or before it (v.post_ln), fc1, GELU (erf), fc2
    (inspect/ref_vision.py:109-118)."""
    d = s.width
    if prefix is not None:
        y = layernorm(x.reshape(-1, 4 * d), wt(prefix + ".norm.weight"), wt(prefix + ".norm.bias"))
        fc1, b1, fc2, b2 = prefix + ".fc1.weight", prefix + ".fc1.bias", prefix + ".fc2.weight", prefix + ".fc2.bias"
    else:
        y = layernorm(x, wt("v.post_ln.weight"), wt("v.post_ln.bias")).reshape(-1, 4 * d)
        fc1, b1, fc2, b2 = "mm.0.weight", "mm.0.bias", "mm.2.weight", "mm.2.bias"
    y = gelu_erf(y @ wt(fc1).T + wt(b1))
    return (y @ wt(fc2).T + wt(b2)).astype(np.float32)


def attention(q, k, v):
    """Softmax attention of every patch over every patch, head by head
    (inspect/ref_vision.py:124-129)."""
    n, heads, hd = q.shape
    att = np.empty((n, heads, hd), np.float32)
    for hh in range(heads):
        sc = (q[:, hh] @ k[:, hh].T) / math.sqrt(hd)
        sc = np.exp(sc - sc.max(-1, keepdims=True))
        sc /= sc.sum(-1, keepdims=True)
        att[:, hh] = sc @ v[:, hh]
    return att


def encode(px, wt, s: VShape = VShape()):
    """The tower on the RGBA picture PX (H x W x 4, H and W multiples of 32):
    dict(embed (N x width), blk0 (after block 0), merged (N/4 x OUT), ds (three
    N/4 x OUT)) -- inspect/ref_vision.py:72-148, src/cuda-vision.lisp:34-101."""
    h, w = px.shape[:2]
    assert h % (PATCH * MERGE) == 0 and w % (PATCH * MERGE) == 0
    d, heads, hd = s.width, s.heads, s.head_dim
    gh, gw = h // PATCH, w // PATCH
    rows, cols = merge_order(gh, gw)
    n = gh * gw
    pw = wt("v.patch_embd.weight") + wt("v.patch_embd.weight.1")
    x = patches(px, rows, cols) @ pw.reshape(d, -1).T + wt("v.patch_embd.bias")
    table = wt("v.position_embd.weight").reshape(-1, d)
    side = int(round(math.sqrt(table.shape[0])))
    x = (x + pos_embed(table, rows, cols, gh, gw, side)).astype(np.float32)
    out = {"embed": x.copy()}
    cos, sin = rotary(rows, cols, hd)
    ds = []
    for i in range(s.depth):
        p = "v.blk.%d." % i
        hn = layernorm(x, wt(p + "ln1.weight"), wt(p + "ln1.bias"))
        qkv = (hn @ wt(p + "attn_qkv.weight").T + wt(p + "attn_qkv.bias")).reshape(n, 3, heads, hd)
        q, k, v = rope(qkv[:, 0], cos, sin), rope(qkv[:, 1], cos, sin), qkv[:, 2]
        att = attention(q, k, v)
        x = x + att.reshape(n, d) @ wt(p + "attn_out.weight").T + wt(p + "attn_out.bias")
        hn = layernorm(x, wt(p + "ln2.weight"), wt(p + "ln2.bias"))
        x = (x + gelu_tanh(hn @ wt(p + "ffn_up.weight").T + wt(p + "ffn_up.bias")) @ wt(p + "ffn_down.weight").T
             + wt(p + "ffn_down.bias")).astype(np.float32)
        if i == 0:
            out["blk0"] = x.copy()
        if i in s.deepstack:
            ds.append(merger(x, wt, s, "v.deepstack.%d" % i))
    out["merged"] = merger(x, wt, s)
    out["ds"] = ds
    return out


def encode_flops(n, s: VShape = VShape()):
    """Multiply-add FLOPs of one picture of N patches: the products (patch
    embedding, the blocks' four, the four mergers' two each) and attention's two."""
    d, f, o, m = s.width, s.ffn, s.out, n // 4
    blocks = s.depth * (2 * n * d * (3 * d + d + 2 * f) + 4 * n * n * d)
    mergers = (len(s.deepstack) + 1) * 2 * m * (4 * d * 4 * d + 4 * d * o)
    return 2 * n * d * 3 * PATCH * PATCH + blocks + mergers
