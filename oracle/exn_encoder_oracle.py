"""exn_encoder_oracle -- the CPU restatement of the prompt encoder as ex-nihilo reads it:
Qwen3-VL-8B's text model, every token's state after its last block before the final
norm, float32 numpy.

TEST INFRASTRUCTURE ONLY.  Tests use this module for the expected values; the product path
(libexn-hip.so and the exn_hip host package) never imports it.

The reference runs this model through illatio (il::load-model, il::cuda-forward-n,
il::forward-batch: src/encoder.lisp:41-48,143-183), a dependency the reference tree
does not vendor and pins to no version (ex-nihilo.asd:9 names "illatio" only;
github.com/modus-lisp/illatio).  So the forward here restates the published model,
transformers' Qwen3-VL text model, with the shape docs/design.md:42-50 gives: 36
layers of 4096, 32 query heads and 8 key/value heads of 128 (query head h reads
key/value head h // 4), FFN 12288 (SwiGLU), RMSNorm eps 1e-6 before attention and
before the MLP and over each head of q and k, RoPE theta 5e6 by rotate_half (dims i
and i + 64 turn together), causal attention; and the reference's own parts around it:
  - src/encoder.lisp:26-39 (mrope-table): frequency j < 64 turns by the token's h
    position where j mod 3 = 1, by its w position where j mod 3 = 2, below 60; by its
    t position elsewhere;
  - src/encoder.lisp:69-110 (call-with-picture-rows): the picture's rows replace the
    image pads' embeddings; deepstack set j is added to them after layer j;
  - src/encoder.lisp:112-141 (encode-edit-prompt): the positions of an edit prompt --
    (i, i, i) before the picture, (a0, a0 + r, a0 + c) on it, then (p0 + i) x 3 from
    p0 = a0 + max(gh, gw);
  - src/encoder.lisp:143-183 (encoder-states): the states after the last block, before
    the final norm.
Against illatio's own arithmetic (its quantisation and order of operations) this is
parity unpinned.  tests/test_encoder_oracle.py pins the model it computes: against
transformers' Qwen3VLTextModel (transformers 5.15.0, installed here; the published
implementation this restates) with the same weights, on an edit prompt's (t, h, w)
positions with picture rows and deepstack sets, within float32 rounding; and by the
mathematics: the M-RoPE table on text positions against 1-D RoPE, causality (a prefix's
states do not change when tokens follow), grouped heads against the same model with every
key/value head repeated, rotate_half as a rotation, RMSNorm's closed form.  The synthetic weights (Q8_0 matrices, fp32 norms) come from the counter
generator of oracle/exn_oracle.py, tensor ids from ENC_ID0 on.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from oracle import exn_oracle as xo

EPS = 1e-6
ROPE_BASE = 5e6
ENC_ID0 = 8000
INPUT_IDS, INPUT_PICTURE = 8998, 8999


@dataclass(frozen=True)
class EShape:
    """docs/design.md:42-45.  LAYERS is the loop bound the tests shorten; VOCAB is the
    synthetic model's (the real one has 151936 rows)."""
    width: int = 4096
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 8192


LAYER_SLOTS = ("attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
               "attn_q_norm.weight", "attn_k_norm.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight",
               "ffn_down.weight")


def enc_expected(s: EShape = EShape()):
    """(name, (rows, cols) or (n,)) of every tensor the encoder reads: llama.cpp's qwen3vl
    names in te-q8_0.gguf, a matrix (out, in)."""
    d, kv, f = s.width, s.kv_heads * s.head_dim, s.ffn
    shapes = {"attn_norm.weight": (d,), "attn_q.weight": (d, d), "attn_k.weight": (kv, d), "attn_v.weight": (kv, d),
              "attn_output.weight": (d, d), "attn_q_norm.weight": (s.head_dim,), "attn_k_norm.weight": (s.head_dim,),
              "ffn_norm.weight": (d,), "ffn_gate.weight": (f, d), "ffn_up.weight": (f, d), "ffn_down.weight": (d, f)}
    r = [("token_embd.weight", (s.vocab, d))]
    for i in range(s.layers):
        r += [("blk.%d.%s" % (i, slot), shapes[slot]) for slot in LAYER_SLOTS]
    return r


class SynthEncoder:
    """wt(name) -> fp32: matrices Q8_0 from the counter generator, dequantised exactly;
    norm weights 1 + 0.05 z.  Tensor id: ENC_ID0 + its index in enc_expected for 36 layers."""

    def __init__(self, seed, s: EShape = EShape(), keep=True):
        self.seed, self.s, self.keep = seed, s, keep
        full = EShape(s.width, 36, s.heads, s.kv_heads, s.head_dim, s.ffn, s.vocab)
        self.ids = {n: ENC_ID0 + i for i, (n, _) in enumerate(enc_expected(full))}
        self.shapes = dict(enc_expected(s))
        self.cache = {}

    def q8(self, name):
        rows, cols = self.shapes[name]
        return xo.q8_0_synth_fast(self.seed, self.ids[name], rows, cols)

    def __call__(self, name):
        if name not in self.cache:
            shape = self.shapes[name]
            if len(shape) == 1:
                v = np.float32(1.0) + np.float32(0.05) * xo.normal(self.seed, self.ids[name], shape[0])
            else:
                v = xo.dequant_fast(*self.q8(name))
            if not self.keep and len(shape) > 1 and name != "token_embd.weight":
                return v          # full depth: a layer's matrices made again when read
            self.cache[name] = v
        return self.cache[name]


def synth_ids(seed, n, vocab):
    """N token ids below VOCAB from the generator."""
    z = xo.words(xo.key(seed, INPUT_IDS), np.arange(n, dtype=np.uint64))
    return (z % np.uint64(vocab)).astype(np.int32)


def synth_picture_rows(seed, m, width=4096):
    """The vision tower's outputs for an M-row picture: merged (m, width) and three
    deepstack sets (3, m, width), ~ N(0, 1)."""
    z = xo.normal(seed, INPUT_PICTURE, 4 * m * width).reshape(4, m, width)
    return z[0], z[1:]


# --- positions and M-RoPE ----------------------------------------------------------------

def text_positions(n, start=0):
    p = np.arange(start, start + n, dtype=np.int64)
    return np.stack([p, p, p], 1)


def edit_positions(a0, gh, gw, after):
    """src/encoder.lisp:125-129: A0 text tokens, the picture's gh x gw rows, AFTER tokens."""
    before = text_positions(a0)
    r, c = np.divmod(np.arange(gh * gw), gw)
    pic = np.stack([np.full(gh * gw, a0), a0 + r, a0 + c], 1)
    return np.concatenate([before, pic, text_positions(after, a0 + max(gh, gw))]).astype(np.int64)


def mrope_tables(pos3, base=ROPE_BASE, hd=128):
    """cos, sin (n, hd/2) of each token's angles (src/encoder.lisp:26-39): frequency j at
    base^(-2j/hd), turned by axis (j mod 3) of the token's (t, h, w) below 60, by t above."""
    half = hd // 2
    j = np.arange(half)
    axis = np.where(j < 60, j % 3, 0)
    inv = base ** (-(2.0 * j) / hd)
    ang = pos3[:, axis].astype(np.float64) * inv
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_half(x, cos, sin):
    """x (n, heads, hd) turned by rotate_half: dims i and i + hd/2 by angle i."""
    half = x.shape[-1] // 2
    c = np.concatenate([cos, cos], -1)[:, None, :]
    s = np.concatenate([sin, sin], -1)[:, None, :]
    rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
    return x * c + rot * s


def rmsnorm(x, w, eps=EPS):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def silu(x):
    return x / (1 + np.exp(-x))


# --- the forward ----------------------------------------------------------------------------

def _keep(x):
    return x


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def layer(wt, i, x, cos, sin, s: EShape = EShape(), bf16=False):
    """Block i of the text model on rows x (n, width): causal grouped-query attention, SwiGLU.
    BF16: round where the GPU's products and attention round (matrices and the products'
    inputs to bf16, q, k, v to fp16) -- a model of that arithmetic, to tell its rounding from
    a mistake; the restatement of the model is BF16 false."""
    rb, rh = (xo.bf16_round, _f16) if bf16 else (_keep, _keep)
    w = lambda name: rb(wt(name))
    p = "blk.%d." % i
    n = x.shape[0]
    h = rb(rmsnorm(x, wt(p + "attn_norm.weight")))
    q = (h @ w(p + "attn_q.weight").T).reshape(n, s.heads, s.head_dim)
    k = (h @ w(p + "attn_k.weight").T).reshape(n, s.kv_heads, s.head_dim)
    v = (h @ w(p + "attn_v.weight").T).reshape(n, s.kv_heads, s.head_dim)
    q = rh(rope_half(rmsnorm(q, wt(p + "attn_q_norm.weight")), cos, sin))
    k = rh(rope_half(rmsnorm(k, wt(p + "attn_k_norm.weight")), cos, sin))
    v = rh(v)
    g = s.heads // s.kv_heads
    k, v = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)          # query head h reads kv head h // g
    att = rb(xo.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), 0, n))
    x = x + att.reshape(n, s.width) @ w(p + "attn_output.weight").T
    h = rb(rmsnorm(x, wt(p + "ffn_norm.weight")))
    ff = rb(silu(h @ w(p + "ffn_gate.weight").T) * (h @ w(p + "ffn_up.weight").T))
    return (x + ff @ w(p + "ffn_down.weight").T).astype(np.float32)


def states(wt, ids, pos3=None, picture=None, s: EShape = EShape(), base=ROPE_BASE, bf16=False):
    """encoder-states (src/encoder.lisp:143-183): every token's state after the last block,
    before the final norm, (n, width).  POS3: (n, 3) positions, text positions 0.. when
    None.  PICTURE: (a0, merged (m, width), deep (3, m, width)) -- rows a0 .. a0 + m - 1
    take merged's rows after the embedding and deep[j] added after layer j
    (call-with-picture-rows, :69-110)."""
    n = len(ids)
    x = wt("token_embd.weight")[np.asarray(ids)].astype(np.float32)
    if picture is not None:
        a0, merged, deep = picture
        x[a0:a0 + len(merged)] = merged
    cos, sin = mrope_tables(text_positions(n) if pos3 is None else pos3, base, s.head_dim)
    for i in range(s.layers):
        x = layer(wt, i, x, cos, sin, s, bf16)
        if picture is not None and i < len(deep):
            x[a0:a0 + len(merged)] += deep[i]
    return x
