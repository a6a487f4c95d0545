"""exn_oracle -- the CPU restatement of ex-nihilo's DiT step, float32 numpy.

TEST INFRASTRUCTURE ONLY.  Tests, the smoke check and the CPU-baseline leg of
the benchmark use this module for the expected values; the product path (libexn-hip.so
and the exn_hip host package) never imports it.

It restates, function by function (citations are into the reference tree):
  - inspect/ref_dit.py (all of it): linear, layernorm, rmsnorm, gelu_tanh,
    silu, timestep_embedding, positions, rope_tables, rope, attention, forward;
  - src/host.lisp:9-50: dit-positions with a reference picture (edit mode);
  - src/cuda/dit.cu:60-66: the xa_lim mask (prompt causal, a reference
    picture's block whole, image rows all keys);
  - src/cuda-dit.lisp:137-243: the step driver's prefix K/V cache (the
    cached pass runs the image rows only against the kept prompt K/V) and
    the edit insertion of the reference picture's rows;
  - src/generate.lisp:7-9,133-135: the Turbo sigma list and the Euler update;
  - src/weights.lisp:19-45: tensor names and ggml dims;
  - src/cuda-dit.lisp:110-126: the int8 product of the reference's default
    *int8* mode (Q8_0 matrices times activations quantised to Q8_0 by blocks
    of 32, n >= 16 rows).  Its kernels (quant_q8, MM_Q8_MMA2) live in illatio,
    which the reference does not vendor and pins to no version; quant_q8_0 and
    linear_w8a8 restate ggml's published CUDA forms (the activation quantiser
    of its batched Q8_0 product and the Q8_0 block dot product), which the
    reference's note names as their model ("ggml's way for a batch",
    :111-113).  Against illatio's own arithmetic this is parity unpinned;
and the synthetic inputs (a counter-based generator, defined in synth.c),
whose C twin is oracle/liboracle.so.

How each function is pinned (tests/test_oracle.py): forward against vectors
written by the reference's own inspect/ref_dit.py at tiny shapes
(tests/golden/); the pieces by closed forms, invariants and float64 brute
force; the Q8_0 codec and generator against the C twin and numpy's own
IEEE conversions.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field

import numpy as np

# --- model shape (src/weights.lisp:19-20; inspect/ref_dit.py:19-20) ---------------

AXES = (16, 56, 56)                      # RoPE head-dim split, inspect/ref_dit.py:20
THETA = 10000.0                          # inspect/ref_dit.py:72
EPS = 1e-6                               # src/cuda/dit.cu:30,53
TURBO_SIGMAS = (1.0, 0.978453, 0.95418, 0.926626, 0.89508, 0.845148, 0.704534, 0.414568, 0.0)  # src/generate.lisp:7-9


@dataclass(frozen=True)
class Shape:
    """dit-shape (src/weights.lisp:19-20); the reference fixes every field but
    LAYERS is the loop bound the tests shorten (cf. *dit-layers*,
    src/metal-dit.lisp:112)."""
    width: int = 4096
    layers: int = 32
    head_dim: int = 128
    ffn: int = 12288
    latent: int = 64
    context: int = 4096
    freq: int = 256

    @property
    def heads(self) -> int:
        return self.width // self.head_dim


def dit_expected(sh: Shape = Shape()):
    """[(name, ggml dims)] in the reference's order, contiguous axis first
    (src/weights.lisp:22-45).  The index in this list is the tensor id the
    synthetic generator keys on."""
    w, f = sh.width, sh.ffn
    out = [("img_in.weight", (sh.latent, w)),
           ("txt_in.text_norm.weight", (sh.context,)),
           ("txt_in.in_layer.weight", (sh.context, w)),
           ("txt_in.out_layer.weight", (w, w)),
           ("time_text_embed.timestep_embedder.linear_1.weight", (sh.freq, w)),
           ("time_text_embed.timestep_embedder.linear_2.weight", (w, w)),
           ("modulation.1.weight", (w, 4 * w)),
           ("norm_out.linear.weight", (w, w)),
           ("proj_out.weight", (w, sh.latent))]
    for i in range(sh.layers):
        b = "transformer_blocks.%d." % i
        out += [(b + "attn.norm_q.weight", (sh.head_dim,)),
                (b + "attn.norm_k.weight", (sh.head_dim,)),
                (b + "attn.to_q.weight", (w, w)),
                (b + "attn.to_k.weight", (w, w)),
                (b + "attn.to_v.weight", (w, w)),
                (b + "attn.to_out.0.weight", (w, w)),
                (b + "img_mlp.gate_up.weight", (w, 2 * f)),
                (b + "img_mlp.out.weight", (f, w))]
    return out


def tensor_id(name: str) -> int:
    """The generator's tensor id: the tensor's index in dit_expected's order
    for 32 layers (edge tensors 0..8, then 9 + 8*layer + slot)."""
    edge = [n for n, _ in dit_expected(Shape(layers=0))]
    if name in edge:
        return edge.index(name)
    assert name.startswith("transformer_blocks."), name
    rest = name[len("transformer_blocks."):]
    layer, slot = rest.split(".", 1)
    slots = ["attn.norm_q.weight", "attn.norm_k.weight", "attn.to_q.weight", "attn.to_k.weight",
             "attn.to_v.weight", "attn.to_out.0.weight", "img_mlp.gate_up.weight", "img_mlp.out.weight"]
    return 9 + 8 * int(layer) + slots.index(slot)


# ids of the synthetic step inputs, past every weight's
INPUT_CONTEXT, INPUT_LATENT, INPUT_REF_LATENT = 1001, 1002, 1003

# --- the counter-based generator (definition: synth.c's header) -------------------

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
NORMAL_SCALE = np.float32(1.3214498960651507e-05)   # 1 / (4 * sd of a 16-bit uniform)
D_SCALE = np.float32(2.6428997921303017e-09)        # 2e-4 * NORMAL_SCALE


def mix64(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def key(seed: int, tensor: int) -> np.uint64:
    with np.errstate(over="ignore"):
        return mix64(np.uint64(seed) * _G + np.uint64(tensor) + np.uint64(1))


def words(k, idx):
    with np.errstate(over="ignore"):
        return mix64(np.uint64(k) + (np.asarray(idx, dtype=np.uint64) + np.uint64(1)) * _G)


def _sum2(w):
    s = np.zeros(w.shape, dtype=np.int64)
    for c in range(4):
        s += ((w >> np.uint64(16 * c)) & np.uint64(0xFFFF)).astype(np.int64)
    return (2 * s - 262140).astype(np.float32)


def normal(seed: int, tensor: int, n: int) -> np.ndarray:
    """n unit normals (Irwin-Hall of 4), float32, element i from word(key, i)."""
    return _sum2(words(key(seed, tensor), np.arange(n, dtype=np.uint64))) * NORMAL_SCALE


def q8_0_synth(seed: int, tensor: int, rows: int, cols: int):
    """A rows x cols Q8_0 matrix as SoA: qs int8 (rows, cols), d fp16 (rows, cols/32)."""
    assert cols % 32 == 0
    nb = rows * (cols // 32)
    k = key(seed, tensor)
    base = np.arange(nb, dtype=np.uint64) * np.uint64(5)
    qs = np.empty((nb, 32), dtype=np.int8)
    for w in range(4):
        x = words(k, base + np.uint64(w))
        for j in range(8):
            u = ((x >> np.uint64(8 * j)) & np.uint64(0xFF)).astype(np.int32)
            qs[:, 8 * w + j] = ((u * 255 + 128) >> 8) - 127
    z = _sum2(words(k, base + np.uint64(4))) * D_SCALE
    d = np.abs(z).astype(np.float16)                  # numpy's conversion: IEEE RNE, subnormals kept
    return qs.reshape(rows, cols), d.reshape(rows, cols // 32)


def q8_0_to_blocks(qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """SoA -> GGUF block_q8_0 records (uint8, 34 bytes a block: fp16 d, int8 qs[32])."""
    nb = qs.size // 32
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 0:2] = d.reshape(nb).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = qs.reshape(nb, 32).view(np.uint8)
    return out.reshape(-1)


def dequant_q8_0_blocks(blocks: np.ndarray) -> np.ndarray:
    """GGUF block_q8_0 -> fp32: fp32(d) * q (what gguf-py's quants.dequantize
    gives ref_dit.py, inspect/ref_dit.py:28-30).  Exact in fp32."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)      # (nb, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(-1)


def dequant_q8_0(qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """SoA Q8_0 -> fp32 with qs's shape."""
    rows = qs.shape[0]
    q = qs.reshape(rows, -1, 32).astype(np.float32)
    return (q * d.astype(np.float32).reshape(rows, -1, 1)).reshape(qs.shape)


# --- the W8A8 product (src/cuda-dit.lisp:110-126) ------------------------------------

def quant_q8_0(x):
    """Activations to Q8_0 by blocks of 32, as quant_q8 does ahead of the reference's int8
    products (src/cuda-dit.lisp:120-123), after ggml's CUDA activation quantiser: amax = max |x|
    over the block, d = amax / 127, q = round(x / d) half away from zero (0 when amax is 0), the
    divisions float32 and correctly rounded; d is kept as fp16 and the products use that.
    X: (n, K) float32, K a multiple of 32.  Returns (q int8 (n, K), d float16 (n, K / 32))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, K = x.shape
    b = x.reshape(n, K // 32, 32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float32)
    safe = np.where(amax != 0, d, np.float32(1)).astype(np.float32)
    v = (b / safe[:, :, None]).astype(np.float32)
    q = np.sign(v) * np.floor(np.abs(v.astype(np.float64)) + 0.5)      # half away from zero, exact
    q = np.where(amax[:, :, None] != 0, q, 0)
    return q.astype(np.int8).reshape(n, K), d.astype(np.float16)


def linear_w8a8(x, qs, d, gain=1.0):
    """Y = X W^T the reference's int8 way (src/cuda-dit.lisp:119-124: quant_q8, then illatio's
    MM_Q8_MMA2 after ggml's Q8_0 x Q8_0 dot product): X quantised by quant_q8_0; per 32-block
    the integer dot product, exact; then y = fma(float(isum), dx * dw, y) in float32 over the
    blocks in order, the scale product (exact: 11 x 11 bits) rounded, the fused multiply-add
    rounded once (the C twin's fmaf).  W: Q8_0 SoA (qs int8 (N, K), d float16 (N, K / 32));
    GAIN, a power of two, scales dw."""
    lib = clib()
    if lib is None:
        raise RuntimeError("linear_w8a8 takes its fused multiply-adds from oracle/liboracle.so (make -C oracle)")
    xq, xd = quant_q8_0(x)
    n, K = xq.shape
    xqf, wqf = xq.astype(np.float32), np.asarray(qs).astype(np.float32)
    dx = xd.astype(np.float32)
    dw = (np.asarray(d).astype(np.float32) * np.float32(gain)).astype(np.float32)
    N = wqf.shape[0]
    y = np.zeros((n, N), np.float32)
    for blk in range(K // 32):
        c = slice(32 * blk, 32 * blk + 32)
        isum = np.ascontiguousarray(xqf[:, c] @ wqf[:, c].T, dtype=np.float32)   # exact: below 2^20
        lib.exo_w8a8_fma(_ptr(isum), _ptr(np.ascontiguousarray(dx[:, blk])), _ptr(np.ascontiguousarray(dw[:, blk])),
                         n, N, _ptr(y))
    return y


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even, NaN quiet."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


# --- the C twin (liboracle.so), for full-size weights ----------------------------

_LIB = None


def clib():
    """oracle/liboracle.so (built by `make -C oracle`), or None."""
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liboracle.so")
        if not os.path.exists(path):
            return None
        lib = ctypes.CDLL(path)
        u64, i64, vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p
        lib.exo_key.restype = u64; lib.exo_key.argtypes = [u64, u64]
        lib.exo_word.restype = u64; lib.exo_word.argtypes = [u64, u64]
        lib.exo_f16_rne.restype = ctypes.c_uint16; lib.exo_f16_rne.argtypes = [ctypes.c_float]
        lib.exo_f16_to_f32.restype = ctypes.c_float; lib.exo_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.exo_bf16_rne_n.argtypes = [vp, vp, i64]
        lib.exo_q8_0_synth.argtypes = [u64, u64, i64, i64, vp, vp]
        lib.exo_q8_0_synth_blocks.argtypes = [u64, u64, i64, i64, vp]
        lib.exo_normal.argtypes = [u64, u64, i64, vp]
        lib.exo_dequant_q8_0_blocks.argtypes = [vp, i64, vp]
        lib.exo_dequant_q8_0.argtypes = [vp, vp, i64, vp]
        lib.exo_w8a8_fma.argtypes = [vp, vp, vp, i64, i64, vp]
        _LIB = lib
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def q8_0_synth_fast(seed, tensor, rows, cols):
    """q8_0_synth through the C twin (identical output, tests hold them equal)."""
    lib = clib()
    if lib is None:
        return q8_0_synth(seed, tensor, rows, cols)
    qs = np.empty((rows, cols), dtype=np.int8)
    d = np.empty((rows, cols // 32), dtype=np.uint16)
    lib.exo_q8_0_synth(seed, tensor, rows, cols, _ptr(qs), _ptr(d))
    return qs, d.view(np.float16)


def dequant_fast(qs, d):
    lib = clib()
    if lib is None:
        return dequant_q8_0(qs, d)
    out = np.empty(qs.shape, dtype=np.float32)
    lib.exo_dequant_q8_0(_ptr(np.ascontiguousarray(qs)), _ptr(np.ascontiguousarray(d).view(np.uint16)),
                         qs.size, _ptr(out))
    return out


# --- synthetic weights --------------------------------------------------------------

def synth_vector(seed: int, name: str, n: int) -> np.ndarray:
    """The norms' weights: norm_q, norm_k ~ 1 + 0.05 z; txt_in.text_norm ~
    0.05 z (zero-centred, used as 1 + w: src/cuda-dit.lisp:67-68)."""
    z = normal(seed, tensor_id(name), n)
    if name == "txt_in.text_norm.weight":
        return np.float32(0.05) * z
    return np.float32(1.0) + np.float32(0.05) * z


class SynthWeights:
    """wt(name) -> fp32 (out, in) matrix or vector, as ref_dit.py's Weights
    gives them (inspect/ref_dit.py:23-30), from the counter generator.
    Matrices are Q8_0 and dequantised exactly; `q8(name)` gives the SoA
    codes.  GAIN (float32) multiplies every matrix: the tiny golden shapes use
    4 so that a 256-wide linear keeps unit gain and the timestep path gives
    gates far from zero.  Dequantised matrices are cached per name up to
    `cache_bytes`."""

    def __init__(self, seed: int, shape: Shape = Shape(), cache_bytes: int = 2 << 30, gain: float = 1.0,
                 keep_q8: bool = False):
        self.seed, self.shape, self.gain = seed, shape, np.float32(gain)
        self.dims = dict(dit_expected(shape))
        self.cache, self.cache_bytes = {}, cache_bytes
        self.keep_q8, self.q8cache = keep_q8, {}

    def q8(self, name):
        """The SoA codes (kept per name when keep_q8: 1.06 bytes a weight, not 4)."""
        if name in self.q8cache:
            return self.q8cache[name]
        dims = self.dims[name]
        c = q8_0_synth_fast(self.seed, tensor_id(name), dims[1], dims[0])
        if self.keep_q8:
            self.q8cache[name] = c
        return c

    def __call__(self, name):
        dims = self.dims[name]
        if len(dims) == 1:
            return synth_vector(self.seed, name, dims[0])
        if name in self.cache:
            return self.cache[name]
        m = dequant_fast(*self.q8(name))
        if self.gain != 1:
            m = m * self.gain
        if sum(v.nbytes for v in self.cache.values()) + m.nbytes <= self.cache_bytes:
            self.cache[name] = m
        return m


def synth_inputs(seed: int, p: int, h: int, w: int, shape: Shape = Shape(), ref_hw=None):
    """The step's synthetic inputs: context (p x context) ~ N(0,1), latent
    (latent x h x w) ~ N(0,1), and, for an edit, a reference latent."""
    ctx = normal(seed, INPUT_CONTEXT, p * shape.context).reshape(p, shape.context)
    lat = normal(seed, INPUT_LATENT, shape.latent * h * w).reshape(shape.latent, h, w)
    if ref_hw is None:
        return ctx, lat
    rh, rw = ref_hw
    ref = normal(seed, INPUT_REF_LATENT, shape.latent * rh * rw).reshape(shape.latent, rh, rw)
    return ctx, lat, ref


# --- the pieces (inspect/ref_dit.py:33-105) ---------------------------------------

def linear(x, w):
    """Y = X W^T, w (out, in) -- inspect/ref_dit.py:33-34."""
    return x @ w.T


def mm(wt, name, x, w8a8=False):
    """The reference's product dispatch for matrix NAME (src/cuda-dit.lisp:115-126): with W8A8
    (its default *int8*), a Q8_0 matrix (WT has its codes) times at least 16 rows goes the int8
    way (linear_w8a8); everything else is linear(x, wt(name))."""
    if w8a8 and x.shape[0] >= 16 and hasattr(wt, "q8"):
        qs, d = wt.q8(name)
        return linear_w8a8(x, qs, d, getattr(wt, "gain", 1.0))
    return linear(x, wt(name))


def layernorm(x, eps=EPS):
    """No affine -- inspect/ref_dit.py:37-40; src/cuda/dit.cu:17-32."""
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps)


def rmsnorm(x, w, eps=EPS):
    """inspect/ref_dit.py:43-44."""
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def gelu_tanh(x):
    """inspect/ref_dit.py:47-48; src/cuda/dit.cu:194-199."""
    return 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def silu(x):
    """inspect/ref_dit.py:51-52; src/cuda/dit.cu:201-206."""
    return x / (1 + np.exp(-x))


def timestep_embedding(t, dim=256, period=10000.0):
    """cos then sin of t times dim/2 frequencies, float32 as ref_dit.py
    computes it (inspect/ref_dit.py:55-59; host.lisp:9-15 does the same in
    double and rounds)."""
    half = dim // 2
    f = np.exp(-math.log(period) * np.arange(half, dtype=np.float32) / half)
    a = t * f
    return np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32)


def image_positions(frame, h, w):
    """src/host.lisp:32-35: an h x w block at FRAME, rows and columns centred."""
    r, c = np.meshgrid(np.arange(h), np.arange(w), indexing="ij")
    pos = np.stack([np.full(h * w, frame), (r - (h - h // 2)).reshape(-1), (c - (w - w // 2)).reshape(-1)], 1)
    return pos


def positions(p, h, w, ref=None):
    """Every row's (frame, row, col): src/host.lisp:37-50 (inspect/ref_dit.py:
    62-69 for the plain case).  P counts the whole prefix; REF = (a, rh, rw)
    puts a rh x rw reference picture after the first a text rows, framed at a,
    the remaining text from a + max(rh, rw) on, the image after it."""
    if ref is None:
        txt = np.repeat(np.arange(p)[:, None], 3, 1)
        return np.concatenate([txt, image_positions(p, h, w)]).astype(np.float32)
    a, rh, rw = ref
    after = p - a - rh * rw
    pos0 = a + max(rh, rw)
    parts = [np.repeat(np.arange(a)[:, None], 3, 1), image_positions(a, rh, rw),
             np.repeat((pos0 + np.arange(after))[:, None], 3, 1), image_positions(pos0 + after, h, w)]
    return np.concatenate(parts).astype(np.float32)


def rope_tables(pos, theta=THETA):
    """cos, sin: tokens x 64, the three axes' pairs in turn (inspect/ref_dit.py:72-79)."""
    angs = []
    for a, d in enumerate(AXES):
        omega = 1.0 / theta ** (np.arange(0, d, 2, dtype=np.float64) / d)
        angs.append(pos[:, a:a + 1].astype(np.float64) * omega[None, :])
    ang = np.concatenate(angs, axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x, cos, sin):
    """Interleaved pairs (2i, 2i+1) turned by the token's angle i (inspect/ref_dit.py:82-88)."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c, s = cos[:, None, :], sin[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def xa_lim(g, p, l, b0, b1):
    """Row g of the sequence sees keys 0..xa_lim(g) (src/cuda/dit.cu:60-66)."""
    g = np.asarray(g)
    return np.where(g >= p, l - 1, np.where((g >= b0) & (g < b1), b1 - 1, g))


def attention(q, k, v, q0, p, b0=0, b1=0, head_chunk=4):
    """softmax(Q K^T / sqrt(hd) + mask) V with xa_lim's mask: query t is row
    q0 + t of the sequence, K and V are the l rows 0..l-1 (inspect/ref_dit.py:
    91-105 for the plain first pass; src/cuda/dit.cu:208-336 for q0, b0, b1).
    q: (n, H, hd); k, v: (l, H, hd)."""
    n, heads, hd = q.shape
    l = k.shape[0]
    scale = np.float32(1.0 / math.sqrt(hd))
    lim = xa_lim(q0 + np.arange(n), p, l, b0, b1)
    mask = np.arange(l)[None, :] > lim[:, None]          # True: hidden
    out = np.empty_like(q)
    for h0 in range(0, heads, head_chunk):
        hs = slice(h0, min(heads, h0 + head_chunk))
        qh = np.ascontiguousarray(q[:, hs].transpose(1, 0, 2))          # (h, n, hd)
        kt = np.ascontiguousarray(k[:, hs].transpose(1, 2, 0))          # (h, hd, l)
        vh = np.ascontiguousarray(v[:, hs].transpose(1, 0, 2))          # (h, l, hd)
        s = np.matmul(qh, kt) * scale
        s = np.where(mask[None], np.asarray(-np.inf, dtype=s.dtype), s)
        s = s - s.max(-1, keepdims=True)
        e = np.exp(s)
        pr = e / e.sum(-1, keepdims=True)
        out[:, hs] = np.matmul(pr, vh).transpose(1, 0, 2)
    return out


# --- the step (inspect/ref_dit.py:108-153 with src/cuda-dit.lisp:137-243) ----------

@dataclass
class PrefixCache:
    """The kept prompt K/V (src/cuda-dit.lisp:44-50,148-151,207-218,232-233):
    per layer, K and V of rows 0..p-1, under KEY; LENGTH is p."""
    key: object = None
    length: int = 0
    kv: dict = field(default_factory=dict)


def modulation(wt, sigma, shape=Shape()):
    """[embed(1000 sigma), embed(0)] -> linear_1, SiLU, linear_2, SiLU; then
    modulation.1 (2 x 4W: scale1, gate1, scale2, gate2) and norm_out's scale
    from row 0 (inspect/ref_dit.py:112-118,150)."""
    t = sigma * 1000.0
    emb = np.stack([timestep_embedding(t, shape.freq), timestep_embedding(0.0, shape.freq)])
    emb = linear(silu(linear(emb, wt("time_text_embed.timestep_embedder.linear_1.weight"))),
                 wt("time_text_embed.timestep_embedder.linear_2.weight"))
    emb = silu(emb)
    mod = linear(emb, wt("modulation.1.weight"))
    sc = linear(emb[0:1], wt("norm_out.linear.weight"))
    return emb, mod, sc


def block(wt, il, x, mod_rows, cos, sin, kfull, vfull, q0, p, b0, b1, shape=Shape(), w8a8=False):
    """One block (inspect/ref_dit.py:132-148): X's rows are sequence rows
    q0..q0+n-1; MOD_ROWS (n, 4W) their modulation rows; KFULL/VFULL receive
    this pass's K, V at rows q0.. and hold the kept prefix below.  W8A8: the
    products as the reference's int8 mode takes them (mm).  Returns the new X
    (float32)."""
    W, H, HD, F = shape.width, shape.heads, shape.head_dim, shape.ffn
    n = x.shape[0]
    scale1, gate1, scale2, gate2 = (mod_rows[:, i * W:(i + 1) * W] for i in range(4))
    b = "transformer_blocks.%d." % il
    y = layernorm(x) * (1.0 + scale1)
    q = mm(wt, b + "attn.to_q.weight", y, w8a8).reshape(n, H, HD)
    k = mm(wt, b + "attn.to_k.weight", y, w8a8).reshape(n, H, HD)
    v = mm(wt, b + "attn.to_v.weight", y, w8a8).reshape(n, H, HD)
    q = rope(rmsnorm(q, wt(b + "attn.norm_q.weight")), cos, sin)
    k = rope(rmsnorm(k, wt(b + "attn.norm_k.weight")), cos, sin)
    kfull[q0:q0 + n] = k
    vfull[q0:q0 + n] = v
    a = attention(q, kfull, vfull, q0, p, b0, b1).reshape(n, W)
    x = x + np.tanh(gate1) * mm(wt, b + "attn.to_out.0.weight", a, w8a8)
    y = layernorm(x) * (1.0 + scale2)
    gu = mm(wt, b + "img_mlp.gate_up.weight", y, w8a8)
    y = silu(gu[:, :F]) * gu[:, F:]
    x = x + np.tanh(gate2) * mm(wt, b + "img_mlp.out.weight", y, w8a8)
    return x.astype(np.float32)


def prompt_rows(wt, ctx, shape=Shape(), w8a8=False):
    """txt_in: RMSNorm with (1 + w), linear, GELU-tanh, linear (inspect/ref_dit.py:120-121)."""
    txt = rmsnorm(ctx, 1.0 + wt("txt_in.text_norm.weight"))
    return mm(wt, "txt_in.out_layer.weight", gelu_tanh(mm(wt, "txt_in.in_layer.weight", txt, w8a8)), w8a8)


def tokens(latent):
    """A channel-major latent (c, h, w) as h*w rows of c (inspect/ref_dit.py:122)."""
    c, h, w = latent.shape
    return latent.reshape(c, h * w).T


def forward(wt, ctx, latent, sigma, shape=Shape(), ref=None, cache: PrefixCache | None = None,
            prefix_key=None, dump=None, layers=None, w8a8=False):
    """The velocity at SIGMA, dit-velocity's contract (src/cuda-dit.lisp:137-144):
    CTX the encoder's P x context states, LATENT (64, h, w) channel-major.
    REF = (a, ref_latent (64, rh, rw)): an edit's reference picture, put in the
    prefix after the first a text rows.  With CACHE and PREFIX_KEY, the first
    call keeps each layer's prefix K/V and a later call with the same key and
    prefix length runs only the image rows.  DUMP (a dict) receives 'txt'
    (the prompt rows, uncached pass only) and 'blk' (x after each block).
    W8A8: every product of a Q8_0 matrix with at least 16 rows the reference's
    int8 way (mm; src/cuda-dit.lisp:110-126).  Without REF, CACHE and W8A8
    this is ref_dit.forward, step for step."""
    W, H, HD = shape.width, shape.heads, shape.head_dim
    L = shape.layers if layers is None else layers
    ptext = ctx.shape[0]
    c, h, w = latent.shape
    nimg = h * w
    nref = 0 if ref is None else ref[1].shape[1] * ref[1].shape[2]
    a = 0 if ref is None else ref[0]
    p = ptext + nref
    cached = (cache is not None and prefix_key is not None and cache.key == prefix_key and cache.length == p)
    n0 = p if cached else 0
    l = p + nimg
    emb, mod, sc = modulation(wt, sigma, shape)
    img = mm(wt, "img_in.weight", tokens(latent), w8a8)
    if cached:
        x = img.astype(np.float32)
    else:
        txt = prompt_rows(wt, ctx, shape, w8a8)
        if dump is not None:
            dump["txt"] = txt.astype(np.float32)
        if ref is None:
            pre = txt
        else:
            rimg = mm(wt, "img_in.weight", tokens(ref[1]), w8a8)
            pre = np.concatenate([txt[:a], rimg, txt[a:]])
        x = np.concatenate([pre, img]).astype(np.float32)
    n = x.shape[0]
    rows = np.where(n0 + np.arange(n) < p, 1, 0)              # prompt rows: modulation row 1 (t = 0)
    mod_rows = mod[rows]
    pos = positions(p, h, w, None if ref is None else (a, ref[1].shape[1], ref[1].shape[2]))
    cos, sin = rope_tables(pos[n0:])
    b0, b1 = (a, a + nref) if ref is not None else (0, 0)
    if cache is not None and not cached:
        cache.key, cache.length, cache.kv = None, 0, {}
    if dump is not None:
        dump["blk"] = []
    for il in range(L):
        kfull = np.zeros((l, H, HD), dtype=np.float32)
        vfull = np.zeros((l, H, HD), dtype=np.float32)
        if cached:
            kfull[:p], vfull[:p] = cache.kv[il]
        x = block(wt, il, x, mod_rows, cos, sin, kfull, vfull, n0, p, b0, b1, shape, w8a8)
        if cache is not None and prefix_key is not None and not cached:
            cache.kv[il] = (kfull[:p].copy(), vfull[:p].copy())
        if dump is not None:
            dump["blk"].append(x.copy())
    if cache is not None and prefix_key is not None and not cached:
        cache.key, cache.length = prefix_key, p
    xi = x[p - n0:]
    xi = layernorm(xi) * (1.0 + sc)
    v = mm(wt, "proj_out.weight", xi, w8a8)                  # (h*w) x 64
    return v.T.reshape(c, h, w).astype(np.float32)


class Overrides:
    """The synthetic weights WT with some matrices replaced (OVER: name -> fp32 matrix)."""

    def __init__(self, wt, over):
        self.wt, self.over = wt, over

    def __call__(self, name):
        return self.over[name] if name in self.over else self.wt(name)


# Weights at the magnitudes real checkpoints reach, for parity off the unit-scale synthetic data.
# txt_in_8e5: txt_in's in_layer scaled so its GELU's rows reach about 8e5 (the magnitude the
# reference records for the real weights, src/metal-dit.lisp:5-7), and the prompt rows of the
# residual stream about 7e5 after out_layer.  img_in_outliers: eight of img_in's 4096 output
# channels scaled by 80, so every image row of the residual stream carries outlier channels
# through the blocks (they then hold most of each row's variance).
MAGNITUDE_CASES = {
    "txt_in_8e5": ("txt_in.in_layer.weight", None, 2e5),
    "img_in_outliers": ("img_in.weight", (17, 400, 1033, 1999, 2048, 2900, 3511, 4000), 80.0),
}


def magnitude_overrides(wt, case):
    """The replaced matrices of MAGNITUDE_CASES[case] (fp32, scaled exactly by a power-of-two-
    free factor applied once in fp32)."""
    name, rows, scale = MAGNITUDE_CASES[case]
    m = np.array(wt(name), np.float32, copy=True)
    if rows is None:
        m *= np.float32(scale)
    else:
        m[list(rows)] *= np.float32(scale)
    return {name: m}


def euler(wt, ctx, latent, shape=Shape(), sigmas=TURBO_SIGMAS, ref=None, prefix_key="prompt",
          layers=None, on_step=None, w8a8=False):
    """The Turbo schedule's Euler loop: z <- z + (s' - s) v, (s' - s) as a
    single float (src/generate.lisp:133-135; edit: :95-97).  The prefix cache
    is used as generate uses it (:prefix-key prompt)."""
    z = latent.astype(np.float32).copy()
    cache = PrefixCache()
    for s, s2 in zip(sigmas[:-1], sigmas[1:]):
        v = forward(wt, ctx, z, s, shape, ref=ref, cache=cache, prefix_key=prefix_key, layers=layers, w8a8=w8a8)
        z = z + np.float32(s2 - s) * v
        if on_step is not None:
            on_step(s, v, z)
    return z


def rel_l2(got, want):
    """||got - want|| / ||want||, in float64."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-300))


# --- work counts (what the benchmark's roofline divides by) ------------------------

def gemm_flops_per_row(shape=Shape()):
    """Per sequence row and block: q, k, v, out (W x W each), gate_up (W x 2F), down (F x W)."""
    W, F = shape.width, shape.ffn
    return 2 * (4 * W * W + W * 2 * F + F * W)


def visible_pairs(n, q0, p, l, b0=0, b1=0):
    """Visible (query, key) pairs under xa_lim for queries q0..q0+n-1."""
    lim = xa_lim(q0 + np.arange(n), p, l, b0, b1)
    return int((lim + 1).sum())


def step_flops(nimg, p, cached, shape=Shape(), nref=0, a=0):
    """Algorithmic FLOPs of one step: block GEMMs, attention (QK^T and PV,
    2 * 2 * hd per head per visible pair) and the edge GEMMs."""
    ptot = p + nref
    n0 = ptot if cached else 0
    n = nimg if cached else ptot + nimg
    l = ptot + nimg
    b0, b1 = (a, a + nref) if nref else (0, 0)
    L, W = shape.layers, shape.width
    gemm = L * n * gemm_flops_per_row(shape)
    att = L * 4 * shape.head_dim * shape.heads * visible_pairs(n, n0, ptot, l, b0, b1)
    edge = 2 * (2 * shape.freq * W + 2 * W * W + 2 * W * 4 * W + W * W)       # timestep, modulation, norm_out
    edge += 2 * nimg * (shape.latent * W + W * shape.latent)                 # img_in, proj_out
    if not cached:
        edge += 2 * p * (shape.context * W + W * W) + 2 * nref * shape.latent * W   # txt_in, reference img_in
    return {"gemm": gemm, "attention": att, "edge": edge, "total": gemm + att + edge}
