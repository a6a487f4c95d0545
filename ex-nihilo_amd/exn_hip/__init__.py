"""exn_hip -- the host side of libexn-hip.so in Python: a ctypes binding of
include/exn_hip.h and the reference's DiT backend trio on top of it.

The reference's host is Common Lisp (src/cuda-dit.lisp); its trio is

    (upload-dit path &key device)                                  src/cuda-dit.lisp:52
    (dit-velocity d context p latent h w sigma &key prefix-key ref) src/cuda-dit.lisp:137
    (dit-release d)                                                 src/cuda-dit.lisp:99

and generate's Euler loop (src/generate.lisp:112-137) calls it.  This module
mirrors those names, argument meanings and error behaviour (a failed call
raises ExnError carrying the library's message, as the reference signals a
Lisp error) for hosts that are not SBCL -- the tests and the benchmark.  The
SBCL binding is ../lisp/hip-dit.lisp.  There is no CPU fallback: without the
built library or a GPU every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# the build beside the package, or another build of it named by EXN_HIP_LIB (the sanitized host build)
LIB_PATH = os.environ.get("EXN_HIP_LIB") or os.path.join(os.path.dirname(HERE), "libexn-hip.so")

OK, ENODEV, EINVAL, ENOMEM, EHIP, ESTATE = 0, 1, 2, 3, 4, 5
Q8_0, F32, BF16, F16 = 8, 0, 30, 1
DT_F32, DT_BF16, DT_F16 = 0, 1, 2
WIDTH, HEADS, HEAD_DIM, FFN, LATENT = 4096, 32, 128, 12288, 64
# Qwen-Image-2.1-Turbo's schedule (src/generate.lisp:7-9)
TURBO_SIGMAS = (1.0, 0.978453, 0.95418, 0.926626, 0.89508, 0.845148, 0.704534, 0.414568, 0.0)


class ExnError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("exn error %d: %s" % (code, msg))
        self.code = code


_lib = None
vp = c_void_p

# name -> (restype, argtypes); every function of include/exn_hip.h
SIGNATURES = {
    "exn_last_error": (c_char_p, []),
    "exn_version": (c_int, []),
    "exn_device_count": (c_int, [POINTER(c_int)]),
    "exn_open": (c_int, [c_int, POINTER(vp)]),
    "exn_close": (c_int, [vp]),
    "exn_set_stream": (c_int, [vp, vp]),
    "exn_sync": (c_int, [vp]),
    "exn_alloc": (c_int, [vp, c_size_t, POINTER(vp)]),
    "exn_free": (c_int, [vp, vp]),
    "exn_upload": (c_int, [vp, vp, vp, c_size_t]),
    "exn_download": (c_int, [vp, vp, vp, c_size_t]),
    "exn_copy": (c_int, [vp, vp, vp, c_size_t]),
    "exn_weight_q8_0": (c_int, [vp, vp, c_int64, c_int64, POINTER(vp)]),
    "exn_weight_f32": (c_int, [vp, vp, c_int64, c_int64, POINTER(vp)]),
    "exn_weight_bf16": (c_int, [vp, vp, c_int64, c_int64, POINTER(vp)]),
    "exn_weight_q8_0_synth": (c_int, [vp, c_uint64, c_uint64, c_int64, c_int64, POINTER(vp)]),
    "exn_weight_info": (c_int, [vp, POINTER(c_int64), POINTER(c_int64), POINTER(c_int)]),
    "exn_weight_free": (c_int, [vp]),
    "exn_dequant": (c_int, [vp, vp, vp, vp]),
    "exn_mm": (c_int, [vp, vp, vp, c_int, vp, c_int, c_int64]),
    "exn_mm_noalloc": (c_int, [vp, vp, vp, c_int, vp, c_int, c_int64]),
    "exn_quant_q8": (c_int, [vp, vp, c_int, c_int64, c_int64, c_int64, vp, vp]),
    "exn_mm_w8a8": (c_int, [vp, vp, vp, vp, c_int64, vp, c_int]),
    "exn_mm_gate_add": (c_int, [vp, vp, vp, c_int64, vp, c_int, c_int, c_int, vp]),
    "exn_mm_swiglu": (c_int, [vp, vp, vp, vp, c_int64]),
    "exn_weight_pairs": (c_int, [vp, vp]),
    "exn_weight_resident": (c_int, [vp, vp, c_int]),
    "exn_ln_mod": (c_int, [vp, c_int, c_int, c_int, c_int, vp, c_int64, vp, vp, c_int]),
    "exn_rms": (c_int, [vp, c_int, c_int, c_float, vp, vp, vp, c_int]),
    "exn_gate_add": (c_int, [vp, c_int64, c_int, c_int, c_int, c_int, vp, vp, vp]),
    "exn_swiglu": (c_int, [vp, c_int64, c_int, vp, vp]),
    "exn_gelu_tanh": (c_int, [vp, c_int64, vp]),
    "exn_silu": (c_int, [vp, c_int64, vp]),
    "exn_qkv_prep": (c_int, [vp, vp, c_int64, vp, vp, vp, vp, vp, vp, c_int64, c_int64]),
    "exn_mm_qkv": (c_int, [vp, vp, vp, c_int64, vp, vp, vp, vp, vp, vp, c_int64, c_int64]),
    "exn_attend": (c_int, [vp, vp, vp, vp, vp, c_int, c_int, c_int, c_int, c_int64, c_int, c_int, c_float]),
    "exn_euler": (c_int, [vp, c_int64, vp, vp, c_float]),
    "exn_dit_create": (c_int, [vp, c_int, POINTER(vp)]),
    "exn_dit_set": (c_int, [vp, c_char_p, c_int, vp, c_int64, c_int64]),
    "exn_dit_synth": (c_int, [vp, c_uint64]),
    "exn_dit_check": (c_int, [vp]),
    "exn_dit_resident": (c_int, [vp, c_int]),
    "exn_dit_w8a8": (c_int, [vp, c_int]),
    "exn_dit_velocity": (c_int, [vp, vp, c_int, vp, c_int, c_int, c_double, c_uint64, c_int, vp, c_int, c_int, vp]),
    "exn_dit_velocity_dev": (c_int, [vp, vp, c_int, vp, c_int, c_int, c_double, c_uint64, c_int, vp, c_int, c_int,
                                     vp]),
    "exn_dit_generate_dev": (c_int, [vp, vp, c_int, vp, c_int, c_int, vp, c_int, c_int, vp, c_int, c_int]),
    "exn_dit_trace": (c_int, [vp, vp, c_int64]),
    "exn_dit_profile": (c_int, [vp, c_int]),
    "exn_dit_profile_every": (c_int, [vp, c_int]),
    "exn_dit_profile_read": (c_int, [vp, c_int, POINTER(c_double), POINTER(c_int64), POINTER(c_double),
                                     POINTER(c_double)]),
    "exn_dit_rope_table": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int64, vp, vp]),
    "exn_dit_release": (c_int, [vp]),
    "exn_dit_destroy": (c_int, [vp]),
    "exn_dit_memory": (c_int, [vp, POINTER(c_int64), POINTER(c_int64)]),
    "exn_vae_create": (c_int, [vp, POINTER(vp)]),
    "exn_vae_set": (c_int, [vp, c_char_p, c_int, vp, POINTER(c_int64), c_int]),
    "exn_vae_synth": (c_int, [vp, c_uint64]),
    "exn_vae_check": (c_int, [vp]),
    "exn_vae_check_encoder": (c_int, [vp]),
    "exn_vae_tiles": (c_int, [vp, c_int]),
    "exn_vae_encode": (c_int, [vp, vp, c_int, c_int, vp]),
    "exn_vae_encode_dev": (c_int, [vp, vp, c_int, c_int, vp]),
    "exn_vae_decode": (c_int, [vp, vp, c_int, c_int, vp]),
    "exn_vae_decode_dev": (c_int, [vp, vp, c_int, c_int, vp]),
    "exn_vae_release": (c_int, [vp]),
    "exn_vae_destroy": (c_int, [vp]),
    "exn_vae_memory": (c_int, [vp, POINTER(c_int64), POINTER(c_int64)]),
    "exn_vae_conv": (c_int, [vp, c_int, c_int, c_int, vp, vp, vp, vp, vp, c_int, c_int, c_int, c_int, c_int, vp,
                             c_int64]),
    "exn_vae_rms_silu": (c_int, [vp, c_int64, c_int, vp, vp, vp, c_int]),
    "exn_vae_dupup_add": (c_int, [vp, c_int, c_int, c_int, c_int, c_int, vp, vp]),
    "exn_vae_avgdown_add": (c_int, [vp, c_int, c_int, c_int, c_int, c_int, vp, vp]),
    "exn_vision_create": (c_int, [vp, POINTER(vp)]),
    "exn_vision_set": (c_int, [vp, c_char_p, c_int, vp, POINTER(c_int64), c_int]),
    "exn_vision_synth": (c_int, [vp, c_uint64]),
    "exn_vision_check": (c_int, [vp]),
    "exn_vision_encode": (c_int, [vp, vp, c_int, c_int, vp, vp]),
    "exn_vision_encode_dev": (c_int, [vp, vp, c_int, c_int, vp, vp]),
    "exn_vision_trace": (c_int, [vp, c_int]),
    "exn_vision_traced": (c_int, [vp, c_int, vp]),
    "exn_vision_release": (c_int, [vp]),
    "exn_vision_destroy": (c_int, [vp]),
    "exn_vision_memory": (c_int, [vp, POINTER(c_int64), POINTER(c_int64)]),
    "exn_vis_gemm": (c_int, [vp, vp, vp, vp, vp, vp, c_int64, c_int64, c_int64, c_int]),
    "exn_vis_attend": (c_int, [vp, c_int, c_int, vp, vp, vp, vp]),
    "exn_vis_ln": (c_int, [vp, c_int64, c_int, vp, vp, vp, vp]),
    "exn_dit_stats": (c_int, [vp, c_int]),
    "exn_dit_stats_read": (c_int, [vp, vp, vp, c_int64]),
    "exn_enc_create": (c_int, [vp, c_int, c_double, POINTER(vp)]),
    "exn_enc_set": (c_int, [vp, c_char_p, c_int, vp, c_int64, c_int64]),
    "exn_enc_synth": (c_int, [vp, c_uint64, c_int64]),
    "exn_enc_check": (c_int, [vp]),
    "exn_enc_states": (c_int, [vp, vp, c_int, vp, c_int, c_int, vp, vp, vp]),
    "exn_enc_states_dev": (c_int, [vp, vp, c_int, vp, c_int, c_int, vp, vp, vp]),
    "exn_enc_rope_table": (c_int, [vp, c_int, c_double, vp]),
    "exn_enc_release": (c_int, [vp]),
    "exn_enc_destroy": (c_int, [vp]),
    "exn_enc_memory": (c_int, [vp, POINTER(c_int64), POINTER(c_int64)]),
    "exn_enc_resident": (c_int, [vp, c_int]),
}


def lib():
    """libexn-hip.so, loaded once.  Raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ExnError(ENODEV, "%s is not built (make -C ex-nihilo_amd)" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def check(code):
    if code != OK:
        raise ExnError(code, lib().exn_last_error().decode(errors="replace"))
    return code


def call(name, *args):
    return check(getattr(lib(), name)(*args))


def ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(vp)


# --- context and device buffers -------------------------------------------------------

class Context:
    """A device and its stream (exn_open)."""

    def __init__(self, device: int = 0):
        h = vp()
        call("exn_open", device, ctypes.byref(h))
        self.h = h
        self.device = device

    def sync(self):
        call("exn_sync", self.h)

    def close(self):
        if self.h:
            call("exn_close", self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class DevBuf:
    """Device memory of a numpy dtype and shape (exn_alloc), freed on close/GC."""

    def __init__(self, ctx: Context, shape, dtype):
        self.ctx, self.shape, self.dtype = ctx, tuple(np.atleast_1d(shape)), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        h = vp()
        call("exn_alloc", ctx.h, max(self.nbytes, 1), ctypes.byref(h))
        self.h = h

    @classmethod
    def of(cls, ctx, a: np.ndarray):
        a = np.ascontiguousarray(a)
        b = cls(ctx, a.shape, a.dtype)
        b.upload(a)
        return b

    @property
    def ptr(self):
        return self.h.value

    def at(self, byte_offset: int):
        return vp(self.h.value + byte_offset)

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        call("exn_upload", self.ctx.h, self.h, ptr(a), a.nbytes)

    def get(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        call("exn_download", self.ctx.h, ptr(out), self.h, self.nbytes)
        return out

    def free(self):
        if getattr(self, "h", None) and self.ctx.h:
            call("exn_free", self.ctx.h, self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A matrix on the device (exn_weight_*): ROWS outputs of COLS inputs."""

    def __init__(self, ctx, handle, rows, cols):
        self.ctx, self.h, self.rows, self.cols = ctx, handle, rows, cols

    @classmethod
    def q8_0(cls, ctx, blocks: np.ndarray, rows: int, cols: int):
        h = vp()
        call("exn_weight_q8_0", ctx.h, ptr(np.ascontiguousarray(blocks, dtype=np.uint8)), rows, cols, ctypes.byref(h))
        return cls(ctx, h, rows, cols)

    @classmethod
    def f32(cls, ctx, m: np.ndarray):
        m = np.ascontiguousarray(m, dtype=np.float32)
        h = vp()
        call("exn_weight_f32", ctx.h, ptr(m), m.shape[0], m.shape[1], ctypes.byref(h))
        return cls(ctx, h, m.shape[0], m.shape[1])

    @classmethod
    def bf16(cls, ctx, bits: np.ndarray):
        """A BF16 matrix from its bit patterns (uint16, rows x cols)."""
        b = np.ascontiguousarray(bits, dtype=np.uint16)
        h = vp()
        call("exn_weight_bf16", ctx.h, ptr(b), b.shape[0], b.shape[1], ctypes.byref(h))
        return cls(ctx, h, b.shape[0], b.shape[1])

    @classmethod
    def synth(cls, ctx, seed: int, tensor: int, rows: int, cols: int):
        h = vp()
        call("exn_weight_q8_0_synth", ctx.h, seed, tensor, rows, cols, ctypes.byref(h))
        return cls(ctx, h, rows, cols)

    def pairs(self):
        call("exn_weight_pairs", self.ctx.h, self.h)
        return self

    def resident(self, bf16: bool = True):
        """Keep (or drop) the matrix's resident bf16 expansion, which products then use."""
        call("exn_weight_resident", self.ctx.h, self.h, 1 if bf16 else 0)
        return self

    def free(self):
        # a weight's memory belongs to its context: once that is closed there is nothing to free
        if getattr(self, "h", None) and self.ctx.h:
            call("exn_weight_free", self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# --- the backend trio (src/cuda-dit.lisp) -------------------------------------------------

DIT_PREFIX = "model.diffusion_model."


class Dit:
    """The DiT on the device: weights, scratch and the kept prompt K/V (gdit)."""

    def __init__(self, ctx: Context, layers: int = 32):
        h = vp()
        call("exn_dit_create", ctx.h, layers, ctypes.byref(h))
        self.ctx, self.h, self.layers = ctx, h, layers
        self._keys = {}

    def set(self, name: str, kind: int, data: np.ndarray, dims):
        """One tensor by its GGUF name (with or without the model prefix) and ggml dims."""
        if name.startswith(DIT_PREFIX):
            name = name[len(DIT_PREFIX):]
        d0 = dims[0]
        d1 = dims[1] if len(dims) > 1 else 1
        call("exn_dit_set", self.h, name.encode(), kind, ptr(np.ascontiguousarray(data)), d0, d1)

    def synth(self, seed: int):
        call("exn_dit_synth", self.h, seed)

    def check(self):
        call("exn_dit_check", self.h)

    def resident(self, bf16: bool = True):
        """Block matrices from resident bf16 expansions (the default) or from Q8_0."""
        call("exn_dit_resident", self.h, 1 if bf16 else 0)

    def w8a8(self, on: bool = True):
        """The reference's *int8* products (its default) for every Q8_0 matrix with at least 16
        rows, or (off, this library's default) the bf16 products."""
        call("exn_dit_w8a8", self.h, 1 if on else 0)

    def prefix_key(self, key) -> int:
        """A 64-bit key for a Lisp-style prefix key (EQUAL objects -> one key)."""
        if key is None:
            return 0
        if key not in self._keys:
            self._keys[key] = len(self._keys) + 1
        return self._keys[key]

    def memory(self):
        w, s = c_int64(), c_int64()
        call("exn_dit_memory", self.h, ctypes.byref(w), ctypes.byref(s))
        return w.value, s.value

    PROFILE_CLASSES = ("qkv", "attend", "out", "gate_up", "down", "ln_mod", "qkv_prep", "edge")

    def profile(self, on, classes=None, every=1):
        """Record HIP event pairs around the step's launches: all classes, or those named;
        around every EVERY-th launch of each only."""
        mask = 0
        if on:
            mask = -1 if classes is None else sum(1 << self.PROFILE_CLASSES.index(c) for c in classes)
        call("exn_dit_profile_every", self.h, every)
        call("exn_dit_profile", self.h, mask)

    def profile_read(self):
        """{class: (ms, launches, flops, bytes)} over the recorded launches."""
        out = {}
        for i, name in enumerate(self.PROFILE_CLASSES):
            ms, n, f, b = c_double(), c_int64(), c_double(), c_double()
            call("exn_dit_profile_read", self.h, i, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(f), ctypes.byref(b))
            out[name] = (ms.value, n.value, f.value, b.value)
        return out

    def profile_top(self, k=6):
        """EXN_PROFILE's report (src/tenant.lisp:53-62): the K classes with the most GPU time,
        [(class, ms)] largest first, and the total ms."""
        rows = sorted(((c, v[0]) for c, v in self.profile_read().items() if v[1]), key=lambda r: -r[1])
        return rows[:k], sum(r[1] for r in rows)

    STATS_SLOTS = ("x", "att", "ff", "txt")

    def stats(self, on: bool = True):
        """*dit-trace*'s numbers (exn_dit_stats) for every velocity while on."""
        call("exn_dit_stats", self.h, 1 if on else 0)

    def stats_read(self):
        """The last velocity's (max finite |x|, values not finite), each (layers + 1) x 4: row 0
        before the blocks, row 1 + l after block l; columns STATS_SLOTS."""
        k = (self.layers + 1) * 4
        mx, bad = np.zeros(k, np.float32), np.zeros(k, np.int64)
        call("exn_dit_stats_read", self.h, ptr(mx), ptr(bad), k)
        return mx.reshape(-1, 4), bad.reshape(-1, 4)

    def release(self):
        call("exn_dit_release", self.h)

    def destroy(self):
        if self.h:
            call("exn_dit_destroy", self.h)
            self.h = None


def upload_dit(tensors=None, *, device: int = 0, layers: int = 32, seed: int | None = None, ctx=None) -> Dit:
    """upload-dit (src/cuda-dit.lisp:52-86).  TENSORS: an iterable of
    (name, kind, data, ggml dims) as read from the GGUF (block_q8_0 bytes for
    Q8_0); or SEED: the synthetic weights made on the device.  The model is
    checked against dit-expected (src/weights.lisp:47-61) before return."""
    ctx = ctx or Context(device)
    d = Dit(ctx, layers)
    if seed is not None:
        d.synth(seed)
    for name, kind, data, dims in tensors or ():
        d.set(name, kind, data, dims)
    d.check()
    return d


def dit_velocity(d: Dit, context: np.ndarray, p: int, latent: np.ndarray, h: int, w: int, sigma: float,
                 prefix_key=None, ref=None) -> np.ndarray:
    """dit-velocity (src/cuda-dit.lisp:137-144): CONTEXT (P x 4096 fp32),
    LATENT (64 x H x W fp32, channel-major) -> the velocity, same shape.
    REF = (a, ref_latent, rh, rw): an edit's reference picture."""
    ctxa = np.ascontiguousarray(context, dtype=np.float32).reshape(-1)
    lat = np.ascontiguousarray(latent, dtype=np.float32).reshape(-1)
    if lat.size != 64 * h * w:
        raise ExnError(EINVAL, "latent of %d floats for %d x %d" % (lat.size, h, w))
    v = np.empty((64, h, w), np.float32)
    if ref is not None:
        a, rl, rh, rw = ref
        rl = np.ascontiguousarray(rl, dtype=np.float32).reshape(-1)
        refargs = (a, ptr(rl), rh, rw)
    else:
        refargs = (0, None, 0, 0)
    call("exn_dit_velocity", d.h, ptr(ctxa) if p > 0 else None, p, ptr(lat), h, w, float(sigma),
         d.prefix_key(prefix_key), *refargs, ptr(v))
    return v


def rope_table(p: int, h: int, w: int, ref=None):
    """The library's host-side dit-positions and rope-table (src/host.lisp:19-50), the
    tables a step uploads: P text rows, an H x W image, REF = (a, rh, rw) for an edit's
    reference picture.  Returns (positions: rows x 3 int32, cs: rows x 128 float32,
    the cos and sin of each of the 64 pairs interleaved)."""
    edit = ref is not None
    a, rh, rw = ref if edit else (0, 0, 0)
    rows = p + (rh * rw if edit else 0) + h * w
    pos = np.empty((rows, 3), np.int32)
    cs = np.empty((rows, 128), np.float32)
    call("exn_dit_rope_table", p, h, w, 1 if edit else 0, a, rh, rw, rows, ptr(pos), ptr(cs))
    return pos, cs


def dit_release(d: Dit):
    """dit-release (src/cuda-dit.lisp:99-108)."""
    d.release()


def prompt_key(context: np.ndarray, p: int, ref=None):
    """A prefix key that names the prompt by its content, as generate's key is the prompt
    itself (src/generate.lisp:134): the context rows and, for an edit, the reference
    picture and where it sits.  Two prompts share kept K/V only if these are equal."""
    import hashlib
    hsh = hashlib.sha256(np.ascontiguousarray(context, dtype=np.float32).tobytes())
    if ref is not None:
        a, rl, rh, rw = ref
        hsh.update(np.array([a, rh, rw], np.int64).tobytes())
        hsh.update(np.ascontiguousarray(rl, dtype=np.float32).tobytes())
    return ("prompt", p, hsh.hexdigest())


def generate_latent(d: Dit, context: np.ndarray, p: int, z: np.ndarray, h: int, w: int,
                    sigmas=TURBO_SIGMAS, prefix_key=None, ref=None) -> np.ndarray:
    """generate's Euler loop (src/generate.lisp:133-135) on host arrays:
    z <- z + (s' - s) v, (s' - s) rounded to a single float.  The prompt's K/V are
    kept from the first step under PREFIX_KEY, by default a key made from the
    context (and reference picture) itself (prompt_key)."""
    if prefix_key is None:
        prefix_key = prompt_key(context, p, ref)
    z = np.array(z, dtype=np.float32, copy=True)
    for s, s2 in zip(sigmas[:-1], sigmas[1:]):
        v = dit_velocity(d, context, p, z, h, w, s, prefix_key=prefix_key, ref=ref)
        z = z + np.float32(s2 - s) * v
    return z


# --- the VAE: upload-vae, vae-decode, vae-encode, vae-release (src/cuda-vae.lisp) ----------

class Vae:
    """The decoder and encoder on the device: their tensors and scratch (gvae)."""

    def __init__(self, ctx: Context):
        h = vp()
        call("exn_vae_create", ctx.h, ctypes.byref(h))
        self.ctx, self.h = ctx, h

    def set(self, name: str, kind: int, data: np.ndarray, shape):
        """One tensor by its safetensors name and shape (BF16 bit patterns as uint16, or F32)."""
        dims = (c_int64 * len(shape))(*shape)
        call("exn_vae_set", self.h, name.encode(), kind, ptr(np.ascontiguousarray(data)), dims, len(shape))

    def synth(self, seed: int):
        call("exn_vae_synth", self.h, seed)

    def check(self):
        call("exn_vae_check", self.h)

    def check_encoder(self):
        call("exn_vae_check_encoder", self.h)

    def memory(self):
        w, s = c_int64(), c_int64()
        call("exn_vae_memory", self.h, ctypes.byref(w), ctypes.byref(s))
        return w.value, s.value

    def release(self):
        call("exn_vae_release", self.h)

    def destroy(self):
        if self.h:
            call("exn_vae_destroy", self.h)
            self.h = None


def upload_vae(tensors=None, *, device: int = 0, seed: int | None = None, ctx=None) -> Vae:
    """upload-vae (src/cuda-vae.lisp:15-26): TENSORS an iterable of (name, kind,
    data, shape) as read from the safetensors, or SEED: the synthetic decoder made
    on the device.  Checked against the decoder's tensor list before return."""
    ctx = ctx or Context(device)
    v = Vae(ctx)
    if seed is not None:
        v.synth(seed)
    for name, kind, data, shape in tensors or ():
        v.set(name, kind, data, shape)
    v.check()
    return v


def vae_decode(v: Vae, latent: np.ndarray, h: int, w: int):
    """vae-decode (src/cuda-vae.lisp:94-136): LATENT (64 x H x W floats,
    channel-major, denormalized) -> (the picture as 16H x 16W x 4 floats, RGBA
    in -1..1, channels last; its height; its width)."""
    lat = np.ascontiguousarray(latent, dtype=np.float32).reshape(-1)
    if lat.size != 64 * h * w:
        raise ExnError(EINVAL, "latent of %d floats for %d x %d" % (lat.size, h, w))
    px = np.empty((16 * h, 16 * w, 4), np.float32)
    call("exn_vae_decode", v.h, ptr(lat), h, w, ptr(px))
    return px, 16 * h, 16 * w


def vae_encode(v: Vae, px: np.ndarray, h: int, w: int) -> np.ndarray:
    """vae-encode (src/cuda-vae.lisp:138-190): PX (H x W x 4 floats, RGBA in -1..1, rows of
    W pixels; H and W multiples of 16) -> the latent's mean, 64 x H/16 x W/16 floats
    channel-major, as vae_decode takes it (denormalized)."""
    x = np.ascontiguousarray(px, dtype=np.float32).reshape(-1)
    if x.size != h * w * 4:
        raise ExnError(EINVAL, "picture of %d floats for %d x %d RGBA" % (x.size, h, w))
    z = np.empty((64, h // 16, w // 16), np.float32)
    call("exn_vae_encode", v.h, ptr(x), h, w, ptr(z))
    return z


def vae_release(v: Vae):
    """vae-release (src/cuda-vae.lisp:28-33): the scratch freed."""
    v.release()


# --- the vision tower: load-vision, vision-encode, vision-release (src/cuda-vision.lisp) -----

VISION_WIDTH, VISION_OUT = 1152, 4096


class Vision:
    """Qwen3-VL's vision tower on the device: its tensors and scratch (q3vision)."""

    def __init__(self, ctx: Context):
        h = vp()
        call("exn_vision_create", ctx.h, ctypes.byref(h))
        self.ctx, self.h = ctx, h

    def set(self, name: str, kind: int, data: np.ndarray, shape):
        """One tensor by its GGUF name and row-major shape (F16 / BF16 bit patterns as uint16, or F32)."""
        dims = (c_int64 * len(shape))(*shape)
        call("exn_vision_set", self.h, name.encode(), kind, ptr(np.ascontiguousarray(data)), dims, len(shape))

    def synth(self, seed: int):
        call("exn_vision_synth", self.h, seed)

    def check(self):
        call("exn_vision_check", self.h)

    def trace(self, on: bool):
        call("exn_vision_trace", self.h, 1 if on else 0)

    def traced(self, which: int, n: int):
        """After a traced encode of N patches: the rows after the embedding (0) or block 0 (1)."""
        out = np.empty((n, VISION_WIDTH), np.float32)
        call("exn_vision_traced", self.h, which, ptr(out))
        return out

    def memory(self):
        w, s = c_int64(), c_int64()
        call("exn_vision_memory", self.h, ctypes.byref(w), ctypes.byref(s))
        return w.value, s.value

    def release(self):
        call("exn_vision_release", self.h)

    def destroy(self):
        if self.h:
            call("exn_vision_destroy", self.h)
            self.h = None


def load_vision(tensors=None, *, device: int = 0, seed: int | None = None, ctx=None) -> Vision:
    """load-vision (src/cuda-vision.lisp:15-30): TENSORS an iterable of (name, kind,
    data, shape) as read from the mmproj GGUF, or SEED: the synthetic tower made on
    the device.  Checked against the tower's tensor list before return."""
    ctx = ctx or Context(device)
    v = Vision(ctx)
    if seed is not None:
        v.synth(seed)
    for name, kind, data, shape in tensors or ():
        v.set(name, kind, data, shape)
    v.check()
    return v


def vision_encode(v: Vision, px: np.ndarray, h: int, w: int):
    """vision-encode (src/cuda-vision.lisp:34-101): PX (H x W x 4 floats, RGBA in
    -1..1; H, W multiples of 32) -> (merged M x 4096, deepstack 3 x M x 4096, M),
    M = H W / 1024, rows in merge-block order."""
    p = np.ascontiguousarray(px, dtype=np.float32).reshape(-1)
    if p.size != h * w * 4:
        raise ExnError(EINVAL, "picture of %d floats for %d x %d RGBA" % (p.size, h, w))
    m = (h // 32) * (w // 32)
    merged = np.empty((m, VISION_OUT), np.float32)
    deep = np.empty((3, m, VISION_OUT), np.float32)
    call("exn_vision_encode", v.h, ptr(p), h, w, ptr(merged), ptr(deep))
    return merged, deep, m


def vision_release(v: Vision):
    """vision-release (src/cuda-vision.lisp:103-107): the scratch freed."""
    v.release()


# --- the prompt encoder: load-encoder, encoder-states (src/encoder.lisp) -------------------

ENC_ROPE_BASE = 5e6


class Encoder:
    """Qwen3-VL-8B's text model on the device (illatio's model, for encoder-states)."""

    def __init__(self, ctx: Context, layers: int = 36, rope_base: float = ENC_ROPE_BASE):
        h = vp()
        call("exn_enc_create", ctx.h, layers, rope_base, ctypes.byref(h))
        self.ctx, self.h, self.layers = ctx, h, layers

    def set(self, name: str, kind: int, data: np.ndarray, d0: int, d1: int):
        """One tensor by its GGUF name and ggml dims (Q8_0 block records as uint8, or F32)."""
        call("exn_enc_set", self.h, name.encode(), kind, ptr(np.ascontiguousarray(data)), d0, d1)

    def synth(self, seed: int, vocab: int = 8192):
        call("exn_enc_synth", self.h, seed, vocab)

    def check(self):
        call("exn_enc_check", self.h)

    def resident(self, on: bool):
        """The products from resident bf16 expansions (the default) or from Q8_0 alone."""
        call("exn_enc_resident", self.h, 1 if on else 0)

    def memory(self):
        w, s = c_int64(), c_int64()
        call("exn_enc_memory", self.h, ctypes.byref(w), ctypes.byref(s))
        return w.value, s.value

    def release(self):
        call("exn_enc_release", self.h)

    def destroy(self):
        if self.h:
            call("exn_enc_destroy", self.h)
            self.h = None


def load_encoder(tensors=None, *, device: int = 0, layers: int = 36, seed: int | None = None, vocab: int = 8192,
                 ctx=None) -> Encoder:
    """load-encoder (src/encoder.lisp:41-48): TENSORS an iterable of (name, kind, data, d0,
    d1) as read from te-q8_0.gguf, or SEED: the synthetic model made on the device."""
    ctx = ctx or Context(device)
    e = Encoder(ctx, layers)
    if seed is not None:
        e.synth(seed, vocab)
    for name, kind, data, d0, d1 in tensors or ():
        e.set(name, kind, data, d0, d1)
    e.check()
    return e


def encoder_states(e: Encoder, ids, pos=None, picture=None):
    """encoder-states (src/encoder.lisp:143-183): every token's state after the last block,
    before the final norm, (n, 4096).  POS: (n, 3) (t, h, w) positions or None (text 0..n-1);
    PICTURE: (a0, merged (m, 4096), deep (3, m, 4096) or None) -- the picture's rows."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n = len(ids)
    p = None if pos is None else np.ascontiguousarray(pos, dtype=np.int32).reshape(n, 3)
    out = np.empty((n, WIDTH), np.float32)
    if picture is None:
        call("exn_enc_states", e.h, ptr(ids), n, None if p is None else ptr(p), 0, 0, None, None, ptr(out))
    else:
        a0, merged, deep = picture
        mg = np.ascontiguousarray(merged, dtype=np.float32)
        dp = None if deep is None else np.ascontiguousarray(deep, dtype=np.float32)
        call("exn_enc_states", e.h, ptr(ids), n, None if p is None else ptr(p), a0, len(mg), ptr(mg),
             None if dp is None else ptr(dp), ptr(out))
    return out


def enc_rope_table(n: int, pos=None, base: float = ENC_ROPE_BASE):
    """mrope-table (src/encoder.lisp:26-39) as the library computes it (host only): (n, 128),
    cos and sin of pair j at columns 2j, 2j + 1."""
    cs = np.empty((n, 128), np.float32)
    p = None if pos is None else np.ascontiguousarray(pos, dtype=np.int32).reshape(n, 3)
    call("exn_enc_rope_table", None if p is None else ptr(p), n, base, ptr(cs))
    return cs
