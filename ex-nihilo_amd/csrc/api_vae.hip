// api_vae.hip -- the VAE decoder and encoder (src/cuda-vae.lisp): weights and drivers.
#include "api_host.h"

// --- the VAE decoder: upload-vae, vae-decode, vae-release (src/cuda-vae.lisp) ----------

namespace {

struct VStage {
  int in, out;
  bool up, tup;
};
// (in, out, spatial up, temporal up), deepest first: src/weights.lisp:65-67
const VStage kVaeStages[5] = {{1152, 1152, true, true}, {1152, 1152, true, true}, {1152, 576, true, true},
                              {576, 288, true, false},  {288, 144, false, false}};
const int kVaeZ = 64, kVaeOut = 4;

// src/weights.lisp:69-98 (vae-expected), the video-only time_conv tensors left out
std::vector<VExpect> vae_expected() {
  std::vector<VExpect> r;
  const int top = kVaeStages[0].in;
  auto add = [&](const std::string& n, std::vector<int64_t> s) { r.push_back(VExpect{n, s}); };
  auto conv = [&](const std::string& n, int64_t o, int64_t i, int64_t k, bool frames) {
    if (frames) add(n + ".weight", {o, i, 1, k, k});
    else add(n + ".weight", {o, i, k, k});
    add(n + ".bias", {o});
  };
  auto res = [&](const std::string& p, int i, int o) {
    add(p + ".residual.0.gamma", {i, 1, 1, 1});
    conv(p + ".residual.2", o, i, 3, true);
    add(p + ".residual.3.gamma", {o, 1, 1, 1});
    conv(p + ".residual.6", o, o, 3, true);
    if (i != o) conv(p + ".shortcut", o, i, 1, true);
  };
  conv("conv2", kVaeZ, kVaeZ, 1, true);
  conv("decoder.conv1", top, kVaeZ, 3, true);
  res("decoder.middle.0", top, top);
  add("decoder.middle.1.norm.gamma", {top, 1, 1});
  conv("decoder.middle.1.to_qkv", 3 * top, top, 1, false);
  conv("decoder.middle.1.proj", top, top, 1, false);
  res("decoder.middle.2", top, top);
  char p[96];
  for (int s = 0; s < 5; ++s) {
    for (int j = 0; j < 3; ++j) {
      snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.%d", s, j);
      res(p, j == 0 ? kVaeStages[s].in : kVaeStages[s].out, kVaeStages[s].out);
    }
    if (kVaeStages[s].up) {
      snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.3.resample.1", s);
      conv(p, kVaeStages[s].out, kVaeStages[s].out, 3, false);
    }
  }
  add("decoder.head.0.gamma", {kVaeStages[4].out, 1, 1, 1});
  conv("decoder.head.2", kVaeOut, kVaeStages[4].out, 3, true);
  return r;
}

// the encoder (a picture to a latent): (in, out, spatial down, temporal down), the picture's
// end first: src/weights.lisp:100-102
const VStage kVaeEncStages[5] = {{96, 96, true, false}, {96, 192, true, true}, {192, 384, true, true},
                                 {384, 768, true, true}, {768, 768, false, false}};
const int kVaeIn = 4;

// src/weights.lisp:104-134 (vae-encoder-expected), the video-only time_conv tensors left out
std::vector<VExpect> vae_encoder_expected() {
  std::vector<VExpect> r;
  const int top = kVaeEncStages[4].out;
  auto add = [&](const std::string& n, std::vector<int64_t> s) { r.push_back(VExpect{n, s}); };
  auto conv = [&](const std::string& n, int64_t o, int64_t i, int64_t k, bool frames) {
    if (frames) add(n + ".weight", {o, i, 1, k, k});
    else add(n + ".weight", {o, i, k, k});
    add(n + ".bias", {o});
  };
  auto res = [&](const std::string& p, int i, int o) {
    add(p + ".residual.0.gamma", {i, 1, 1, 1});
    conv(p + ".residual.2", o, i, 3, true);
    add(p + ".residual.3.gamma", {o, 1, 1, 1});
    conv(p + ".residual.6", o, o, 3, true);
    if (i != o) conv(p + ".shortcut", o, i, 1, true);
  };
  conv("encoder.conv1", kVaeEncStages[0].in, kVaeIn, 3, true);
  char p[96];
  for (int s = 0; s < 5; ++s) {
    const VStage& st = kVaeEncStages[s];
    for (int j = 0; j < 2; ++j) {
      snprintf(p, sizeof p, "encoder.downsamples.%d.downsamples.%d", s, j);
      res(p, j == 0 ? st.in : st.out, st.out);
    }
    if (st.up) {
      snprintf(p, sizeof p, "encoder.downsamples.%d.downsamples.2.resample.1", s);
      conv(p, st.out, st.out, 3, false);
    }
  }
  res("encoder.middle.0", top, top);
  add("encoder.middle.1.norm.gamma", {top, 1, 1});
  conv("encoder.middle.1.to_qkv", 3 * top, top, 1, false);
  conv("encoder.middle.1.proj", top, top, 1, false);
  res("encoder.middle.2", top, top);
  add("encoder.head.0.gamma", {top, 1, 1, 1});
  conv("encoder.head.2", 2 * kVaeZ, top, 3, true);
  conv("conv1", 2 * kVaeZ, 2 * kVaeZ, 1, true);
  return r;
}

// a decoder tensor on the device: a convolution's weights as bf16 rows of (tap, channel), K
// padded with zeros to kp (a multiple of 64); anything else as fp32
struct VT {
  void* p = nullptr;
  bool conv = false;
  int64_t o = 0, n = 0;
  int ci = 0, taps = 0, kp = 0;
};

bool is_conv_weight(const VExpect& e) {
  return e.shape.size() >= 4 && e.name.size() > 7 && e.name.compare(e.name.size() - 7, 7, ".weight") == 0;
}

}  // namespace

struct exn_vae {
  exn_ctx* ctx = nullptr;
  std::vector<VExpect> expect;   // the decoder's tensors, then (from n_dec on) the encoder's
  size_t n_dec = 0;
  std::map<std::string, VT> t;
  std::map<std::string, Buf> bufs;
  float* part = nullptr;   // split-K partial sums of the small convolutions (a decode's scratch)
  int64_t part_cap = 0;
  int wide_only = 0;       // exn_vae_tiles: 256-pixel tiles only
};

// split-K scratch: a split convolution has S x tiles <= 256 workgroups of 256 pixels x at most
// 288 channels, so 256 x 256 x 288 floats hold any of its partials
static const int64_t kVaePartCap = (int64_t)256 * 256 * 288;

static int vae_buf(exn_vae* v, const char* key, size_t bytes, void** out) {
  Buf& b = v->bufs[key];
  if (b.bytes < bytes) {
    HIPCHK(hipStreamSynchronize(v->ctx->stream));
    dev_free(b.p);
    b.p = nullptr;
    b.bytes = 0;
    TRY(dev_alloc(&b.p, bytes));
    b.bytes = bytes;
  }
  *out = b.p;
  return EXN_OK;
}

static const VExpect* vae_find(const exn_vae* v, const char* name, int* index) {
  for (size_t i = 0; i < v->expect.size(); ++i)
    if (v->expect[i].name == name) {
      if (index) *index = (int)i;
      return &v->expect[i];
    }
  return nullptr;
}

// fp32 values of tensor E (device, file order) -> its device form
static int vae_store(exn_vae* v, const VExpect& e, const float* f32) {
  VT& t = v->t[e.name];
  int64_t n = 1;
  for (auto d : e.shape) n *= d;
  if (is_conv_weight(e)) {
    const int64_t o = e.shape[0];
    const int ci = (int)e.shape[1], taps = (int)(e.shape.back() * e.shape[e.shape.size() - 2]);
    const int kp = (taps * ci + 63) / 64 * 64;
    if (!t.p) TRY(dev_alloc(&t.p, (size_t)o * kp * 2));
    t.conv = true;
    t.o = o;
    t.ci = ci;
    t.taps = taps;
    t.kp = kp;
    t.n = n;
    HIPCHK(vae_pack_conv(v->ctx->stream, o, ci, taps, kp, f32, (uint16_t*)t.p));
  } else {
    if (!t.p) TRY(dev_alloc(&t.p, (size_t)n * 4));
    t.conv = false;
    t.n = n;
    HIPCHK(hipMemcpyAsync(t.p, f32, (size_t)n * 4, hipMemcpyDeviceToDevice, v->ctx->stream));
  }
  return EXN_OK;
}

static const VT* vae_t(const exn_vae* v, const std::string& name) {
  auto it = v->t.find(name);
  return it == v->t.end() ? nullptr : &it->second;
}


int exn_vae_create(exn_ctx* ctx, exn_vae** out) {
  TRY(use(ctx));
  if (!out) FAIL(EXN_EINVAL, "null output");
  exn_vae* v = new exn_vae();
  v->ctx = ctx;
  v->expect = vae_expected();
  v->n_dec = v->expect.size();
  for (auto& e : vae_encoder_expected()) v->expect.push_back(e);
  *out = v;
  return EXN_OK;
}

int exn_vae_release(exn_vae* v) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  for (auto& kv : v->bufs) dev_free(kv.second.p);
  v->bufs.clear();
  v->part = nullptr;
  v->part_cap = 0;
  return EXN_OK;
}

int exn_vae_destroy(exn_vae* v) {
  if (!v) return EXN_OK;
  TRY(exn_vae_release(v));
  for (auto& kv : v->t) dev_free(kv.second.p);
  delete v;
  return EXN_OK;
}

int exn_vae_set(exn_vae* v, const char* name, int kind, const void* data, const int64_t* dims, int ndims) {
  if (!v || !name || !data || !dims) FAIL(EXN_EINVAL, "vae set: null argument");
  TRY(use(v->ctx));
  const VExpect* e = vae_find(v, name, nullptr);
  if (!e) FAIL(EXN_EINVAL, "vae set: no decoder or encoder tensor %s", name);
  if (kind != EXN_F32 && kind != EXN_BF16) FAIL(EXN_EINVAL, "vae set %s: kind %d (F32 or BF16 only)", name, kind);
  bool same = ndims == (int)e->shape.size();
  for (int i = 0; same && i < ndims; ++i) same = dims[i] == e->shape[i];
  if (!same) {
    std::string want;
    for (auto d : e->shape) want += (want.empty() ? "" : " ") + std::to_string(d);
    FAIL(EXN_EINVAL, "vae set %s: shape is not (%s)", name, want.c_str());
  }
  int64_t n = 1;
  for (auto d : e->shape) n *= d;
  std::vector<float> f((size_t)n);
  if (kind == EXN_F32) {
    memcpy(f.data(), data, (size_t)n * 4);
  } else {
    const uint16_t* b = (const uint16_t*)data;
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)b[i] << 16;
      memcpy(&f[(size_t)i], &u, 4);
    }
  }
  float* tmp = nullptr;
  TRY(ctx_tmp(v->ctx, (size_t)n * 4, (void**)&tmp));
  HIPCHK(hipMemcpyAsync(tmp, f.data(), (size_t)n * 4, hipMemcpyHostToDevice, v->ctx->stream));
  TRY(vae_store(v, *e, tmp));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

// every decoder and encoder tensor from the counter generator (the oracle's SynthVae): value =
// bf16(base + scale * normal), normal i of key(seed, 4000 + the tensor's index), the encoder's
// after the decoder's
int exn_vae_synth(exn_vae* v, uint64_t seed) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  for (size_t i = 0; i < v->expect.size(); ++i) {
    const VExpect& e = v->expect[i];
    int64_t n = 1;
    for (auto d : e.shape) n *= d;
    const std::string& nm = e.name;
    auto ends = [&](const char* s) { return nm.size() >= strlen(s) && nm.compare(nm.size() - strlen(s), strlen(s), s) == 0; };
    double base = 0.0, scale;
    if (ends(".gamma")) {
      base = 1.0;
      scale = 0.1;
    } else if (ends(".bias")) {
      scale = 0.02;
    } else {
      int64_t fan = 1;
      for (size_t k = 1; k < e.shape.size(); ++k) fan *= e.shape[k];
      double g = 1.0;
      if (nm.find(".residual.6.") != std::string::npos || nm.rfind("decoder.middle.1.proj", 0) == 0 ||
          nm.rfind("encoder.middle.1.proj", 0) == 0)
        g = 0.5;
      if (nm.rfind("decoder.head.2", 0) == 0) g = 1.2;
      scale = g / sqrt((double)fan);
    }
    float* tmp = nullptr;
    TRY(ctx_tmp(v->ctx, (size_t)n * 4, (void**)&tmp));
    HIPCHK(synth_normal(v->ctx->stream, gen_key(seed, 4000 + i), n, (float)base, (float)scale, base != 0.0, tmp));
    if (!is_conv_weight(e)) HIPCHK(vae_round_bf16(v->ctx->stream, n, tmp));
    TRY(vae_store(v, e, tmp));
  }
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

int exn_vae_check(exn_vae* v) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  for (size_t i = 0; i < v->n_dec; ++i)
    if (!vae_t(v, v->expect[i].name)) FAIL(EXN_ESTATE, "decoder: missing %s", v->expect[i].name.c_str());
  return EXN_OK;
}

int exn_vae_tiles(exn_vae* v, int small) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  v->wide_only = small ? 0 : 1;
  return EXN_OK;
}

int exn_vae_check_encoder(exn_vae* v) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  for (size_t i = v->n_dec; i < v->expect.size(); ++i)
    if (!vae_t(v, v->expect[i].name)) FAIL(EXN_ESTATE, "encoder: missing %s", v->expect[i].name.c_str());
  return EXN_OK;
}

int exn_vae_memory(exn_vae* v, int64_t* weights, int64_t* scratch) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  int64_t w = 0, s = 0;
  for (auto& kv : v->t) w += kv.second.conv ? kv.second.o * kv.second.kp * 2 : kv.second.n * 4;
  for (auto& kv : v->bufs) s += (int64_t)kv.second.bytes;
  if (weights) *weights = w;
  if (scratch) *scratch = s;
  return EXN_OK;
}


// one convolution of the decoder: NAME's weights and bias over X (bf16 pixel rows, h x w of the
// output), RES added when given
static int vae_conv_named(exn_vae* v, const std::string& name, int up, int out, const uint16_t* x, const float* res,
                          void* y, int h, int w, const float* keep = nullptr, int kcin = 0, int ft = 0,
                          uint16_t* y2 = nullptr, const float* gamma = nullptr, uint16_t* yr = nullptr) {
  const VT* wt = vae_t(v, name + ".weight");
  const VT* b = vae_t(v, name + ".bias");
  if (!wt || !b) FAIL(EXN_ESTATE, "decoder: missing %s", name.c_str());
  const VaeEpi ep{res, keep, kcin, ft, y2, v->part, v->part_cap, gamma, yr, v->wide_only};
  HIPCHK(vae_conv(v->ctx->stream, wt->taps, up, out, x, (const uint16_t*)wt->p, (const float*)b->p, ep, y, h, w,
                  wt->ci, (int)wt->o, wt->kp));
  return EXN_OK;
}

static const float* vae_vec(const exn_vae* v, const std::string& name) {
  const VT* t = vae_t(v, name);
  return t ? (const float*)t->p : nullptr;
}

// a width whose output channels one convolution tile holds: the norm can ride in its store
static bool vae_one_tile(int c) { return c == 96 || c == 144 || c == 192 || c == 288; }

// OUT = conv(silu(norm(conv(silu(norm(X)))))) + (X, or its 1 x 1 shortcut): src/cuda-vae.lisp's
// resblock, inspect/ref_vae.py:59-65.  OUT fp32, or bf16 when OUT_BF16 (a product's input next);
// XB: X in bf16 when the caller has it (the shortcut's input), else cast here; XRS: silu(norm(X))
// in bf16 when the step that wrote X made it, else made here.  At a one-tile width the inner
// norm rides in the first convolution's store, and with GNEXT the second leaves
// silu(norm(OUT) x GNEXT) in YNEXT for the next block or the head (*MADE then true).  T1, T3, U
// bf16 scratch, T2 fp32 scratch; YNEXT may be T1.
static int vae_resblock(exn_vae* v, const std::string& p, const float* x, const uint16_t* xb, const uint16_t* xrs,
                        void* out, bool out_bf16, int i, int o, int h, int w, uint16_t* t1, float* t2, uint16_t* u,
                        uint16_t* t3, const float* gnext = nullptr, uint16_t* ynext = nullptr, bool* made = nullptr) {
  hipStream_t s = v->ctx->stream;
  const int64_t n = (int64_t)h * w;
  const float* g0 = vae_vec(v, p + ".residual.0.gamma");
  const float* g3 = vae_vec(v, p + ".residual.3.gamma");
  if (!g0 || !g3) FAIL(EXN_ESTATE, "decoder: missing %s gammas", p.c_str());
  if (made) *made = false;
  if (!xrs) {
    HIPCHK(vae_rms_silu(s, n, i, x, g0, t1, 1));
    xrs = t1;
  }
  const bool one = vae_one_tile(o);
  if (one) {
    TRY(vae_conv_named(v, p + ".residual.2", 0, VAE_RMS, xrs, nullptr, nullptr, h, w, nullptr, 0, 0, nullptr, g3, t3));
  } else {
    TRY(vae_conv_named(v, p + ".residual.2", 0, VAE_F32, xrs, nullptr, t2, h, w));
    HIPCHK(vae_rms_silu(s, n, o, t2, g3, t3, 1));
  }
  const float* res = x;
  if (i != o) {
    if (!xb) {
      HIPCHK(f32_to_bf16(s, x, u, n * i));
      xb = u;
    }
    TRY(vae_conv_named(v, p + ".shortcut", 0, VAE_F32, xb, nullptr, t2, h, w));
    res = t2;
  }
  if (one && gnext && ynext && !out_bf16) {
    TRY(vae_conv_named(v, p + ".residual.6", 0, VAE_F32, t3, res, out, h, w, nullptr, 0, 0, nullptr, gnext, ynext));
    if (made) *made = true;
    return EXN_OK;
  }
  return vae_conv_named(v, p + ".residual.6", 0, out_bf16 ? VAE_BF16 : VAE_F32, t3, res, out, h, w);
}

// one head over the n pixels, c wide (inspect/ref_vae.py:68-76): OUT = proj(softmax(q k^T /
// sqrt(c)) v) + X
static int vae_attention(exn_vae* v, const std::string& p, const float* x, float* out, int h, int w, int c,
                         uint16_t* t1) {
  hipStream_t s = v->ctx->stream;
  const int64_t n = (int64_t)h * w, np = (n + 63) / 64 * 64;
  float *qkv, *S;
  uint16_t *q, *k, *vt, *P, *ao;
  TRY(vae_buf(v, "qkv", (size_t)n * 3 * c * 4, (void**)&qkv));
  TRY(vae_buf(v, "q", (size_t)n * c * 2, (void**)&q));
  TRY(vae_buf(v, "k", (size_t)n * c * 2, (void**)&k));
  TRY(vae_buf(v, "vt", (size_t)c * np * 2, (void**)&vt));
  TRY(vae_buf(v, "S", (size_t)n * np * 4, (void**)&S));
  TRY(vae_buf(v, "P", (size_t)n * np * 2, (void**)&P));
  TRY(vae_buf(v, "ao", (size_t)n * c * 2, (void**)&ao));
  const float* g = vae_vec(v, p + ".norm.gamma");
  if (!g) FAIL(EXN_ESTATE, "decoder: missing %s.norm.gamma", p.c_str());
  HIPCHK(vae_rms_silu(s, n, c, x, g, t1, 0));
  TRY(vae_conv_named(v, p + ".to_qkv", 0, 0, t1, nullptr, qkv, h, w));
  HIPCHK(vae_split_qkv(s, n, np, c, qkv, q, k, vt));
  EpiArgs ea{};
  ea.y = S;
  ea.ldy = np;
  HIPCHK(gemm_wbf16(s, q, c, k, n, n, c, EPI_F32, ea));
  HIPCHK(vae_softmax_rows(s, (int)n, (int)np, (float)(1.0 / sqrt((double)c)), S, P));
  ea.y = ao;
  ea.ldy = c;
  HIPCHK(gemm_wbf16(s, P, np, vt, n, c, np, EPI_BF16, ea));
  return vae_conv_named(v, p + ".proj", 0, 0, ao, x, out, h, w);
}

static int vae_decode(exn_vae* v, const float* latent, int h, int w, float* rgba) {
  hipStream_t s = v->ctx->stream;
  const int top = kVaeStages[0].in;
  // the most values any picture of the decode holds (pixels x channels), and the widest
  int64_t most = (int64_t)h * w * top;
  {
    int64_t hh = h, ww = w;
    for (auto& st : kVaeStages) {
      most = std::max(most, hh * ww * std::max(st.in, st.out));
      if (st.up) {
        hh *= 2;
        ww *= 2;
      }
      most = std::max(most, hh * ww * st.out);
    }
  }
  float *A, *B, *C, *t2;
  uint16_t *t1, *u, *xs;
  TRY(vae_buf(v, "A", (size_t)most * 4, (void**)&A));
  TRY(vae_buf(v, "B", (size_t)most * 4, (void**)&B));
  TRY(vae_buf(v, "C", (size_t)most * 4, (void**)&C));
  TRY(vae_buf(v, "t2", (size_t)most * 4, (void**)&t2));
  TRY(vae_buf(v, "t1", (size_t)most * 2, (void**)&t1));
  TRY(vae_buf(v, "u", (size_t)most * 2, (void**)&u));
  TRY(vae_buf(v, "xs", (size_t)most * 2, (void**)&xs));
  uint16_t* t3;
  TRY(vae_buf(v, "t3", (size_t)most * 2, (void**)&t3));
  TRY(vae_buf(v, "part", (size_t)kVaePartCap * 4, (void**)&v->part));
  v->part_cap = kVaePartCap;
  int hh = h, ww = w;
  const int64_t n0 = (int64_t)h * w;
  // the latent's pixels, conv2 (1 x 1), decoder.conv1 (3 x 3 to the top width)
  HIPCHK(vae_latent_pixels(s, n0, kVaeZ, latent, t1));
  TRY(vae_conv_named(v, "conv2", 0, VAE_BF16, t1, nullptr, u, hh, ww));
  TRY(vae_conv_named(v, "decoder.conv1", 0, VAE_F32, u, nullptr, A, hh, ww));
  TRY(vae_resblock(v, "decoder.middle.0", A, nullptr, nullptr, B, false, top, top, hh, ww, t1, t2, u, t3));
  TRY(vae_attention(v, "decoder.middle.1", B, C, hh, ww, top, t1));
  TRY(vae_resblock(v, "decoder.middle.2", C, nullptr, nullptr, A, false, top, top, hh, ww, t1, t2, u, t3));
  const float* ghead = vae_vec(v, "decoder.head.0.gamma");
  if (!ghead) FAIL(EXN_ESTATE, "decoder: missing decoder.head.0.gamma");
  // the residual.0 gamma of block j of stage si (the norm its input takes)
  auto g0_of = [&](int si, int j) {
    char q[96];
    snprintf(q, sizeof q, "decoder.upsamples.%d.upsamples.%d.residual.0.gamma", si, j);
    return vae_vec(v, q);
  };
  char p[96];
  const uint16_t* a_bf16 = nullptr;   // A in bf16, when the step that wrote A kept a copy
  const uint16_t* a_rs = nullptr;     // silu(norm(A)) for the stage's first block, when made (in t1)
  bool made = false;
  for (int si = 0; si < 5; ++si) {
    const VStage& st = kVaeStages[si];
    // A holds the stage's input, kept for DupUp3D; the last block of an upsampling stage
    // writes bf16 straight for the resample convolution.  At one-tile widths each block's
    // second convolution leaves the next block's (or the head's) normed input in t1.
    snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.0", si);
    TRY(vae_resblock(v, p, A, a_bf16, a_rs, B, false, st.in, st.out, hh, ww, t1, t2, u, t3, g0_of(si, 1), t1, &made));
    const uint16_t* b_rs = made ? t1 : nullptr;
    snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.1", si);
    TRY(vae_resblock(v, p, B, nullptr, b_rs, C, false, st.out, st.out, hh, ww, t1, t2, u, t3, g0_of(si, 2), t1,
                     &made));
    const uint16_t* c_rs = made ? t1 : nullptr;
    snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.2", si);
    if (st.up) {
      TRY(vae_resblock(v, p, C, nullptr, c_rs, u, true, st.out, st.out, hh, ww, t1, t2, u, t3));
      // nearest x2 folded into the convolution's loads, DupUp3D of the stage's input into its
      // store, a bf16 copy when the next stage's first block takes a 1 x 1 shortcut of it, and
      // that block's normed input when the width is one tile
      const bool copy = si + 1 < 5 && kVaeStages[si + 1].in != kVaeStages[si + 1].out;
      const bool norm = si + 1 < 5 && vae_one_tile(st.out);
      // the fp32 output is dead when the next block has both bf16 inputs (its norm and its
      // shortcut's), adds the shortcut (in != out), and its stage keeps nothing for a DupUp3D
      const bool dead = copy && norm && !kVaeStages[si + 1].up;
      snprintf(p, sizeof p, "decoder.upsamples.%d.upsamples.3.resample.1", si);
      TRY(vae_conv_named(v, p, 1, VAE_DUPUP, u, nullptr, dead ? nullptr : C, 2 * hh, 2 * ww, A, st.in,
                         st.tup ? 2 : 1, copy ? xs : nullptr, norm ? g0_of(si + 1, 0) : nullptr, norm ? t1 : nullptr));
      a_bf16 = copy ? xs : nullptr;
      a_rs = norm ? t1 : nullptr;
      hh *= 2;
      ww *= 2;
      std::swap(A, C);
    } else {
      TRY(vae_resblock(v, p, C, nullptr, c_rs, B, false, st.out, st.out, hh, ww, t1, t2, u, t3,
                       si + 1 < 5 ? g0_of(si + 1, 0) : ghead, t1, &made));
      a_bf16 = nullptr;
      a_rs = made ? t1 : nullptr;
      std::swap(A, B);
    }
  }
  // the head: norm, SiLU, 3 x 3 to RGBA, clamped
  if (!a_rs) {
    HIPCHK(vae_rms_silu(s, (int64_t)hh * ww, kVaeStages[4].out, A, ghead, t1, 1));
    a_rs = t1;
  }
  return vae_conv_named(v, "decoder.head.2", 0, VAE_CLAMP, a_rs, nullptr, rgba, hh, ww);
}

// the encoder (src/cuda-vae.lisp:138-190): RGBA (h x w x 4 fp32, -1 .. 1) -> the latent's mean
// (64 x h/16 x w/16 fp32, channel-major, as the decoder takes it).  The first convolution runs
// as a 1 x 1 product over each pixel's 3 x 3 RGBA neighbourhood (36 values, padded to 64); a
// stage is two residual blocks, then a stride-2 convolution plus AvgDown3D of the stage's input
// (or, without the spatial step, the input added); the middle; the head's norm, SiLU, 3 x 3 to
// the mean and log-variance and conv1 (1 x 1), of which the mean is kept.
static int vae_encode(exn_vae* v, const float* rgba, int h, int w, float* latent) {
  hipStream_t s = v->ctx->stream;
  const int top = kVaeEncStages[4].out;
  int64_t most = (int64_t)h * w * kVaeEncStages[0].in;
  {
    int64_t hh = h, ww = w;
    for (auto& st : kVaeEncStages) {
      most = std::max(most, hh * ww * std::max(st.in, st.out));
      if (st.up) {
        hh /= 2;
        ww /= 2;
      }
    }
  }
  float *A, *B, *C, *t2;
  uint16_t *t1, *u, *t3;
  TRY(vae_buf(v, "A", (size_t)most * 4, (void**)&A));
  TRY(vae_buf(v, "B", (size_t)most * 4, (void**)&B));
  TRY(vae_buf(v, "C", (size_t)most * 4, (void**)&C));
  TRY(vae_buf(v, "t2", (size_t)most * 4, (void**)&t2));
  TRY(vae_buf(v, "t1", (size_t)most * 2, (void**)&t1));
  TRY(vae_buf(v, "u", (size_t)most * 2, (void**)&u));
  TRY(vae_buf(v, "t3", (size_t)most * 2, (void**)&t3));
  TRY(vae_buf(v, "part", (size_t)kVaePartCap * 4, (void**)&v->part));
  v->part_cap = kVaePartCap;
  int hh = h, ww = w;
  // the residual.0 gamma of block j of stage si (the norm its input takes)
  auto g0_of = [&](int si, int j) {
    char q[96];
    snprintf(q, sizeof q, "encoder.downsamples.%d.downsamples.%d.residual.0.gamma", si, j);
    return vae_vec(v, q);
  };
  // encoder.conv1: RGBA neighbourhoods (u, 64 bf16 a pixel) x the weights' (tap, channel) rows;
  // at a one-tile width it leaves the first block's normed input in t1 too
  const uint16_t* a_rs = nullptr;
  {
    const VT* wt = vae_t(v, "encoder.conv1.weight");
    const VT* b = vae_t(v, "encoder.conv1.bias");
    if (!wt || !b || wt->kp != 64) FAIL(EXN_ESTATE, "encoder: encoder.conv1 not loaded");
    HIPCHK(vae_rgba_taps(s, h, w, rgba, u));
    const bool one = vae_one_tile((int)wt->o) && g0_of(0, 0);
    const VaeEpi ep{nullptr, nullptr, 0, 0, nullptr, v->part, v->part_cap, one ? g0_of(0, 0) : nullptr,
                    one ? t1 : nullptr, v->wide_only};
    HIPCHK(vae_conv(s, 1, 0, VAE_F32, u, (const uint16_t*)wt->p, (const float*)b->p, ep, A, h, w, 64, (int)wt->o, 64));
    a_rs = one ? t1 : nullptr;
  }
  char p[96];
  for (int si = 0; si < 5; ++si) {
    const VStage& st = kVaeEncStages[si];
    // A: the stage's input, kept for AvgDown3D (or the add) at the stage's end.  At one-tile
    // widths the first block's second convolution leaves the second block's normed input in t1.
    snprintf(p, sizeof p, "encoder.downsamples.%d.downsamples.0", si);
    bool made = false;
    TRY(vae_resblock(v, p, A, nullptr, a_rs, B, false, st.in, st.out, hh, ww, t1, t2, u, t3, g0_of(si, 1), t1,
                     &made));
    const uint16_t* b_rs = made ? t1 : nullptr;
    a_rs = nullptr;
    snprintf(p, sizeof p, "encoder.downsamples.%d.downsamples.1", si);
    if (st.up) {
      // the second block in bf16 for the stride-2 convolution, into C at half size, then
      // AvgDown3D of A added
      TRY(vae_resblock(v, p, B, nullptr, b_rs, u, true, st.out, st.out, hh, ww, t1, t2, u, t3));
      snprintf(p, sizeof p, "encoder.downsamples.%d.downsamples.2.resample.1", si);
      TRY(vae_conv_named(v, p, 2, VAE_F32, u, nullptr, C, hh / 2, ww / 2));
      HIPCHK(vae_avgdown_add(s, st.in, st.out, st.tup ? 2 : 1, hh, ww, A, C));
      hh /= 2;
      ww /= 2;
    } else {
      TRY(vae_resblock(v, p, B, nullptr, b_rs, C, false, st.out, st.out, hh, ww, t1, t2, u, t3));
      HIPCHK(vae_add(s, (int64_t)hh * ww * st.out, A, C));
    }
    std::swap(A, C);
  }
  TRY(vae_resblock(v, "encoder.middle.0", A, nullptr, nullptr, B, false, top, top, hh, ww, t1, t2, u, t3));
  TRY(vae_attention(v, "encoder.middle.1", B, C, hh, ww, top, t1));
  TRY(vae_resblock(v, "encoder.middle.2", C, nullptr, nullptr, A, false, top, top, hh, ww, t1, t2, u, t3));
  const float* ghead = vae_vec(v, "encoder.head.0.gamma");
  if (!ghead) FAIL(EXN_ESTATE, "encoder: missing encoder.head.0.gamma");
  const int64_t n = (int64_t)hh * ww;
  HIPCHK(vae_rms_silu(s, n, top, A, ghead, t1, 1));
  TRY(vae_conv_named(v, "encoder.head.2", 0, VAE_BF16, t1, nullptr, u, hh, ww));
  TRY(vae_conv_named(v, "conv1", 0, VAE_F32, u, nullptr, t2, hh, ww));
  HIPCHK(vae_pixels_latent(s, n, kVaeZ, 2 * kVaeZ, t2, latent));
  return EXN_OK;
}


int exn_vae_encode_dev(exn_vae* v, const float* rgba, int h, int w, float* latent) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  // the first stage's bf16 picture (96 channels) is one buffer of under 2^31 bytes
  if (!rgba || !latent || h <= 0 || w <= 0 || h % 16 || w % 16 ||
      (int64_t)h * w * kVaeEncStages[0].out * 2 >= ((int64_t)1 << 31))
    FAIL(EXN_EINVAL, "vae encode: picture %d x %d (multiples of 16, under 2^31 / 192 pixels)", h, w);
  TRY(exn_vae_check_encoder(v));
  return vae_encode(v, rgba, h, w, latent);
}

int exn_vae_encode(exn_vae* v, const float* rgba, int h, int w, float* latent) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  // the first stage's bf16 picture (96 channels) is one buffer of under 2^31 bytes
  if (!rgba || !latent || h <= 0 || w <= 0 || h % 16 || w % 16 ||
      (int64_t)h * w * kVaeEncStages[0].out * 2 >= ((int64_t)1 << 31))
    FAIL(EXN_EINVAL, "vae encode: picture %d x %d (multiples of 16, under 2^31 / 192 pixels)", h, w);
  const int64_t npx = (int64_t)h * w * kVaeIn, nz = (int64_t)kVaeZ * (h / 16) * (w / 16);
  float *dp, *dz;
  TRY(vae_buf(v, "h_px", (size_t)npx * 4, (void**)&dp));
  TRY(vae_buf(v, "h_z", (size_t)nz * 4, (void**)&dz));
  HIPCHK(hipMemcpyAsync(dp, rgba, (size_t)npx * 4, hipMemcpyHostToDevice, v->ctx->stream));
  TRY(exn_vae_encode_dev(v, dp, h, w, dz));
  HIPCHK(hipMemcpyAsync(latent, dz, (size_t)nz * 4, hipMemcpyDeviceToHost, v->ctx->stream));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

int exn_vae_decode_dev(exn_vae* v, const float* latent, int h, int w, float* rgba) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  if (!latent || !rgba || h <= 0 || w <= 0 || (int64_t)h * w > (1 << 16))
    FAIL(EXN_EINVAL, "vae decode: latent %d x %d", h, w);
  TRY(exn_vae_check(v));
  return vae_decode(v, latent, h, w, rgba);
}

int exn_vae_decode(exn_vae* v, const float* latent, int h, int w, float* rgba) {
  if (!v) FAIL(EXN_EINVAL, "null decoder");
  TRY(use(v->ctx));
  if (!latent || !rgba || h <= 0 || w <= 0 || (int64_t)h * w > (1 << 16))
    FAIL(EXN_EINVAL, "vae decode: latent %d x %d", h, w);
  const int64_t nz = (int64_t)kVaeZ * h * w, npx = (int64_t)256 * h * w * kVaeOut;
  float *dz, *dp;
  TRY(vae_buf(v, "h_z", (size_t)nz * 4, (void**)&dz));
  TRY(vae_buf(v, "h_px", (size_t)npx * 4, (void**)&dp));
  HIPCHK(hipMemcpyAsync(dz, latent, (size_t)nz * 4, hipMemcpyHostToDevice, v->ctx->stream));
  TRY(exn_vae_decode_dev(v, dz, h, w, dp));
  HIPCHK(hipMemcpyAsync(rgba, dp, (size_t)npx * 4, hipMemcpyDeviceToHost, v->ctx->stream));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

// op-level entry points of the decoder's kernels (tests)
int exn_vae_conv(exn_ctx* ctx, int taps, int up, int outdt, const uint16_t* x, const uint16_t* wt, const float* bias,
                 const float* res, void* y, int h, int w, int c, int cout, int kp, float* part, int64_t part_cap) {
  TRY(use(ctx));
  if (!x || !wt || !bias || !y || (taps != 1 && taps != 9) || outdt < 0 || outdt > 2 || part_cap < 0)
    FAIL(EXN_EINVAL, "vae conv arguments");
  const VaeEpi ep{res, nullptr, 0, 0, nullptr, part, part ? part_cap : 0};
  const hipError_t e = vae_conv(ctx->stream, taps, up, outdt, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (e == hipErrorInvalidValue)
    FAIL(EXN_EINVAL, "vae conv: taps %d up %d out %d, %d x %d x %d -> %d, kp %d", taps, up, outdt, h, w, c, cout, kp);
  HIPCHK(e);
  return EXN_OK;
}

int exn_vae_rms_silu(exn_ctx* ctx, int64_t n, int c, const float* x, const float* gamma, uint16_t* y, int silu) {
  TRY(use(ctx));
  if (!x || !gamma || !y || c % 4 || n < 0) FAIL(EXN_EINVAL, "vae rms arguments");
  HIPCHK(vae_rms_silu(ctx->stream, n, c, x, gamma, y, silu));
  return EXN_OK;
}

int exn_vae_dupup_add(exn_ctx* ctx, int cin, int cout, int ft, int h, int w, const float* x, float* y) {
  TRY(use(ctx));
  if (!x || !y || cin <= 0 || cout <= 0 || ft < 1 || (int64_t)cout * ft * 4 % cin) FAIL(EXN_EINVAL, "dupup arguments");
  HIPCHK(vae_dupup_add(ctx->stream, cin, cout, ft, h, w, x, y));
  return EXN_OK;
}

int exn_vae_avgdown_add(exn_ctx* ctx, int cin, int cout, int ft, int h, int w, const float* x, float* y) {
  TRY(use(ctx));
  if (!x || !y || cin <= 0 || cout <= 0 || ft < 1 || (int64_t)cin * ft * 4 % cout || h <= 0 || w <= 0 || h % 2 ||
      w % 2)
    FAIL(EXN_EINVAL, "avgdown arguments");
  HIPCHK(vae_avgdown_add(ctx->stream, cin, cout, ft, h, w, x, y));
  return EXN_OK;
}
