// api_vision.hip -- the vision tower (src/cuda-vision.lisp): weights and driver.
#include "api_host.h"

// --- the vision tower (replaces src/cuda-vision.lisp's q3vision) ------------------------------

namespace {

// the tower's dimensions (src/host.lisp:104-112; inspect/ref_vision.py:20-22)
const int kVisD = 1152, kVisHeads = 16, kVisHd = 72, kVisF = 4304, kVisDepth = 27, kVisOut = 4096, kVisSide = 48;
const int kVisDeep[3] = {8, 16, 24};

// every tensor the tower reads, as inspect/ref_vision.py names them, row-major shapes
std::vector<VExpect> vision_expected() {
  std::vector<VExpect> r;
  const int64_t d = kVisD, f = kVisF, o = kVisOut;
  auto add = [&](const std::string& n, std::vector<int64_t> s) { r.push_back(VExpect{n, s}); };
  add("v.patch_embd.weight", {d, 3, 16, 16});
  add("v.patch_embd.weight.1", {d, 3, 16, 16});
  add("v.patch_embd.bias", {d});
  add("v.position_embd.weight", {(int64_t)kVisSide * kVisSide, d});
  char p[64];
  for (int i = 0; i < kVisDepth; ++i) {
    snprintf(p, sizeof p, "v.blk.%d.", i);
    const std::string b = p;
    add(b + "ln1.weight", {d});
    add(b + "ln1.bias", {d});
    add(b + "attn_qkv.weight", {3 * d, d});
    add(b + "attn_qkv.bias", {3 * d});
    add(b + "attn_out.weight", {d, d});
    add(b + "attn_out.bias", {d});
    add(b + "ln2.weight", {d});
    add(b + "ln2.bias", {d});
    add(b + "ffn_up.weight", {f, d});
    add(b + "ffn_up.bias", {f});
    add(b + "ffn_down.weight", {d, f});
    add(b + "ffn_down.bias", {d});
  }
  for (int j = 0; j < 3; ++j) {
    snprintf(p, sizeof p, "v.deepstack.%d.", kVisDeep[j]);
    const std::string b = p;
    add(b + "norm.weight", {4 * d});
    add(b + "norm.bias", {4 * d});
    add(b + "fc1.weight", {4 * d, 4 * d});
    add(b + "fc1.bias", {4 * d});
    add(b + "fc2.weight", {o, 4 * d});
    add(b + "fc2.bias", {o});
  }
  add("v.post_ln.weight", {d});
  add("v.post_ln.bias", {d});
  add("mm.0.weight", {4 * d, 4 * d});
  add("mm.0.bias", {4 * d});
  add("mm.2.weight", {o, 4 * d});
  add("mm.2.bias", {o});
  return r;
}

// fp16 bits -> fp32, subnormals, infinities and NaNs kept
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t u;
  if (e == 0x1F) {
    u = sign | 0x7F800000u | (m << 13);
  } else if (e != 0) {
    u = sign | ((e + 112) << 23) | (m << 13);
  } else if (m == 0) {
    u = sign;
  } else {
    float f = (float)m * 5.9604644775390625e-08f;   // m * 2^-24, exact
    memcpy(&u, &f, 4);
    u |= sign;
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

struct exn_vision {
  exn_ctx* ctx = nullptr;
  std::vector<VExpect> expect;
  std::map<std::string, float*> t;   // fp32 device copies
  std::map<std::string, Buf> bufs;
  float* pw = nullptr;                // the two patch kernels summed
  bool pw_ok = false;
  int side = 0;                       // the position table's side
  bool trace = false;
  int64_t traced_n = 0;               // patches of the traced encode
};

static int vis_buf(exn_vision* v, const char* key, size_t bytes, float** out) {
  Buf& b = v->bufs[key];
  if (b.bytes < bytes) {
    HIPCHK(hipStreamSynchronize(v->ctx->stream));
    dev_free(b.p);
    b.p = nullptr;
    b.bytes = 0;
    TRY(dev_alloc(&b.p, bytes));
    b.bytes = bytes;
  }
  *out = (float*)b.p;
  return EXN_OK;
}

static const VExpect* vis_find(const exn_vision* v, const char* name) {
  for (auto& e : v->expect)
    if (e.name == name) return &e;
  return nullptr;
}

static const float* vis_t(const exn_vision* v, const std::string& name) {
  auto it = v->t.find(name);
  return it == v->t.end() ? nullptr : it->second;
}

// N fp32 values (device, DATA) into tensor NAME's device copy
static int vis_store(exn_vision* v, const std::string& name, int64_t n, const float* data) {
  float*& p = v->t[name];
  if (!p) TRY(dev_alloc((void**)&p, (size_t)n * 4));
  HIPCHK(hipMemcpyAsync(p, data, (size_t)n * 4, hipMemcpyDeviceToDevice, v->ctx->stream));
  if (name.rfind("v.patch_embd.weight", 0) == 0) v->pw_ok = false;
  return EXN_OK;
}


int exn_vision_create(exn_ctx* ctx, exn_vision** out) {
  TRY(use(ctx));
  if (!out) FAIL(EXN_EINVAL, "null output");
  exn_vision* v = new exn_vision();
  v->ctx = ctx;
  v->expect = vision_expected();
  *out = v;
  return EXN_OK;
}

int exn_vision_release(exn_vision* v) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  TRY(use(v->ctx));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  for (auto& kv : v->bufs) dev_free(kv.second.p);
  v->bufs.clear();
  v->traced_n = 0;
  return EXN_OK;
}

int exn_vision_destroy(exn_vision* v) {
  if (!v) return EXN_OK;
  TRY(exn_vision_release(v));
  for (auto& kv : v->t) dev_free(kv.second);
  dev_free(v->pw);
  delete v;
  return EXN_OK;
}

int exn_vision_set(exn_vision* v, const char* name, int kind, const void* data, const int64_t* dims, int ndims) {
  if (!v || !name || !data || !dims) FAIL(EXN_EINVAL, "vision set: null argument");
  TRY(use(v->ctx));
  const VExpect* e = vis_find(v, name);
  if (!e) FAIL(EXN_EINVAL, "vision set: no tower tensor %s", name);
  if (kind != EXN_F32 && kind != EXN_F16 && kind != EXN_BF16)
    FAIL(EXN_EINVAL, "vision set %s: kind %d (F32, F16 or BF16 only)", name, kind);
  const bool table = e->name == "v.position_embd.weight";
  bool same = ndims == (int)e->shape.size();
  for (int i = 0; same && i < ndims; ++i) same = dims[i] == e->shape[i] || (table && i == 0);
  int side = 0;
  if (same && table) {
    side = (int)std::lround(std::sqrt((double)dims[0]));
    same = side >= 2 && (int64_t)side * side == dims[0];
  }
  if (!same) {
    std::string want;
    for (auto d : e->shape) want += (want.empty() ? "" : " ") + std::to_string(d);
    FAIL(EXN_EINVAL, "vision set %s: shape is not (%s)%s", name, want.c_str(), table ? ", S square" : "");
  }
  int64_t n = 1;
  for (int i = 0; i < ndims; ++i) n *= dims[i];
  std::vector<float> f((size_t)n);
  if (kind == EXN_F32) {
    memcpy(f.data(), data, (size_t)n * 4);
  } else if (kind == EXN_F16) {
    const uint16_t* h = (const uint16_t*)data;
    for (int64_t i = 0; i < n; ++i) f[(size_t)i] = half_to_float(h[i]);
  } else {
    const uint16_t* b = (const uint16_t*)data;
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)b[i] << 16;
      memcpy(&f[(size_t)i], &u, 4);
    }
  }
  if (table && v->t.count(e->name) && v->side != side) {
    HIPCHK(hipStreamSynchronize(v->ctx->stream));
    dev_free(v->t[e->name]);
    v->t.erase(e->name);
  }
  float* tmp = nullptr;
  TRY(ctx_tmp(v->ctx, (size_t)n * 4, (void**)&tmp));
  HIPCHK(hipMemcpyAsync(tmp, f.data(), (size_t)n * 4, hipMemcpyHostToDevice, v->ctx->stream));
  TRY(vis_store(v, e->name, n, tmp));
  if (table) v->side = side;
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

// every tower tensor from the counter generator (the oracle's SynthVision): value = base +
// scale * normal i of key(seed, 6000 + the tensor's index), matrices then rounded to fp16
int exn_vision_synth(exn_vision* v, uint64_t seed) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  TRY(use(v->ctx));
  for (size_t i = 0; i < v->expect.size(); ++i) {
    const VExpect& e = v->expect[i];
    const std::string& nm = e.name;
    int64_t n = 1;
    for (auto d : e.shape) n *= d;
    double base = 0.0, scale;
    bool f16 = true;
    if (e.shape.size() == 1) {
      f16 = false;
      const bool bias = nm.size() > 5 && nm.compare(nm.size() - 5, 5, ".bias") == 0;
      base = bias ? 0.0 : 1.0;
      scale = bias ? 0.02 : 0.1;
    } else if (nm == "v.position_embd.weight") {
      scale = 1.0;
    } else {
      int64_t fan = 1;
      for (size_t k = 1; k < e.shape.size(); ++k) fan *= e.shape[k];
      auto ends = [&](const char* s) { return nm.size() >= strlen(s) && nm.compare(nm.size() - strlen(s), strlen(s), s) == 0; };
      double g = 1.0;
      if (nm.rfind("v.patch_embd", 0) == 0) g = 0.7;
      else if (ends("attn_qkv.weight")) g = 2.0;
      else if (ends("attn_out.weight") || ends("ffn_down.weight")) g = 0.5;
      scale = g / sqrt((double)fan);
    }
    float* tmp = nullptr;
    TRY(ctx_tmp(v->ctx, (size_t)n * 4, (void**)&tmp));
    HIPCHK(synth_normal(v->ctx->stream, gen_key(seed, 6000 + i), n, (float)base, (float)scale, 1, tmp));
    if (f16) HIPCHK(round_f16(v->ctx->stream, n, tmp));
    if (nm == "v.position_embd.weight" && v->t.count(nm) && v->side != kVisSide) {
      HIPCHK(hipStreamSynchronize(v->ctx->stream));
      dev_free(v->t[nm]);
      v->t.erase(nm);
    }
    TRY(vis_store(v, nm, n, tmp));
    if (nm == "v.position_embd.weight") v->side = kVisSide;
  }
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

int exn_vision_check(exn_vision* v) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  for (auto& e : v->expect)
    if (!vis_t(v, e.name)) FAIL(EXN_ESTATE, "vision tower: missing %s", e.name.c_str());
  return EXN_OK;
}

int exn_vision_memory(exn_vision* v, int64_t* weights, int64_t* scratch_bytes) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  int64_t w = 0, s = 0;
  for (auto& e : v->expect) {
    if (!vis_t(v, e.name)) continue;
    int64_t n = 1;
    for (auto d : e.shape) n *= d;
    if (e.name == "v.position_embd.weight") n = (int64_t)v->side * v->side * kVisD;
    w += n * 4;
  }
  if (v->pw) w += (int64_t)kVisD * 768 * 4;
  for (auto& kv : v->bufs) s += (int64_t)kv.second.bytes;
  if (weights) *weights = w;
  if (scratch_bytes) *scratch_bytes = s;
  return EXN_OK;
}

int exn_vision_trace(exn_vision* v, int on) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  v->trace = on != 0;
  return EXN_OK;
}


// a merger (src/cuda-vision.lisp:71-82; inspect/ref_vision.py:109-118): four patches' rows as
// one row of 4608, LayerNorm after (deepstack, PREFIX) or before (v.post_ln), fc1, GELU (erf),
// fc2 into OUT (M x 4096)
static int vis_merger(exn_vision* v, const float* x, int n, float* out, const char* prefix) {
  hipStream_t s = v->ctx->stream;
  const int m = n / 4, d4 = 4 * kVisD;
  float *t1, *t2;
  TRY(vis_buf(v, "mt1", (size_t)n * kVisD * 4, &t1));
  TRY(vis_buf(v, "mt2", (size_t)m * d4 * 4, &t2));
  std::string fc1 = "mm.0", fc2 = "mm.2";
  if (prefix) {
    const std::string p = prefix;
    HIPCHK(vis_ln(s, m, d4, x, vis_t(v, p + ".norm.weight"), vis_t(v, p + ".norm.bias"), t1));
    fc1 = p + ".fc1";
    fc2 = p + ".fc2";
  } else {
    HIPCHK(vis_ln(s, n, kVisD, x, vis_t(v, "v.post_ln.weight"), vis_t(v, "v.post_ln.bias"), t1));
  }
  HIPCHK(vis_gemm(s, t1, vis_t(v, fc1 + ".weight"), vis_t(v, fc1 + ".bias"), nullptr, t2, m, d4, d4, 2));
  HIPCHK(vis_gemm(s, t2, vis_t(v, fc2 + ".weight"), vis_t(v, fc2 + ".bias"), nullptr, out, m, kVisOut, d4, 0));
  return EXN_OK;
}

// vision-encode on the device (src/cuda-vision.lisp:34-101)
static int vis_encode(exn_vision* v, const float* px, int h, int w, float* merged, float* deep) {
  hipStream_t s = v->ctx->stream;
  const int gh = h / 16, gw = w / 16, n = gh * gw, m = n / 4, D = kVisD;
  if (!v->pw_ok) {
    if (!v->pw) TRY(dev_alloc((void**)&v->pw, (size_t)D * 768 * 4));
    HIPCHK(vis_sum(s, (int64_t)D * 768, vis_t(v, "v.patch_embd.weight"), vis_t(v, "v.patch_embd.weight.1"), v->pw));
    v->pw_ok = true;
  }
  float *pat, *pe, *cs, *x, *hb, *qkv, *q, *k, *vt, *att, *up;
  TRY(vis_buf(v, "pat", (size_t)n * 768 * 4, &pat));
  TRY(vis_buf(v, "pe", (size_t)n * D * 4, &pe));
  TRY(vis_buf(v, "cs", (size_t)n * 144 * 4, &cs));
  TRY(vis_buf(v, "x", (size_t)n * D * 4, &x));
  TRY(vis_buf(v, "hb", (size_t)n * D * 4, &hb));
  TRY(vis_buf(v, "qkv", (size_t)n * 3 * D * 4, &qkv));
  TRY(vis_buf(v, "q", (size_t)n * D * 4, &q));
  TRY(vis_buf(v, "k", (size_t)n * D * 4, &k));
  TRY(vis_buf(v, "vt", (size_t)n * D * 4, &vt));
  TRY(vis_buf(v, "att", (size_t)n * D * 4, &att));
  TRY(vis_buf(v, "up", (size_t)n * kVisF * 4, &up));
  HIPCHK(vis_prep(s, px, w, gh, gw, vis_t(v, "v.position_embd.weight"), v->side, D, pat, pe, cs));
  HIPCHK(vis_gemm(s, pat, v->pw, vis_t(v, "v.patch_embd.bias"), pe, x, n, D, 768, 0));
  float* tr = nullptr;
  if (v->trace) {
    TRY(vis_buf(v, "trace", (size_t)2 * n * D * 4, &tr));
    HIPCHK(hipMemcpyAsync(tr, x, (size_t)n * D * 4, hipMemcpyDeviceToDevice, s));
  }
  const float qscale = (float)(1.4426950408889634 / sqrt((double)kVisHd));
  char p[64];
  for (int i = 0; i < kVisDepth; ++i) {
    snprintf(p, sizeof p, "v.blk.%d.", i);
    const std::string b = p;
    HIPCHK(vis_ln(s, n, D, x, vis_t(v, b + "ln1.weight"), vis_t(v, b + "ln1.bias"), hb));
    HIPCHK(vis_gemm(s, hb, vis_t(v, b + "attn_qkv.weight"), vis_t(v, b + "attn_qkv.bias"), nullptr, qkv, n, 3 * D, D, 0));
    HIPCHK(vis_heads(s, n, kVisHeads, qkv, cs, qscale, q, k, vt));
    HIPCHK(vis_attend(s, n, kVisHeads, q, k, vt, att));
    HIPCHK(vis_gemm(s, att, vis_t(v, b + "attn_out.weight"), vis_t(v, b + "attn_out.bias"), x, x, n, D, D, 0));
    HIPCHK(vis_ln(s, n, D, x, vis_t(v, b + "ln2.weight"), vis_t(v, b + "ln2.bias"), hb));
    HIPCHK(vis_gemm(s, hb, vis_t(v, b + "ffn_up.weight"), vis_t(v, b + "ffn_up.bias"), nullptr, up, n, kVisF, D, 1));
    HIPCHK(vis_gemm(s, up, vis_t(v, b + "ffn_down.weight"), vis_t(v, b + "ffn_down.bias"), x, x, n, D, kVisF, 0));
    if (i == 0 && tr) HIPCHK(hipMemcpyAsync(tr + (size_t)n * D, x, (size_t)n * D * 4, hipMemcpyDeviceToDevice, s));
    for (int j = 0; j < 3; ++j)
      if (kVisDeep[j] == i) {
        snprintf(p, sizeof p, "v.deepstack.%d", i);
        TRY(vis_merger(v, x, n, deep + (size_t)j * m * kVisOut, p));
      }
  }
  TRY(vis_merger(v, x, n, merged, nullptr));
  if (tr) v->traced_n = n;
  return EXN_OK;
}


int exn_vision_encode_dev(exn_vision* v, const float* px, int h, int w, float* merged, float* deepstack) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  TRY(use(v->ctx));
  if (!px || !merged || !deepstack || h <= 0 || w <= 0 || h % 32 || w % 32 || (int64_t)(h / 16) * (w / 16) > 16384)
    FAIL(EXN_EINVAL, "vision encode: picture %d x %d (multiples of 32, at most 16384 patches)", h, w);
  TRY(exn_vision_check(v));
  return vis_encode(v, px, h, w, merged, deepstack);
}

int exn_vision_encode(exn_vision* v, const float* px, int h, int w, float* merged, float* deepstack) {
  if (!v) FAIL(EXN_EINVAL, "null vision tower");
  TRY(use(v->ctx));
  if (!px || !merged || !deepstack || h <= 0 || w <= 0 || h % 32 || w % 32 || (int64_t)(h / 16) * (w / 16) > 16384)
    FAIL(EXN_EINVAL, "vision encode: picture %d x %d (multiples of 32, at most 16384 patches)", h, w);
  const int64_t npx = (int64_t)h * w * 4, m = (int64_t)(h / 32) * (w / 32);
  float *dp, *dm;
  TRY(vis_buf(v, "h_px", (size_t)npx * 4, &dp));
  TRY(vis_buf(v, "h_out", (size_t)4 * m * kVisOut * 4, &dm));
  HIPCHK(hipMemcpyAsync(dp, px, (size_t)npx * 4, hipMemcpyHostToDevice, v->ctx->stream));
  TRY(exn_vision_encode_dev(v, dp, h, w, dm, dm + m * kVisOut));
  HIPCHK(hipMemcpyAsync(merged, dm, (size_t)m * kVisOut * 4, hipMemcpyDeviceToHost, v->ctx->stream));
  HIPCHK(hipMemcpyAsync(deepstack, dm + m * kVisOut, (size_t)3 * m * kVisOut * 4, hipMemcpyDeviceToHost,
                        v->ctx->stream));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

int exn_vision_traced(exn_vision* v, int which, float* out) {
  if (!v || !out || which < 0 || which > 1) FAIL(EXN_EINVAL, "vision traced: arguments");
  TRY(use(v->ctx));
  auto it = v->bufs.find("trace");
  if (!v->traced_n || it == v->bufs.end()) FAIL(EXN_ESTATE, "vision traced: no traced encode");
  const size_t rows = (size_t)v->traced_n * kVisD;
  HIPCHK(hipMemcpyAsync(out, (const float*)it->second.p + which * rows, rows * 4, hipMemcpyDeviceToHost,
                        v->ctx->stream));
  HIPCHK(hipStreamSynchronize(v->ctx->stream));
  return EXN_OK;
}

int exn_vis_gemm(exn_ctx* ctx, const float* x, const float* w, const float* bias, const float* r, float* y, int64_t m,
                 int64_t n, int64_t k, int act) {
  TRY(use(ctx));
  if (!x || !w || !bias || !y || act < 0 || act > 2) FAIL(EXN_EINVAL, "vis gemm arguments");
  const hipError_t e = vis_gemm(ctx->stream, x, w, bias, r, y, m, n, k, act);
  if (e == hipErrorInvalidValue) FAIL(EXN_EINVAL, "vis gemm: %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  HIPCHK(e);
  return EXN_OK;
}

int exn_vis_attend(exn_ctx* ctx, int n, int heads, const float* q, const float* k, const float* vt, float* att) {
  TRY(use(ctx));
  if (!q || !k || !vt || !att || n <= 0 || heads <= 0) FAIL(EXN_EINVAL, "vis attend arguments");
  const hipError_t e = vis_attend(ctx->stream, n, heads, q, k, vt, att);
  if (e == hipErrorInvalidValue) FAIL(EXN_EINVAL, "vis attend: n %d (a multiple of 4)", n);
  HIPCHK(e);
  return EXN_OK;
}

int exn_vis_ln(exn_ctx* ctx, int64_t rows, int width, const float* x, const float* w, const float* b, float* y) {
  TRY(use(ctx));
  if (!x || !w || !b || !y || rows < 0) FAIL(EXN_EINVAL, "vis ln arguments");
  const hipError_t e = vis_ln(ctx->stream, rows, width, x, w, b, y);
  if (e == hipErrorInvalidValue) FAIL(EXN_EINVAL, "vis ln: width %d (a multiple of 4, at most 5120)", width);
  HIPCHK(e);
  return EXN_OK;
}
