// api_encoder.hip -- the prompt encoder's text model (src/encoder.lisp): weights and driver.
#include "api_host.h"

// --- the prompt encoder (replaces illatio's qwen3 forward under src/encoder.lisp) -------------

namespace {

enum { E_ATTN_NORM, E_Q, E_K, E_V, E_OUT, E_QNORM, E_KNORM, E_FFN_NORM, E_GATE, E_UP, E_DOWN, E_SLOTS };
const char* const kEncSlot[E_SLOTS] = {"attn_norm.weight", "attn_q.weight",      "attn_k.weight",
                                       "attn_v.weight",    "attn_output.weight", "attn_q_norm.weight",
                                       "attn_k_norm.weight", "ffn_norm.weight",  "ffn_gate.weight",
                                       "ffn_up.weight",    "ffn_down.weight"};
// ggml dims of each slot: d0 (contiguous, the inputs), d1 (rows; 1 for a vector)
const int64_t kEncDims[E_SLOTS][2] = {{4096, 1},     {4096, 4096}, {4096, 1024},  {4096, 1024},
                                      {4096, 4096},  {128, 1},     {128, 1},      {4096, 1},
                                      {4096, 12288}, {4096, 12288}, {12288, 4096}};
const int kEncGroup = 4;   // query heads a key/value head (32 / 8)

// A head's rotate_half pairs (i, i + 64) stored as adjacent dims (2i, 2i + 1): q and k rows (and
// their norm weights) are permuted alike, which leaves q.k and each head's RMS unchanged, so the
// DiT's pairwise rotary (dims 2i, 2i + 1 by angle i) applies.
int enc_perm(int i) { return i < 64 ? 2 * i : 2 * (i - 64) + 1; }

// the key/value heads' rows in the q | k | v matrix: 8 heads of 128 each for k and for v
constexpr int kEncKV = 8 * EXN_HD;

// the layer-matrix row of each source row of SLOT: q (32 heads) | k (8) | v (8), the rotary's
// pairs of q and k adjacent; or gate/up interleaved by 32
std::vector<int32_t> enc_rows(int slot) {
  std::vector<int32_t> m;
  if (slot == E_Q) {
    for (int r = 0; r < EXN_W; ++r) m.push_back((r / EXN_HD) * EXN_HD + enc_perm(r % EXN_HD));
  } else if (slot == E_K) {
    for (int r = 0; r < kEncKV; ++r) m.push_back(EXN_W + (r / EXN_HD) * EXN_HD + enc_perm(r % EXN_HD));
  } else if (slot == E_V) {
    for (int r = 0; r < kEncKV; ++r) m.push_back(EXN_W + kEncKV + r);
  } else if (slot == E_GATE || slot == E_UP) {
    for (int r = 0; r < EXN_F; ++r) m.push_back(64 * (r / 32) + (slot == E_UP ? 32 : 0) + r % 32);
  }
  return m;
}

struct EncLayer {
  exn_w* qkv = nullptr;      // q | k | v, 4096 + 1024 + 1024 rows (the rotary's pairs adjacent)
  exn_w* out = nullptr;
  exn_w* gate_up = nullptr;  // gate / up interleaved by 32
  exn_w* down = nullptr;
  float* vec[E_SLOTS] = {};  // the norms' weights (q and k norms permuted as their rows)
  unsigned have = 0;         // slots set, a bit each
};

}  // namespace

struct exn_enc {
  exn_ctx* ctx = nullptr;
  int layers = 36;
  double base = 5e6;
  int64_t vocab = 0;
  int8_t* eqs = nullptr;     // token_embd: Q8_0 codes and scales, or fp32 rows
  uint16_t* ed = nullptr;
  float* ef = nullptr;
  std::vector<EncLayer> L;
  std::map<std::string, Buf> bufs;
  float* one_gate = nullptr;  // +inf a column: the gated residual's tanh(gate) is exactly 1
  std::map<int, int32_t*> maps;  // device row maps by slot
  bool bf16 = true;           // the matrices run from resident bf16 expansions (exn_enc_resident)
};

static int enc_buf(exn_enc* e, const char* key, size_t bytes, void** out, bool zero = false) {
  Buf& b = e->bufs[key];
  if (b.bytes < bytes) {
    HIPCHK(hipStreamSynchronize(e->ctx->stream));
    dev_free(b.p);
    b.p = nullptr;
    b.bytes = 0;
    TRY(dev_alloc(&b.p, bytes));
    b.bytes = bytes;
    if (zero) HIPCHK(hipMemsetAsync(b.p, 0, bytes, e->ctx->stream));
  }
  *out = b.p;
  return EXN_OK;
}

static int enc_map(exn_enc* e, int slot, int32_t** out) {
  int32_t*& m = e->maps[slot];
  if (!m) {
    const std::vector<int32_t> h = enc_rows(slot);
    TRY(dev_alloc((void**)&m, h.size() * 4));
    HIPCHK(hipMemcpyAsync(m, h.data(), h.size() * 4, hipMemcpyHostToDevice, e->ctx->stream));
    HIPCHK(hipStreamSynchronize(e->ctx->stream));
  }
  *out = m;
  return EXN_OK;
}

// the Q8_0 layer matrix slot S writes into (made on first use)
static int enc_matrix(exn_enc* e, EncLayer& L, int slot, exn_w** out) {
  exn_w** w = slot == E_OUT ? &L.out : slot == E_DOWN ? &L.down : (slot == E_GATE || slot == E_UP) ? &L.gate_up : &L.qkv;
  if (!*w) {
    const int64_t rows = slot == E_OUT ? EXN_W : slot == E_DOWN ? EXN_W : (slot == E_GATE || slot == E_UP) ? 2 * EXN_F
                                                                                                   : EXN_W + 2 * kEncKV;
    const int64_t cols = slot == E_DOWN ? EXN_F : EXN_W;
    TRY(w_new(e->ctx, EXN_Q8_0, rows, cols, w));
    if (slot == E_GATE || slot == E_UP) (*w)->pairs = true;
  }
  *out = *w;
  return EXN_OK;
}

// slot S's weight vector (N floats, device, DATA) into the layer, q and k norms permuted
static int enc_vector(exn_enc* e, EncLayer& L, int slot, const float* host) {
  const int n = (int)kEncDims[slot][0];
  std::vector<float> v(host, host + n);
  if (slot == E_QNORM || slot == E_KNORM)
    for (int i = 0; i < n; ++i) v[(size_t)enc_perm(i)] = host[i];
  if (!L.vec[slot]) TRY(dev_alloc((void**)&L.vec[slot], (size_t)n * 4));
  HIPCHK(hipMemcpyAsync(L.vec[slot], v.data(), (size_t)n * 4, hipMemcpyHostToDevice, e->ctx->stream));
  HIPCHK(hipStreamSynchronize(e->ctx->stream));
  L.have |= 1u << slot;
  return EXN_OK;
}


int exn_enc_create(exn_ctx* ctx, int layers, double rope_base, exn_enc** out) {
  TRY(use(ctx));
  if (!out || layers < 1 || layers > 64 || !(rope_base > 1.0)) FAIL(EXN_EINVAL, "encoder: layers %d, rope base %g", layers, rope_base);
  exn_enc* e = new exn_enc();
  e->ctx = ctx;
  e->layers = layers;
  e->base = rope_base;
  e->L.resize((size_t)layers);
  std::vector<float> inf((size_t)EXN_W, INFINITY);
  int r = dev_alloc((void**)&e->one_gate, (size_t)EXN_W * 4);
  if (r == EXN_OK && hipMemcpy(e->one_gate, inf.data(), (size_t)EXN_W * 4, hipMemcpyHostToDevice) != hipSuccess) {
    exn::set_error("encoder: gate upload");
    r = EXN_EHIP;
  }
  if (r != EXN_OK) {
    dev_free(e->one_gate);
    delete e;
    return r;
  }
  *out = e;
  return EXN_OK;
}

int exn_enc_release(exn_enc* e) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  TRY(use(e->ctx));
  HIPCHK(hipStreamSynchronize(e->ctx->stream));
  for (auto& kv : e->bufs) dev_free(kv.second.p);
  e->bufs.clear();
  return EXN_OK;
}

int exn_enc_destroy(exn_enc* e) {
  if (!e) return EXN_OK;
  TRY(exn_enc_release(e));
  for (auto& L : e->L) {
    exn_weight_free(L.qkv);
    exn_weight_free(L.out);
    exn_weight_free(L.gate_up);
    exn_weight_free(L.down);
    for (auto* p : L.vec) dev_free(p);
  }
  for (auto& kv : e->maps) dev_free(kv.second);
  dev_free(e->eqs);
  dev_free(e->ed);
  dev_free(e->ef);
  dev_free(e->one_gate);
  delete e;
  return EXN_OK;
}

int exn_enc_set(exn_enc* e, const char* name, int kind, const void* data, int64_t d0, int64_t d1) {
  if (!e || !name || !data) FAIL(EXN_EINVAL, "encoder set: null argument");
  TRY(use(e->ctx));
  const std::string nm = name;
  if (nm == "output_norm.weight" || nm == "output.weight") return EXN_OK;   // past the states read
  if (nm == "token_embd.weight") {
    if (d0 != EXN_W || d1 < 1 || d1 > (1 << 20) || (kind != EXN_Q8_0 && kind != EXN_F32))
      FAIL(EXN_EINVAL, "encoder set token_embd: %lld x %lld of kind %d (4096 x vocab, Q8_0 or F32)", (long long)d0,
           (long long)d1, kind);
    HIPCHK(hipStreamSynchronize(e->ctx->stream));
    dev_free(e->eqs);
    dev_free(e->ed);
    dev_free(e->ef);
    e->eqs = nullptr;
    e->ed = nullptr;
    e->ef = nullptr;
    e->vocab = 0;
    if (kind == EXN_Q8_0) {
      TRY(dev_alloc((void**)&e->eqs, (size_t)(d1 * d0)));
      TRY(dev_alloc((void**)&e->ed, (size_t)(d1 * d0 / 32) * 2));
      TRY(upload_q8_blocks(e->ctx, data, d1, d0, nullptr, e->eqs, e->ed));
    } else {
      TRY(dev_alloc((void**)&e->ef, (size_t)(d1 * d0) * 4));
      HIPCHK(hipMemcpy(e->ef, data, (size_t)(d1 * d0) * 4, hipMemcpyHostToDevice));
    }
    e->vocab = d1;
    return EXN_OK;
  }
  int il = -1, slot = -1;
  {
    int pos = 0;
    if (sscanf(name, "blk.%d.%n", &il, &pos) == 1 && pos > 0)
      for (int k = 0; k < E_SLOTS; ++k)
        if (strcmp(name + pos, kEncSlot[k]) == 0) slot = k;
  }
  if (il < 0 || il >= e->layers || slot < 0) FAIL(EXN_EINVAL, "encoder set: no tensor %s in %d layers", name, e->layers);
  if (d0 != kEncDims[slot][0] || d1 != kEncDims[slot][1])
    FAIL(EXN_EINVAL, "encoder set %s: dims %lld x %lld, not %lld x %lld", name, (long long)d0, (long long)d1,
         (long long)kEncDims[slot][0], (long long)kEncDims[slot][1]);
  EncLayer& L = e->L[(size_t)il];
  if (d1 == 1) {
    if (kind != EXN_F32) FAIL(EXN_EINVAL, "encoder set %s: a norm's weights are F32", name);
    return enc_vector(e, L, slot, (const float*)data);
  }
  if (kind != EXN_Q8_0) FAIL(EXN_EINVAL, "encoder set %s: kind %d (the encoder's matrices are Q8_0)", name, kind);
  exn_w* w = nullptr;
  TRY(enc_matrix(e, L, slot, &w));
  w->wx_ok = false;   // the expansion, if kept, is remade before the next use
  int32_t* map = nullptr;
  if (slot != E_OUT && slot != E_DOWN) TRY(enc_map(e, slot, &map));
  TRY(upload_q8_blocks(e->ctx, data, d1, d0, map, w->qs, w->d));
  TRY(retile(w));
  L.have |= 1u << slot;
  return EXN_OK;
}

// every tensor from the counter generator (the oracle's SynthEncoder): Q8_0 matrices, norm
// weights 1 + 0.05 z, a token embedding of VOCAB rows; tensor id 8000 + its index (token_embd
// 0, then 11 a layer in slot order)
int exn_enc_synth(exn_enc* e, uint64_t seed, int64_t vocab) {
  if (!e || vocab < 1 || vocab > (1 << 20)) FAIL(EXN_EINVAL, "encoder synth: vocab %lld", (long long)vocab);
  TRY(use(e->ctx));
  hipStream_t s = e->ctx->stream;
  HIPCHK(hipStreamSynchronize(s));
  dev_free(e->eqs);
  dev_free(e->ed);
  dev_free(e->ef);
  e->eqs = nullptr;
  e->ed = nullptr;
  e->ef = nullptr;
  TRY(dev_alloc((void**)&e->eqs, (size_t)(vocab * EXN_W)));
  TRY(dev_alloc((void**)&e->ed, (size_t)(vocab * EXN_W / 32) * 2));
  HIPCHK(synth_q8(s, gen_key(seed, 8000), vocab, EXN_W, EXN_W / 32, nullptr, e->eqs, e->ed));
  e->vocab = vocab;
  for (int il = 0; il < e->layers; ++il) {
    EncLayer& L = e->L[(size_t)il];
    for (int slot = 0; slot < E_SLOTS; ++slot) {
      const uint64_t key = gen_key(seed, 8000 + 1 + 11 * (uint64_t)il + slot);
      if (kEncDims[slot][1] == 1) {
        const int n = (int)kEncDims[slot][0];
        float* tmp = nullptr;
        TRY(ctx_tmp(e->ctx, (size_t)n * 4, (void**)&tmp));
        HIPCHK(synth_normal(s, key, n, 1.f, 0.05f, 1, tmp));
        std::vector<float> h((size_t)n);
        HIPCHK(hipMemcpyAsync(h.data(), tmp, (size_t)n * 4, hipMemcpyDeviceToHost, s));
        HIPCHK(hipStreamSynchronize(s));
        TRY(enc_vector(e, L, slot, h.data()));
        continue;
      }
      exn_w* w = nullptr;
      TRY(enc_matrix(e, L, slot, &w));
      w->wx_ok = false;
      int32_t* map = nullptr;
      if (slot != E_OUT && slot != E_DOWN) TRY(enc_map(e, slot, &map));
      HIPCHK(synth_q8(s, key, kEncDims[slot][1], kEncDims[slot][0], kEncDims[slot][0] / 32, map, w->qs, w->d));
      TRY(retile(w));
      L.have |= 1u << slot;
    }
  }
  HIPCHK(hipStreamSynchronize(s));
  return EXN_OK;
}

int exn_enc_check(exn_enc* e) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  if (!e->vocab) FAIL(EXN_ESTATE, "encoder: missing token_embd.weight");
  for (int il = 0; il < e->layers; ++il)
    for (int slot = 0; slot < E_SLOTS; ++slot)
      if (!(e->L[(size_t)il].have >> slot & 1u)) FAIL(EXN_ESTATE, "encoder: missing blk.%d.%s", il, kEncSlot[slot]);
  return EXN_OK;
}

// the layers' matrices multiplied from resident bf16 expansions (1, the default, 14 GB beside
// the 7.4 GB of Q8_0, made by the first prompt of more than 256 tokens: shorter ones run every
// product through the few-row kernel, which streams the Q8_0 codes) or from Q8_0 alone,
// dequantised in the products (0: any expansions are dropped)
int exn_enc_resident(exn_enc* e, int bf16) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  TRY(use(e->ctx));
  e->bf16 = bf16 != 0;
  if (!e->bf16)
    for (auto& L : e->L)
      for (exn_w* m : {L.qkv, L.out, L.gate_up, L.down})
        if (m) TRY(w_resident(m, false));
  HIPCHK(hipStreamSynchronize(e->ctx->stream));
  return EXN_OK;
}

int exn_enc_memory(exn_enc* e, int64_t* weights, int64_t* scratch_bytes) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  int64_t w = e->vocab * EXN_W * (e->ef ? 4 : 1) + (e->ed ? e->vocab * EXN_W / 16 : 0), s = 0;
  for (auto& L : e->L)
    for (exn_w* m : {L.qkv, L.out, L.gate_up, L.down})
      if (m) w += m->rows * m->cols * 17 / 16 + (m->qt ? tile_q8_bytes(m->rows, m->cols) : 0) +
                  (m->wx ? m->rows * m->cols * 2 : 0);
  for (auto& kv : e->bufs) s += (int64_t)kv.second.bytes;
  if (weights) *weights = w;
  if (scratch_bytes) *scratch_bytes = s;
  return EXN_OK;
}

// mrope-table (src/encoder.lisp:26-39) as the products read it: row t's angle of frequency j
// (< 64) is its position on axis (j mod 3: t, h, w) below 60, t above, times base^(-2j/128);
// cos, sin of pair j at CS[128 t + 2j], [128 t + 2j + 1].  POS: n (t, h, w) triples, or NULL for
// text positions 0 .. n-1.  Host only.
int exn_enc_rope_table(const int32_t* pos, int n, double base, float* cs) {
  if (n < 0 || !cs || !(base > 1.0)) FAIL(EXN_EINVAL, "encoder rope table arguments");
  for (int t = 0; t < n; ++t)
    for (int j = 0; j < 64; ++j) {
      const int axis = j < 60 ? j % 3 : 0;
      const double p = pos ? (double)pos[3 * t + axis] : (double)t;
      const double a = p * std::pow(base, -(2.0 * j) / 128.0);
      cs[(size_t)t * 128 + 2 * j] = (float)std::cos(a);
      cs[(size_t)t * 128 + 2 * j + 1] = (float)std::sin(a);
    }
  return EXN_OK;
}


// encoder-states on the device: IDS (n, validated), CS (n x 128, exn_enc_rope_table's), the
// picture's rows PIC0 .. PIC0 + M - 1 taking MERGED after the embedding and DEEP[j] (3 x M x
// 4096) after layer j; OUT n x 4096
static int enc_states(exn_enc* e, const int32_t* ids, int n, const float* cs, int pic0, int m, const float* merged,
                      const float* deep, float* out) {
  hipStream_t s = e->ctx->stream;
  // expansions made (or remade after a set) once a prompt reads them, then kept: a prompt of at
  // most 256 tokens takes every product from the Q8_0 codes (wop_n) and leaves them unmade
  if (e->bf16 && n > 256)
    for (auto& L : e->L)
      for (exn_w* w : {L.qkv, L.out, L.gate_up, L.down}) TRY(w_resident(w, true));
  const int64_t lcap = ((int64_t)n + 63) / 64 * 64;
  float* x;
  uint16_t *y, *att, *ff, *q, *kc, *vt, *qkv;
  TRY(enc_buf(e, "x", (size_t)n * EXN_W * 4, (void**)&x));
  TRY(enc_buf(e, "y", (size_t)n * EXN_W * 2, (void**)&y));
  TRY(enc_buf(e, "att", (size_t)n * EXN_W * 2, (void**)&att));
  TRY(enc_buf(e, "ff", (size_t)n * EXN_F * 2, (void**)&ff));
  TRY(enc_buf(e, "q", (size_t)n * EXN_W * 2, (void**)&q));
  TRY(enc_buf(e, "kc", (size_t)lcap * EXN_W * 2, (void**)&kc, true));
  TRY(enc_buf(e, "vt", (size_t)lcap * EXN_W * 2, (void**)&vt, true));
  TRY(enc_buf(e, "qkv", (size_t)n * (EXN_W + 2 * kEncKV) * 2, (void**)&qkv));
  // a prompt of at most 1024 tokens is about one row of 256-row tiles: its products split K
  // over the chip (the DiT's prompt-row path), the partial sums then added in order; a longer
  // one splits the products of fewer tiles than 192 (out and down, 16 column tiles)
  float* part = nullptr;
  const bool split = n <= 1024;
  TRY(enc_buf(e, "part", (size_t)kSplitCap * 4, (void**)&part));
  auto splits = [&](const exn_w* w) { return split || ((int64_t)n + 255) / 256 * ((w->rows + 255) / 256) < 192; };
  // the product through EPI; with NSUM, a split product's sums are left in PART for the caller
  // (*NSUM partials, 0 where it ran whole)
  auto mm = [&](const exn_w* w, const uint16_t* xin, int64_t lda, Epi epi, const EpiArgs& a,
                int* nsum = nullptr) -> hipError_t {
    if (nsum) *nsum = 0;
    if (splits(w)) {
      const hipError_t r =
          gemm_split_rows(s, xin, lda, wop_n(w, n), n, w->rows, w->cols, epi, a, part, kSplitCap, 8, nsum);
      if (r != hipErrorNotSupported) return r;
    }
    return gemm_any(s, w, xin, lda, n, epi, a);
  };
  // a gated-residual product into x, then the RMS norm NW of the new rows into y: a split
  // product's sums and the norm in one pass
  auto mm_norm = [&](const exn_w* w, const uint16_t* xin, int64_t lda, const EpiArgs& a, const float* nw) -> hipError_t {
    int ns = 0;
    const hipError_t r = mm(w, xin, lda, EPI_GATE_ADD, a, &ns);
    if (r != hipSuccess) return r;
    if (ns > 0) return split_sum_rms(s, ns, n, w->rows, part, a, 1e-6f, nw, y);
    return rms_norm(s, n, EXN_W, 1e-6f, x, nw, y, 1);
  };
  HIPCHK(enc_embed(s, ids, n, e->vocab, e->eqs, e->ed, e->ef, EXN_W, x));
  if (m > 0)
    HIPCHK(hipMemcpyAsync(x + (int64_t)pic0 * EXN_W, merged, (size_t)m * EXN_W * 4, hipMemcpyDeviceToDevice, s));
  EpiArgs ea;
  if (e->layers > 0) HIPCHK(rms_norm(s, n, EXN_W, 1e-6f, x, e->L[0].vec[E_ATTN_NORM], y, 1));
  for (int il = 0; il < e->layers; ++il) {
    const EncLayer& L = e->L[(size_t)il];
    // y: the layer's attention-normed rows.  q | k | v of the 8 key/value heads (fp16 rows, or
    // the split product's partial sums), then the q/k norms, the rotary and the K/V stores, each
    // key/value head for its 4 query heads
    ea = EpiArgs{};
    ea.y = qkv;
    ea.ldy = EXN_W + 2 * kEncKV;
    int ns = 0;
    HIPCHK(mm(L.qkv, y, EXN_W, EPI_F16, ea, &ns));
    if (ns > 0)
      HIPCHK(qkv_prep_part(s, part, ns, n, L.vec[E_QNORM], L.vec[E_KNORM], cs, q, kc, vt, 0, lcap, n, kEncGroup));
    else
      HIPCHK(qkv_prep(s, qkv, n, L.vec[E_QNORM], L.vec[E_KNORM], cs, q, kc, vt, 0, lcap, n, kEncGroup));
    HIPCHK(attend(s, q, kc, vt, att, n, 0, n, n, lcap, 0, 0, 1.f));
    ea = EpiArgs{};
    ea.resid = x;
    ea.ldy = EXN_W;
    ea.gate = e->one_gate;
    HIPCHK(mm_norm(L.out, att, EXN_W, ea, L.vec[E_FFN_NORM]));
    ea = EpiArgs{};
    ea.y = ff;
    ea.ldy = EXN_F;
    HIPCHK(mm(L.gate_up, y, EXN_W, EPI_SWIGLU, ea));
    ea = EpiArgs{};
    ea.resid = x;
    ea.ldy = EXN_W;
    ea.gate = e->one_gate;
    // the next layer's attention norm goes with the sums, unless a picture's deep rows are
    // added in between
    const bool deep_add = m > 0 && il < 3 && deep;
    if (il + 1 < e->layers && !deep_add) {
      HIPCHK(mm_norm(L.down, ff, EXN_F, ea, e->L[(size_t)il + 1].vec[E_ATTN_NORM]));
      continue;
    }
    HIPCHK(mm(L.down, ff, EXN_F, EPI_GATE_ADD, ea));
    if (deep_add)
      HIPCHK(gate_add(s, (int64_t)m * EXN_W, EXN_W, 0, 0, 0, x + (int64_t)pic0 * EXN_W, deep + (int64_t)il * m * EXN_W,
                      e->one_gate));
    if (il + 1 < e->layers) HIPCHK(rms_norm(s, n, EXN_W, 1e-6f, x, e->L[(size_t)il + 1].vec[E_ATTN_NORM], y, 1));
  }
  HIPCHK(hipMemcpyAsync(out, x, (size_t)n * EXN_W * 4, hipMemcpyDeviceToDevice, s));
  return EXN_OK;
}


int exn_enc_states_dev(exn_enc* e, const int32_t* ids, int n, const float* cs, int pic0, int m, const float* merged,
                       const float* deep, float* out) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  TRY(use(e->ctx));
  if (!ids || !cs || !out || n < 1 || n > 65536 || m < 0 || (m > 0 && (!merged || pic0 < 0 || pic0 + m > n)))
    FAIL(EXN_EINVAL, "encoder states: n %d, picture rows %d at %d", n, m, pic0);
  TRY(exn_enc_check(e));
  return enc_states(e, ids, n, cs, pic0, m, merged, deep, out);
}

int exn_enc_states(exn_enc* e, const int32_t* ids, int n, const int32_t* pos, int pic0, int m, const float* merged,
                   const float* deep, float* out) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  TRY(use(e->ctx));
  if (!ids || !out || n < 1 || n > 65536 || m < 0 || (m > 0 && (!merged || pic0 < 0 || pic0 + m > n)))
    FAIL(EXN_EINVAL, "encoder states: n %d, picture rows %d at %d", n, m, pic0);
  TRY(exn_enc_check(e));
  for (int t = 0; t < n; ++t)
    if (ids[t] < 0 || ids[t] >= e->vocab) FAIL(EXN_EINVAL, "encoder states: token %d is %d (vocab %lld)", t, ids[t], (long long)e->vocab);
  std::vector<float> cs((size_t)n * 128);
  TRY(exn_enc_rope_table(pos, n, e->base, cs.data()));
  hipStream_t s = e->ctx->stream;
  int32_t* dids;
  float *dcs, *dpic = nullptr, *dout;
  TRY(enc_buf(e, "h_ids", (size_t)n * 4, (void**)&dids));
  TRY(enc_buf(e, "h_cs", cs.size() * 4, (void**)&dcs));
  TRY(enc_buf(e, "h_out", (size_t)n * EXN_W * 4, (void**)&dout));
  if (m > 0) {
    TRY(enc_buf(e, "h_pic", (size_t)(deep ? 4 : 1) * m * EXN_W * 4, (void**)&dpic));
    HIPCHK(hipMemcpyAsync(dpic, merged, (size_t)m * EXN_W * 4, hipMemcpyHostToDevice, s));
    if (deep) HIPCHK(hipMemcpyAsync(dpic + (int64_t)m * EXN_W, deep, (size_t)3 * m * EXN_W * 4, hipMemcpyHostToDevice, s));
  }
  HIPCHK(hipMemcpyAsync(dids, ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(dcs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, s));
  TRY(enc_states(e, dids, n, dcs, pic0, m, dpic, deep && m > 0 ? dpic + (int64_t)m * EXN_W : nullptr, dout));
  HIPCHK(hipMemcpyAsync(out, dout, (size_t)n * EXN_W * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  return EXN_OK;
}
