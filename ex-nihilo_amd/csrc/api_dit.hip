// api_dit.hip -- the DiT: upload-dit's model, dit-velocity's step driver and dit-release
// (src/cuda-dit.lisp), the Euler loop, profiling and the trace.
#include "api_host.h"

// --- the model ---------------------------------------------------------------------

namespace {

// dit-expected (src/weights.lisp:22-45): ggml dims (contiguous first) and the synthetic tensor id
struct Expect {
  int64_t d0, d1;  // d1 = 1 for a vector
  int id;
};

enum Slot { S_NORM_Q = 0, S_NORM_K, S_TO_Q, S_TO_K, S_TO_V, S_TO_OUT, S_GATE_UP, S_OUT };
static const char* kSlots[8] = {"attn.norm_q.weight",   "attn.norm_k.weight",   "attn.to_q.weight",
                                "attn.to_k.weight",     "attn.to_v.weight",     "attn.to_out.0.weight",
                                "img_mlp.gate_up.weight", "img_mlp.out.weight"};
static const char* kEdge[9] = {"img_in.weight",
                               "txt_in.text_norm.weight",
                               "txt_in.in_layer.weight",
                               "txt_in.out_layer.weight",
                               "time_text_embed.timestep_embedder.linear_1.weight",
                               "time_text_embed.timestep_embedder.linear_2.weight",
                               "modulation.1.weight",
                               "norm_out.linear.weight",
                               "proj_out.weight"};

static Expect edge_expect(int i) {
  static const int64_t dims[9][2] = {{EXN_LAT, EXN_W}, {EXN_W, 1},     {EXN_W, EXN_W}, {EXN_W, EXN_W}, {EXN_FREQ, EXN_W},
                                     {EXN_W, EXN_W},   {EXN_W, 4 * EXN_W}, {EXN_W, EXN_W}, {EXN_W, EXN_LAT}};
  return Expect{dims[i][0], dims[i][1], i};
}

static Expect slot_expect(int layer, int s) {
  static const int64_t dims[8][2] = {{EXN_HD, 1},    {EXN_HD, 1},    {EXN_W, EXN_W}, {EXN_W, EXN_W},
                                     {EXN_W, EXN_W}, {EXN_W, EXN_W}, {EXN_W, 2 * EXN_F}, {EXN_F, EXN_W}};
  return Expect{dims[s][0], dims[s][1], 9 + 8 * layer + s};
}

struct Layer {
  exn_w* qkv = nullptr;      // to_q | to_k | to_v rows: 12288 x 4096
  exn_w* out = nullptr;      // to_out.0
  exn_w* gate_up = nullptr;  // 24576 x 4096, gate/up interleaved by 32 rows
  exn_w* down = nullptr;     // img_mlp.out: 4096 x 12288
  float* norm_q = nullptr;
  float* norm_k = nullptr;
  uint8_t have = 0;          // bit per slot
};

}  // namespace

struct exn_dit {
  exn_ctx* ctx = nullptr;
  int layers = 32;
  exn_w* edge[9] = {};      // index as kEdge; [1] unused (text_norm is a vector)
  float* text_norm = nullptr;  // 1 + w
  bool have_edge[9] = {};
  std::vector<Layer> L;
  int32_t* pair_map = nullptr;  // device row map of the gate_up interleave
  bool bf16 = true;             // block matrices run from resident bf16 expansions (exn_dit_resident)
  bool int8 = false;            // the reference's *int8* products (exn_dit_w8a8)
  // scratch
  std::map<std::string, Buf> bufs;
  // kept prompt K/V: per layer K [32][lcap][128] and V^T [32][128][lcap], bf16
  int64_t lcap = 0;
  std::vector<uint16_t*> kc, vt;
  uint64_t kept_key = 0;
  int kept_len = 0;
  bool kept = false;
  // the rotary table for sequence rows 0..l-1 (cos, sin of 64 pairs)
  float* cs = nullptr;
  int64_t cs_rows = 0;
  std::vector<int> cs_key;
  // the residual stream after each block, copied out when set (exn_dit_trace)
  float* trace = nullptr;
  int64_t trace_cap = 0;
  // *dit-trace*'s numbers (exn_dit_stats): (layers + 1) x 4 records of the last velocity
  bool stats_on = false;
  uint32_t* stats = nullptr;   // the "stats" scratch buffer while a velocity with stats_on holds it
  int64_t stats_records = 0;
  // per-launch event pairs by kernel class (exn_dit_profile)
  struct Rec {
    int cls;
    hipEvent_t a, b;
    double flops, bytes;
  };
  unsigned prof = 0;   // bit per kernel class recorded
  int prof_every = 1;  // events around every prof_every-th launch of a recorded class
  int64_t prof_seen[EXN_PROF_CLASSES] = {};
  std::vector<Rec> recs;
  std::vector<hipEvent_t> pool;
  size_t pool_used = 0;
  // the totals of records already folded (the record list is bounded: see prof_fold)
  double fold_ms[EXN_PROF_CLASSES] = {}, fold_flops[EXN_PROF_CLASSES] = {}, fold_bytes[EXN_PROF_CLASSES] = {};
  int64_t fold_n[EXN_PROF_CLASSES] = {};
};

// at most this many recorded launches hold events at once; past it the records so far are
// waited for, summed into the per-class totals and their events reused
static const size_t kProfRecs = 4096;

static void prof_clear(exn_dit* d) {
  d->recs.clear();
  d->pool_used = 0;
  for (int c = 0; c < EXN_PROF_CLASSES; ++c) {
    d->fold_ms[c] = d->fold_flops[c] = d->fold_bytes[c] = 0;
    d->fold_n[c] = 0;
  }
}

static void prof_fold(exn_dit* d) {
  if (hipStreamSynchronize(d->ctx->stream) != hipSuccess) return;
  for (const auto& r : d->recs) {
    float e = 0.f;
    if (hipEventElapsedTime(&e, r.a, r.b) != hipSuccess) continue;
    d->fold_ms[r.cls] += e;
    d->fold_flops[r.cls] += r.flops;
    d->fold_bytes[r.cls] += r.bytes;
    ++d->fold_n[r.cls];
  }
  d->recs.clear();
  d->pool_used = 0;
}

static hipEvent_t prof_event(exn_dit* d) {
  if (d->pool_used == d->pool.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    d->pool.push_back(e);
  }
  return d->pool[d->pool_used++];
}

// a recorded launch: the start event before it, the end event after it
struct ProfScope {
  exn_dit* d;
  int cls;
  double flops, bytes;
  hipEvent_t a = nullptr;
  ProfScope(exn_dit* d_, int c, double f, double b) : d(d_), cls(c), flops(f), bytes(b) {
    if (!(d->prof >> cls & 1u) || d->prof_seen[cls]++ % d->prof_every != 0) return;
    if (d->recs.size() >= kProfRecs) prof_fold(d);
    if ((a = prof_event(d))) (void)hipEventRecord(a, d->ctx->stream);
  }
  ~ProfScope() {
    if (!a) return;
    hipEvent_t b = prof_event(d);
    if (!b) return;
    (void)hipEventRecord(b, d->ctx->stream);
    d->recs.push_back(exn_dit::Rec{cls, a, b, flops, bytes});
  }
};

static int dit_buf(exn_dit* d, const char* key, size_t bytes, void** out) {
  Buf& b = d->bufs[key];
  if (b.bytes < bytes) {
    HIPCHK(hipStreamSynchronize(d->ctx->stream));
    dev_free(b.p);
    b.p = nullptr;
    b.bytes = 0;
    TRY(dev_alloc(&b.p, bytes));
    b.bytes = bytes;
  }
  *out = b.p;
  return EXN_OK;
}

static void dit_free_scratch(exn_dit* d) {
  for (auto& kv : d->bufs) dev_free(kv.second.p);
  d->bufs.clear();
  for (auto p : d->kc) dev_free(p);
  for (auto p : d->vt) dev_free(p);
  d->kc.clear();
  d->vt.clear();
  d->lcap = 0;
  d->kept = false;
  d->kept_key = 0;
  d->kept_len = 0;
  dev_free(d->cs);
  d->cs = nullptr;
  d->cs_rows = 0;
  d->cs_key.clear();
}

// find NAME in dit-expected: edge index (>= 0) or layer/slot
static bool lookup(const exn_dit* d, const char* name, int* edge, int* layer, int* slot) {
  *edge = *layer = *slot = -1;
  for (int i = 0; i < 9; ++i)
    if (!strcmp(name, kEdge[i])) {
      *edge = i;
      return true;
    }
  const char* pre = "transformer_blocks.";
  if (strncmp(name, pre, strlen(pre))) return false;
  const char* r = name + strlen(pre);
  char* end = nullptr;
  const long li = strtol(r, &end, 10);
  if (end == r || *end != '.' || li < 0 || li >= d->layers) return false;
  for (int s = 0; s < 8; ++s)
    if (!strcmp(end + 1, kSlots[s])) {
      *layer = (int)li;
      *slot = s;
      return true;
    }
  return false;
}


int exn_dit_create(exn_ctx* ctx, int layers, exn_dit** out) {
  TRY(use(ctx));
  if (!out) FAIL(EXN_EINVAL, "null output");
  *out = nullptr;
  if (layers < 1 || layers > 32) FAIL(EXN_EINVAL, "layers %d: 1..32", layers);
  exn_dit* d = new exn_dit();
  d->ctx = ctx;
  d->layers = layers;
  d->L.resize((size_t)layers);
  const std::vector<int32_t> map = pair_rows(2 * EXN_F);
  int r = dev_alloc((void**)&d->pair_map, map.size() * 4);
  if (r == EXN_OK) {
    hipError_t e = hipMemcpy(d->pair_map, map.data(), map.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      exn::set_error("pair map upload: %s", hipGetErrorString(e));
      r = EXN_EHIP;
    }
  }
  if (r != EXN_OK) {
    dev_free(d->pair_map);
    delete d;
    return r;
  }
  *out = d;
  return EXN_OK;
}

int exn_dit_destroy(exn_dit* d) {
  if (!d) return EXN_OK;
  (void)hipSetDevice(d->ctx->device);
  (void)hipStreamSynchronize(d->ctx->stream);
  dit_free_scratch(d);
  for (auto& w : d->edge) exn_weight_free(w);
  for (auto& l : d->L) {
    exn_weight_free(l.qkv);
    exn_weight_free(l.out);
    exn_weight_free(l.gate_up);
    exn_weight_free(l.down);
    dev_free(l.norm_q);
    dev_free(l.norm_k);
  }
  dev_free(d->text_norm);
  dev_free(d->pair_map);
  for (auto e : d->pool) (void)hipEventDestroy(e);
  delete d;
  return EXN_OK;
}

int exn_dit_profile(exn_dit* d, int on) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  if (on) {
    HIPCHK(hipStreamSynchronize(d->ctx->stream));
    prof_clear(d);
  }
  d->prof = on < 0 ? (1u << EXN_PROF_CLASSES) - 1u : (unsigned)on & ((1u << EXN_PROF_CLASSES) - 1u);
  return EXN_OK;
}

int exn_dit_profile_every(exn_dit* d, int every) {
  if (!d || every < 1) FAIL(EXN_EINVAL, "profile sampling %d", every);
  d->prof_every = every;
  for (auto& c : d->prof_seen) c = 0;
  return EXN_OK;
}

int exn_dit_profile_read(exn_dit* d, int cls, double* ms, int64_t* launches, double* flops, double* bytes) {
  if (!d || cls < 0 || cls >= EXN_PROF_CLASSES) FAIL(EXN_EINVAL, "profile class %d", cls);
  TRY(use(d->ctx));
  HIPCHK(hipStreamSynchronize(d->ctx->stream));
  double t = d->fold_ms[cls], f = d->fold_flops[cls], b = d->fold_bytes[cls];
  int64_t c = d->fold_n[cls];
  for (const auto& r : d->recs) {
    if (r.cls != cls) continue;
    float e = 0.f;
    HIPCHK(hipEventElapsedTime(&e, r.a, r.b));
    t += e;
    f += r.flops;
    b += r.bytes;
    ++c;
  }
  if (ms) *ms = t;
  if (launches) *launches = c;
  if (flops) *flops = f;
  if (bytes) *bytes = b;
  return EXN_OK;
}

int exn_dit_trace(exn_dit* d, float* buf, int64_t cap) {
  if (!d || (buf && cap < 0)) FAIL(EXN_EINVAL, "trace arguments");
  d->trace = buf;
  d->trace_cap = buf ? cap : 0;
  return EXN_OK;
}

int exn_dit_stats(exn_dit* d, int on) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  d->stats_on = on != 0;
  return EXN_OK;
}

int exn_dit_stats_read(exn_dit* d, float* maxabs, int64_t* nonfinite, int64_t records) {
  if (!d || records < 0 || (records && (!maxabs || !nonfinite))) FAIL(EXN_EINVAL, "stats read arguments");
  TRY(use(d->ctx));
  if (!d->stats) FAIL(EXN_ESTATE, "no velocity has recorded its numbers since the last release (exn_dit_stats)");
  const int64_t k = std::min(records, d->stats_records);
  std::vector<uint32_t> h((size_t)(4 * d->stats_records));
  HIPCHK(hipMemcpyAsync(h.data(), d->stats, h.size() * 4, hipMemcpyDeviceToHost, d->ctx->stream));
  HIPCHK(hipStreamSynchronize(d->ctx->stream));
  for (int64_t i = 0; i < k; ++i) {
    uint32_t m = h[(size_t)(4 * i)];
    memcpy(&maxabs[i], &m, 4);
    nonfinite[i] = (int64_t)((uint64_t)h[(size_t)(4 * i + 2)] | ((uint64_t)h[(size_t)(4 * i + 3)] << 32));
  }
  return EXN_OK;
}

int exn_dit_release(exn_dit* d) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  HIPCHK(hipStreamSynchronize(d->ctx->stream));
  dit_free_scratch(d);
  d->stats = nullptr;
  d->stats_records = 0;
  return EXN_OK;
}

int exn_dit_memory(exn_dit* d, int64_t* weights, int64_t* scratch) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  int64_t w = 0, s = 0;
  auto wb = [](const exn_w* x) -> int64_t {
    if (!x) return 0;
    const int64_t e = x->rows * x->cols;
    return (x->qs ? e + e / 16 : 0) + (x->qt ? tile_q8_bytes(x->rows, x->cols) : 0) + (x->wb ? 2 * e : 0) +
           (x->wf ? 4 * e : 0) + (x->wx ? 2 * e : 0);
  };
  for (auto x : d->edge) w += wb(x);
  for (auto& l : d->L) w += wb(l.qkv) + wb(l.out) + wb(l.gate_up) + wb(l.down) + 2 * 4 * EXN_HD;
  for (auto& kv : d->bufs) s += (int64_t)kv.second.bytes;
  s += (int64_t)(d->kc.size() + d->vt.size()) * d->lcap * EXN_W * 2 + d->cs_rows * 128 * 4;
  if (weights) *weights = w;
  if (scratch) *scratch = s;
  return EXN_OK;
}

// the layer's fused matrix and the rows a tensor takes in it
static int layer_target(exn_dit* d, int layer, int slot, exn_w** w, int64_t* row0, const int32_t** map) {
  Layer& L = d->L[(size_t)layer];
  *row0 = 0;
  *map = nullptr;
  exn_w** slotp = nullptr;
  int64_t rows = EXN_W, cols = EXN_W;
  switch (slot) {
    case S_TO_Q: case S_TO_K: case S_TO_V:
      slotp = &L.qkv; rows = 3 * EXN_W; *row0 = (int64_t)(slot - S_TO_Q) * EXN_W; break;
    case S_TO_OUT: slotp = &L.out; break;
    case S_GATE_UP: slotp = &L.gate_up; rows = 2 * EXN_F; *map = d->pair_map; break;
    case S_OUT: slotp = &L.down; cols = EXN_F; break;
    default: FAIL(EXN_EINVAL, "not a matrix slot");
  }
  if (!*slotp) {
    TRY(w_new(d->ctx, EXN_Q8_0, rows, cols, slotp));
    if (slot == S_GATE_UP) (*slotp)->pairs = true;
  }
  *w = *slotp;
  return EXN_OK;
}

static int set_vector(exn_dit* d, float** dst, int kind, const void* data, int64_t n, bool plus_one) {
  std::vector<float> v((size_t)n);
  if (kind == EXN_F32) {
    memcpy(v.data(), data, (size_t)n * 4);
  } else if (kind == EXN_BF16) {
    const uint16_t* b = (const uint16_t*)data;
    for (int64_t i = 0; i < n; ++i) {
      const uint32_t u = (uint32_t)b[i] << 16;
      memcpy(&v[(size_t)i], &u, 4);
    }
  } else {
    FAIL(EXN_EINVAL, "a vector of kind %d (F32 or BF16 expected)", kind);
  }
  if (plus_one)
    for (auto& x : v) x = 1.f + x;
  if (!*dst) TRY(dev_alloc((void**)dst, (size_t)n * 4));
  HIPCHK(hipMemcpy(*dst, v.data(), (size_t)n * 4, hipMemcpyHostToDevice));
  return EXN_OK;
}

// a layer matrix given a BF16 or F32 slot: from then on its products read wb, which holds every
// slot's rows in bf16 -- the Q8_0 slots' dequantised exactly and rounded, bf16(fp32(d) * q), as the
// resident expansion holds them
static int make_dense(exn_w* w) {
  if (w->dense) return EXN_OK;
  TRY(dev_alloc((void**)&w->wb, (size_t)(w->rows * w->cols) * 2));
  HIPCHK(dequant_q8(w->ctx->stream, w->qs, w->d, w->rows * w->cols, nullptr, w->wb));
  HIPCHK(hipStreamSynchronize(w->ctx->stream));
  dev_free(w->wx);
  w->wx = nullptr;
  w->wx_ok = false;
  w->dense = true;
  return EXN_OK;
}

// ROWS rows of fp32 (KIND EXN_F32, rounded to bf16, RNE) or bf16 host data into a dense layer
// matrix's wb from row ROW0, or (PAIRED: the gate_up matrix) to the rows of the 32-row interleave
static int set_dense_rows(exn_ctx* ctx, exn_w* w, int64_t row0, bool paired, int kind, const void* data,
                          int64_t rows) {
  const int64_t cols = w->cols, count = rows * cols;
  if (!paired) return upload_bf16_from(ctx, data, kind == EXN_F32, count, w->wb + row0 * cols);
  void* t = nullptr;
  TRY(ctx_tmp(ctx, (size_t)count * (kind == EXN_F32 ? 6 : 2), &t));
  uint16_t* tb = (uint16_t*)t;
  if (kind == EXN_F32) {
    float* tf = (float*)(tb + count);
    HIPCHK(hipMemcpyAsync(tf, data, (size_t)count * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(f32_to_bf16(ctx->stream, tf, tb, count));
  } else {
    HIPCHK(hipMemcpyAsync(tb, data, (size_t)count * 2, hipMemcpyHostToDevice, ctx->stream));
  }
  const std::vector<int32_t> map = pair_rows(rows);
  for (int64_t rr = 0; rr < rows; rr += 32)
    HIPCHK(hipMemcpyAsync(w->wb + (row0 + map[(size_t)rr]) * cols, tb + rr * cols, (size_t)(32 * cols) * 2,
                          hipMemcpyDeviceToDevice, ctx->stream));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

int exn_dit_set(exn_dit* d, const char* name, int kind, const void* data, int64_t d0, int64_t d1) {
  if (!d || !name || !data) FAIL(EXN_EINVAL, "null argument");
  TRY(use(d->ctx));
  d->kept = false;   // K/V kept from other weights are not this model's
  int edge, layer, slot;
  if (!lookup(d, name, &edge, &layer, &slot)) FAIL(EXN_EINVAL, "%s: not a tensor of the DiT", name);
  const Expect ex = edge >= 0 ? edge_expect(edge) : slot_expect(layer, slot);
  if (d0 != ex.d0 || d1 != ex.d1)
    FAIL(EXN_EINVAL, "%s is (%lld %lld), not (%lld %lld)", name, (long long)d0, (long long)d1, (long long)ex.d0,
         (long long)ex.d1);
  exn_ctx* ctx = d->ctx;
  if (ex.d1 == 1) {  // a vector
    if (edge == 1) {
      TRY(set_vector(d, &d->text_norm, kind, data, d0, true));
      d->have_edge[1] = true;
    } else {
      Layer& L = d->L[(size_t)layer];
      TRY(set_vector(d, slot == S_NORM_Q ? &L.norm_q : &L.norm_k, kind, data, d0, false));
      L.have |= (uint8_t)(1u << slot);
    }
    return EXN_OK;
  }
  if (kind != EXN_Q8_0 && kind != EXN_F32 && kind != EXN_BF16) FAIL(EXN_EINVAL, "%s: kind %d", name, kind);
  const int64_t rows = d1, cols = d0;
  if (edge >= 0) {
    exn_weight_free(d->edge[edge]);
    d->edge[edge] = nullptr;
    int r = kind == EXN_Q8_0 ? exn_weight_q8_0(ctx, data, rows, cols, &d->edge[edge])
            : kind == EXN_F32 ? exn_weight_f32(ctx, (const float*)data, rows, cols, &d->edge[edge])
                              : exn_weight_bf16(ctx, (const uint16_t*)data, rows, cols, &d->edge[edge]);
    TRY(r);
    d->have_edge[edge] = true;
    return EXN_OK;
  }
  exn_w* w = nullptr;
  int64_t row0 = 0;
  const int32_t* map = nullptr;
  TRY(layer_target(d, layer, slot, &w, &row0, &map));
  if (kind == EXN_Q8_0) {
    TRY(upload_q8_blocks(ctx, data, rows, cols, map, w->qs + row0 * cols, w->d + row0 * (cols / 32)));
    w->wx_ok = false;
    TRY(retile(w));
    if (w->dense) {  // the slot's rows into the dense rows too (gate_up's slot is the whole matrix)
      HIPCHK(dequant_q8(ctx->stream, w->qs + row0 * cols, w->d + row0 * (cols / 32), rows * cols, nullptr,
                        w->wb + row0 * cols));
      HIPCHK(hipStreamSynchronize(ctx->stream));
    }
  } else {
    // upload-dit takes BF16 and F32 matrices too (src/cuda-dit.lisp:77-80); the block products take
    // bf16 operands, so F32 rows are rounded to bf16 here
    TRY(make_dense(w));
    TRY(set_dense_rows(ctx, w, row0, map != nullptr, kind, data, rows));
  }
  d->L[(size_t)layer].have |= (uint8_t)(1u << slot);
  return EXN_OK;
}

int exn_dit_synth(exn_dit* d, uint64_t seed) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  d->kept = false;
  hipStream_t s = d->ctx->stream;
  for (int i = 0; i < 9; ++i) {
    const Expect ex = edge_expect(i);
    const uint64_t key = gen_key(seed, (uint64_t)ex.id);
    if (i == 1) {
      if (!d->text_norm) TRY(dev_alloc((void**)&d->text_norm, EXN_W * 4));
      HIPCHK(synth_normal(s, key, EXN_W, 1.f, 0.05f, 1, d->text_norm));  // used as 1 + 0.05 z
    } else {
      if (!d->edge[i] || d->edge[i]->kind != EXN_Q8_0) {
        exn_weight_free(d->edge[i]);
        d->edge[i] = nullptr;
        TRY(w_new(d->ctx, EXN_Q8_0, ex.d1, ex.d0, &d->edge[i]));
      }
      HIPCHK(synth_q8(s, key, ex.d1, ex.d0, ex.d0 / 32, nullptr, d->edge[i]->qs, d->edge[i]->d));
      TRY(retile(d->edge[i]));
    }
    d->have_edge[i] = true;
  }
  for (int layer = 0; layer < d->layers; ++layer) {
    Layer& L = d->L[(size_t)layer];
    for (int sl = 0; sl < 8; ++sl) {
      const Expect ex = slot_expect(layer, sl);
      const uint64_t key = gen_key(seed, (uint64_t)ex.id);
      if (sl == S_NORM_Q || sl == S_NORM_K) {
        float** v = sl == S_NORM_Q ? &L.norm_q : &L.norm_k;
        if (!*v) TRY(dev_alloc((void**)v, EXN_HD * 4));
        HIPCHK(synth_normal(s, key, EXN_HD, 1.f, 0.05f, 1, *v));
      } else {
        exn_w* w = nullptr;
        int64_t row0 = 0;
        const int32_t* map = nullptr;
        TRY(layer_target(d, layer, sl, &w, &row0, &map));
        HIPCHK(synth_q8(s, key, ex.d1, ex.d0, ex.d0 / 32, map, w->qs + row0 * ex.d0, w->d + row0 * (ex.d0 / 32)));
        w->wx_ok = false;
        TRY(retile(w));
        if (w->dense) {  // every slot of the matrix is made Q8_0 again here
          HIPCHK(hipStreamSynchronize(s));
          dev_free(w->wb);
          w->wb = nullptr;
          w->dense = false;
        }
      }
      L.have |= (uint8_t)(1u << sl);
    }
  }
  HIPCHK(hipStreamSynchronize(s));
  return EXN_OK;
}

int exn_dit_resident(exn_dit* d, int bf16) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  if (d->bf16 != (bf16 != 0)) d->kept = false;   // the other product path: K/V recomputed
  d->bf16 = bf16 != 0;
  for (auto& l : d->L)
    for (exn_w* w : {l.qkv, l.out, l.gate_up, l.down})
      if (w) TRY(w_resident(w, d->bf16));
  HIPCHK(hipStreamSynchronize(d->ctx->stream));
  return EXN_OK;
}

int exn_dit_w8a8(exn_dit* d, int on) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  if (d->int8 != (on != 0)) d->kept = false;   // other products: K/V recomputed
  d->int8 = on != 0;
  return EXN_OK;
}

int exn_dit_check(exn_dit* d) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  std::string missing;
  int count = 0;
  for (int i = 0; i < 9; ++i)
    if (!d->have_edge[i]) {
      if (count++ < 8) missing += std::string("\n  missing ") + kEdge[i];
    }
  for (int l = 0; l < d->layers; ++l)
    for (int s = 0; s < 8; ++s)
      if (!(d->L[(size_t)l].have & (1u << s))) {
        if (count++ < 8) missing += "\n  missing transformer_blocks." + std::to_string(l) + "." + kSlots[s];
      }
  if (count) FAIL(EXN_ESTATE, "%d tensors missing:%s%s", count, missing.c_str(), count > 8 ? "\n  ..." : "");
  return EXN_OK;
}


// --- a step (dit-velocity, src/cuda-dit.lisp:137-243) --------------------------------

// every row's (frame, row, col) -- dit-positions (src/host.lisp:37-50)
static void positions(int p, int h, int w, int a, int rh, int rw, bool edit, std::vector<int>& pos) {
  pos.clear();
  auto image = [&](int frame, int hh, int ww) {
    for (int r = 0; r < hh; ++r)
      for (int c = 0; c < ww; ++c) {
        pos.push_back(frame);
        pos.push_back(r - (hh - hh / 2));
        pos.push_back(c - (ww - ww / 2));
      }
  };
  auto text = [&](int x) { pos.push_back(x); pos.push_back(x); pos.push_back(x); };
  if (!edit) {
    for (int i = 0; i < p; ++i) text(i);
    image(p, h, w);
  } else {
    const int after = p - a - rh * rw, start = a + (rh > rw ? rh : rw);
    for (int i = 0; i < a; ++i) text(i);
    image(a, rh, rw);
    for (int i = 0; i < after; ++i) text(start + i);
    image(start + after, h, w);
  }
}

// rope-table (src/host.lisp:19-30): cos, sin of each row's 64 angles, in double, rounded
static void rope_table(const std::vector<int>& pos, std::vector<float>& cs) {
  static const int axes[3] = {16, 56, 56};
  const size_t rows = pos.size() / 3;
  cs.assign(rows * 128, 0.f);
  for (size_t t = 0; t < rows; ++t) {
    int j = 0;
    for (int a = 0; a < 3; ++a)
      for (int i = 0; i < axes[a] / 2; ++i, ++j) {
        const double ang = (double)pos[3 * t + a] * (1.0 / std::pow(10000.0, (double)(2 * i) / axes[a]));
        cs[t * 128 + 2 * j] = (float)std::cos(ang);
        cs[t * 128 + 2 * j + 1] = (float)std::sin(ang);
      }
  }
}

// timestep-embedding (src/host.lisp:9-15) of t and of 0, in double on the device: 2 x 256 floats
__global__ void k_time_embed(double t, float* __restrict__ emb) {
  const int j = threadIdx.x;  // 128 threads
  const double f = exp(-log(10000.0) * j / 128.0);
  const double a = t * f;
  emb[j] = (float)cos(a);
  emb[128 + j] = (float)sin(a);
  emb[256 + j] = 1.f;
  emb[256 + 128 + j] = 0.f;
}

static int ensure_kv(exn_dit* d, int64_t l, int keep_rows) {
  const int64_t need = (l + 63) / 64 * 64;
  if (d->lcap >= need && (int)d->kc.size() == d->layers) return EXN_OK;
  const int64_t lcap = need + 256;  // room for a longer prompt without moving again
  hipStream_t s = d->ctx->stream;
  std::vector<uint16_t*> kc((size_t)d->layers, nullptr), vt((size_t)d->layers, nullptr);
  int r = EXN_OK;
  for (int i = 0; i < d->layers && r == EXN_OK; ++i) {
    r = dev_alloc((void**)&kc[(size_t)i], (size_t)(EXN_H * lcap * EXN_HD) * 2);
    if (r == EXN_OK) r = dev_alloc((void**)&vt[(size_t)i], (size_t)(EXN_H * lcap * EXN_HD) * 2);
    if (r == EXN_OK) {
      // keys past l are masked, but V^T's columns there enter P V with P = 0: keep them finite
      if (hipMemsetAsync(kc[(size_t)i], 0, (size_t)(EXN_H * lcap * EXN_HD) * 2, s) != hipSuccess ||
          hipMemsetAsync(vt[(size_t)i], 0, (size_t)(EXN_H * lcap * EXN_HD) * 2, s) != hipSuccess)
        r = EXN_EHIP;
    }
    if (r == EXN_OK && keep_rows > 0 && i < (int)d->kc.size()) {  // carry the kept prompt rows over
      // V^T's key columns are permuted inside aligned groups of 16 (vt_pos): whole groups move
      const int64_t vcols = (keep_rows + 15) / 16 * 16;
      if (hipMemcpy2DAsync(kc[(size_t)i], (size_t)(lcap * EXN_HD * 2), d->kc[(size_t)i], (size_t)(d->lcap * EXN_HD * 2),
                           (size_t)(keep_rows * EXN_HD * 2), EXN_H, hipMemcpyDeviceToDevice, s) != hipSuccess ||
          hipMemcpy2DAsync(vt[(size_t)i], (size_t)(lcap * 2), d->vt[(size_t)i], (size_t)(d->lcap * 2),
                           (size_t)(vcols * 2), EXN_H * EXN_HD, hipMemcpyDeviceToDevice, s) != hipSuccess)
        r = EXN_EHIP;
    }
  }
  if (r == EXN_OK && hipStreamSynchronize(s) != hipSuccess) r = EXN_EHIP;
  if (r != EXN_OK) {
    for (auto p : kc) dev_free(p);
    for (auto p : vt) dev_free(p);
    if (r == EXN_EHIP) exn::set_error("prefix K/V allocation: %s", hipGetErrorString(hipGetLastError()));
    return r;
  }
  for (auto p : d->kc) dev_free(p);
  for (auto p : d->vt) dev_free(p);
  d->kc = kc;
  d->vt = vt;
  d->lcap = lcap;
  return EXN_OK;
}

static int ensure_rope(exn_dit* d, int p, int h, int w, int a, int rh, int rw, bool edit) {
  const std::vector<int> key = {p, h, w, a, rh, rw, edit ? 1 : 0};
  if (d->cs && d->cs_key == key) return EXN_OK;
  std::vector<int> pos;
  positions(p, h, w, a, rh, rw, edit, pos);
  std::vector<float> cs;
  rope_table(pos, cs);
  const int64_t rows = (int64_t)(pos.size() / 3);
  HIPCHK(hipStreamSynchronize(d->ctx->stream));
  if (d->cs_rows < rows) {
    dev_free(d->cs);
    d->cs = nullptr;
    d->cs_rows = 0;
    TRY(dev_alloc((void**)&d->cs, (size_t)rows * 128 * 4));
    d->cs_rows = rows;
  }
  HIPCHK(hipMemcpy(d->cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  d->cs_key = key;
  return EXN_OK;
}

static int velocity(exn_dit* d, const float* context, int ptext, const float* latent, int h, int w, double sigma,
                    uint64_t prefix_key, int ref_a, const float* ref_latent, int rh, int rw, float* v) {
  TRY(exn_dit_check(d));
  if (h <= 0 || w <= 0 || ptext < 0 || !latent || !v) FAIL(EXN_EINVAL, "velocity: h %d, w %d, p %d", h, w, ptext);
  const bool edit = ref_latent != nullptr;
  if (edit && (rh <= 0 || rw <= 0 || ref_a < 0 || ref_a > ptext)) FAIL(EXN_EINVAL, "reference picture: a %d, %d x %d", ref_a, rh, rw);
  if (d->bf16)
    for (auto& l : d->L)
      for (exn_w* m : {l.qkv, l.out, l.gate_up, l.down}) TRY(w_resident(m, true));
  exn_ctx* ctx = d->ctx;
  hipStream_t s = ctx->stream;
  const int64_t nimg = (int64_t)h * w;
  const int nref = edit ? rh * rw : 0, a = edit ? ref_a : 0;
  const int p = ptext + nref;  // the prefix: text and the reference picture
  const bool cached = prefix_key != 0 && d->kept && d->kept_key == prefix_key && d->kept_len == p;
  const int n0 = cached ? p : 0;
  const int64_t n = cached ? nimg : p + nimg, l = p + nimg;
  if (!cached && ptext > 0 && !context) FAIL(EXN_EINVAL, "velocity: null context on an uncached pass");
  if (l > (1 << 24)) FAIL(EXN_EINVAL, "sequence of %lld rows", (long long)l);

  TRY(ensure_kv(d, l, cached ? p : 0));
  TRY(ensure_rope(d, p, h, w, a, rh, rw, edit));
  if (!cached) d->kept = false;

  float *emb, *e1, *e2, *mod, *sc, *x, *vrows, *tok;
  uint16_t *y, *qkv, *q, *att, *ff;
  TRY(dit_buf(d, "emb", 512 * 4, (void**)&emb));
  TRY(dit_buf(d, "e1", 2 * EXN_W * 4, (void**)&e1));
  TRY(dit_buf(d, "e2", 2 * EXN_W * 4, (void**)&e2));
  TRY(dit_buf(d, "mod", 2 * 4 * EXN_W * 4, (void**)&mod));
  TRY(dit_buf(d, "sc", EXN_W * 4, (void**)&sc));
  TRY(dit_buf(d, "x", (size_t)(l * EXN_W) * 4, (void**)&x));
  TRY(dit_buf(d, "y", (size_t)(l * EXN_W) * 2, (void**)&y));
  TRY(dit_buf(d, "qkv", (size_t)(l * 3 * EXN_W) * 2, (void**)&qkv));
  float* part = nullptr;   // split-K partials: an uncached pass's prompt rows, image rows past whole waves
  const int64_t nh = std::max<int64_t>(0, std::min<int64_t>(p - n0, n));
  TRY(dit_buf(d, "split", (size_t)kSplitCap * 4, (void**)&part));
  TRY(dit_buf(d, "q", (size_t)(l * EXN_W) * 2, (void**)&q));
  TRY(dit_buf(d, "att", (size_t)(l * EXN_W) * 2, (void**)&att));
  TRY(dit_buf(d, "ff", (size_t)(l * EXN_F) * 2, (void**)&ff));
  // *dit-trace*'s numbers (src/metal-dit.lisp:206-213,254-257) when exn_dit_stats is on: record
  // 4 row + slot, row 0 before the blocks (slot 0 the stream, 3 txt_in's GELU rows), row 1 + l
  // after block l (0 the stream, 1 the attention's output, 2 the MLP's inner rows)
  uint32_t* st = nullptr;
  if (d->stats_on) {
    d->stats_records = (int64_t)(d->layers + 1) * 4;
    TRY(dit_buf(d, "stats", (size_t)d->stats_records * 16, (void**)&st));
    d->stats = st;
    HIPCHK(tensor_stats_clear(s, st, d->stats_records));
  }
  auto stat = [&](int row, int slot, const void* t, int bf16, int64_t count) -> hipError_t {
    return st ? tensor_stats(s, t, bf16, count, st + 4 * (4 * row + slot)) : hipSuccess;
  };
  TRY(dit_buf(d, "tok", (size_t)((nimg > nref ? nimg : nref) * EXN_LAT) * 4, (void**)&tok));
  TRY(dit_buf(d, "vrows", (size_t)(nimg * EXN_LAT) * 4, (void**)&vrows));
  // split-K partials of the edge products with few tiles (proj_out's 64 columns, txt_in over few
  // prompt rows): S slices of M x N with S <= 1024 / tiles of 64 x 64, so S M N <= 1024 x 4096
  // whatever the shape.  The cap never binds, so a product's split follows its own shape only and
  // a prompt's rows come out the same over any picture (the kept K/V stay valid).
  float* epart = nullptr;
  const int64_t epart_cap = (int64_t)1024 * 64 * 64;
  TRY(dit_buf(d, "epart", (size_t)epart_cap * 4, (void**)&epart));

  // the int8 mode (exn_dit_w8a8) takes a Q8_0 matrix's products of at least 16 rows the
  // reference's int8 way (src/cuda-dit.lisp:119-124): the fp32 activations quantised to Q8_0
  // (xq, xd), then the int8 product with per-block scales
  auto int8_ok = [&](const exn_w* W, int64_t m) {
    return d->int8 && W && W->kind == EXN_Q8_0 && !W->dense && W->qs && m >= 16;
  };
  int8_t* xq = nullptr;
  uint16_t* xd = nullptr;
  if (d->int8) {
    TRY(dit_buf(d, "i8q", (size_t)(std::max<int64_t>(l, 256) * EXN_F), (void**)&xq));
    TRY(dit_buf(d, "i8d", (size_t)(std::max<int64_t>(l, 256) * (EXN_F / 32)) * 2, (void**)&xd));
  }
  // an edge product in fp32: Y (m rows, ldy apart) = X (m rows of the matrix's inputs) W^T
  auto edge_mm = [&](int e, const float* xin, int64_t m, float* yout, int gelu) {
    const exn_w* W = d->edge[e];
    if (int8_ok(W, m)) {
      hipError_t r = quant_q8(s, xin, 0, W->cols, m, W->cols, xq, xd);
      if (r == hipSuccess) r = gemm_w8a8(s, xq, xd, m, W->qs, W->d, W->rows, W->cols, yout, W->rows, 0);
      if (r == hipSuccess && gelu) r = gelu_tanh(s, m * W->rows, yout);
      return r;
    }
    return gemm_f32(s, xin, W->cols, W->qs, W->d, W->wb, W->wf, m, W->rows, W->cols, yout, W->rows, gelu, epart,
                    epart_cap);
  };
  {
  ProfScope prologue(d, EXN_PROF_EDGE, 0, 0);
  // the timestep: t and 0 through the embedder, SiLU, the shared modulation (src/cuda-dit.lisp:157-167)
  hipLaunchKernelGGL(k_time_embed, dim3(1), dim3(128), 0, s, 1000.0 * sigma, emb);
  HIPCHK(hipGetLastError());
  auto gv = [&](int e, const float* xin, int64_t m, float* yout, int act) {
    const exn_w* W = d->edge[e];
    return gemv_q8(s, xin, W->cols, W->qs, W->d, W->wb, W->wf, m, W->rows, W->cols, yout, W->rows, act);
  };
  HIPCHK(gv(4, emb, 2, e1, 1));
  HIPCHK(gv(5, e1, 2, e2, 1));
  HIPCHK(gv(6, e2, 2, mod, 0));
  HIPCHK(gv(7, e2, 1, sc, 0));

  // the joint sequence: the prompt through txt_in (unless cached), the image through img_in
  if (!cached && ptext > 0) {
    float *t1, *h1;
    TRY(dit_buf(d, "t1", (size_t)(ptext * EXN_W) * 4, (void**)&t1));
    TRY(dit_buf(d, "h1", (size_t)(ptext * EXN_W) * 4, (void**)&h1));
    HIPCHK(rms_norm(s, ptext, EXN_W, 1e-6f, context, d->text_norm, t1, 0));
    HIPCHK(edge_mm(2, t1, ptext, h1, 1));
    HIPCHK(stat(0, 3, h1, 0, ptext * EXN_W));
    float* txt = x;
    if (edit) TRY(dit_buf(d, "txt", (size_t)(ptext * EXN_W) * 4, (void**)&txt));
    HIPCHK(edge_mm(3, h1, ptext, txt, 0));
    if (edit) {  // text before the picture, the picture through img_in, the text after
      HIPCHK(hipMemcpyAsync(x, txt, (size_t)a * EXN_W * 4, hipMemcpyDeviceToDevice, s));
      HIPCHK(hipMemcpyAsync(x + (int64_t)(a + nref) * EXN_W, txt + (int64_t)a * EXN_W, (size_t)(ptext - a) * EXN_W * 4,
                            hipMemcpyDeviceToDevice, s));
    }
  }
  if (!cached && edit) {
    HIPCHK(latent_rows(s, ref_latent, nref, tok));
    HIPCHK(edge_mm(0, tok, nref, x + (int64_t)a * EXN_W, 0));
  }
  HIPCHK(latent_rows(s, latent, nimg, tok));
  HIPCHK(edge_mm(0, tok, nimg, x + (int64_t)(p - n0) * EXN_W, 0));
  }
  EpiArgs ea{};

  // the blocks (src/cuda-dit.lisp:196-231)
  const int ms = 4 * EXN_W;
  const int b0 = a, b1 = a + nref;
  double pairs = 0;  // visible (query, key) pairs under xa_lim
  for (int64_t g = n0; g < n0 + n; ++g)
    pairs += (double)(g >= p ? l : (g >= b0 && g < b1 ? b1 : g + 1));
  const double nd = (double)n, Wd = EXN_W, Fd = EXN_F;
  const double ln_bytes = nd * Wd * (4 + 2), qkv_bytes = nd * 3 * Wd * 2 * 2 + nd * 128 * 4;
  if (d->trace && n * EXN_W <= d->trace_cap)
    HIPCHK(hipMemcpyAsync(d->trace, x, (size_t)(n * EXN_W) * 4, hipMemcpyDeviceToDevice, s));
  HIPCHK(stat(0, 0, x, 0, n * EXN_W));
  float *a32 = nullptr, *h32 = nullptr, *gu32 = nullptr, *ff32 = nullptr;   // the int8 block's fp32 rows
  for (int il = 0; il < d->layers; ++il) {
    Layer& L = d->L[(size_t)il];
    if (int8_ok(L.qkv, n) && int8_ok(L.out, n) && int8_ok(L.gate_up, n) && int8_ok(L.down, n) && L.gate_up->pairs) {
      // the reference's *int8* block (src/cuda-dit.lisp:196-231 with mm at :119-124): each
      // product's fp32 input quantised, the int8 product to fp32 (QKV: fp16 rows for qkv_prep),
      // and the elementwise steps apart, as the reference runs them
      if (!a32) {
        TRY(dit_buf(d, "a32", (size_t)(l * EXN_W) * 4, (void**)&a32));
        TRY(dit_buf(d, "h32", (size_t)(l * EXN_W) * 4, (void**)&h32));
        TRY(dit_buf(d, "gu32", (size_t)(l * 2 * EXN_F) * 4, (void**)&gu32));
        TRY(dit_buf(d, "ff32", (size_t)(l * EXN_F) * 4, (void**)&ff32));
      }
      {
        ProfScope ps(d, EXN_PROF_LN_MOD, 0, nd * Wd * 8);
        HIPCHK(ln_mod(s, (int)n, n0, p, ms, x, EXN_W, mod + 0 * EXN_W, a32, 0));
      }
      {
        ProfScope ps(d, EXN_PROF_QKV, 2 * nd * 3 * Wd * Wd, nd * Wd * 5 + 3 * Wd * Wd * 1.0625 + nd * 3 * Wd * 2);
        HIPCHK(quant_q8(s, a32, 0, EXN_W, n, EXN_W, xq, xd));
        HIPCHK(gemm_w8a8(s, xq, xd, n, L.qkv->qs, L.qkv->d, 3 * EXN_W, EXN_W, qkv, 3 * EXN_W, 1));
      }
      {
        ProfScope ps(d, EXN_PROF_QKV_PREP, 0, qkv_bytes);
        HIPCHK(qkv_prep(s, qkv, n, L.norm_q, L.norm_k, d->cs, q, d->kc[(size_t)il], d->vt[(size_t)il], n0, d->lcap, n));
      }
      {
        ProfScope ps(d, EXN_PROF_ATTEND, 4.0 * EXN_HD * EXN_H * pairs, nd * Wd * 2 * 3 + 2.0 * l * Wd * 2);
        HIPCHK(attend(s, q, d->kc[(size_t)il], d->vt[(size_t)il], a32, (int)n, n0, p, (int)l, d->lcap, b0, b1, 1.f, 1));
      }
      {
        ProfScope ps(d, EXN_PROF_OUT, 2 * nd * Wd * Wd, nd * Wd * 5 + Wd * Wd * 1.0625 + nd * Wd * 4 * 4);
        HIPCHK(quant_q8(s, a32, 0, EXN_W, n, EXN_W, xq, xd));
        HIPCHK(gemm_w8a8(s, xq, xd, n, L.out->qs, L.out->d, EXN_W, EXN_W, h32, EXN_W, 0));
        HIPCHK(gate_add(s, n * EXN_W, EXN_W, n0, p, ms, x, h32, mod + 1 * EXN_W));
      }
      {
        ProfScope ps(d, EXN_PROF_LN_MOD, 0, nd * Wd * 8);
        HIPCHK(ln_mod(s, (int)n, n0, p, ms, x, EXN_W, mod + 2 * EXN_W, a32, 0));
      }
      {
        ProfScope ps(d, EXN_PROF_GATE_UP, 2 * nd * Wd * 2 * Fd, nd * Wd * 5 + 2 * Fd * Wd * 1.0625 + nd * Fd * 16);
        HIPCHK(quant_q8(s, a32, 0, EXN_W, n, EXN_W, xq, xd));
        HIPCHK(gemm_w8a8(s, xq, xd, n, L.gate_up->qs, L.gate_up->d, 2 * EXN_F, EXN_W, gu32, 2 * EXN_F, 0));
        HIPCHK(swiglu_pairs(s, n, EXN_F, gu32, ff32));
      }
      {
        ProfScope ps(d, EXN_PROF_DOWN, 2 * nd * Fd * Wd, nd * Fd * 5 + Fd * Wd * 1.0625 + nd * Wd * 4 * 4);
        HIPCHK(quant_q8(s, ff32, 0, EXN_F, n, EXN_F, xq, xd));
        HIPCHK(gemm_w8a8(s, xq, xd, n, L.down->qs, L.down->d, EXN_W, EXN_F, h32, EXN_W, 0));
        HIPCHK(gate_add(s, n * EXN_W, EXN_W, n0, p, ms, x, h32, mod + 3 * EXN_W));
      }
      HIPCHK(stat(il + 1, 0, x, 0, n * EXN_W));
      HIPCHK(stat(il + 1, 1, a32, 0, n * EXN_W));
      HIPCHK(stat(il + 1, 2, ff32, 0, n * EXN_F));
      if (d->trace && (int64_t)(il + 2) * n * EXN_W <= d->trace_cap)
        HIPCHK(hipMemcpyAsync(d->trace + (int64_t)(il + 1) * n * EXN_W, x, (size_t)(n * EXN_W) * 4,
                              hipMemcpyDeviceToDevice, s));
      continue;
    }
    {
      ProfScope ps(d, EXN_PROF_LN_MOD, 0, ln_bytes);
      HIPCHK(ln_mod(s, (int)n, n0, p, ms, x, EXN_W, mod + 0 * EXN_W, y, 1));
    }
    // the QKV product with qk-norm, RoPE and the K/V^T stores in its epilogue (bf16 or Q8_0
    // weights), else (shapes the fused path does not take) the product to fp16 rows and
    // qkv_prep over them.  An uncached pass's prompt rows (at most 256) go apart first, through
    // the few-row product with its K split, whose partial sums qkv_prep_part reads (fp16 rows and
    // qkv_prep where the product ran whole), so that the image rows' fused product runs
    // whole waves of tiles (4096 rows: 768 tiles, 3 waves, where the 256 prompt rows with them
    // make 816, a fourth wave of 48).  Every pass computes its image rows alike.
    int64_t qh = 0;   // the rows done apart
    if (nh > 0 && nh < n && nh <= 256) {
      int ns = 0;   // the partial sums left in part (0: fp16 rows in qkv)
      {
        ProfScope ps(d, EXN_PROF_QKV, 2.0 * nh * 3 * Wd * Wd, nh * Wd * 2 + 3 * Wd * Wd * 1.0625 + nh * 3 * Wd * 2);
        ea = EpiArgs{};
        ea.y = qkv;
        ea.ldy = 3 * EXN_W;
        const hipError_t r = gemm_split_rows(s, y, EXN_W, wop_n(L.qkv, nh), nh, 3 * EXN_W, EXN_W, EPI_F16, ea, part,
                                             kSplitCap, 8, &ns);
        if (r != hipErrorNotSupported) HIPCHK(r);
        if (r == hipSuccess) qh = nh;
      }
      if (qh) {
        ProfScope ps(d, EXN_PROF_QKV_PREP, 0, (double)nh * (3 * Wd * (ns > 0 ? 4.0 * ns : 2.0) + 3 * Wd * 2 + 128 * 4));
        if (ns > 0)
          HIPCHK(qkv_prep_part(s, part, ns, nh, L.norm_q, L.norm_k, d->cs, q, d->kc[(size_t)il], d->vt[(size_t)il], n0,
                               d->lcap, n));
        else
          HIPCHK(qkv_prep(s, qkv, nh, L.norm_q, L.norm_k, d->cs, q, d->kc[(size_t)il], d->vt[(size_t)il], n0, d->lcap,
                          n));
      }
    }
    const double nq = nd - (double)qh;
    bool fused = false;
    {
      ProfScope ps(d, EXN_PROF_QKV, 2 * nq * 3 * Wd * Wd, nq * Wd * 2 + 3 * Wd * Wd * 1.0625 + nq * 3 * Wd * 2);
      ea = EpiArgs{};
      ea.n0 = n0 + (int)qh;
      ea.wq = L.norm_q;
      ea.wk = L.norm_k;
      ea.cs = d->cs;
      ea.qscale = QK_QSCALE;
      ea.q = q + qh * EXN_HD;
      ea.qld = n;
      ea.kc = d->kc[(size_t)il];
      ea.vt = d->vt[(size_t)il];
      ea.lcap = d->lcap;
      const hipError_t r = gemm_qkv(s, y + qh * EXN_W, EXN_W, wop(L.qkv), n - qh, EXN_W, ea);
      if (r != hipErrorNotSupported) HIPCHK(r);
      fused = r == hipSuccess;
    }
    if (!fused) {
      {
        ProfScope ps(d, EXN_PROF_QKV, 2 * nq * 3 * Wd * Wd, nq * Wd * 2 + 3 * Wd * Wd * 1.0625 + nq * 3 * Wd * 2);
        ea = EpiArgs{};
        ea.y = qkv + qh * 3 * EXN_W;
        ea.ldy = 3 * EXN_W;
        HIPCHK(gemm_any(s, L.qkv, y + qh * EXN_W, EXN_W, n - qh, EPI_F16, ea));
      }
      ProfScope ps(d, EXN_PROF_QKV_PREP, 0, qkv_bytes * nq / nd);
      HIPCHK(qkv_prep(s, qkv + qh * 3 * EXN_W, n - qh, L.norm_q, L.norm_k, d->cs, q + qh * EXN_HD, d->kc[(size_t)il],
                      d->vt[(size_t)il], n0 + qh, d->lcap, n));
    }
    // The last block's prompt rows: once their K/V are kept (the QKV product above), nothing
    // reads what the rest of the block makes of them -- the step's output is the image rows'
    // -- so the attention and the products from here on take rows r0.. only, the image rows,
    // tiled as in a cached pass.  A traced pass, or one recording its numbers, takes every row.
    const int64_t r0 = il + 1 == d->layers && !d->trace && !st ? nh : 0;
    const int64_t nr = n - r0, nhr = nh - r0;
    const double ndr = (double)nr;
    {
      ProfScope ps(d, EXN_PROF_ATTEND, 4.0 * EXN_HD * EXN_H * pairs, ndr * Wd * 2 * 2 + 2.0 * l * Wd * 2);
      HIPCHK(attend(s, q + r0 * EXN_HD, d->kc[(size_t)il], d->vt[(size_t)il], att + r0 * EXN_W, (int)nr, n0 + (int)r0,
                    p, (int)l, d->lcap, b0, b1, 1.f, 0, n));
    }
    {
      ProfScope ps(d, EXN_PROF_OUT, 2 * ndr * Wd * Wd, ndr * Wd * 2 + Wd * Wd * 1.0625 + ndr * Wd * 4 * 2);
      ea = EpiArgs{};
      ea.resid = x + r0 * EXN_W;
      ea.ldy = EXN_W;
      ea.gate = mod + 1 * EXN_W;
      ea.n0 = n0 + (int)r0;
      ea.p = p;
      ea.mstride = ms;
      HIPCHK(block_mm(s, L.out, att + r0 * EXN_W, EXN_W, nr, nhr, EPI_GATE_ADD, ea, part));
    }
    {
      ProfScope ps(d, EXN_PROF_LN_MOD, 0, ln_bytes * ndr / nd);
      HIPCHK(ln_mod(s, (int)nr, n0 + (int)r0, p, ms, x + r0 * EXN_W, EXN_W, mod + 2 * EXN_W, y + r0 * EXN_W, 1));
    }
    {
      ProfScope ps(d, EXN_PROF_GATE_UP, 2 * ndr * Wd * 2 * Fd, ndr * Wd * 2 + 2 * Fd * Wd * 1.0625 + ndr * Fd * 2);
      ea = EpiArgs{};
      ea.y = ff + r0 * EXN_F;
      ea.ldy = EXN_F;
      HIPCHK(block_mm(s, L.gate_up, y + r0 * EXN_W, EXN_W, nr, nhr, EPI_SWIGLU, ea, part));
    }
    {
      ProfScope ps(d, EXN_PROF_DOWN, 2 * ndr * Fd * Wd, ndr * Fd * 2 + Fd * Wd * 1.0625 + ndr * Wd * 4 * 2);
      ea = EpiArgs{};
      ea.resid = x + r0 * EXN_W;
      ea.ldy = EXN_W;
      ea.gate = mod + 3 * EXN_W;
      ea.n0 = n0 + (int)r0;
      ea.p = p;
      ea.mstride = ms;
      HIPCHK(block_mm(s, L.down, ff + r0 * EXN_F, EXN_F, nr, nhr, EPI_GATE_ADD, ea, part));
    }
    HIPCHK(stat(il + 1, 0, x, 0, n * EXN_W));
    HIPCHK(stat(il + 1, 1, att, 1, n * EXN_W));
    HIPCHK(stat(il + 1, 2, ff, 1, n * EXN_F));
    if (d->trace && (int64_t)(il + 2) * n * EXN_W <= d->trace_cap)
      HIPCHK(hipMemcpyAsync(d->trace + (int64_t)(il + 1) * n * EXN_W, x, (size_t)(n * EXN_W) * 4,
                            hipMemcpyDeviceToDevice, s));
  }
  if (prefix_key != 0 && !cached) {
    d->kept = true;
    d->kept_key = prefix_key;
    d->kept_len = p;
  }
  // the image's rows: LayerNorm * (1 + scale(t)), proj_out (src/cuda-dit.lisp:235-243)
  ProfScope epilogue(d, EXN_PROF_EDGE, 0, 0);
  float* yf;
  TRY(dit_buf(d, "yf", (size_t)(nimg * EXN_W) * 4, (void**)&yf));
  HIPCHK(ln_mod(s, (int)nimg, 0, 0, 0, x + (int64_t)(p - n0) * EXN_W, EXN_W, sc, yf, 0));
  HIPCHK(edge_mm(8, yf, nimg, vrows, 0));
  HIPCHK(rows_to_latent(s, vrows, nimg, v));
  return EXN_OK;
}


int exn_dit_velocity_dev(exn_dit* d, const float* context, int p, const float* latent, int h, int w, double sigma,
                         uint64_t prefix_key, int ref_a, const float* ref_latent, int rh, int rw, float* v) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  return velocity(d, context, p, latent, h, w, sigma, prefix_key, ref_a, ref_latent, rh, rw, v);
}

int exn_dit_velocity(exn_dit* d, const float* context, int p, const float* latent, int h, int w, double sigma,
                     uint64_t prefix_key, int ref_a, const float* ref_latent, int rh, int rw, float* v) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  if (h <= 0 || w <= 0 || p < 0 || !latent || !v || (p > 0 && !context))
    FAIL(EXN_EINVAL, "velocity: h %d, w %d, p %d", h, w, p);
  hipStream_t s = d->ctx->stream;
  const int64_t nimg = (int64_t)h * w;
  const int64_t nref = ref_latent ? (int64_t)rh * rw : 0;
  float *dctx = nullptr, *dlat, *dref = nullptr, *dv;
  if (p > 0) TRY(dit_buf(d, "h_ctx", (size_t)p * EXN_W * 4, (void**)&dctx));
  TRY(dit_buf(d, "h_lat", (size_t)nimg * EXN_LAT * 4, (void**)&dlat));
  TRY(dit_buf(d, "h_v", (size_t)nimg * EXN_LAT * 4, (void**)&dv));
  if (ref_latent) {
    if (nref <= 0) FAIL(EXN_EINVAL, "reference picture %d x %d", rh, rw);
    TRY(dit_buf(d, "h_ref", (size_t)nref * EXN_LAT * 4, (void**)&dref));
    HIPCHK(hipMemcpyAsync(dref, ref_latent, (size_t)nref * EXN_LAT * 4, hipMemcpyHostToDevice, s));
  }
  if (p > 0) HIPCHK(hipMemcpyAsync(dctx, context, (size_t)p * EXN_W * 4, hipMemcpyHostToDevice, s));
  HIPCHK(hipMemcpyAsync(dlat, latent, (size_t)nimg * EXN_LAT * 4, hipMemcpyHostToDevice, s));
  TRY(velocity(d, dctx, p, dlat, h, w, sigma, prefix_key, ref_a, dref, rh, rw, dv));
  HIPCHK(hipMemcpyAsync(v, dv, (size_t)nimg * EXN_LAT * 4, hipMemcpyDeviceToHost, s));
  HIPCHK(hipStreamSynchronize(s));
  return EXN_OK;
}

int exn_dit_generate_dev(exn_dit* d, const float* context, int p, float* z, int h, int w, const double* sigmas,
                         int nsig, int ref_a, const float* ref_latent, int rh, int rw) {
  if (!d) FAIL(EXN_EINVAL, "null model");
  TRY(use(d->ctx));
  if (!z || !sigmas || nsig < 2) FAIL(EXN_EINVAL, "generate: %d sigmas", nsig);
  static std::atomic<uint64_t> counter{0};
  const uint64_t key = 0x6765000000000000ull + (++counter);  // a fresh key, as edit's (:edit k) is
  const int64_t count = (int64_t)h * w * EXN_LAT;
  float* v = nullptr;
  TRY(dit_buf(d, "gen_v", (size_t)count * 4, (void**)&v));
  for (int i = 0; i + 1 < nsig; ++i) {
    TRY(velocity(d, context, p, z, h, w, sigmas[i], key, ref_a, ref_latent, rh, rw, v));
    HIPCHK(euler(d->ctx->stream, count, z, v, (float)(sigmas[i + 1] - sigmas[i])));
  }
  return EXN_OK;
}

int exn_dit_rope_table(int p, int h, int w, int edit, int ref_a, int rh, int rw, int64_t rows_cap, int32_t* pos,
                       float* cs) {
  if (p < 0 || h <= 0 || w <= 0 || (edit && (rh <= 0 || rw <= 0 || ref_a < 0 || ref_a > p)))
    FAIL(EXN_EINVAL, "rope table: p %d, %d x %d, edit %d (a %d, %d x %d)", p, h, w, edit, ref_a, rh, rw);
  const int nref = edit ? rh * rw : 0;
  const int64_t rows = (int64_t)p + nref + (int64_t)h * w;
  if (rows > rows_cap) FAIL(EXN_EINVAL, "rope table: %lld rows, room for %lld", (long long)rows, (long long)rows_cap);
  std::vector<int> pv;
  positions(p + nref, h, w, edit ? ref_a : 0, rh, rw, edit != 0, pv);
  if (pos)
    for (size_t i = 0; i < pv.size(); ++i) pos[i] = pv[i];
  if (cs) {
    std::vector<float> c;
    rope_table(pv, c);
    memcpy(cs, c.data(), c.size() * 4);
  }
  return EXN_OK;
}
