// api_weights.hip -- weight matrices: Q8_0 records to codes, scales and the tiled operand,
// bf16 and fp32 rows, the synthetic generator, the resident bf16 expansion, gate/up pairing.
#include "api_host.h"

// --- weights ----------------------------------------------------------------------

int w_new(exn_ctx* ctx, int kind, int64_t rows, int64_t cols, exn_w** out) {
  if (!out) FAIL(EXN_EINVAL, "null output");
  *out = nullptr;
  if (rows <= 0 || cols <= 0) FAIL(EXN_EINVAL, "matrix %lld x %lld", (long long)rows, (long long)cols);
  if (kind == EXN_Q8_0 && cols % 32) FAIL(EXN_EINVAL, "Q8_0 matrix of %lld columns: not a multiple of 32", (long long)cols);
  exn_w* w = new exn_w();
  w->ctx = ctx;
  w->kind = kind;
  w->rows = rows;
  w->cols = cols;
  int r = EXN_OK;
  if (kind == EXN_Q8_0) {
    r = dev_alloc((void**)&w->qs, (size_t)(rows * cols));
    if (r == EXN_OK) r = dev_alloc((void**)&w->d, (size_t)(rows * cols / 32) * 2);
    if (r == EXN_OK && cols % 64 == 0) r = dev_alloc((void**)&w->qt, (size_t)tile_q8_bytes(rows, cols));
  } else if (kind == EXN_F32) {
    r = dev_alloc((void**)&w->wf, (size_t)(rows * cols) * 4);
  } else {
    r = dev_alloc((void**)&w->wb, (size_t)(rows * cols) * 2);
  }
  if (r != EXN_OK) {
    dev_free(w->qs);
    dev_free(w->d);
    dev_free(w->qt);
    dev_free(w->wb);
    dev_free(w->wf);
    delete w;
    return r;
  }
  *out = w;
  return EXN_OK;
}

int exn_weight_free(exn_w* w) {
  if (!w) return EXN_OK;
  if (w->ctx) {
    (void)hipSetDevice(w->ctx->device);
    (void)hipStreamSynchronize(w->ctx->stream);
  }
  if (!w->view) {
    dev_free(w->qs);
    dev_free(w->d);
    dev_free(w->qt);
    dev_free(w->wb);
    dev_free(w->wf);
    dev_free(w->wx);
  }
  delete w;
  return EXN_OK;
}

// GGUF block_q8_0 records (host) -> qs, d at the given rows (row_map: device int32, or null)
int upload_q8_blocks(exn_ctx* ctx, const void* blocks, int64_t rows, int64_t cols, const int32_t* row_map,
                            int8_t* qs, uint16_t* d) {
  const int64_t kb = cols / 32;
  const size_t bytes = (size_t)(rows * kb) * 34;
  void* staging = nullptr;
  TRY(ctx_tmp(ctx, bytes, &staging));
  HIPCHK(hipMemcpyAsync(staging, blocks, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIPCHK(repack_q8_blocks(ctx->stream, (const uint8_t*)staging, kb, rows, row_map, qs, d));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

// a Q8_0 matrix's tiled copy (the block products' operand) from its codes and scales, after any
// write to them (on the context's stream, ahead of any product that reads it)
int retile(exn_w* w) {
  if (w->kind != EXN_Q8_0 || !w->qt) return EXN_OK;
  HIPCHK(tile_q8(w->ctx->stream, w->qs, w->d, w->rows, w->cols, w->qt));
  return EXN_OK;
}

int exn_weight_q8_0(exn_ctx* ctx, const void* blocks, int64_t rows, int64_t cols, exn_w** out) {
  TRY(use(ctx));
  if (!blocks) FAIL(EXN_EINVAL, "null blocks");
  TRY(w_new(ctx, EXN_Q8_0, rows, cols, out));
  int r = upload_q8_blocks(ctx, blocks, rows, cols, nullptr, (*out)->qs, (*out)->d);
  if (r == EXN_OK) r = retile(*out);
  if (r != EXN_OK) {
    exn_weight_free(*out);
    *out = nullptr;
  }
  return r;
}

int upload_bf16_from(exn_ctx* ctx, const void* data, bool is_f32, int64_t count, uint16_t* dst) {
  if (is_f32) {
    void* staging = nullptr;
    TRY(ctx_tmp(ctx, (size_t)count * 4, &staging));
    HIPCHK(hipMemcpyAsync(staging, data, (size_t)count * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPCHK(f32_to_bf16(ctx->stream, (const float*)staging, dst, count));
  } else {
    HIPCHK(hipMemcpyAsync(dst, data, (size_t)count * 2, hipMemcpyHostToDevice, ctx->stream));
  }
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

int exn_weight_f32(exn_ctx* ctx, const float* data, int64_t rows, int64_t cols, exn_w** out) {
  TRY(use(ctx));
  if (!data) FAIL(EXN_EINVAL, "null data");
  TRY(w_new(ctx, EXN_F32, rows, cols, out));
  hipError_t e = hipMemcpyAsync((*out)->wf, data, (size_t)(rows * cols) * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    exn_weight_free(*out);
    *out = nullptr;
    FAIL(EXN_EHIP, "exn_weight_f32 upload: %s", hipGetErrorString(e));
  }
  return EXN_OK;
}

int exn_weight_bf16(exn_ctx* ctx, const uint16_t* data, int64_t rows, int64_t cols, exn_w** out) {
  TRY(use(ctx));
  if (!data) FAIL(EXN_EINVAL, "null data");
  TRY(w_new(ctx, EXN_BF16, rows, cols, out));
  int r = upload_bf16_from(ctx, data, false, rows * cols, (*out)->wb);
  if (r != EXN_OK) {
    exn_weight_free(*out);
    *out = nullptr;
  }
  return r;
}

uint64_t gen_key(uint64_t seed, uint64_t tensor) {
  auto mix = [](uint64_t z) {
    z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27; z *= 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  return mix(seed * 0x9E3779B97F4A7C15ull + tensor + 1);
}

int exn_weight_q8_0_synth(exn_ctx* ctx, uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, exn_w** out) {
  TRY(use(ctx));
  TRY(w_new(ctx, EXN_Q8_0, rows, cols, out));
  hipError_t e = synth_q8(ctx->stream, gen_key(seed, tensor), rows, cols, cols / 32, nullptr, (*out)->qs, (*out)->d);
  if (e == hipSuccess && (*out)->qt) e = tile_q8(ctx->stream, (*out)->qs, (*out)->d, rows, cols, (*out)->qt);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    exn_weight_free(*out);
    *out = nullptr;
    FAIL(EXN_EHIP, "synthetic weights: %s", hipGetErrorString(e));
  }
  return EXN_OK;
}

int exn_weight_info(const exn_w* w, int64_t* rows, int64_t* cols, int* kind) {
  if (!w) FAIL(EXN_EINVAL, "null weight");
  if (rows) *rows = w->rows;
  if (cols) *cols = w->cols;
  if (kind) *kind = w->kind;
  return EXN_OK;
}

int exn_dequant(exn_ctx* ctx, const exn_w* w, float* f32, uint16_t* bf16) {
  TRY(use(ctx));
  if (!w) FAIL(EXN_EINVAL, "null weight");
  if (w->kind != EXN_Q8_0) FAIL(EXN_EINVAL, "exn_dequant: not a Q8_0 matrix");
  HIPCHK(dequant_q8(ctx->stream, w->qs, w->d, w->rows * w->cols, f32, bf16));
  return EXN_OK;
}

// keep (bf16 = 1) or drop (0) a Q8_0 matrix's bf16 expansion; products use it while it is kept
// (a dense layer matrix has its bf16 rows already)
int w_resident(exn_w* w, bool bf16) {
  if (w->kind != EXN_Q8_0 || w->dense) return EXN_OK;
  if (!bf16) {
    if (w->wx) {
      HIPCHK(hipStreamSynchronize(w->ctx->stream));
      dev_free(w->wx);
    }
    w->wx = nullptr;
    w->wx_ok = false;
    return EXN_OK;
  }
  if (w->wx_ok) return EXN_OK;
  if (!w->wx) TRY(dev_alloc((void**)&w->wx, (size_t)(w->rows * w->cols) * 2));
  HIPCHK(dequant_q8(w->ctx->stream, w->qs, w->d, w->rows * w->cols, nullptr, w->wx));
  w->wx_ok = true;
  return EXN_OK;
}

int exn_weight_resident(exn_ctx* ctx, exn_w* w, int bf16) {
  TRY(use(ctx));
  if (!w) FAIL(EXN_EINVAL, "null weight");
  TRY(w_resident(w, bf16 != 0));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

std::vector<int32_t> pair_rows(int64_t rows) {
  // gate row i (i < rows/2) -> 64*(i/32) + i%32; up row i -> 64*(i/32) + 32 + i%32
  const int64_t f = rows / 2;
  std::vector<int32_t> map((size_t)rows);
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t i = r < f ? r : r - f;
    map[(size_t)r] = (int32_t)(64 * (i / 32) + (r < f ? 0 : 32) + i % 32);
  }
  return map;
}

int exn_weight_pairs(exn_ctx* ctx, exn_w* w) {
  TRY(use(ctx));
  if (!w) FAIL(EXN_EINVAL, "null weight");
  if (w->pairs) return EXN_OK;
  if (w->kind != EXN_Q8_0 || w->rows % 64) FAIL(EXN_EINVAL, "pairs: a Q8_0 matrix of a multiple of 64 rows");
  const std::vector<int32_t> map = pair_rows(w->rows);
  const int64_t kb = w->cols / 32;
  int8_t* qs = nullptr;
  uint16_t* d = nullptr;
  int32_t* dmap = nullptr;
  TRY(dev_alloc((void**)&qs, (size_t)(w->rows * w->cols)));
  int r = dev_alloc((void**)&d, (size_t)(w->rows * kb) * 2);
  if (r == EXN_OK) r = dev_alloc((void**)&dmap, map.size() * 4);
  if (r != EXN_OK) {
    dev_free(qs);
    dev_free(d);
    return r;
  }
  // permute whole rows with 2D copies: source row r -> destination row map[r]
  hipError_t e = hipMemcpyAsync(dmap, map.data(), map.size() * 4, hipMemcpyHostToDevice, w->ctx->stream);
  for (int64_t rr = 0; rr < w->rows && e == hipSuccess; rr += 32) {
    const int64_t dst = map[(size_t)rr];
    e = hipMemcpyAsync(qs + dst * w->cols, w->qs + rr * w->cols, (size_t)(32 * w->cols), hipMemcpyDeviceToDevice,
                       w->ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(d + dst * kb, w->d + rr * kb, (size_t)(32 * kb) * 2, hipMemcpyDeviceToDevice, w->ctx->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(w->ctx->stream);
  dev_free(dmap);
  if (e != hipSuccess) {
    dev_free(qs);
    dev_free(d);
    FAIL(EXN_EHIP, "pairs: %s", hipGetErrorString(e));
  }
  dev_free(w->qs);
  dev_free(w->d);
  w->qs = qs;
  w->d = d;
  w->pairs = true;
  TRY(retile(w));
  HIPCHK(hipStreamSynchronize(w->ctx->stream));
  if (w->wx) {
    w->wx_ok = false;
    TRY(w_resident(w, true));
    HIPCHK(hipStreamSynchronize(w->ctx->stream));
  }
  return EXN_OK;
}
