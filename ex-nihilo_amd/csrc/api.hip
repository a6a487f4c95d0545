// api.hip -- libexn-hip.so's C ABI (include/exn_hip.h): errors, contexts, device memory,
// the op-level entry points and the block products' dispatch the models share.
#include "api_host.h"

namespace exn {

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
}

}  // namespace exn

// the bf16 rows the MFMA products stream, if the matrix has them: a BF16 matrix's, a dense layer
// matrix's, or a Q8_0 matrix's resident expansion; null for Q8_0 without it (dequantised in the
// product) and for F32 (multiplied in fp32)
const uint16_t* wbf(const exn_w* w) {
  if (w->kind == EXN_BF16 || w->dense) return w->wb;
  if (w->kind == EXN_Q8_0 && w->wx_ok) return w->wx;
  return nullptr;
}

// the operand a block product streams: the bf16 rows, else the Q8_0 codes and scales (dequantised
// in the product); an F32 matrix has neither (its products run in fp32)
WOp wop(const exn_w* w) {
  if (const uint16_t* b = wbf(w)) return WOp{b, nullptr, nullptr, nullptr};
  if (w->kind == EXN_Q8_0) return WOp{nullptr, w->qs, w->d, w->qt};
  return WOp{nullptr, nullptr, nullptr, nullptr};
}

// the operand of a product over N rows: a Q8_0 matrix's product of at most 256 rows in the few-row
// kernel's shapes streams the tiled codes even where a resident bf16 expansion exists -- the same
// B operands and the same sums bit for bit, from half the bytes, which is faster there; else wop
WOp wop_n(const exn_w* w, int64_t n) {
  if (n <= 256 && w->kind == EXN_Q8_0 && !w->dense && w->qt && w->cols % 256 == 0 && w->rows % (n > 128 ? 128 : 256) == 0)
    return WOp{nullptr, w->qs, w->d, w->qt};
  return wop(w);
}

int dev_alloc(void** p, size_t bytes) {
  *p = nullptr;
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) {
    *p = nullptr;
    (void)hipGetLastError();
    FAIL(e == hipErrorOutOfMemory ? EXN_ENOMEM : EXN_EHIP, "hipMalloc(%zu bytes): %s", bytes, hipGetErrorString(e));
  }
  return EXN_OK;
}

void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

int use(exn_ctx* ctx) {
  if (!ctx) FAIL(EXN_EINVAL, "null context");
  HIPCHK(hipSetDevice(ctx->device));
  return EXN_OK;
}

// --- the no-allocation product's scratch (exn_mm_noalloc) -----------------------------
// A file-scope device array: every GPU the library runs on holds its own copy until the process
// ends.  In host code the name `scratch` is a stand-in, not a device address: host code only ever
// uses the address hipGetSymbolAddress gives for the current device, taken once a device by
// exn_open and kept per device (g_scratch) and in the context.  Every call on one GPU shares
// that GPU's array, so calls that overlap on one GPU (two streams, two threads) race.
static const size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static std::map<int, void*> g_scratch;

// this device's scratch address (the device current)
static int scratch_address(int device, void** out) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  auto it = g_scratch.find(device);
  if (it != g_scratch.end()) {
    *out = it->second;
    return EXN_OK;
  }
  void* p = nullptr;
  HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  g_scratch[device] = p;
  *out = p;
  return EXN_OK;
}

int ctx_tmp(exn_ctx* ctx, size_t bytes, void** out) {
  if (ctx->tmp_bytes < bytes) {
    HIPCHK(hipStreamSynchronize(ctx->stream));
    dev_free(ctx->tmp);
    ctx->tmp = nullptr;
    ctx->tmp_bytes = 0;
    TRY(dev_alloc(&ctx->tmp, bytes));
    ctx->tmp_bytes = bytes;
  }
  *out = ctx->tmp;
  return EXN_OK;
}


const char* exn_last_error(void) { return g_err.c_str(); }

int exn_version(void) { return 1; }

int exn_device_count(int* n) {
  if (!n) FAIL(EXN_EINVAL, "null count");
  *n = 0;
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    FAIL(EXN_ENODEV, "no GPU: %s", hipGetErrorString(e));
  }
  *n = c;
  return EXN_OK;
}

int exn_open(int device, exn_ctx** out) {
  if (!out) FAIL(EXN_EINVAL, "null output");
  *out = nullptr;
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  if (e != hipSuccess || c == 0) {
    (void)hipGetLastError();
    FAIL(EXN_ENODEV, "no GPU (%s)", e != hipSuccess ? hipGetErrorString(e) : "0 devices");
  }
  if (device < 0 || device >= c) FAIL(EXN_ENODEV, "device %d of %d", device, c);
  HIPCHK(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    FAIL(EXN_ENODEV, "device %d is %s; libexn-hip.so is built for gfx950 only", device, prop.gcnArchName);
  // the device's scratch address, once a device; should it fail, exn_mm_noalloc tries again
  // and reports why, and nothing else needs it
  void* sp = nullptr;
  if (scratch_address(device, &sp) != EXN_OK) sp = nullptr;
  exn_ctx* ctx = new exn_ctx();
  ctx->device = device;
  ctx->scratch = sp;
  e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    FAIL(EXN_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  ctx->stream = ctx->own;
  *out = ctx;
  return EXN_OK;
}

int exn_close(exn_ctx* ctx) {
  if (!ctx) return EXN_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  dev_free(ctx->tmp);
  if (ctx->own) (void)hipStreamDestroy(ctx->own);
  delete ctx;
  return EXN_OK;
}

int exn_set_stream(exn_ctx* ctx, void* stream) {
  TRY(use(ctx));
  ctx->stream = stream ? (hipStream_t)stream : ctx->own;
  return EXN_OK;
}

int exn_sync(exn_ctx* ctx) {
  TRY(use(ctx));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

int exn_alloc(exn_ctx* ctx, size_t bytes, void** dptr) {
  TRY(use(ctx));
  if (!dptr) FAIL(EXN_EINVAL, "null output");
  return dev_alloc(dptr, bytes);
}

int exn_free(exn_ctx* ctx, void* dptr) {
  TRY(use(ctx));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  dev_free(dptr);
  return EXN_OK;
}

int exn_upload(exn_ctx* ctx, void* dst, const void* src, size_t bytes) {
  TRY(use(ctx));
  if (!dst || (!src && bytes)) FAIL(EXN_EINVAL, "null pointer");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIPCHK(hipStreamSynchronize(ctx->stream));  // the host buffer may be reused on return
  return EXN_OK;
}

int exn_download(exn_ctx* ctx, void* dst, const void* src, size_t bytes) {
  TRY(use(ctx));
  if (!dst || (!src && bytes)) FAIL(EXN_EINVAL, "null pointer");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIPCHK(hipStreamSynchronize(ctx->stream));
  return EXN_OK;
}

int exn_copy(exn_ctx* ctx, void* dst, const void* src, size_t bytes) {
  TRY(use(ctx));
  if (!dst || (!src && bytes)) FAIL(EXN_EINVAL, "null pointer");
  HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return EXN_OK;
}

// --- ops ----------------------------------------------------------------------------

static int check_gemm(const exn_w* w, int64_t n) {
  if (!w) FAIL(EXN_EINVAL, "null weight");
  if (n < 0) FAIL(EXN_EINVAL, "n = %lld", (long long)n);
  if (w->cols % 64) FAIL(EXN_EINVAL, "a product over %lld inputs: not a multiple of 64", (long long)w->cols);
  return EXN_OK;
}

// a bf16-operand product on any matrix but an F32 one (which multiplies in fp32: exn_mm)
hipError_t gemm_any(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, Epi epi,
                           const EpiArgs& ea) {
  if (n == 0) return hipSuccess;
  const WOp o = wop_n(w, n);
  if (o.wb) return gemm_wbf16(s, x, lda, o.wb, n, w->rows, w->cols, epi, ea);
  if (w->kind == EXN_Q8_0) return gemm_q8(s, x, lda, o, n, w->rows, w->cols, epi, ea);
  return hipErrorInvalidValue;
}

// EA with every row pointer K rows on (the gated residual's or the output's)
static EpiArgs rows_on(const EpiArgs& ea, Epi epi, int64_t k) {
  EpiArgs eb = ea;
  eb.n0 = ea.n0 + (int)k;
  if (epi == EPI_GATE_ADD) eb.resid = ea.resid + k * ea.ldy;
  else if (epi == EPI_F32) eb.y = (float*)ea.y + k * ea.ldy;
  else eb.y = (uint16_t*)ea.y + k * ea.ldy;
  return eb;
}

// a block product's image rows as whole tiles; where they would leave a last wave of
// workgroups at most half full (6144 rows through to_out and down: 384 tiles, 1.5 waves), the
// rows of the whole waves as tiles and the rest with K split over the chip (2048 rows: 128
// tiles, 2 ways), the rest then taking half a wave's time instead of a whole one
static hipError_t rows_mm(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, Epi epi,
                          const EpiArgs& ea, float* part) {
  const int64_t ct = (w->rows + 255) / 256, tiles = (n + 255) / 256 * ct, full = tiles / 256 * 256;
  if (part && w->kind != EXN_F32 && (epi == EPI_GATE_ADD || epi == EPI_SWIGLU) && full > 0 && tiles > full &&
      tiles - full <= 128 && full % ct == 0) {
    const int64_t n1 = full / ct * 256;   // the whole waves' rows
    hipError_t r = gemm_any(s, w, x, lda, n1, epi, ea);
    if (r != hipSuccess) return r;
    const EpiArgs eb = rows_on(ea, epi, n1);
    r = gemm_split_rows(s, x + n1 * lda, lda, wop_n(w, n - n1), n - n1, w->rows, w->cols, epi, eb, part, kSplitCap);
    if (r != hipErrorNotSupported) return r;
    return gemm_any(s, w, x + n1 * lda, lda, n - n1, epi, eb);
  }
  return gemm_any(s, w, x, lda, n, epi, ea);
}

// a block product over a pass's n rows: its first nh rows (the prompt's, in a pass that has
// them) apart -- with K split over the chip when they are about one row of tiles, else by
// rows_mm (an edit's 4608 prompt rows through to_out and down: 288 tiles) -- and the image
// rows after them by rows_mm, so that the 4096 image rows of a 1024^2 picture fill whole
// waves.  The image rows are tiled alike in every pass whatever comes before them, and a tile's
// rows are the same bits however the rows are tiled, so a cached pass's image rows match the
// uncached pass's.
hipError_t block_mm(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, int64_t nh,
                           Epi epi, const EpiArgs& ea, float* part) {
  if (nh > 0 && nh < n) {
    hipError_t r = hipErrorNotSupported;
    if (nh <= 1024 && part && w->kind != EXN_F32)
      r = gemm_split_rows(s, x, lda, wop_n(w, nh), nh, w->rows, w->cols, epi, ea, part, kSplitCap);
    if (r == hipErrorNotSupported) r = rows_mm(s, w, x, lda, nh, epi, ea, part);
    if (r != hipSuccess) return r;
    return rows_mm(s, w, x + nh * lda, lda, n - nh, epi, rows_on(ea, epi, nh), part);
  }
  return rows_mm(s, w, x, lda, n, epi, ea, part);
}

// exn_mm's checks and its products that need no scratch: an F32 matrix in fp32 (d41_mm_f32), n <= 4
// fp32 rows through the GEMV, bf16 rows through the MFMA product.  *DONE is false when what is left is
// an fp32-rows MFMA product, whose bf16 copy of X the caller stages.
static int mm_direct(exn_ctx* ctx, const exn_w* w, const void* x, int xdt, void* y, int ydt, int64_t n, bool* done) {
  *done = true;
  TRY(check_gemm(w, n));
  if (!x || !y) FAIL(EXN_EINVAL, "null pointer");
  if (w->pairs) FAIL(EXN_EINVAL, "exn_mm on a paired gate_up matrix: use exn_mm_swiglu");
  if ((xdt != EXN_DT_F32 && xdt != EXN_DT_BF16) || (ydt != EXN_DT_F32 && ydt != EXN_DT_BF16 && ydt != EXN_DT_F16))
    FAIL(EXN_EINVAL, "dtype");
  if (w->kind == EXN_F32) {  // fp32 weights are multiplied in fp32, as the reference's d41_mm_f32
    if (xdt != EXN_DT_F32 || ydt != EXN_DT_F32)
      FAIL(EXN_EINVAL, "an F32 matrix multiplies fp32 rows into fp32 rows (d41_mm_f32)");
    if (n <= 4)
      HIPCHK(gemv_q8(ctx->stream, (const float*)x, w->cols, nullptr, nullptr, nullptr, w->wf, n, w->rows, w->cols,
                     (float*)y, w->rows, 0));
    else
      HIPCHK(gemm_f32(ctx->stream, (const float*)x, w->cols, nullptr, nullptr, nullptr, w->wf, n, w->rows, w->cols,
                      (float*)y, w->rows, 0));
    return EXN_OK;
  }
  if (xdt == EXN_DT_F32 && n <= 4 && ydt == EXN_DT_F32) {
    HIPCHK(gemv_q8(ctx->stream, (const float*)x, w->cols, w->qs, w->d, w->kind == EXN_BF16 ? w->wb : nullptr, nullptr,
                   n, w->rows, w->cols, (float*)y, w->rows, 0));
    return EXN_OK;
  }
  if (xdt == EXN_DT_F32) {
    *done = false;
    return EXN_OK;
  }
  EpiArgs ea{};
  ea.y = y;
  ea.ldy = w->rows;
  HIPCHK(gemm_any(ctx->stream, w, (const uint16_t*)x, w->cols, n,
                  ydt == EXN_DT_F32 ? EPI_F32 : (ydt == EXN_DT_F16 ? EPI_F16 : EPI_BF16), ea));
  return EXN_OK;
}

// the MFMA product of fp32 rows X through their bf16 copy XB (n x cols, staged by the caller)
static int mm_staged(exn_ctx* ctx, const exn_w* w, const float* x, uint16_t* xb, void* y, int ydt, int64_t n) {
  HIPCHK(f32_to_bf16(ctx->stream, x, xb, n * w->cols));
  EpiArgs ea{};
  ea.y = y;
  ea.ldy = w->rows;
  HIPCHK(gemm_any(ctx->stream, w, xb, w->cols, n,
                  ydt == EXN_DT_F32 ? EPI_F32 : (ydt == EXN_DT_F16 ? EPI_F16 : EPI_BF16), ea));
  return EXN_OK;
}

int exn_mm(exn_ctx* ctx, const exn_w* w, const void* x, int xdt, void* y, int ydt, int64_t n) {
  TRY(use(ctx));
  bool done = false;
  TRY(mm_direct(ctx, w, x, xdt, y, ydt, n, &done));
  if (done) return EXN_OK;
  void* t = nullptr;
  TRY(ctx_tmp(ctx, (size_t)(n * w->cols) * 2, &t));
  return mm_staged(ctx, w, (const float*)x, (uint16_t*)t, y, ydt, n);
}

int exn_mm_noalloc(exn_ctx* ctx, const exn_w* w, const void* x, int xdt, void* y, int ydt, int64_t n) {
  TRY(use(ctx));
  if (!ctx->scratch) TRY(scratch_address(ctx->device, &ctx->scratch));
  bool done = false;
  if (w && n >= 0 && xdt == EXN_DT_F32 && w->kind != EXN_F32 && !(n <= 4 && ydt == EXN_DT_F32) &&
      (size_t)n * (size_t)w->cols * 2 > kScratchBytes)
    FAIL(EXN_EINVAL, "exn_mm_noalloc: %lld rows of %lld fp32 inputs need %zu bytes of bf16 staging, past the %zu-byte "
         "scratch", (long long)n, (long long)w->cols, (size_t)n * (size_t)w->cols * 2, kScratchBytes);
  TRY(mm_direct(ctx, w, x, xdt, y, ydt, n, &done));
  if (done) return EXN_OK;
  return mm_staged(ctx, w, (const float*)x, (uint16_t*)ctx->scratch, y, ydt, n);
}

int exn_mm_gate_add(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, int64_t n, float* resid, int n0, int p,
                    int mstride, const float* gate) {
  TRY(use(ctx));
  TRY(check_gemm(w, n));
  if (!x_bf16 || !resid || !gate) FAIL(EXN_EINVAL, "null pointer");
  if (w->pairs) FAIL(EXN_EINVAL, "a paired gate_up matrix");
  if (w->kind == EXN_F32) FAIL(EXN_EINVAL, "exn_mm_gate_add: a Q8_0 or BF16 matrix (bf16 products)");
  EpiArgs ea{};
  ea.resid = resid;
  ea.ldy = w->rows;
  ea.gate = gate;
  ea.n0 = n0;
  ea.p = p;
  ea.mstride = mstride;
  HIPCHK(gemm_any(ctx->stream, w, x_bf16, w->cols, n, EPI_GATE_ADD, ea));
  return EXN_OK;
}

int exn_mm_swiglu(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, uint16_t* ff, int64_t n) {
  TRY(use(ctx));
  TRY(check_gemm(w, n));
  if (!x_bf16 || !ff) FAIL(EXN_EINVAL, "null pointer");
  if (!w->pairs) FAIL(EXN_EINVAL, "exn_mm_swiglu wants a matrix interleaved by exn_weight_pairs");
  if (w->kind == EXN_F32) FAIL(EXN_EINVAL, "exn_mm_swiglu: a Q8_0 or BF16 matrix (bf16 products)");
  EpiArgs ea{};
  ea.y = ff;
  ea.ldy = w->rows / 2;
  HIPCHK(gemm_any(ctx->stream, w, x_bf16, w->cols, n, EPI_SWIGLU, ea));
  return EXN_OK;
}

int exn_ln_mod(exn_ctx* ctx, int n, int n0, int p, int mstride, const float* x, int64_t ldx, const float* mod,
               void* out, int outdt) {
  TRY(use(ctx));
  if (n < 0 || !x || !mod || !out || ldx % 4) FAIL(EXN_EINVAL, "ln_mod arguments");
  HIPCHK(ln_mod(ctx->stream, n, n0, p, mstride, x, ldx, mod, out, outdt == EXN_DT_BF16));
  return EXN_OK;
}

int exn_rms(exn_ctx* ctx, int n, int width, float eps, const float* x, const float* w, void* y, int ydt) {
  TRY(use(ctx));
  if (n < 0 || width <= 0 || width % 4 || !x || !w || !y) FAIL(EXN_EINVAL, "rms arguments");
  HIPCHK(rms_norm(ctx->stream, n, width, eps, x, w, y, ydt == EXN_DT_BF16));
  return EXN_OK;
}

int exn_gate_add(exn_ctx* ctx, int64_t count, int width, int n0, int p, int mstride, float* x, const float* h,
                 const float* gate) {
  TRY(use(ctx));
  if (count < 0 || count % 4 || width <= 0 || width % 4 || !x || !h || !gate) FAIL(EXN_EINVAL, "gate_add arguments");
  HIPCHK(gate_add(ctx->stream, count, width, n0, p, mstride, x, h, gate));
  return EXN_OK;
}

int exn_swiglu(exn_ctx* ctx, int64_t n, int f, const uint16_t* gu, uint16_t* out) {
  TRY(use(ctx));
  if (n < 0 || f <= 0 || f % 8 || !gu || !out) FAIL(EXN_EINVAL, "swiglu arguments");
  HIPCHK(swiglu(ctx->stream, n, f, gu, out));
  return EXN_OK;
}

int exn_gelu_tanh(exn_ctx* ctx, int64_t count, float* x) {
  TRY(use(ctx));
  if (count < 0 || !x) FAIL(EXN_EINVAL, "gelu arguments");
  HIPCHK(gelu_tanh(ctx->stream, count, x));
  return EXN_OK;
}

int exn_silu(exn_ctx* ctx, int64_t count, float* x) {
  TRY(use(ctx));
  if (count < 0 || !x) FAIL(EXN_EINVAL, "silu arguments");
  HIPCHK(silu(ctx->stream, count, x));
  return EXN_OK;
}

int exn_qkv_prep(exn_ctx* ctx, const uint16_t* qkv, int64_t n, const float* wq, const float* wk, const float* cs,
                 uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap) {
  TRY(use(ctx));
  if (n < 0 || row0 < 0 || row0 + n > lcap || !qkv || !wq || !wk || !cs || !q || !k || !vt)
    FAIL(EXN_EINVAL, "qkv_prep arguments");
  HIPCHK(qkv_prep(ctx->stream, qkv, n, wq, wk, cs, q, k, vt, row0, lcap, n));
  return EXN_OK;
}

int exn_mm_qkv(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, int64_t n, const float* wq, const float* wk,
               const float* cs, uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap) {
  TRY(use(ctx));
  TRY(check_gemm(w, n));
  if (!x_bf16 || !wq || !wk || !cs || !q || !k || !vt) FAIL(EXN_EINVAL, "null pointer");
  if (w->rows != 3 * EXN_W || w->cols != EXN_W || w->pairs)
    FAIL(EXN_EINVAL, "exn_mm_qkv: the fused q | k | v matrix (12288 x 4096) only");
  if (w->kind == EXN_F32) FAIL(EXN_EINVAL, "exn_mm_qkv: a Q8_0 or BF16 matrix (bf16 products)");
  EpiArgs ea{};
  ea.n0 = (int)row0;
  ea.wq = wq;
  ea.wk = wk;
  ea.cs = cs;
  ea.qscale = QK_QSCALE;
  ea.q = q;
  ea.kc = k;
  ea.vt = vt;
  ea.lcap = lcap;
  if (row0 < 0 || row0 > INT32_MAX) FAIL(EXN_EINVAL, "row0");
  const hipError_t r = gemm_qkv(ctx->stream, x_bf16, EXN_W, wop(w), n, EXN_W, ea);
  if (r == hipErrorNotSupported)
    FAIL(EXN_EINVAL, "exn_mm_qkv: 16-byte aligned arrays, lcap a multiple of 64, row0 + n <= lcap");
  HIPCHK(r);
  return EXN_OK;
}

int exn_attend(exn_ctx* ctx, const uint16_t* q, const uint16_t* k, const uint16_t* vt, uint16_t* out, int n, int q0,
               int p, int l, int64_t lcap, int b0, int b1, float scale) {
  TRY(use(ctx));
  if (n < 0 || q0 < 0 || l <= 0 || l > lcap || lcap % 64 || q0 + n > l || p < 0 || p > l || b0 < 0 || b1 < b0 ||
      b1 > p || !q || !k || !vt || !out)
    FAIL(EXN_EINVAL, "attend arguments (n %d, q0 %d, p %d, l %d, lcap %lld, b0 %d, b1 %d)", n, q0, p, l,
         (long long)lcap, b0, b1);
  HIPCHK(attend(ctx->stream, q, k, vt, out, n, q0, p, l, lcap, b0, b1, scale));
  return EXN_OK;
}

int exn_quant_q8(exn_ctx* ctx, const void* x, int xdt, int64_t ldx, int64_t n, int64_t k, int8_t* q, uint16_t* d) {
  TRY(use(ctx));
  if (!x || !q || !d || n < 0 || k <= 0 || k % 32 || ldx < k || (xdt != EXN_DT_F32 && xdt != EXN_DT_BF16))
    FAIL(EXN_EINVAL, "quant_q8: n %lld, k %lld, ldx %lld, dtype %d", (long long)n, (long long)k, (long long)ldx, xdt);
  HIPCHK(quant_q8(ctx->stream, x, xdt == EXN_DT_BF16, ldx, n, k, q, d));
  return EXN_OK;
}

int exn_mm_w8a8(exn_ctx* ctx, const exn_w* w, const int8_t* xq, const uint16_t* xd, int64_t n, void* y, int ydt) {
  TRY(use(ctx));
  if (!w || w->kind != EXN_Q8_0 || w->dense || !w->qs) FAIL(EXN_EINVAL, "mm_w8a8: the matrix is not Q8_0");
  if (!xq || !xd || !y || n < 0 || (ydt != EXN_DT_F32 && ydt != EXN_DT_F16)) FAIL(EXN_EINVAL, "mm_w8a8 arguments");
  HIPCHK(gemm_w8a8(ctx->stream, xq, xd, n, w->qs, w->d, w->rows, w->cols, y, w->rows, ydt == EXN_DT_F16));
  return EXN_OK;
}

int exn_euler(exn_ctx* ctx, int64_t count, float* z, const float* v, float ds) {
  TRY(use(ctx));
  if (count < 0 || !z || !v) FAIL(EXN_EINVAL, "euler arguments");
  HIPCHK(euler(ctx->stream, count, z, v, ds));
  return EXN_OK;
}
