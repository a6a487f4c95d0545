// api.hip -- libexn-hip.so's C ABI (include/exn_hip.h): contexts, device
// memory, weights, the op-level entry points, and the DiT step driver that
// replaces the reference's CUDA backend (src/cuda-dit.lisp).
#include "exn_common.h"
#include "../../include/exn_hip.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

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

using namespace exn;

#define FAIL(code, ...)        \
  do {                         \
    exn::set_error(__VA_ARGS__); \
    return code;               \
  } while (0)

#define HIPCHK(expr)                                                                          \
  do {                                                                                        \
    hipError_t e_ = (expr);                                                                   \
    if (e_ != hipSuccess) FAIL(e_ == hipErrorOutOfMemory ? EXN_ENOMEM : EXN_EHIP, "%s: %s (%s:%d)", #expr, \
                               hipGetErrorString(e_), __FILE__, __LINE__);                    \
  } while (0)

#define TRY(expr)              \
  do {                         \
    int r_ = (expr);           \
    if (r_ != EXN_OK) return r_; \
  } while (0)

struct exn_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  void* tmp = nullptr;  // scratch of the op-level entry points (fp32 -> bf16 inputs)
  size_t tmp_bytes = 0;
  void* scratch = nullptr;  // this device's static scratch array (exn_mm_noalloc)
};

struct exn_w {
  exn_ctx* ctx = nullptr;
  int kind = EXN_Q8_0;
  int64_t rows = 0, cols = 0;
  int8_t* qs = nullptr;
  uint16_t* d = nullptr;
  uint8_t* qt = nullptr;   // a Q8_0 matrix's tiled copy of qs/d, the block products' operand (cols % 64 == 0)
  uint16_t* wb = nullptr;  // bf16 rows (EXN_BF16 matrices; a dense layer matrix)
  float* wf = nullptr;     // fp32 rows (EXN_F32 matrices)
  uint16_t* wx = nullptr;  // a Q8_0 matrix's resident bf16 expansion, bf16(fp32(d) * q) exactly
  bool wx_ok = false;      // wx matches qs/d
  bool dense = false;      // a layer matrix that has a BF16 or F32 slot: its products read wb, every slot's rows
  bool pairs = false;      // gate/up rows interleaved by 32
  bool view = false;       // rows inside another allocation (not freed here)
};

// the bf16 rows the MFMA products stream, if the matrix has them: a BF16 matrix's, a dense layer
// matrix's, or a Q8_0 matrix's resident expansion; null for Q8_0 without it (dequantised in the
// product) and for F32 (multiplied in fp32)
static const uint16_t* wbf(const exn_w* w) {
  if (w->kind == EXN_BF16 || w->dense) return w->wb;
  if (w->kind == EXN_Q8_0 && w->wx_ok) return w->wx;
  return nullptr;
}

// the operand a block product streams: the bf16 rows, else the Q8_0 codes and scales (dequantised
// in the product); an F32 matrix has neither (its products run in fp32)
static WOp wop(const exn_w* w) {
  if (const uint16_t* b = wbf(w)) return WOp{b, nullptr, nullptr, nullptr};
  if (w->kind == EXN_Q8_0) return WOp{nullptr, w->qs, w->d, w->qt};
  return WOp{nullptr, nullptr, nullptr, nullptr};
}

static int dev_alloc(void** p, size_t bytes) {
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

static void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

static int use(exn_ctx* ctx) {
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

static int ctx_tmp(exn_ctx* ctx, size_t bytes, void** out) {
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

extern "C" {

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

// --- weights ----------------------------------------------------------------------

static int w_new(exn_ctx* ctx, int kind, int64_t rows, int64_t cols, exn_w** out) {
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
static int upload_q8_blocks(exn_ctx* ctx, const void* blocks, int64_t rows, int64_t cols, const int32_t* row_map,
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
static int retile(exn_w* w) {
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

static int upload_bf16_from(exn_ctx* ctx, const void* data, bool is_f32, int64_t count, uint16_t* dst) {
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

static uint64_t gen_key(uint64_t seed, uint64_t tensor) {
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
static int w_resident(exn_w* w, bool bf16) {
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

static std::vector<int32_t> pair_rows(int64_t rows) {
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

// --- ops ----------------------------------------------------------------------------

static int check_gemm(const exn_w* w, int64_t n) {
  if (!w) FAIL(EXN_EINVAL, "null weight");
  if (n < 0) FAIL(EXN_EINVAL, "n = %lld", (long long)n);
  if (w->cols % 64) FAIL(EXN_EINVAL, "a product over %lld inputs: not a multiple of 64", (long long)w->cols);
  return EXN_OK;
}

// a bf16-operand product on any matrix but an F32 one (which multiplies in fp32: exn_mm)
static hipError_t gemm_any(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, Epi epi,
                           const EpiArgs& ea) {
  if (n == 0) return hipSuccess;
  if (const uint16_t* b = wbf(w)) return gemm_wbf16(s, x, lda, b, n, w->rows, w->cols, epi, ea);
  if (w->kind == EXN_Q8_0) return gemm_q8(s, x, lda, wop(w), n, w->rows, w->cols, epi, ea);
  return hipErrorInvalidValue;
}

// split-K scratch of a block product's prompt rows (S x rows x N floats with S x tiles <= 256
// workgroups of 256 x 256: 256^3 floats hold any of them) and of image rows past whole waves
// (2048 rows x 4096 columns, split 2 ways)
static const int64_t kSplitCap = (int64_t)2 * 256 * 256 * 256;

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
    r = gemm_split_rows(s, x + n1 * lda, lda, wop(w), n - n1, w->rows, w->cols, epi, eb, part, kSplitCap);
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
static hipError_t block_mm(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, int64_t nh,
                           Epi epi, const EpiArgs& ea, float* part) {
  if (nh > 0 && nh < n) {
    hipError_t r = hipErrorNotSupported;
    if (nh <= 1024 && part && w->kind != EXN_F32)
      r = gemm_split_rows(s, x, lda, wop(w), nh, w->rows, w->cols, epi, ea, part, kSplitCap);
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

}  // extern "C"

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

struct Buf {
  void* p = nullptr;
  size_t bytes = 0;
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

extern "C" {

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

}  // extern "C"

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
    // qkv_prep over them.  (Splitting an uncached pass's
    // prompt rows off, as the other products do, measured no faster here: 768 + 48 tiles.)
    bool fused = false;
    {
      ProfScope ps(d, EXN_PROF_QKV, 2 * nd * 3 * Wd * Wd, nd * Wd * 2 + 3 * Wd * Wd * 1.0625 + nd * 3 * Wd * 2);
      ea = EpiArgs{};
      ea.n0 = n0;
      ea.wq = L.norm_q;
      ea.wk = L.norm_k;
      ea.cs = d->cs;
      ea.qscale = QK_QSCALE;
      ea.q = q;
      ea.qld = n;
      ea.kc = d->kc[(size_t)il];
      ea.vt = d->vt[(size_t)il];
      ea.lcap = d->lcap;
      const hipError_t r = gemm_qkv(s, y, EXN_W, wop(L.qkv), n, EXN_W, ea);
      if (r != hipErrorNotSupported) HIPCHK(r);
      fused = r == hipSuccess;
    }
    if (!fused) {
      {
        ProfScope ps(d, EXN_PROF_QKV, 2 * nd * 3 * Wd * Wd, nd * Wd * 2 + 3 * Wd * Wd * 1.0625 + nd * 3 * Wd * 2);
        ea = EpiArgs{};
        ea.y = qkv;
        ea.ldy = 3 * EXN_W;
        HIPCHK(gemm_any(s, L.qkv, y, EXN_W, n, EPI_F16, ea));
      }
      ProfScope ps(d, EXN_PROF_QKV_PREP, 0, qkv_bytes);
      HIPCHK(qkv_prep(s, qkv, n, L.norm_q, L.norm_k, d->cs, q, d->kc[(size_t)il], d->vt[(size_t)il], n0, d->lcap, n));
    }
    {
      ProfScope ps(d, EXN_PROF_ATTEND, 4.0 * EXN_HD * EXN_H * pairs, nd * Wd * 2 * 2 + 2.0 * l * Wd * 2);
      HIPCHK(attend(s, q, d->kc[(size_t)il], d->vt[(size_t)il], att, (int)n, n0, p, (int)l, d->lcap, b0, b1, 1.f));
    }
    {
      ProfScope ps(d, EXN_PROF_OUT, 2 * nd * Wd * Wd, nd * Wd * 2 + Wd * Wd * 1.0625 + nd * Wd * 4 * 2);
      ea = EpiArgs{};
      ea.resid = x;
      ea.ldy = EXN_W;
      ea.gate = mod + 1 * EXN_W;
      ea.n0 = n0;
      ea.p = p;
      ea.mstride = ms;
      HIPCHK(block_mm(s, L.out, att, EXN_W, n, nh, EPI_GATE_ADD, ea, part));
    }
    {
      ProfScope ps(d, EXN_PROF_LN_MOD, 0, ln_bytes);
      HIPCHK(ln_mod(s, (int)n, n0, p, ms, x, EXN_W, mod + 2 * EXN_W, y, 1));
    }
    {
      ProfScope ps(d, EXN_PROF_GATE_UP, 2 * nd * Wd * 2 * Fd, nd * Wd * 2 + 2 * Fd * Wd * 1.0625 + nd * Fd * 2);
      ea = EpiArgs{};
      ea.y = ff;
      ea.ldy = EXN_F;
      HIPCHK(block_mm(s, L.gate_up, y, EXN_W, n, nh, EPI_SWIGLU, ea, part));
    }
    {
      ProfScope ps(d, EXN_PROF_DOWN, 2 * nd * Fd * Wd, nd * Fd * 2 + Fd * Wd * 1.0625 + nd * Wd * 4 * 2);
      ea = EpiArgs{};
      ea.resid = x;
      ea.ldy = EXN_W;
      ea.gate = mod + 3 * EXN_W;
      ea.n0 = n0;
      ea.p = p;
      ea.mstride = ms;
      HIPCHK(block_mm(s, L.down, ff, EXN_F, n, nh, EPI_GATE_ADD, ea, part));
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

extern "C" {

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

}  // extern "C"

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

struct VExpect {
  std::string name;
  std::vector<int64_t> shape;
};

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

extern "C" {

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

}  // extern "C"

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

extern "C" {

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

}  // extern "C"

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

extern "C" {

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

}  // extern "C"

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

extern "C" {

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

}  // extern "C"

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

// the layer-matrix row of each source row of SLOT: q | k | v of 32 heads each (key/value head g
// written out for query heads 4g .. 4g + 3, REP the copy), or gate/up interleaved by 32
std::vector<int32_t> enc_rows(int slot, int rep) {
  std::vector<int32_t> m;
  if (slot == E_Q) {
    for (int r = 0; r < EXN_W; ++r) m.push_back((r / EXN_HD) * EXN_HD + enc_perm(r % EXN_HD));
  } else if (slot == E_K || slot == E_V) {
    for (int r = 0; r < 8 * EXN_HD; ++r) {
      const int head = kEncGroup * (r / EXN_HD) + rep, i = r % EXN_HD;
      m.push_back((slot == E_K ? EXN_W : 2 * EXN_W) + head * EXN_HD + (slot == E_K ? enc_perm(i) : i));
    }
  } else if (slot == E_GATE || slot == E_UP) {
    for (int r = 0; r < EXN_F; ++r) m.push_back(64 * (r / 32) + (slot == E_UP ? 32 : 0) + r % 32);
  }
  return m;
}

struct EncLayer {
  exn_w* qkv = nullptr;      // q | k | v, 3 x 4096 rows (the rotary's pairs adjacent)
  exn_w* out = nullptr;
  exn_w* gate_up = nullptr;  // gate / up interleaved by 32
  exn_w* down = nullptr;
  float* vec[E_SLOTS] = {};  // the norms' weights (q and k norms permuted as their rows)
  unsigned have = 0;         // slots set, a bit each (K and V: all four copies)
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
  std::map<int, int32_t*> maps;  // device row maps by slot * 4 + copy
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

static int enc_map(exn_enc* e, int slot, int rep, int32_t** out) {
  int32_t*& m = e->maps[slot * 4 + rep];
  if (!m) {
    const std::vector<int32_t> h = enc_rows(slot, rep);
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
    const int64_t rows = slot == E_OUT ? EXN_W : slot == E_DOWN ? EXN_W : (slot == E_GATE || slot == E_UP) ? 2 * EXN_F : 3 * EXN_W;
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

extern "C" {

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
  const int copies = (slot == E_K || slot == E_V) ? kEncGroup : 1;
  for (int rep = 0; rep < copies; ++rep) {
    int32_t* map = nullptr;
    if (slot != E_OUT && slot != E_DOWN) TRY(enc_map(e, slot, rep, &map));
    TRY(upload_q8_blocks(e->ctx, data, d1, d0, map, w->qs, w->d));
  }
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
      const int copies = (slot == E_K || slot == E_V) ? kEncGroup : 1;
      for (int rep = 0; rep < copies; ++rep) {
        int32_t* map = nullptr;
        if (slot != E_OUT && slot != E_DOWN) TRY(enc_map(e, slot, rep, &map));
        HIPCHK(synth_q8(s, key, kEncDims[slot][1], kEncDims[slot][0], kEncDims[slot][0] / 32, map, w->qs, w->d));
      }
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

// the layers' matrices multiplied from resident bf16 expansions (1, the default, 16 GB beside
// the 8.4 GB of Q8_0) or from Q8_0 alone, dequantised in the products (0)
int exn_enc_resident(exn_enc* e, int bf16) {
  if (!e) FAIL(EXN_EINVAL, "null encoder");
  TRY(use(e->ctx));
  e->bf16 = bf16 != 0;
  for (auto& L : e->L)
    for (exn_w* m : {L.qkv, L.out, L.gate_up, L.down})
      if (m) TRY(w_resident(m, e->bf16));
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

}  // extern "C"

// encoder-states on the device: IDS (n, validated), CS (n x 128, exn_enc_rope_table's), the
// picture's rows PIC0 .. PIC0 + M - 1 taking MERGED after the embedding and DEEP[j] (3 x M x
// 4096) after layer j; OUT n x 4096
static int enc_states(exn_enc* e, const int32_t* ids, int n, const float* cs, int pic0, int m, const float* merged,
                      const float* deep, float* out) {
  hipStream_t s = e->ctx->stream;
  if (e->bf16)   // expansions made (or remade after a set) once, then kept
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
  // a prompt of at most 1024 tokens is about one row of 256-row tiles: its products split K
  // over the chip (the DiT's prompt-row path), the partial sums then added in order; a longer
  // one splits the products of fewer tiles than 192 (out and down, 16 column tiles)
  float* part = nullptr;
  const bool split = n <= 1024;
  TRY(enc_buf(e, "part", (size_t)kSplitCap * 4, (void**)&part));
  auto mm = [&](const exn_w* w, const uint16_t* xin, int64_t lda, Epi epi, const EpiArgs& a) -> hipError_t {
    if (split || ((int64_t)n + 255) / 256 * ((w->rows + 255) / 256) < 192) {
      const hipError_t r = gemm_split_rows(s, xin, lda, wop(w), n, w->rows, w->cols, epi, a, part, kSplitCap);
      if (r != hipErrorNotSupported) return r;
    }
    return gemm_any(s, w, xin, lda, n, epi, a);
  };
  HIPCHK(enc_embed(s, ids, n, e->vocab, e->eqs, e->ed, e->ef, EXN_W, x));
  if (m > 0)
    HIPCHK(hipMemcpyAsync(x + (int64_t)pic0 * EXN_W, merged, (size_t)m * EXN_W * 4, hipMemcpyDeviceToDevice, s));
  EpiArgs ea;
  for (int il = 0; il < e->layers; ++il) {
    const EncLayer& L = e->L[(size_t)il];
    HIPCHK(rms_norm(s, n, EXN_W, 1e-6f, x, L.vec[E_ATTN_NORM], y, 1));
    ea = EpiArgs{};
    ea.n0 = 0;
    ea.wq = L.vec[E_QNORM];
    ea.wk = L.vec[E_KNORM];
    ea.cs = cs;
    ea.qscale = QK_QSCALE;
    ea.q = q;
    ea.qld = n;
    ea.kc = kc;
    ea.vt = vt;
    ea.lcap = lcap;
    const hipError_t r = split ? hipErrorNotSupported : gemm_qkv(s, y, EXN_W, wop(L.qkv), n, EXN_W, ea);
    if (r == hipErrorNotSupported) {
      TRY(enc_buf(e, "qkv", (size_t)n * 3 * EXN_W * 2, (void**)&qkv));
      ea = EpiArgs{};
      ea.y = qkv;
      ea.ldy = 3 * EXN_W;
      HIPCHK(mm(L.qkv, y, EXN_W, EPI_F16, ea));
      HIPCHK(qkv_prep(s, qkv, n, L.vec[E_QNORM], L.vec[E_KNORM], cs, q, kc, vt, 0, lcap, n));
    } else {
      HIPCHK(r);
    }
    HIPCHK(attend(s, q, kc, vt, att, n, 0, n, n, lcap, 0, 0, 1.f));
    ea = EpiArgs{};
    ea.resid = x;
    ea.ldy = EXN_W;
    ea.gate = e->one_gate;
    HIPCHK(mm(L.out, att, EXN_W, EPI_GATE_ADD, ea));
    HIPCHK(rms_norm(s, n, EXN_W, 1e-6f, x, L.vec[E_FFN_NORM], y, 1));
    ea = EpiArgs{};
    ea.y = ff;
    ea.ldy = EXN_F;
    HIPCHK(mm(L.gate_up, y, EXN_W, EPI_SWIGLU, ea));
    ea = EpiArgs{};
    ea.resid = x;
    ea.ldy = EXN_W;
    ea.gate = e->one_gate;
    HIPCHK(mm(L.down, ff, EXN_F, EPI_GATE_ADD, ea));
    if (m > 0 && il < 3 && deep)
      HIPCHK(gate_add(s, (int64_t)m * EXN_W, EXN_W, 0, 0, 0, x + (int64_t)pic0 * EXN_W, deep + (int64_t)il * m * EXN_W,
                      e->one_gate));
  }
  HIPCHK(hipMemcpyAsync(out, x, (size_t)n * EXN_W * 4, hipMemcpyDeviceToDevice, s));
  return EXN_OK;
}

extern "C" {

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

}  // extern "C"
