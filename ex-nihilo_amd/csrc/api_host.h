// api_host.h -- what the library's host-side files share (internal, not part of the C ABI):
// the status macros, the context, weight and scratch-buffer structures, device memory, and
// the block products' dispatch.  The C ABI itself is include/exn_hip.h.
#pragma once

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
void set_error(const char* fmt, ...);
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

struct Buf {
  void* p = nullptr;
  size_t bytes = 0;
};

struct VExpect {
  std::string name;
  std::vector<int64_t> shape;
};

// split-K scratch of a block product's prompt rows (S x rows x N floats with S x tiles <= 256
// workgroups of 256 x 256: 256^3 floats hold any of them) and of image rows past whole waves
// (2048 rows x 4096 columns, split 2 ways)
constexpr int64_t kSplitCap = (int64_t)2 * 256 * 256 * 256;

// shared helpers (api.hip: contexts, memory, the block products; api_weights.hip: weights)
const uint16_t* wbf(const exn_w* w);
WOp wop(const exn_w* w);
WOp wop_n(const exn_w* w, int64_t n);
int dev_alloc(void** p, size_t bytes);
void dev_free(void* p);
int use(exn_ctx* ctx);
int ctx_tmp(exn_ctx* ctx, size_t bytes, void** out);
hipError_t gemm_any(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, Epi epi, const EpiArgs& ea);
hipError_t block_mm(hipStream_t s, const exn_w* w, const uint16_t* x, int64_t lda, int64_t n, int64_t nh, Epi epi, const EpiArgs& ea, float* part);
int w_new(exn_ctx* ctx, int kind, int64_t rows, int64_t cols, exn_w** out);
int upload_q8_blocks(exn_ctx* ctx, const void* blocks, int64_t rows, int64_t cols, const int32_t* row_map, int8_t* qs, uint16_t* d);
int retile(exn_w* w);
int upload_bf16_from(exn_ctx* ctx, const void* data, bool is_f32, int64_t count, uint16_t* dst);
uint64_t gen_key(uint64_t seed, uint64_t tensor);
int w_resident(exn_w* w, bool bf16);
std::vector<int32_t> pair_rows(int64_t rows);
