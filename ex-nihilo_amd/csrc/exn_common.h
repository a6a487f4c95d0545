// exn_common.h -- shared definitions of libexn-hip.so's kernels and host code.
// gfx950 (CDNA4) only: 64-wide wavefronts, bf16 MFMA, 160 KB LDS per CU.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int32_t int32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace exn {

// --- device helpers ------------------------------------------------------------

// two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// two floats -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  f16x2 v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_lo(uint32_t u) {
  return (float)__builtin_bit_cast(f16x2, u)[0];
}
__device__ __forceinline__ float f16_hi(uint32_t u) {
  return (float)__builtin_bit_cast(f16x2, u)[1];
}

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }

// fp16 bits (the low 16 of H) -> fp32 by v_cvt_f32_f16: exact, subnormals included (the
// kernels run in the default mode, which keeps fp16 denormals); one instruction, no branch
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// v from the lane the DPP control names (quad_perm 0x00-0xFF, row_mirror 0x140,
// row_half_mirror 0x141), within rows of 16 lanes
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The sum of v over each row of 16 lanes, in every lane of the row: pairs (xor 1), quads
// (xor 2), then the two quads of each half (half mirror) and the two halves (mirror).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);   // row_half_mirror: lane i <-> 7 - i of each half row
  v += dpp_f<0x140>(v);   // row_mirror: lane i <-> 15 - i
  return v;
}

// gfx950's v_permlane16_swap / v_permlane32_swap on two copies of a value: a and b come back
// holding the lane's own value and its partner's (lane ^ 16, lane ^ 32), in either order.
// Written as inline asm: given the same value twice, the compiler's builtins return what it
// treats as one value, and a sum or max over the pair folds away.  The s_nop covers the
// VALU write -> permlane read hazard of the copies.
__device__ __forceinline__ void xswap16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void xswap32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// The sum of v over the wave, in every lane, without LDS: rows of 16 by DPP, then the row
// pairs and the halves by lane swaps.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  float a = v, b = v;
  xswap16(a, b);
  v = a + b;
  a = v;
  b = v;
  xswap32(a, b);
  return a + b;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ROCm device-library tanh and exp (ocml)
__device__ __forceinline__ float tanh_f(float x) { return tanhf(x); }

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

// SiLU for a value rounded to bf16 next: x / (1 + 2^(-x log2 e)) with the hardware exp2
// and reciprocal (about 1 ulp each); -0 once 2^(-x log2 e) overflows (x below about -88),
// x itself once it vanishes against 1 (x above about 17).
__device__ __forceinline__ float silu_bf16out(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

__device__ __forceinline__ float gelu_tanh_f(float v) {
  return 0.5f * v * (1.f + tanh_f(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

// --- host-side status ------------------------------------------------------------

void set_error(const char* fmt, ...);

}  // namespace exn

// The DiT's fixed dimensions (src/weights.lisp:19-20): width, heads x head dim, FFN.
#define EXN_W 4096
#define EXN_H 32
#define EXN_HD 128
#define EXN_F 12288
#define EXN_LAT 64
#define EXN_FREQ 256

// --- kernel launchers (defined in the .hip files, called by the api*.hip entry points) -----------

namespace exn {

// V^T's column of key k: within every aligned group of 16 keys, bits 2 and 3 of the
// index swapped.  The attention's P V^T product then finds the 8 keys a lane feeds
// one MFMA step (16u + 8(j/4) + 4hi + j%4, j = 0..7) in 16 contiguous bytes.
__host__ __device__ inline int64_t vt_pos(int64_t k) { return k ^ ((((k >> 2) ^ (k >> 3)) & 1) * 12); }

// q's scale: 1/sqrt(128) x log2(e), so that the attention's scores come out in log2 units
constexpr float QK_QSCALE = 0.08838834764831845f * 1.4426950408889634f;

enum Epi { EPI_F32 = 0, EPI_BF16 = 1, EPI_GATE_ADD = 2, EPI_SWIGLU = 3, EPI_GELU_BF16 = 4, EPI_F16 = 5, EPI_QKV = 6,
           EPI_PART = 7 };   // EPI_PART: split K, fp32 sums of workgroup z's k-steps into y + z M ldy

struct EpiArgs {
  void* y;             // EPI_F32 / EPI_BF16 / EPI_GELU_BF16: output rows (ldy elements apart); EPI_SWIGLU: bf16 out (N/2 wide)
  int64_t ldy;         // output row stride in elements
  float* resid;        // EPI_GATE_ADD: the fp32 residual rows, ldy apart
  const float* gate;   // EPI_GATE_ADD: gate rows (row 0, row 1 = gate + mstride)
  int n0, p, mstride;  // EPI_GATE_ADD, EPI_QKV: the sequence row of output row 0; EPI_GATE_ADD: the prefix length,
                       // the modulation row stride
  // EPI_QKV: the fused QKV product (N = 3 x 4096: q | k | v, heads of 128 columns) straight into
  // the attention's layouts -- q and k RMS-normed over each head (weights wq, wk, eps 1e-6) and
  // rotated by cs ([sequence row][128]: cos, sin of each pair), q times qscale; Q [32][M][128],
  // K [32][lcap][128] at key n0 + m, V^T [32][128][lcap] at column vt_pos(n0 + m), all fp16
  const float* wq;
  const float* wk;
  const float* cs;
  float qscale;
  uint16_t* q;
  uint16_t* kc;
  uint16_t* vt;
  int64_t lcap;
  int64_t qld;   // EPI_QKV: Q's rows a head (the pass's; 0: M)
};

// The block products' Q8_0 operand, tiled: for each block of 256 rows (rows past N zero) and each
// k-step of 64 columns, QT_CHUNK contiguous bytes -- the 256 rows' 64 codes (row r at 64 r, the
// order the product's LDS stage holds them), then their two fp16 scales (row r at QT_SCALES + 4 r).
// Chunk (nb, t) is at (nb K/64 + t) QT_CHUNK.  One k-step of a tile is then one contiguous run of
// 17 KB: its DMA touches whole cache lines, and a wave's scale loads one line.
#define QT_CHUNK 17408
#define QT_SCALES 16384
inline int64_t tile_q8_bytes(int64_t rows, int64_t cols) { return (rows + 255) / 256 * (cols / 64) * QT_CHUNK; }
// QT from the SoA codes QS (N x K int8) and scales D (N x K/32 fp16); K % 64 == 0
hipError_t tile_q8(hipStream_t s, const int8_t* qs, const uint16_t* d, int64_t N, int64_t K, uint8_t* qt);

// A kernel's dynamic LDS limit raised to BYTES (hipFuncSetAttribute) once for each device it
// launches on, the current one: thread-safe, and each device's kernels get their own attribute
hipError_t ensure_lds(const void* kern, int bytes);

// a weight matrix as a block product streams it: bf16 rows WB (N x K), or, when WB is null, Q8_0:
// the tiled copy QT (the pipelined product's operand) and the SoA codes QS (N x K int8) and scales
// QD (N x K/32 fp16) that the other kernels read
struct WOp {
  const uint16_t* wb;
  const int8_t* qs;
  const uint16_t* qd;
  const uint8_t* qt;
};

// Y = X W^T with X bf16 (M x K, lda) and W Q8_0 (W.qt, or W.qs/W.qd where the pipeline does not fit)
hipError_t gemm_q8(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N, int64_t K,
                   Epi epi, const EpiArgs& ea);
hipError_t gemm_wbf16(hipStream_t s, const uint16_t* x, int64_t lda, const uint16_t* w,
                      int64_t M, int64_t N, int64_t K, Epi epi, const EpiArgs& ea);
// rows 0 .. M-1 of a product too short to fill the chip (a pass's prompt rows) with its K split
// over S workgroups a tile into PART (S x M x N floats, at most PART_CAP), then the sums in
// order through the epilogue: EPI_GATE_ADD, EPI_SWIGLU, EPI_F32, EPI_BF16 or EPI_F16.  With
// NSUM the sums are left to the caller (split_sum_rms, qkv_prep_part): *NSUM = S, or 0 where
// the product ran whole through the epilogue instead
hipError_t gemm_split_rows(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                           int64_t K, Epi epi, const EpiArgs& ea, float* part, int64_t part_cap, int smax = 8,
                           int* nsum = nullptr);
// the QKV product with the q/k norm, RoPE and the K/V^T stores fused (EPI_QKV), bf16 or Q8_0
// weights; hipErrorNotSupported when the shapes or alignments do not fit the fused path
hipError_t gemm_qkv(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t K,
                    const EpiArgs& ea);
// the edge products: Y = X W^T all fp32 on the SIMD lanes (K % 32 == 0); optional GELU-tanh on Y.
// W is read from wf32 (fp32 rows) when given, else wbf16 (bf16 rows), else qs/d (Q8_0).
// ... with K split when the product has few tiles over a long K and PART (S x M x N floats, at
// most PART_CAP) is given
hipError_t gemm_f32(hipStream_t s, const float* x, int64_t ldx, const int8_t* qs, const uint16_t* d,
                    const uint16_t* wbf16, const float* wf32, int64_t M, int64_t N, int64_t K, float* y, int64_t ldy,
                    int gelu, float* part = nullptr, int64_t part_cap = 0);
// small M (<= 4): Y = X W^T, X fp32, fp32 sums; optional SiLU on the output; W as gemm_f32 reads it
hipError_t gemv_q8(hipStream_t s, const float* x, int64_t ldx, const int8_t* qs, const uint16_t* d,
                   const uint16_t* wbf16, const float* wf32, int64_t M, int64_t N, int64_t K, float* y, int64_t ldy,
                   int silu);

hipError_t synth_q8(hipStream_t s, uint64_t key, int64_t rows, int64_t cols, int64_t row_stride_blocks,
                    const int32_t* row_map, int8_t* qs, uint16_t* d);
hipError_t synth_normal(hipStream_t s, uint64_t key, int64_t n, float base, float scale, int add_base, float* out);
hipError_t dequant_q8(hipStream_t s, const int8_t* qs, const uint16_t* d, int64_t n, float* f32, uint16_t* bf16);
hipError_t repack_q8_blocks(hipStream_t s, const uint8_t* blocks, int64_t nblocks_row, int64_t rows,
                            const int32_t* row_map, int8_t* qs, uint16_t* d);
hipError_t f32_to_bf16(hipStream_t s, const float* x, uint16_t* y, int64_t n);

hipError_t ln_mod(hipStream_t s, int n, int n0, int p, int mstride, const float* x, int64_t ldx,
                  const float* mod, void* out, int out_bf16);
hipError_t rms_norm(hipStream_t s, int n, int width, float eps, const float* x, const float* w, void* out, int out_bf16);
// a split product's S partial sums (S x M x N, S <= 8, N = 4096) through EPI_GATE_ADD's store
// into EA's residual, then rms_norm of the finished rows (W, EPS) into bf16 Y, in one pass
hipError_t split_sum_rms(hipStream_t s, int S, int64_t M, int64_t N, const float* part, const EpiArgs& ea, float eps,
                         const float* w, uint16_t* y);
hipError_t gate_add(hipStream_t s, int64_t count, int width, int n0, int p, int mstride, float* x, const float* h,
                    const float* gate);
hipError_t swiglu(hipStream_t s, int64_t n, int f, const uint16_t* gu, uint16_t* out);
hipError_t swiglu_pairs(hipStream_t s, int64_t n, int f, const float* gu, float* out);
hipError_t gelu_tanh(hipStream_t s, int64_t count, float* x);
hipError_t silu(hipStream_t s, int64_t count, float* x);
hipError_t qkv_prep(hipStream_t s, const uint16_t* qkv, int64_t n, const float* wq, const float* wk,
                    const float* cs, uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap,
                    int64_t qld, int kv_group = 1);
// qkv_prep on the fp16 rows a split QKV product's S partial sums (S x n rows, in order, S <= 8)
// make
hipError_t qkv_prep_part(hipStream_t s, const float* part, int S, int64_t n, const float* wq, const float* wk,
                         const float* cs, uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap,
                         int64_t qld, int kv_group = 1);
hipError_t latent_rows(hipStream_t s, const float* latent, int64_t nimg, float* rows);
hipError_t rows_to_latent(hipStream_t s, const float* rows, int64_t nimg, float* latent);
hipError_t euler(hipStream_t s, int64_t count, float* z, const float* v, float ds);
// the largest finite |x| and the count of values that are not finite of COUNT values of X (fp32,
// or bf16 when BF16), folded into a 16-byte record REC = {max |x| bits, 0, 64-bit count};
// tensor_stats_clear zeroes RECORDS of them
hipError_t tensor_stats(hipStream_t s, const void* x, int bf16, int64_t count, uint32_t* rec);
hipError_t tensor_stats_clear(hipStream_t s, uint32_t* rec, int64_t records);
// W8A8 (w8a8.hip): activation rows to Q8_0, and the int8 product with per-block scales
hipError_t quant_q8(hipStream_t s, const void* x, int xbf16, int64_t ldx, int64_t n, int64_t K, int8_t* q,
                    uint16_t* d);
hipError_t gemm_w8a8(hipStream_t s, const int8_t* xq, const uint16_t* xd, int64_t M, const int8_t* wq,
                     const uint16_t* wd, int64_t N, int64_t K, void* y, int64_t ldy, int f16out);
// Q [32][QLD][128] (QLD 0: N), queries Q0 .. Q0 + N - 1 over keys 0 .. L - 1 under xa_lim
hipError_t attend(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, void* out,
                  int n, int q0, int p, int l, int64_t lcap, int b0, int b1, float scale, int of32 = 0,
                  int64_t qld = 0);

// the VAE decoder (vae.hip).  vae_conv's outputs: fp32 (+ bias, + res when given), bf16 (+ bias,
// + res when given), fp32 (+ bias) clamped to -1 .. 1, fp32 (+ bias, + DupUp3D of keep: kcin
// channels at half size, frame ft - 1 of ft); taps 9 or 1; up 1: the input is the half-size
// picture; up 2: stride 2 over the double-size input (zero padding below and to the right)
enum VaeOut { VAE_F32 = 0, VAE_BF16 = 1, VAE_CLAMP = 2, VAE_DUPUP = 3, VAE_PART = 4, VAE_RMS = 5 };
struct VaeEpi {
  const float* res;    // VAE_F32 / VAE_BF16: added when not null (the output's layout)
  const float* keep;   // VAE_DUPUP: the stage's input, pixel rows of kcin
  int kcin, ft;
  uint16_t* y2;        // VAE_F32 / VAE_DUPUP: when not null, a bf16 copy of the output too
  // scratch for split-K partial sums (S x pixels x cout floats, part_cap floats): when given, a
  // 3 x 3 convolution of too few tiles to fill the chip splits its K over S workgroups (VAE_PART
  // partials, then a sum in fixed order with bias and res)
  float* part;
  int64_t part_cap;
  // when gamma is given (a convolution whose one channel tile holds every output channel: cout
  // 96, 144, 192 or 288): yr = silu(rms(output) x gamma) in bf16 too, the next block's or the
  // head's normed input; VAE_RMS writes yr only
  const float* gamma;
  uint16_t* yr;
  // 1: 256-pixel tiles always (the 128-pixel ones of large pictures off; the same sums, a test's
  // switch)
  int wide_only;
};
hipError_t vae_conv(hipStream_t s, int taps, int up, int out, const uint16_t* x, const uint16_t* wt,
                    const float* bias, const VaeEpi& ep, void* y, int h, int w, int c, int cout, int kp);
hipError_t vae_rms_silu(hipStream_t s, int64_t P, int C, const float* x, const float* gamma, uint16_t* y, int silu);
hipError_t vae_dupup_add(hipStream_t s, int cin, int cout, int ft, int h, int w, const float* x, float* y);
hipError_t vae_latent_pixels(hipStream_t s, int64_t P, int C, const float* z, uint16_t* y);
// the encoder's: AvgDown3D's shortcut (y, h/2 x w/2, += that of x, h x w), y += x, the first
// convolution's RGBA neighbourhoods as rows of 64 bf16, the mean's channels out of pixel rows
hipError_t vae_avgdown_add(hipStream_t s, int cin, int cout, int ft, int h, int w, const float* x, float* y);
hipError_t vae_add(hipStream_t s, int64_t n, const float* x, float* y);
hipError_t vae_rgba_taps(hipStream_t s, int h, int w, const float* x, uint16_t* y);
hipError_t vae_pixels_latent(hipStream_t s, int64_t P, int C, int ld, const float* x, float* z);
hipError_t vae_split_qkv(hipStream_t s, int64_t n, int64_t np, int c, const float* qkv, uint16_t* q, uint16_t* k,
                         uint16_t* vt);
hipError_t vae_softmax_rows(hipStream_t s, int n, int np, float scale, const float* S, uint16_t* P);
hipError_t vae_pack_conv(hipStream_t s, int64_t o, int ci, int taps, int kp, const float* src, uint16_t* dst);
hipError_t vae_round_bf16(hipStream_t s, int64_t n, float* x);

// the vision tower (vision.hip), fp32: patches/positions/rotary of a picture, LayerNorm rows,
// Y = X W^T + bias (+ R) (act 0 none, 1 GELU tanh, 2 GELU erf), heads with the rotary, attention
hipError_t vis_prep(hipStream_t s, const float* px, int w, int gh, int gw, const float* table, int side, int D,
                    float* pat, float* pe, float* cs);
hipError_t vis_ln(hipStream_t s, int64_t rows, int width, const float* x, const float* w, const float* b, float* y);
hipError_t vis_gemm(hipStream_t s, const float* x, const float* w, const float* bias, const float* r, float* y,
                    int64_t M, int64_t N, int64_t K, int act);
hipError_t vis_heads(hipStream_t s, int n, int heads, const float* qkv, const float* cs, float qscale, float* q,
                     float* k, float* vt);
hipError_t vis_attend(hipStream_t s, int n, int heads, const float* q, const float* k, const float* vt, float* att);
hipError_t vis_sum(hipStream_t s, int64_t n, const float* a, const float* b, float* y);
hipError_t round_f16(hipStream_t s, int64_t n, float* x);

// the prompt encoder (encoder.hip): the token embedding's rows, Q8_0 (qs, d) or fp32 (f32)
hipError_t enc_embed(hipStream_t s, const int32_t* ids, int n, int64_t vocab, const int8_t* qs, const uint16_t* d,
                     const float* f32, int width, float* out);

}  // namespace exn
