/* exn_hip.h -- the C ABI of libexn-hip.so: ex-nihilo's DiT denoising step on
 * one MI355X (gfx950), hand-written HIP kernels behind plain C entry points.
 *
 * It replaces the CUDA layer under the reference's DiT backend trio
 * (upload-dit / dit-velocity / dit-release, src/cuda-dit.lisp:52,137,99):
 * illatio's device, memory and launch calls (il::open-cuda, il::cuda-alloc,
 * il::cuda-upload, il::cuda-download, il::cuda-copy-dd, il::launch) and the
 * kernels they launch (src/cuda/dit.cu; illatio's repack_q8, quant_q8,
 * MM_Q8_MMA2, d4_mm_q8_0, g53_mm_bf16, d41_mm_f32, v_rms).  A host binds it
 * with any C FFI (sb-alien in ex-nihilo_amd/lisp/hip-dit.lisp, ctypes in exn_hip).
 *
 * Conventions:
 *   - Every call returns an int status, EXN_OK (0) or an EXN_E* code; the
 *     message of the calling thread's last failure is exn_last_error().
 *     No call aborts the process.
 *   - Matrices follow ggml's order (src/weights.lisp:23-24): ROWS outputs of
 *     COLS inputs, each row contiguous along COLS; Y = X W^T.
 *   - Device pointers are plain addresses (void*); a byte offset into a
 *     buffer, the reference's (cons buf off), is the pointer plus the offset.
 *   - Work is ordered on the context's stream; exn_download and the
 *     host-pointer velocity call synchronise, everything else is
 *     asynchronous.  One thread at a time per context (the reference
 *     serialises callers with *gpu-lock*, src/server.lisp:24-28).
 */
#ifndef EXN_HIP_H
#define EXN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXN_OK 0
#define EXN_ENODEV 1  /* no GPU, or no device of that index */
#define EXN_EINVAL 2  /* bad argument: size, shape, name, null pointer */
#define EXN_ENOMEM 3  /* device allocation failed */
#define EXN_EHIP 4    /* a HIP runtime call failed */
#define EXN_ESTATE 5  /* out of order: a tensor missing, a model released */

/* weight kinds (the GGUF tensor types the reference accepts, src/cuda-dit.lisp:65-81) */
#define EXN_Q8_0 8
#define EXN_F32 0
#define EXN_BF16 30
#define EXN_F16 1     /* the vision tower's tensors only (mmproj-f16.gguf) */

/* activation dtypes of the op-level entry points */
#define EXN_DT_F32 0
#define EXN_DT_BF16 1
#define EXN_DT_F16 2 /* outputs of exn_mm only */

typedef struct exn_ctx exn_ctx; /* a device and its stream (il::open-cuda / exn-device, src/cuda-dit.lisp:25-40) */
typedef struct exn_w exn_w;     /* a weight matrix on the device (the gdit-w entries, src/cuda-dit.lisp:46) */
typedef struct exn_dit exn_dit; /* a DiT: weights, scratch, kept prompt K/V (the gdit struct, src/cuda-dit.lisp:44-50) */

/* --- status and context ------------------------------------------------------------ */

const char* exn_last_error(void);
int exn_version(void);
int exn_device_count(int* n);
/* il::open-cuda + exn-device (src/cuda-dit.lisp:25-40): EXN_ENODEV cleanly when there is no GPU */
int exn_open(int device, exn_ctx** out);
int exn_close(exn_ctx* ctx);
/* order the context's work on STREAM (a hipStream_t); NULL restores the context's own */
int exn_set_stream(exn_ctx* ctx, void* stream);
int exn_sync(exn_ctx* ctx); /* il::cuda-sync */

/* --- device memory: il::cuda-alloc / cuda-free / cuda-upload / cuda-download / cuda-copy-dd ------------ */

int exn_alloc(exn_ctx* ctx, size_t bytes, void** dptr);
int exn_free(exn_ctx* ctx, void* dptr);
int exn_upload(exn_ctx* ctx, void* dst, const void* src, size_t bytes);
int exn_download(exn_ctx* ctx, void* dst, const void* src, size_t bytes); /* synchronous */
int exn_copy(exn_ctx* ctx, void* dst, const void* src, size_t bytes);

/* --- weights (upload-dit's per-tensor branch, src/cuda-dit.lisp:59-81) ------------------------------ */

/* ROWS x COLS Q8_0 from GGUF block_q8_0 records in host memory (34 bytes a block:
 * fp16 d, 32 int8 q), e.g. the mmapped file itself; repacked on the device as
 * repack_q8 does (src/cuda-dit.lisp:71-76).  COLS % 32 == 0. */
int exn_weight_q8_0(exn_ctx* ctx, const void* blocks, int64_t rows, int64_t cols, exn_w** out);
/* a non-Q8_0 matrix (src/cuda-dit.lisp:77-80), kept as given: fp32 rows, multiplied in fp32
 * (d41_mm_f32, :127-130), or bf16 rows, multiplied on the bf16 MFMA (g53_mm_bf16) */
int exn_weight_f32(exn_ctx* ctx, const float* data, int64_t rows, int64_t cols, exn_w** out);
int exn_weight_bf16(exn_ctx* ctx, const uint16_t* data, int64_t rows, int64_t cols, exn_w** out);
/* test hook, no reference counterpart: a synthetic Q8_0 matrix made on the device by the
 * counter-based generator (seed, tensor id) that the host oracle restates bit for bit */
int exn_weight_q8_0_synth(exn_ctx* ctx, uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, exn_w** out);
int exn_weight_info(const exn_w* w, int64_t* rows, int64_t* cols, int* kind);
int exn_weight_free(exn_w* w);
/* test hook: W dequantised, fp32(d) * q into F32 and its bf16 rounding into BF16 (either may be NULL) */
int exn_dequant(exn_ctx* ctx, const exn_w* w, float* f32, uint16_t* bf16);
/* no reference counterpart (the reference keeps Q8_0 in 24 GB): BF16 = 1 keeps a resident
 * bf16 expansion of a Q8_0 matrix, bf16(fp32(d) * q) -- the values its products round
 * the weights to anyway -- and the products then stream it instead of dequantising in
 * the kernel; 0 drops it.  Costs 2 bytes a weight on top of the 1.0625 of Q8_0. */
int exn_weight_resident(exn_ctx* ctx, exn_w* w, int bf16);

/* --- ops: the kernels of src/cuda/dit.cu and illatio's products, on device pointers ------------------ */

/* mm (src/cuda-dit.lisp:115-130): Y (n rows) = X (n rows) W^T.  X is fp32 or bf16
 * (XDT), Y fp32, bf16 or fp16 (YDT); n <= 4 with fp32 X and Y goes through a GEMV in fp32.
 * An F32 matrix takes fp32 X and Y and multiplies in fp32 (d41_mm_f32); Q8_0 and BF16
 * matrices take bf16 operands (fp32 X rounded to bf16 in a buffer the context grows). */
int exn_mm(exn_ctx* ctx, const exn_w* w, const void* x, int xdt, void* y, int ydt, int64_t n);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops): exn_mm with the same arguments and results,
 * which calls no hipMalloc or hipFree.  The bf16 copy of fp32 X goes to a static device
 * array of 64 MiB a GPU (held until the process ends) instead of a buffer the context grows:
 * n x cols x 2 bytes past 64 MiB is EXN_EINVAL.  Every call on one GPU shares its array,
 * so calls that overlap on one GPU (two streams or threads) race. */
int exn_mm_noalloc(exn_ctx* ctx, const exn_w* w, const void* x, int xdt, void* y, int ydt, int64_t n);
/* the reference's default *int8* products (src/cuda-dit.lisp:110-126), whose kernels live in
 * illatio, after ggml's: quant_q8 (:120-123) takes N rows of K activations (fp32 or bf16,
 * EXN_DT_F32 / EXN_DT_BF16, LDX apart) to Q8_0 by blocks of 32, Q int8 [n][K] and D fp16
 * [n][K/32], d = amax / 127 and q = round(x / d) half away from zero */
int exn_quant_q8(exn_ctx* ctx, const void* x, int xdt, int64_t ldx, int64_t n, int64_t k, int8_t* q, uint16_t* d);
/* the int8 product behind mm (:119-124, illatio's MM_Q8_MMA2): a Q8_0 matrix W (rows x cols)
 * with N rows from exn_quant_q8, per 32-block the exact integer dot product, then
 * y = fma(float(isum), dx * dw, y) in fp32 over the blocks in order; Y [n][rows] fp32 or fp16
 * (EXN_DT_F32 / EXN_DT_F16) */
int exn_mm_w8a8(exn_ctx* ctx, const exn_w* w, const int8_t* xq, const uint16_t* xd, int64_t n, void* y, int ydt);
/* mm, then x_gate_add fused into the product's store (src/cuda/dit.cu:34-41):
 * RESID[t] += tanh(GATE[row]) * (X W^T)[t]; sequence row N0 + t < P takes GATE + MSTRIDE */
int exn_mm_gate_add(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, int64_t n, float* resid, int n0, int p,
                    int mstride, const float* gate);
/* mm on a gate_up matrix uploaded with exn_weight_pairs, then x_swiglu2 (src/cuda/dit.cu:186-192)
 * fused: FF (n x rows/2, bf16) = silu(gate) * up */
int exn_mm_swiglu(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, uint16_t* ff, int64_t n);
/* interleave a gate_up matrix's halves by 32 rows in place (gate rows 0..31, up rows
 * 0..31, gate 32..63, ...) so that exn_mm_swiglu finds each pair in one tile */
int exn_weight_pairs(exn_ctx* ctx, exn_w* w);
/* x_ln_mod (src/cuda/dit.cu:17-32): OUT = LayerNorm(X) * (1 + MOD[row]), width 4096,
 * X rows LDX apart; sequence row N0 + t < P takes MOD + MSTRIDE.  OUT fp32 or bf16. */
int exn_ln_mod(exn_ctx* ctx, int n, int n0, int p, int mstride, const float* x, int64_t ldx, const float* mod,
               void* out, int outdt);
/* v_rms (src/cuda-dit.lisp:176): Y = X / rms(X) * W, eps as given; Y fp32 or bf16 */
int exn_rms(exn_ctx* ctx, int n, int width, float eps, const float* x, const float* w, void* y, int ydt);
/* x_gate_add (src/cuda/dit.cu:34-41), fp32: X += tanh(GATE[row]) * H over COUNT values */
int exn_gate_add(exn_ctx* ctx, int64_t count, int width, int n0, int p, int mstride, float* x, const float* h,
                 const float* gate);
/* x_swiglu2 (src/cuda/dit.cu:186-192), bf16: OUT (n x f) = silu(GU[:, :f]) * GU[:, f:] */
int exn_swiglu(exn_ctx* ctx, int64_t n, int f, const uint16_t* gu, uint16_t* out);
/* x_gelu_tanh, x_silu (src/cuda/dit.cu:194-206), fp32 in place */
int exn_gelu_tanh(exn_ctx* ctx, int64_t count, float* x);
int exn_silu(exn_ctx* ctx, int64_t count, float* x);
/* x_qk_norm_rope (src/cuda/dit.cu:43-58) for q and k, plus v, from one fused QKV
 * product: QKV fp16 rows of 3 x 4096 for tokens 0..n-1 = sequence rows ROW0..;
 * CS 128 floats a sequence row (cos, sin of 64 pairs).  Writes, fp16, Q [32][n][128]
 * scaled by log2(e)/sqrt(128), K into [32][LCAP][128] rows ROW0.., V transposed
 * into [32][128][LCAP]: key k at column k with bits 2 and 3 swapped (a permutation
 * inside every aligned 16 keys, the order exn_attend's P V product reads them in) */
int exn_qkv_prep(exn_ctx* ctx, const uint16_t* qkv, int64_t n, const float* wq, const float* wk, const float* cs,
                 uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap);
/* mm on the fused QKV matrix (src/cuda-dit.lisp:115-130) with x_qk_norm_rope (src/cuda/dit.cu:43-58)
 * in the product's store: X_BF16 [n][4096] times W (12288 x 4096, bf16 or resident Q8_0), then
 * exn_qkv_prep's outputs from the fp32 sums, without the fp16 QKV rows in between.  Arrays
 * 16-byte aligned, LCAP % 64 == 0, ROW0 + n <= LCAP, CS with rows ROW0 .. ROW0 + n - 1. */
int exn_mm_qkv(exn_ctx* ctx, const exn_w* w, const uint16_t* x_bf16, int64_t n, const float* wq, const float* wk,
               const float* cs, uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap);
/* x_attend_mma (src/cuda/dit.cu:208-336) with xa_lim's mask (:60-66): OUT [n][4096]
 * bf16 for queries = sequence rows Q0..Q0+n-1 over keys 0..l-1; Q, K, V^T fp16 in the
 * layouts exn_qkv_prep writes.  SCALE multiplies the scores, which are in log2
 * units (1 for exn_qkv_prep's Q).  LCAP % 64 == 0; K's rows and V^T's columns of
 * keys l..roundup(l, 64)-1 finite (they are read, and masked). */
int exn_attend(exn_ctx* ctx, const uint16_t* q, const uint16_t* k, const uint16_t* vt, uint16_t* out, int n, int q0,
               int p, int l, int64_t lcap, int b0, int b1, float scale);
/* the Euler update of generate's loop (src/generate.lisp:133-135): Z += DS * V */
int exn_euler(exn_ctx* ctx, int64_t count, float* z, const float* v, float ds);

/* --- the model: the backend trio ----------------------------------------------------------------- */

/* an empty DiT of LAYERS blocks (32 in the real model; fewer to look at part of a step, as
 * *dit-layers* does in src/metal-dit.lisp:112) on CTX */
int exn_dit_create(exn_ctx* ctx, int layers, exn_dit** out);
/* one tensor of upload-dit (src/cuda-dit.lisp:59-81), by its name without the
 * "model.diffusion_model." prefix and its ggml dims D0 (contiguous) x D1 (1 for a vector);
 * KIND EXN_Q8_0 (block_q8_0 records), EXN_F32 or EXN_BF16.  Dims and names are held
 * against dit-expected (src/weights.lisp:22-45); txt_in.text_norm.weight is used as 1 + w.
 * Edge matrices are kept as given (F32 multiplied in fp32).  A block matrix given as F32 or
 * BF16 is kept as bf16 rows (F32 rounded to nearest even), the operands its products take;
 * its layer matrix (q | k | v, or gate_up) then runs from bf16 rows, its Q8_0 slots
 * dequantised into them exactly.  Setting or synthesising a tensor drops the kept prompt K/V. */
int exn_dit_set(exn_dit* d, const char* name, int kind, const void* data, int64_t d0, int64_t d1);
/* test hook: every tensor of the model made on the device by the synthetic generator */
int exn_dit_synth(exn_dit* d, uint64_t seed);
/* EXN_OK when every expected tensor is present, else EXN_ESTATE naming each missing one
 * (open-dit's check, src/weights.lisp:47-61) */
int exn_dit_check(exn_dit* d);
/* no reference counterpart: BF16 = 1 (the default) runs the block matrices from resident
 * bf16 expansions (exn_weight_resident; 14 GB for the 7B model), made here for the matrices
 * present and at the next step for any set later; 0 drops them and runs from Q8_0 with the
 * dequantisation inside the product.  A change drops the kept prompt K/V. */
int exn_dit_resident(exn_dit* d, int bf16);
/* *int8* (src/cuda-dit.lisp:110-113): ON = 1 takes every product of a Q8_0 matrix with at
 * least 16 rows the reference's int8 way (exn_quant_q8, exn_mm_w8a8; a block's four when all
 * four qualify) -- the reference's default numerics; 0, this library's default, the bf16
 * products.  A change drops the kept prompt K/V. */
int exn_dit_w8a8(exn_dit* d, int on);
/* dit-velocity (src/cuda-dit.lisp:137-243): CONTEXT (P x 4096 fp32, the encoder's states),
 * LATENT (64 x H x W fp32, channel-major) -> V (64 x H x W), host memory, synchronous.
 * SIGMA is a double, as the reference's schedule (src/generate.lisp:7-9); t = 1000 sigma.
 * PREFIX_KEY != 0 keeps the prompt's K/V after the first call and reuses them while the
 * key and prefix length stay.  REF_LATENT != NULL: an edit's reference picture (64 x RH x
 * RW) put in the prefix after the first REF_A text rows (P counts the text only). */
int exn_dit_velocity(exn_dit* d, const float* context, int p, const float* latent, int h, int w, double sigma,
                     uint64_t prefix_key, int ref_a, const float* ref_latent, int rh, int rw, float* v);
/* the same on device pointers, asynchronous on the context's stream */
int exn_dit_velocity_dev(exn_dit* d, const float* context, int p, const float* latent, int h, int w, double sigma,
                         uint64_t prefix_key, int ref_a, const float* ref_latent, int rh, int rw, float* v);
/* generate's loop (src/generate.lisp:133-135) on the device: Z (device, 64 x H x W) through
 * the NSIG - 1 Euler steps of SIGMAS; the prompt's K/V are made at the first step under a key
 * of the loop's own and kept for the rest */
int exn_dit_generate_dev(exn_dit* d, const float* context, int p, float* z, int h, int w, const double* sigmas,
                         int nsig, int ref_a, const float* ref_latent, int rh, int rw);
/* *dit-trace* (src/metal-dit.lisp:114-124), as a copy: while BUF (device, fp32) is set,
 * each velocity pass copies the residual stream's n rows before the first block to
 * BUF and after block i to BUF + (i + 1) * n * 4096, as far as CAP floats reach;
 * NULL turns it off */
int exn_dit_trace(exn_dit* d, float* buf, int64_t cap);
/* *dit-trace*'s numbers (src/metal-dit.lisp:114-124,206-213,254-257): while ON, each velocity
 * records the largest finite |x| and the count of values that are not finite of, before the
 * blocks, the residual stream entering them (record 0) and, in an uncached pass, txt_in's GELU
 * rows (record 3); after block l, the stream (record 4 (l + 1)), the attention's output (+1)
 * and the MLP's inner rows, SwiGLU's output (+2; the gate_up product's own rows are never
 * stored).  exn_dit_stats_read copies the last velocity's first RECORDS of the (layers + 1) x 4
 * records (a slot with nothing recorded reads 0, 0) into MAXABS and NONFINITE; EXN_ESTATE when
 * none was recorded since the model's last release */
int exn_dit_stats(exn_dit* d, int on);
int exn_dit_stats_read(exn_dit* d, float* maxabs, int64_t* nonfinite, int64_t records);
/* EXN_PROFILE's per-kernel GPU time (src/tenant.lisp:53-62), on the context's stream:
 * exn_dit_profile(d, ON) clears and starts recording a HIP event pair around every
 * launch of the step of the kernel classes in the bit mask ON (1 << EXN_PROF_...; -1
 * for all); (d, 0) stops.  exn_dit_profile_read gives a class's summed milliseconds,
 * launches, and algorithmic FLOPs and HBM bytes (one read of each input, one write of
 * each output) over the recorded launches. */
#define EXN_PROF_QKV 0      /* LayerNormed rows x to_q|to_k|to_v (qk-norm, RoPE, K/V^T stores fused on bf16 weights) */
#define EXN_PROF_ATTEND 1   /* attention */
#define EXN_PROF_OUT 2      /* attention rows x to_out.0, gated residual fused */
#define EXN_PROF_GATE_UP 3  /* LayerNormed rows x gate_up, SwiGLU fused */
#define EXN_PROF_DOWN 4     /* SwiGLU rows x img_mlp.out, gated residual fused */
#define EXN_PROF_LN_MOD 5   /* LayerNorm x (1 + scale) */
#define EXN_PROF_QKV_PREP 6 /* QK RMSNorm + RoPE, V transposed (when the QKV product does not fuse them) */
#define EXN_PROF_EDGE 7     /* timestep, txt_in, img_in, proj_out and the rest */
#define EXN_PROF_CLASSES 8
int exn_dit_profile(exn_dit* d, int on);
/* events around every EVERY-th launch of each recorded class only (default 1): the sampled
 * launches' mean duration at a fraction of the events' cost; restarts the count */
int exn_dit_profile_every(exn_dit* d, int every);
int exn_dit_profile_read(exn_dit* d, int cls, double* ms, int64_t* launches, double* flops, double* bytes);
/* test hook: dit-positions and rope-table (src/host.lisp:19-50) as the step computes them, on
 * the host (no GPU needed): for P text rows, an H x W image and, when EDIT, a RH x RW reference
 * picture after the first REF_A text rows, each sequence row's (frame, row, col) into POS
 * (3 ints a row) and the cos, sin of its 64 angles into CS (128 floats a row, pairs
 * interleaved); either may be NULL.  Rows = P + (EDIT ? RH RW : 0) + H W, at most ROWS_CAP. */
int exn_dit_rope_table(int p, int h, int w, int edit, int ref_a, int rh, int rw, int64_t rows_cap, int32_t* pos,
                       float* cs);
/* dit-release (src/cuda-dit.lisp:99-108): scratch and kept prompt K/V freed, weights kept */
int exn_dit_release(exn_dit* d);
int exn_dit_destroy(exn_dit* d);
/* bytes of device memory the model holds: weights, scratch, kept K/V */
int exn_dit_memory(exn_dit* d, int64_t* weights, int64_t* scratch);

/* --- the VAE decoder and encoder (replace src/cuda-vae.lisp's gvae and src/cuda/vae.cu) --- */
typedef struct exn_vae exn_vae;
/* upload-vae (src/cuda-vae.lisp:15-26) in parts: create, then one exn_vae_set a tensor */
int exn_vae_create(exn_ctx* ctx, exn_vae** out);
/* one decoder or encoder tensor by its safetensors name and shape (NDIMS dims, row-major), KIND
 * EXN_BF16 (the file's bit patterns) or EXN_F32; names and shapes held against vae-expected
 * and vae-encoder-expected (src/weights.lisp:69-134; the video-only time_conv tensors are not
 * taken).  A convolution's (o, i, [1,] k, k) weights are kept as bf16 rows
 * of (ky, kx, ci), as src/host.lisp:73-90 lays them out for the GPU. */
int exn_vae_set(exn_vae* v, const char* name, int kind, const void* data, const int64_t* dims, int ndims);
/* test hook: every decoder and encoder tensor made on the device by the synthetic generator
 * (bf16 values) */
int exn_vae_synth(exn_vae* v, uint64_t seed);
/* EXN_OK when every decoder tensor is present, else EXN_ESTATE naming the first missing one
 * (open-vae's check, src/weights.lisp:136-147) */
int exn_vae_check(exn_vae* v);
/* the same for the encoder's tensors (open-vae checks both, src/weights.lisp:136-147; here a
 * decoder may be loaded alone, and exn_vae_encode makes this check) */
int exn_vae_check_encoder(exn_vae* v);
/* vae-decode (src/cuda-vae.lisp:94-136): LATENT (64 x H x W floats, channel-major,
 * denormalized) -> RGBA (16H x 16W x 4 floats in -1..1, rows of pixels, channels last).
 * Host arrays; exn_vae_decode_dev takes device arrays, on the context's stream. */
int exn_vae_decode(exn_vae* v, const float* latent, int h, int w, float* rgba);
int exn_vae_decode_dev(exn_vae* v, const float* latent, int h, int w, float* rgba);
/* vae-encode (src/cuda-vae.lisp:138-190): RGBA (H x W x 4 floats in -1..1, rows of pixels; H
 * and W multiples of 16, H W < 2^31 / 192) -> the latent's mean (64 x H/16 x W/16 floats, channel-major, as
 * exn_vae_decode takes it: denormalized).  Host arrays; exn_vae_encode_dev takes device
 * arrays, on the context's stream. */
int exn_vae_encode(exn_vae* v, const float* rgba, int h, int w, float* latent);
int exn_vae_encode_dev(exn_vae* v, const float* rgba, int h, int w, float* latent);
/* vae-release (src/cuda-vae.lisp:28-33): the scratch freed, the weights kept */
int exn_vae_release(exn_vae* v);
int exn_vae_destroy(exn_vae* v);
/* bytes of device memory the decoder holds: weights, scratch */
int exn_vae_memory(exn_vae* v, int64_t* weights, int64_t* scratch);
/* test hook, no reference counterpart: SMALL 1 (the default) lets the 96- and 144-wide
 * convolutions of pictures of 2^18 pixels or more run on 128-pixel tiles (two workgroups a CU),
 * 0 keeps every convolution on 256-pixel tiles; each output value is the same sum either way */
int exn_vae_tiles(exn_vae* v, int small);
/* the decoder's and encoder's kernels one at a time (src/cuda/vae.cu's x_conv3 with the 1 x 1
 * products, x_up2 folded in (UP 1), x_conv3s2 (UP 2), bias and residual fused; v_rms with
 * x_silu; x_dupup_add; x_avgdown_add).  X: bf16 pixel rows (H x W x C; H/2 x W/2 x C with UP 1;
 * 2H x 2W x C with UP 2, the output H x W); WT: bf16 rows of (tap, channel), KP long (a
 * multiple of 64, zero past TAPS * C); OUTDT 0 fp32 (+ RES when not null), 1 bf16, 2 fp32
 * clamped to -1..1.  C a multiple of 8, at least 64.  PART (PART_CAP floats, or null): scratch
 * with which a 3 x 3 convolution of fewer 256 x 288 tiles than the chip has CUs splits its K
 * over up to 4 workgroups a tile and sums their partials in order. */
int exn_vae_conv(exn_ctx* ctx, int taps, int up, int outdt, const uint16_t* x, const uint16_t* wt, const float* bias,
                 const float* res, void* y, int h, int w, int c, int cout, int kp, float* part, int64_t part_cap);
int exn_vae_rms_silu(exn_ctx* ctx, int64_t n, int c, const float* x, const float* gamma, uint16_t* y, int silu);
int exn_vae_dupup_add(exn_ctx* ctx, int cin, int cout, int ft, int h, int w, const float* x, float* y);
/* Y (H/2 x W/2 x COUT) += AvgDown3D(X) (H x W x CIN), frame FT - 1 of FT */
int exn_vae_avgdown_add(exn_ctx* ctx, int cin, int cout, int ft, int h, int w, const float* x, float* y);

/* --- the vision tower (replaces src/cuda-vision.lisp's q3vision and src/cuda/qvision.cu) -----
 * Qwen3-VL's ViT, which lets the prompt encoder see a picture to edit: 27 blocks of 1152, 16
 * heads of 72, FFN 4304, a learned 48 x 48 position table resampled to the picture's grid, a 2-D
 * rotary, patches of 16 px in 2 x 2 merge blocks; the merger (four patches to one row of 4096)
 * and three deepstack mergers after blocks 8, 16 and 24.  fp32 throughout, as the reference. */
typedef struct exn_vision exn_vision;
/* load-vision (src/cuda-vision.lisp:15-30) in parts: create, then one exn_vision_set a tensor */
int exn_vision_create(exn_ctx* ctx, exn_vision** out);
/* one tower tensor by its GGUF name (inspect/ref_vision.py's names) and row-major shape (NDIMS
 * dims, a matrix (out, in)), KIND EXN_F32, EXN_F16 or EXN_BF16; kept as fp32 (il::load-f32).
 * v.position_embd.weight is (S, 1152) for a square S (48 x 48 in the model); the two patch
 * kernels (v.patch_embd.weight and .weight.1, one frame given twice) are summed, as
 * vision-tensors does (src/host.lisp:175-190). */
int exn_vision_set(exn_vision* v, const char* name, int kind, const void* data, const int64_t* dims, int ndims);
/* test hook: every tower tensor from the synthetic generator (matrices fp16-valued) */
int exn_vision_synth(exn_vision* v, uint64_t seed);
/* EXN_OK when every tower tensor is present, else EXN_ESTATE naming the first missing one */
int exn_vision_check(exn_vision* v);
/* vision-encode (src/cuda-vision.lisp:34-101): PX, the picture (H x W x 4 floats, RGBA in
 * -1 .. 1, rows of pixels; H and W multiples of 32, H W / 256 patches at most 16384) ->
 * MERGED (M x 4096 floats, M = H W / 1024, in merge-block order: the 32-pixel grid row-major)
 * and DEEPSTACK (3 x M x 4096: after blocks 8, 16, 24).  Host arrays; exn_vision_encode_dev
 * takes device arrays, on the context's stream. */
int exn_vision_encode(exn_vision* v, const float* px, int h, int w, float* merged, float* deepstack);
int exn_vision_encode_dev(exn_vision* v, const float* px, int h, int w, float* merged, float* deepstack);
/* test hook: with ON, each encode keeps the patch rows after the embedding (WHICH 0) and after
 * block 0 (WHICH 1), N x 1152 floats, which exn_vision_traced copies to host memory OUT
 * (ref_vision.py's embed.f32 and blk0.f32) */
int exn_vision_trace(exn_vision* v, int on);
int exn_vision_traced(exn_vision* v, int which, float* out);
/* vision-release (src/cuda-vision.lisp:103-107): scratch freed, weights kept */
int exn_vision_release(exn_vision* v);
int exn_vision_destroy(exn_vision* v);
/* bytes of device memory the tower holds: weights, scratch */
int exn_vision_memory(exn_vision* v, int64_t* weights, int64_t* scratch);
/* the tower's kernels one at a time (device arrays, fp32).  exn_vis_gemm: Y (M x N) = X (M x K)
 * W^T (W: N x K) + BIAS (+ R, M x N, may be Y), then ACT (0 none, 1 GELU tanh form, 2 GELU erf
 * form): d41_mm_f32 with v_bias and v_gelu / x_gelu_tanh; K a multiple of 4, X and W 16-byte
 * aligned.  exn_vis_attend: softmax attention of N patches (a multiple of 4) over themselves,
 * HEADS heads of 72: Q and K [head][N][72] (Q scaled by log2(e)/sqrt(72)), VT [head][72][N],
 * ATT [N][HEADS x 72].  exn_vis_ln: LayerNorm of ROWS rows of WIDTH (eps 1e-6, q3v_layernorm). */
int exn_vis_gemm(exn_ctx* ctx, const float* x, const float* w, const float* bias, const float* r, float* y, int64_t m,
                 int64_t n, int64_t k, int act);
int exn_vis_attend(exn_ctx* ctx, int n, int heads, const float* q, const float* k, const float* vt, float* att);
int exn_vis_ln(exn_ctx* ctx, int64_t rows, int width, const float* x, const float* w, const float* b, float* y);

/* --- the prompt encoder (replaces illatio's qwen3 forward under src/encoder.lisp:41-67,143-183) ---
 * Qwen3-VL-8B's text model read for every token's state after its last block, before the final
 * norm: 36 layers of 4096, 32 query heads and 8 key/value heads of 128, FFN 12288 (SwiGLU),
 * RMSNorm eps 1e-6 (and over each head of q and k), RoPE theta 5e6 with interleaved M-RoPE,
 * causal.  Tokenizing stays the host's (il::tokenize). */
typedef struct exn_enc exn_enc;
/* load-encoder (src/encoder.lisp:41-48) in parts: an empty encoder of LAYERS blocks (36; fewer to
 * look at part of the model) with the model's RoPE base (il::model-rope-base, 5e6) */
int exn_enc_create(exn_ctx* ctx, int layers, double rope_base, exn_enc** out);
/* one tensor of te-q8_0.gguf by its name (token_embd.weight, blk.N.attn_norm / attn_q / attn_k /
 * attn_v / attn_output / attn_q_norm / attn_k_norm / ffn_norm / ffn_gate / ffn_up / ffn_down
 * .weight) and ggml dims D0 (contiguous) x D1 (1 for a vector): matrices EXN_Q8_0 (block_q8_0
 * records; token_embd also EXN_F32), norm weights EXN_F32.  output_norm.weight and output.weight
 * are accepted and not kept (the states are read before them). */
int exn_enc_set(exn_enc* e, const char* name, int kind, const void* data, int64_t d0, int64_t d1);
/* test hook: every tensor from the synthetic generator, a token embedding of VOCAB rows */
int exn_enc_synth(exn_enc* e, uint64_t seed, int64_t vocab);
/* EXN_OK when every tensor is present, else EXN_ESTATE naming the first missing one */
int exn_enc_check(exn_enc* e);
/* encoder-states (src/encoder.lisp:143-183) with call-with-picture-rows (:69-110): IDS (N token
 * ids), POS (N (t, h, w) triples, or NULL for text positions 0 .. N-1; mrope-table, :26-39);
 * when M > 0 rows PIC0 .. PIC0 + M - 1 take MERGED's rows (M x 4096, the vision tower's) after
 * the embedding and DEEP's set j (3 x M x 4096, or NULL) added after layer j; OUT: N x 4096
 * floats.  Host arrays; an id outside the vocabulary is EXN_EINVAL.  exn_enc_states_dev takes
 * device arrays and the rotary table CS (exn_enc_rope_table's N x 128 floats) in place of POS,
 * on the context's stream; there an id outside the vocabulary embeds as a row of zeros. */
int exn_enc_states(exn_enc* e, const int32_t* ids, int n, const int32_t* pos, int pic0, int m, const float* merged,
                   const float* deep, float* out);
int exn_enc_states_dev(exn_enc* e, const int32_t* ids, int n, const float* cs, int pic0, int m, const float* merged,
                       const float* deep, float* out);
/* mrope-table (src/encoder.lisp:26-39) on the host, no GPU needed: row t's frequency j < 64 turns
 * by its position on axis j mod 3 (t, h, w) below 60, by t above, at BASE^(-2j/128); the cos and
 * sin of pair j at CS[128 t + 2j] and [128 t + 2j + 1] (rotate_half's dims j and j + 64). */
int exn_enc_rope_table(const int32_t* pos, int n, double base, float* cs);
/* scratch freed, weights kept; destroy frees both */
int exn_enc_release(exn_enc* e);
int exn_enc_destroy(exn_enc* e);
/* bytes of device memory the encoder holds: weights (with any bf16 expansions), scratch */
int exn_enc_memory(exn_enc* e, int64_t* weights, int64_t* scratch);
/* No reference counterpart (illatio multiplies from Q8_0): BF16 1, the default, runs the
 * layers' products from a resident bf16 expansion of each Q8_0 matrix (bf16(fp32(d) q), the
 * operand values the Q8_0 products make in LDS; 14 GB beside the 7.4 GB of Q8_0, made by the
 * first exn_enc_states of more than 256 tokens and after a matrix is set: shorter prompts
 * stream the Q8_0 codes in every product and leave them unmade); 0 drops them and multiplies
 * from Q8_0. The states are the same either way. */
int exn_enc_resident(exn_enc* e, int bf16);

#ifdef __cplusplus
}
#endif

#endif /* EXN_HIP_H */
