// vision.hip -- Qwen3-VL's vision tower, the picture seen by the prompt encoder when editing
// (src/cuda-vision.lisp, src/cuda/qvision.cu; its numpy reference inspect/ref_vision.py), in
// fp32 as the reference computes it:
//
//   k_vis_prep    each patch's 768 pixels in merge-block order, its learned position resampled
//                 bilinearly from the table and the 2-D rotary's cosines and sines
//                 (src/host.lisp:119-166, which the reference runs on the host);
//   k_vis_gemm    Y = X W^T + b (+ R) (then GELU), fp32 products on v_mfma_f32_16x16x4_f32;
//   k_vis_ln      LayerNorm rows, eps 1e-6;
//   k_vis_heads   QKV rows into heads: q and k turned by the rotary, q scaled for the exp2
//                 softmax, V transposed;
//   k_vis_attend  softmax attention of every patch over every patch, flash-style, fp32 MFMAs.
//
// fp32 MFMAs (157 TFLOP/s dense on MI355X) keep the reference's fp32 products: the tower is
// held to float32 numpy, not to a bf16 tolerance.
#include "exn_common.h"

namespace exn {

typedef __attribute__((address_space(3))) void lds_void;

#define VIS_VOFF_NONE 0x80000000u   // past any extent: the DMA reads zeros

static inline unsigned vgrid(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

// one lane of a 16-byte DMA into LDS from base + voff + soff, zeros where voff passes the extent
__device__ __forceinline__ void vdma16(const void* base, uint32_t extent, lds_void* dst, uint32_t voff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, 0);
}

__device__ __forceinline__ void vis_wait_dma() {
  asm volatile("" ::: "memory");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// --- the picture's patches, positions and rotary ----------------------------------------

// One workgroup a patch k, in merge-block order (block row, block column, then the 2 x 2 inside):
// its pixels as (channel, row, column) from the RGBA picture (W pixels a row); its position row:
// the table (side x side rows of D) at 2 x 2 taps, corners aligned, the weights in double as
// inspect/ref_vision.py:63-69 forms them, the sum in fp32 in its order (:91-94); its 72 cosines,
// then 72 sines: 18 frequencies of the row, 18 of the column, those 36 twice, in double
// (src/host.lisp:154-166).
__global__ void __launch_bounds__(256)
k_vis_prep(const float* __restrict__ px, int W, int gh, int gw, const float* __restrict__ table, int side, int D,
           float* __restrict__ pat, float* __restrict__ pe, float* __restrict__ cs) {
#pragma clang fp contract(off)
  const int k = blockIdx.x, t = threadIdx.x;
  const int blk = k >> 2, in = k & 3, bw = gw >> 1;
  const int r = 2 * (blk / bw) + (in >> 1), c = 2 * (blk % bw) + (in & 1);
  for (int i = t; i < 768; i += 256) {
    const int ch = i >> 8, ky = (i >> 4) & 15, kx = i & 15;
    pat[(int64_t)k * 768 + i] = px[((int64_t)(r * 16 + ky) * W + c * 16 + kx) * 4 + ch];
  }
  int th[2], tw[2];
  double wh[2], ww[2];
  {
    const double sh = (double)r * (side - 1) / (double)max(gh - 1, 1);
    const double sw = (double)c * (side - 1) / (double)max(gw - 1, 1);
    const double fh = floor(sh), fw = floor(sw);
    wh[0] = fmax(1.0 - fabs(sh - fh), 0.0);
    wh[1] = fmax(1.0 - fabs(sh - (fh + 1.0)), 0.0);
    ww[0] = fmax(1.0 - fabs(sw - fw), 0.0);
    ww[1] = fmax(1.0 - fabs(sw - (fw + 1.0)), 0.0);
    th[0] = min((int)fh, side - 1);
    th[1] = min((int)fh + 1, side - 1);
    tw[0] = min((int)fw, side - 1);
    tw[1] = min((int)fw + 1, side - 1);
  }
  float wt[4];
  const float* row[4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      wt[2 * a + b] = (float)(wh[a] * ww[b]);
      row[2 * a + b] = table + (int64_t)(th[a] * side + tw[b]) * D;
    }
  for (int j = t; j < D; j += 256) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) s = s + wt[q] * row[q][j];
    pe[(int64_t)k * D + j] = s;
  }
  if (t < 36) {
    const int i = t % 18;
    const double a = (double)(t < 18 ? r : c) * (1.0 / pow(10000.0, (2.0 * i) / 36.0));
    const float cv = (float)cos(a), sv = (float)sin(a);
    float* o = cs + (int64_t)k * 144;
    o[t] = cv;
    o[t + 36] = cv;
    o[72 + t] = sv;
    o[72 + t + 36] = sv;
  }
}

hipError_t vis_prep(hipStream_t s, const float* px, int w, int gh, int gw, const float* table, int side, int D,
                    float* pat, float* pe, float* cs) {
  const int n = gh * gw;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_vis_prep, dim3(n), dim3(256), 0, s, px, w, gh, gw, table, side, D, pat, pe, cs);
  return hipGetLastError();
}

// --- LayerNorm ----------------------------------------------------------------------------

// one workgroup a row of WIDTH (a multiple of 4, at most 5120): mean, then the mean square about
// it, (x - mean) / sqrt(var + eps) * w + b, as inspect/ref_vision.py:35-38 orders it
__global__ void __launch_bounds__(256)
k_vis_ln(int width, const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b,
         float* __restrict__ y) {
#pragma clang fp contract(off)
  __shared__ float red[2][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, w4 = width >> 2;
  const f32x4* r = (const f32x4*)(x + (int64_t)blockIdx.x * width);
  f32x4 v[5];
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 5; ++e) {
    const int i = t + 256 * e;
    v[e] = i < w4 ? r[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    s += (v[e][0] + v[e][1]) + (v[e][2] + v[e][3]);
  }
  s = wave_sum(s);
  if (lane == 0) red[0][wave] = s;
  __syncthreads();
  const float mean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / (float)width;
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 5; ++e)
    if (t + 256 * e < w4)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d = v[e][j] - mean;
        q += d * d;
      }
  q = wave_sum(q);
  if (lane == 0) red[1][wave] = q;
  __syncthreads();
  const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float)width;
  const float sd = __fsqrt_rn(var + 1e-6f);
  f32x4* o = (f32x4*)(y + (int64_t)blockIdx.x * width);
#pragma unroll
  for (int e = 0; e < 5; ++e) {
    const int i = t + 256 * e;
    if (i < w4) {
      const f32x4 g = ((const f32x4*)w)[i], bb = ((const f32x4*)b)[i];
      f32x4 z;
#pragma unroll
      for (int j = 0; j < 4; ++j) z[j] = __fdiv_rn(v[e][j] - mean, sd) * g[j] + bb[j];
      o[i] = z;
    }
  }
}

hipError_t vis_ln(hipStream_t s, int64_t rows, int width, const float* x, const float* w, const float* b, float* y) {
  if (rows <= 0) return hipSuccess;
  if (width % 4 || width > 5120) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_vis_ln, dim3((unsigned)rows), dim3(256), 0, s, width, x, w, b, y);
  return hipGetLastError();
}

// --- the fp32 product ----------------------------------------------------------------------

// Y (M x N) = X (M x K) W^T (W: N x K, rows K apart) + bias, + R (M x N; may be Y itself: each
// element is read by the thread that then writes it), then GELU (ACT 1: the tanh form, 2: erf).
// Workgroup tiles of (32 RM) x (32 RN), four waves of (16 RM) x (16 RN), each a grid of 16 x 16
// v_mfma_f32_16x16x4_f32 blocks (A: lane l holds row l % 16, k = l / 16; D: lane l holds column
// l % 16, rows 4 (l / 16) + e).  K steps of 32: the tile's X and W rows (128 bytes each) move to
// LDS by DMA, two stages, row r's 16-byte chunk c stored at c ^ (r / 2 % 8) so that the fragment
// reads (16 rows at one chunk) fall in distinct banks.  A lane's fragment is 4 consecutive k of
// its row; MFMA j of a 16-wide k slice takes component j on both sides, so every k is summed
// once, in a different order than a plain loop.  Rows past M or N and k past K read as zeros.
template <int RM, int RN, int ACT>
__global__ void __launch_bounds__(256)
k_vis_gemm(const float* __restrict__ X, const float* __restrict__ Wt, const float* __restrict__ bias,
           const float* R, float* Y, int M, int N, int K) {
  constexpr int BM = 32 * RM, BN = 32 * RN, SA = BM * 128, STAGE = (BM + BN) * 128;
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int wm = (wave >> 1) * 16 * RM, wn = (wave & 1) * 16 * RN;
  const int tm = blockIdx.y * BM, tn = blockIdx.x * BN;
  const float* xb = X + (int64_t)tm * K;
  const float* wb = Wt + (int64_t)tn * K;
  const uint32_t xext = (uint32_t)((int64_t)min(BM, M - tm) * K * 4), wext = (uint32_t)((int64_t)min(BN, N - tn) * K * 4);
  // DMA: instruction i of wave w moves LDS chunks 64 (w R + i) + lane of the A (R = RM) or B
  // (R = RN) rows: row P / 8, LDS chunk P % 8, global chunk (P % 8) ^ (row / 2 % 8)
  uint32_t aoff[RM], boff[RN];
  int akc[RM], bkc[RN];
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    const int P = 64 * (wave * RM + i) + lane, r = P >> 3, c = (P & 7) ^ ((r >> 1) & 7);
    aoff[i] = (uint32_t)(r * K * 4 + c * 16);
    akc[i] = 4 * c;
  }
#pragma unroll
  for (int i = 0; i < RN; ++i) {
    const int P = 64 * (wave * RN + i) + lane, r = P >> 3, c = (P & 7) ^ ((r >> 1) & 7);
    boff[i] = (uint32_t)(r * K * 4 + c * 16);
    bkc[i] = 4 * c;
  }
  auto issue = [&](int kt, int st) {
    const int k0 = kt * 32;
    uint8_t* base = smem + st * STAGE;
#pragma unroll
    for (int i = 0; i < RM; ++i)
      vdma16(xb, xext, (lds_void*)(base + (wave * RM + i) * 1024),
             k0 + akc[i] < K ? aoff[i] + (uint32_t)(k0 * 4) : VIS_VOFF_NONE);
#pragma unroll
    for (int i = 0; i < RN; ++i)
      vdma16(wb, wext, (lds_void*)(base + SA + (wave * RN + i) * 1024),
             k0 + bkc[i] < K ? boff[i] + (uint32_t)(k0 * 4) : VIS_VOFF_NONE);
  };
  // fragment rows: row r at r * 128, its chunk c at 16 (c ^ (r / 2 % 8))
  int ra[RM], sa[RM], rb[RN], sb[RN];
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    const int r = wm + 16 * i + c16;
    ra[i] = r * 128;
    sa[i] = (r >> 1) & 7;
  }
#pragma unroll
  for (int j = 0; j < RN; ++j) {
    const int r = wn + 16 * j + c16;
    rb[j] = SA + r * 128;
    sb[j] = (r >> 1) & 7;
  }
  f32x4 acc[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nk = (K + 31) / 32;
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    vis_wait_dma();   // step kt's rows are in; every wave is done with step kt - 1's stage
    if (kt + 1 < nk) issue(kt + 1, (kt + 1) & 1);
    const uint8_t* st = smem + (kt & 1) * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 4 * h + g;
      f32x4 a[RM], b[RN];
#pragma unroll
      for (int i = 0; i < RM; ++i) a[i] = *(const f32x4*)(st + ra[i] + 16 * (c ^ sa[i]));
#pragma unroll
      for (int j = 0; j < RN; ++j) b[j] = *(const f32x4*)(st + rb[j] + 16 * (c ^ sb[j]));
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
          for (int j = 0; j < RN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
    }
  }
  {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < RN; ++j) {
    const int col = tn + wn + 16 * j + c16;
    if (col >= N) continue;
    const float bj = bias[col];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = tm + wm + 16 * i + 4 * g + e;
        if (row >= M) continue;
        const int64_t o = (int64_t)row * N + col;
        float v = acc[i][j][e] + bj;
        if (R) v = v + R[o];
        if (ACT == 1) v = gelu_tanh_f(v);
        if (ACT == 2) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
        Y[o] = v;
      }
  }
  }
}

template <int RM, int RN, int ACT>
static hipError_t vis_gemm_t(hipStream_t s, const float* x, const float* w, const float* bias, const float* r, float* y,
                             int M, int N, int K) {
  constexpr int lds = 2 * (32 * RM + 32 * RN) * 128;
  {
    const hipError_t e = ensure_lds((const void*)k_vis_gemm<RM, RN, ACT>, lds);
    if (e != hipSuccess) return e;
  }
  dim3 grid(vgrid(N, 32 * RN), vgrid(M, 32 * RM));
  hipLaunchKernelGGL((k_vis_gemm<RM, RN, ACT>), grid, dim3(256), lds, s, x, w, bias, r, y, M, N, K);
  return hipGetLastError();
}

template <int RM, int RN>
static hipError_t vis_gemm_act(hipStream_t s, int act, const float* x, const float* w, const float* bias,
                               const float* r, float* y, int M, int N, int K) {
  switch (act) {
    case 0: return vis_gemm_t<RM, RN, 0>(s, x, w, bias, r, y, M, N, K);
    case 1: return vis_gemm_t<RM, RN, 1>(s, x, w, bias, r, y, M, N, K);
    case 2: return vis_gemm_t<RM, RN, 2>(s, x, w, bias, r, y, M, N, K);
  }
  return hipErrorInvalidValue;
}

// 64 x 64 tiles: on the tower's shapes they ran 0-18% faster than 128 x 128 or 128 x 64 (the
// larger tiles leave a last, partly filled round of workgroups: 864 and 1088 tiles of 128 x 128
// for QKV and ffn_up against 512 a round at two a CU)
hipError_t vis_gemm(hipStream_t s, const float* x, const float* w, const float* bias, const float* r, float* y,
                    int64_t M, int64_t N, int64_t K, int act) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K <= 0 || K % 4 || ((uintptr_t)x & 15) || ((uintptr_t)w & 15) || !bias) return hipErrorInvalidValue;
  if (M * K * 4 >= ((int64_t)1 << 31) || N * K * 4 >= ((int64_t)1 << 31) || M * N >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  return vis_gemm_act<2, 2>(s, act, x, w, bias, r, y, (int)M, (int)N, (int)K);
}

// --- heads, rotary -------------------------------------------------------------------------

// tokens t0 .. t0 + 63 of head h from the QKV rows (n x 3D: q, k, v, each heads x 72): q and k
// turned by the rotary (t cos + rotate_half(t) sin, inspect/ref_vision.py:103-106) into
// [head][n][72], q then times QSCALE; v through LDS into V^T [head][72][n]
__global__ void __launch_bounds__(256)
k_vis_heads(int n, int D, const float* __restrict__ qkv, const float* __restrict__ cs, float qscale,
            float* __restrict__ q, float* __restrict__ k, float* __restrict__ vt) {
#pragma clang fp contract(off)
  __shared__ float vs[72][65];
  const int h = blockIdx.y, t0 = blockIdx.x * 64;
  for (int idx = threadIdx.x; idx < 64 * 72; idx += 256) {
    const int tl = idx / 72, d = idx - 72 * tl, t = t0 + tl;
    if (t >= n) continue;
    const float* row = qkv + (int64_t)t * 3 * D + h * 72;
    const float c = cs[(int64_t)t * 144 + d], sn = cs[(int64_t)t * 144 + 72 + d];
    const int dr = d < 36 ? d + 36 : d - 36;
    const float rq = d < 36 ? -row[dr] : row[dr], rk = d < 36 ? -row[D + dr] : row[D + dr];
    q[((int64_t)h * n + t) * 72 + d] = (row[d] * c + rq * sn) * qscale;
    k[((int64_t)h * n + t) * 72 + d] = row[D + d] * c + rk * sn;
    vs[d][tl] = row[2 * D + d];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 64 * 72; idx += 256) {
    const int d = idx >> 6, tl = idx & 63, t = t0 + tl;
    if (t < n) vt[((int64_t)h * 72 + d) * n + t] = vs[d][tl];
  }
}

hipError_t vis_heads(hipStream_t s, int n, int heads, const float* qkv, const float* cs, float qscale, float* q,
                     float* k, float* vt) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_vis_heads, dim3(vgrid(n, 64), heads), dim3(256), 0, s, n, heads * 72, qkv, cs, qscale, q, k, vt);
  return hipGetLastError();
}

// --- attention ------------------------------------------------------------------------------

// Softmax attention of every patch over every patch (inspect/ref_vision.py:124-129): grid
// (ceil(n / 128), heads), four waves of 32 queries (two blocks of 16).  Taken transposed, as
// S^T = K Q^T (16 x 16 blocks: keys x queries) and O^T += V^T P^T: a lane holds one query's
// scores and its O^T columns, so the online softmax needs lane exchanges only for the tile's max
// and, at the end, the row sum.  q comes scaled by log2(e)/sqrt(72): the scores are in log2
// units and exp2 gives the softmax's exp.  A head dim of 72 is four 16-wide k slices and a tail
// of 8 (two MFMAs, lane group g holding dims 64 + 2 g, + 1); the O^T product runs 80 rows, the
// last 8 on zeros.  64-key tiles of K ([n][72], 288-byte rows) and V^T ([72][n]; row d's 16-byte
// chunk c at c ^ (d % 16), so the 16 rows a fragment read touches fall in distinct banks) move to
// LDS by DMA, two stages; keys past n read as zeros and score -inf.  Every tile holds at least one
// key below n, so the running max is finite after the first.
#define VA_KT 18432    // a K tile: 64 rows x 288 bytes
#define VA_STAGE 36864 // K tile + V^T tile (72 rows x 256 bytes)
__global__ void __launch_bounds__(256, 2)
k_vis_attend(int n, int D, const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ vt,
             float* __restrict__ att) {
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4, h = blockIdx.y;
  const int q0 = blockIdx.x * 128 + wave * 32;
  const float* qh = q + (int64_t)h * n * 72;
  const float* kh = k + (int64_t)h * n * 72;
  const float* vh = vt + (int64_t)h * 72 * n;
  // Q^T fragments (B operand): query q0 + 16 qb + c16, dims 16 c + 4 g .. + 3 and 64 + 2 g, + 1
  f32x4 qf[2][4];
  float qt[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qi = q0 + 16 * qb + c16;
    const float* qr = qh + (int64_t)min(qi, n - 1) * 72;
    const float live = qi < n ? 1.f : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) qf[qb][c] = *(const f32x4*)(qr + 16 * c + 4 * g) * live;
    qt[qb][0] = qr[64 + 2 * g] * live;
    qt[qb][1] = qr[64 + 2 * g + 1] * live;
  }
  auto issue = [&](int t, int st) {
    const int key0 = t * 64;
    uint8_t* base = smem + st * VA_STAGE;
    const uint32_t kext = (uint32_t)((int64_t)(n - key0) * 288), vext = (uint32_t)(((int64_t)72 * n - key0) * 4);
    for (int i = wave; i < 18; i += 4) {
      const int P = 64 * i + lane;
      const int kr = P / 18, kc = P - 18 * kr;
      vdma16(kh + (int64_t)key0 * 72, kext, (lds_void*)(base + i * 1024),
             key0 + kr < n ? (uint32_t)(kr * 288 + kc * 16) : VIS_VOFF_NONE);
      const int d = P >> 4, c = (P & 15) ^ (d & 15);
      vdma16(vh + key0, vext, (lds_void*)(base + VA_KT + i * 1024),
             key0 + 4 * c < n ? (uint32_t)((int64_t)d * n * 4 + c * 16) : VIS_VOFF_NONE);
    }
  };
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4 o[5][2];
#pragma unroll
  for (int db = 0; db < 5; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nt = (n + 63) / 64;
  issue(0, 0);
  for (int t = 0; t < nt; ++t) {
    vis_wait_dma();
    if (t + 1 < nt) issue(t + 1, (t + 1) & 1);
    const uint8_t* kb_ = smem + (t & 1) * VA_STAGE;
    const uint8_t* vb_ = kb_ + VA_KT;
    f32x4 s[4][2];
#pragma unroll
    for (int kp = 0; kp < 4; kp += 2) {
      f32x4 kf[2][4];
      float kt[2][2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint8_t* kr = kb_ + (16 * (kp + u) + c16) * 288;
#pragma unroll
        for (int c = 0; c < 4; ++c) kf[u][c] = *(const f32x4*)(kr + 64 * c + 16 * g);
        kt[u][0] = *(const float*)(kr + 256 + 8 * g);
        kt[u][1] = *(const float*)(kr + 260 + 8 * g);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) s[kp + u][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              s[kp + u][qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[u][c][e], qf[qb][c][e], s[kp + u][qb], 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            s[kp + u][qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kt[u][e], qt[qb][e], s[kp + u][qb], 0, 0, 0);
    }
    if (t * 64 + 64 > n) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t * 64 + 16 * kb + 4 * g + e >= n) {
            s[kb][0][e] = -INFINITY;
            s[kb][1][e] = -INFINITY;
          }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[kb][qb][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m[qb], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[qb] - mn);
      m[qb] = mn;
      float ls = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = __builtin_amdgcn_exp2f(s[kb][qb][e] - mn);
          s[kb][qb][e] = p;
          ls += p;
        }
      l[qb] = l[qb] * alpha + ls;
#pragma unroll
      for (int db = 0; db < 5; ++db) o[db][qb] = o[db][qb] * alpha;
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 vf[5];
#pragma unroll
      for (int db = 0; db < 5; ++db) {
        const int d = 16 * db + c16;
        vf[db] = d < 72 ? *(const f32x4*)(vb_ + d * 256 + 16 * ((4 * kb + g) ^ (d & 15))) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int db = 0; db < 5; ++db)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            o[db][qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[db][e], s[kb][qb][e], o[db][qb], 0, 0, 0);
    }
  }
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float lt = l[qb];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const int qi = q0 + 16 * qb + c16;
    if (qi >= n) continue;
#pragma unroll
    for (int db = 0; db < 5; ++db) {
      const int d0 = 16 * db + 4 * g;
      if (d0 < 72) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __fdiv_rn(o[db][qb][e], lt);
        *(f32x4*)(att + (int64_t)qi * D + h * 72 + d0) = v;
      }
    }
  }
}

hipError_t vis_attend(hipStream_t s, int n, int heads, const float* q, const float* k, const float* vt, float* att) {
  if (n <= 0) return hipSuccess;
  if (n % 4 || (int64_t)n * 288 >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  {
    const hipError_t e = ensure_lds((const void*)k_vis_attend, 2 * VA_STAGE);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_vis_attend, dim3(vgrid(n, 128), heads), dim3(256), 2 * VA_STAGE, s, n, heads * 72, q, k, vt,
                     att);
  return hipGetLastError();
}

// --- the patch kernels' sum --------------------------------------------------------------

__global__ void k_vis_sum(int64_t n, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
}

hipError_t vis_sum(hipStream_t s, int64_t n, const float* a, const float* b, float* y) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_vis_sum, dim3(vgrid(n, 256)), dim3(256), 0, s, n, a, b, y);
  return hipGetLastError();
}

}  // namespace exn
