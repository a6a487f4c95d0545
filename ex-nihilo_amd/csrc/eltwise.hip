// eltwise.hip -- the DiT's bandwidth kernels: coalesced 16-byte accesses, one
// pass over HBM each, fp32 arithmetic.
//
//   ln_mod      LayerNorm (no affine, eps 1e-6) * (1 + mod[row]); row < p takes
//               mod row 1 (t = 0), else row 0 -- src/cuda/dit.cu:17-32
//   rms_norm    x / rms(x) * w (txt_in's text_norm, w = 1 + weight) -- illatio's
//               v_rms at src/cuda-dit.lisp:176
//   gate_add    x += tanh(gate[row]) * h -- src/cuda/dit.cu:34-41
//   swiglu      silu(gu[:, :F]) * gu[:, F:] -- src/cuda/dit.cu:186-192 (and swiglu_pairs:
//               fp32, on gate and up columns interleaved by 32)
//   gelu_tanh   src/cuda/dit.cu:194-199;  silu  src/cuda/dit.cu:201-206
//   qkv_prep    per head: RMSNorm * w, then the interleaved RoPE (src/cuda/dit.cu:
//               43-58) of q and k, and v transposed, into the attention's layouts
//   latent_rows / rows_to_latent   the channel-major latent <-> token rows
//               (src/cuda-dit.lisp:188-191,238-243)
//   euler       z += ds * v, two roundings as the host loop's single floats
//               (src/generate.lisp:133-135)
#include "exn_common.h"

namespace exn {

static inline unsigned grid_of(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

// sum over a 256-thread block; RED must hold 4 floats and not be reused until a barrier
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// one block a row of 4096: 16 values a thread, kept in registers between the passes
__global__ void __launch_bounds__(256)
k_ln_mod(int n, int n0, int p, int mstride, const float* __restrict__ x, int64_t ldx, const float* __restrict__ mod,
         void* __restrict__ out, int out_bf16) {
  __shared__ float red[8];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float* r = x + (int64_t)t * ldx;
  f32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = *(const f32x4*)(r + 4 * tid + 1024 * i);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  const float mean = block_sum256(s, red) * (1.f / 4096.f);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[i][e] -= mean;
      ss += v[i][e] * v[i][e];
    }
  const float inv = rsqrtf(block_sum256(ss, red + 4) * (1.f / 4096.f) + 1e-6f);
  const float* m = mod + (n0 + t < p ? mstride : 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 4 * tid + 1024 * i;
    const f32x4 mv = *(const f32x4*)(m + c);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[i][e] * inv * (1.f + mv[e]);
    if (out_bf16) {
      *(u32x2*)((uint16_t*)out + (int64_t)t * 4096 + c) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {
      *(f32x4*)((float*)out + (int64_t)t * 4096 + c) = o;
    }
  }
}

hipError_t ln_mod(hipStream_t s, int n, int n0, int p, int mstride, const float* x, int64_t ldx, const float* mod,
                  void* out, int out_bf16) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_ln_mod, dim3(n), dim3(256), 0, s, n, n0, p, mstride, x, ldx, mod, out, out_bf16);
  return hipGetLastError();
}

// y = x / sqrt(mean(x^2) + eps) * w, a block a row of WIDTH (a multiple of 4)
__global__ void __launch_bounds__(256)
k_rms(int width, float eps, const float* __restrict__ x, const float* __restrict__ w, void* __restrict__ out,
      int out_bf16) {
  __shared__ float red[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float* r = x + (int64_t)t * width;
  float ss = 0.f;
  for (int c = 4 * tid; c < width; c += 1024) {
    const f32x4 v = *(const f32x4*)(r + c);
    ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
  const float inv = rsqrtf(block_sum256(ss, red) / (float)width + eps);
  for (int c = 4 * tid; c < width; c += 1024) {
    const f32x4 v = *(const f32x4*)(r + c), wv = *(const f32x4*)(w + c);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[e] * inv * wv[e];
    if (out_bf16)
      *(u32x2*)((uint16_t*)out + (int64_t)t * width + c) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    else
      *(f32x4*)((float*)out + (int64_t)t * width + c) = o;
  }
}

hipError_t rms_norm(hipStream_t s, int n, int width, float eps, const float* x, const float* w, void* out,
                    int out_bf16) {
  if (n <= 0) return hipSuccess;
  if (width % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rms, dim3(n), dim3(256), 0, s, width, eps, x, w, out, out_bf16);
  return hipGetLastError();
}

// The S partial sums of a split product (PART: S x M x 4096 floats, in order) into the gated
// residual rows X (ldx; x += tanh(gate) * sum, the gate row as the product's EPI_GATE_ADD takes
// it), then each finished row's RMS norm times W into bf16 Y (4096 wide): the split sum's and
// rms_norm's arithmetic in one pass over the rows.  One block a row; thread t takes columns
// 4t + 1024j in both passes, as both separate kernels do, so the values are theirs bit for bit.
// The row's 4 S partial loads go out before any sum.
template <int S>
__global__ void __launch_bounds__(256)
k_sum_rms(int64_t M, const float* __restrict__ part, float* __restrict__ x, int64_t ldx, const float* __restrict__ gate,
          int n0, int p, int mstride, float eps, const float* __restrict__ w, uint16_t* __restrict__ y) {
  constexpr int64_t N = 4096;
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  float* r = x + m * ldx;
  const float* gr = gate + (n0 + m < p ? mstride : 0);
  f32x4 pv[4][S], xv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = 4 * tid + 1024 * j;
#pragma unroll
    for (int z = 0; z < S; ++z) pv[j][z] = *(const f32x4*)(part + ((int64_t)z * M + m) * N + c);
    xv[j] = *(const f32x4*)(r + c);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = 4 * tid + 1024 * j;
    f32x4 v = pv[j][0];
#pragma unroll
    for (int z = 1; z < S; ++z) v += pv[j][z];
#pragma unroll
    for (int e = 0; e < 4; ++e) xv[j][e] = xv[j][e] + tanh_f(gr[c + e]) * v[e];
    *(f32x4*)(r + c) = xv[j];
    ss += xv[j][0] * xv[j][0] + xv[j][1] * xv[j][1] + xv[j][2] * xv[j][2] + xv[j][3] * xv[j][3];
  }
  const float inv = rsqrtf(block_sum256(ss, red) / (float)N + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = 4 * tid + 1024 * j;
    const f32x4 wv = *(const f32x4*)(w + c);
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = xv[j][e] * inv * wv[e];
    *(u32x2*)(y + m * N + c) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
}

hipError_t split_sum_rms(hipStream_t s, int S, int64_t M, int64_t N, const float* part, const EpiArgs& ea, float eps,
                         const float* w, uint16_t* y) {
  if (M == 0) return hipSuccess;
  if (S < 1 || S > 8 || N != 4096 || ea.ldy % 4) return hipErrorInvalidValue;
  const dim3 g((unsigned)M);
  switch (S) {
#define EXN_SUM_RMS_S(k)                                                                                             \
  case k:                                                                                                            \
    hipLaunchKernelGGL(k_sum_rms<k>, g, dim3(256), 0, s, M, part, ea.resid, ea.ldy, ea.gate, ea.n0, ea.p, ea.mstride, \
                       eps, w, y);                                                                                   \
    break;
    EXN_SUM_RMS_S(1) EXN_SUM_RMS_S(2) EXN_SUM_RMS_S(3) EXN_SUM_RMS_S(4) EXN_SUM_RMS_S(5) EXN_SUM_RMS_S(6)
    EXN_SUM_RMS_S(7) EXN_SUM_RMS_S(8)
#undef EXN_SUM_RMS_S
  }
  return hipGetLastError();
}

// 4 values a thread; COUNT a multiple of 4 and WIDTH of 4
__global__ void k_gate_add(int64_t count4, int width, int n0, int p, int mstride, float* __restrict__ x,
                           const float* __restrict__ h, const float* __restrict__ gate) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count4) return;
  const int64_t e = 4 * i;
  const int t = n0 + (int)(e / width), c = (int)(e % width);
  const f32x4 g = *(const f32x4*)(gate + (t < p ? mstride : 0) + c);
  const f32x4 hv = *(const f32x4*)(h + e);
  f32x4 xv = *(const f32x4*)(x + e);
#pragma unroll
  for (int k = 0; k < 4; ++k) xv[k] += tanh_f(g[k]) * hv[k];
  *(f32x4*)(x + e) = xv;
}

hipError_t gate_add(hipStream_t s, int64_t count, int width, int n0, int p, int mstride, float* x, const float* h,
                    const float* gate) {
  if (count % 4 || width % 4) return hipErrorInvalidValue;
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gate_add, dim3(grid_of(count / 4, 256)), dim3(256), 0, s, count / 4, width, n0, p, mstride, x,
                     h, gate);
  return hipGetLastError();
}

// bf16 gu (n x 2f) -> bf16 out (n x f), 8 values a thread
__global__ void k_swiglu(int64_t count8, int f, const uint16_t* __restrict__ gu, uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count8) return;
  const int64_t e = 8 * i, t = e / f, j = e % f;
  const u32x4 g = *(const u32x4*)(gu + t * 2 * f + j);
  const u32x4 u = *(const u32x4*)(gu + t * 2 * f + f + j);
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float g0 = bf16_lo(g[k]), g1 = bf16_hi(g[k]);
    o[k] = pack_bf16x2(silu_f(g0) * bf16_lo(u[k]), silu_f(g1) * bf16_hi(u[k]));
  }
  *(u32x4*)(out + e) = o;
}

hipError_t swiglu(hipStream_t s, int64_t n, int f, const uint16_t* gu, uint16_t* out) {
  if (f % 8) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_swiglu, dim3(grid_of(n * f / 8, 256)), dim3(256), 0, s, n * f / 8, f, gu, out);
  return hipGetLastError();
}

// x_swiglu2 in fp32 on a gate_up product whose columns hold gate and up interleaved by 32 (the
// device order of the paired gate_up rows): out [n][f] = silu(gate) * up, 4 columns a thread
__global__ void k_swiglu_pairs(int64_t count4, int f, const float* __restrict__ gu, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count4) return;
  const int64_t e = 4 * i, t = e / f, c = e % f;
  const float* r = gu + t * 2 * f + 64 * (c >> 5) + (c & 31);   // gate of column c; up 32 on
  const f32x4 g = *(const f32x4*)r, u = *(const f32x4*)(r + 32);
  f32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = silu_f(g[k]) * u[k];
  *(f32x4*)(out + e) = o;
}

hipError_t swiglu_pairs(hipStream_t s, int64_t n, int f, const float* gu, float* out) {
  if (f % 32) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_swiglu_pairs, dim3(grid_of(n * f / 4, 256)), dim3(256), 0, s, n * f / 4, f, gu, out);
  return hipGetLastError();
}

__global__ void k_gelu(int64_t count, float* __restrict__ x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) x[i] = gelu_tanh_f(x[i]);
}

__global__ void k_silu(int64_t count, float* __restrict__ x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) x[i] = silu_f(x[i]);
}

hipError_t gelu_tanh(hipStream_t s, int64_t count, float* x) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gelu, dim3(grid_of(count, 256)), dim3(256), 0, s, count, x);
  return hipGetLastError();
}

hipError_t silu(hipStream_t s, int64_t count, float* x) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(k_silu, dim3(grid_of(count, 256)), dim3(256), 0, s, count, x);
  return hipGetLastError();
}

// qkv: fp16 rows of q | k | v for tokens 0..n-1, token t being sequence row
// row0 + t: q 32 heads of 128, k and v 32 / G heads each (G query heads a key/value
// head: 1, rows of 3 x 4096, or 4, rows of 6144).  Writes, all fp16 (the attention's
// operands, as the reference's halves): q ([32][n][128], scaled by qscale after the
// rotation), k into kc ([32][lcap][128]) rows row0.., v transposed into vt
// ([32][128][lcap]) columns row0.., query head h taking key/value head h / G.  cs:
// cos, sin for 64 pairs, 128 floats a sequence row.  grid (ceil(n/TB), 32), block 256: TB
// tokens a workgroup, 64, or 32 for passes of at most 512 rows (a prompt's: twice the
// workgroups, and half the registers a thread holds the partial sums' loads in).
// S > 0: the rows are those a split product's S partial sums (S x n rows of fp32, in order)
// give through its fp16 store -- the same sums, in the same order, rounded once -- read from
// the partials (all S of a value's loads out before its sum) instead of fp16 rows written and
// read back
template <int S, int TB>
__global__ void __launch_bounds__(256)
k_qkv_prep(const uint16_t* __restrict__ qkv, const float* __restrict__ part, int64_t n,
           const float* __restrict__ wq, const float* __restrict__ wk, const float* __restrict__ cs, float qscale,
           uint16_t* __restrict__ q, uint16_t* __restrict__ kc, uint16_t* __restrict__ vt, int64_t row0, int64_t lcap,
           int64_t qld, int g) {
  static_assert(TB == 64 || TB == 32, "64 or 32 tokens a workgroup");
  constexpr int RQ = TB / 16;   // a wave's rounds of 4 tokens
  __shared__ uint16_t tile[TB][128 + 2];
  const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t ld = 4096 + 2 * (4096 / g);                      // a row of qkv
  const int64_t ko = 4096 + (h / g) * 128, vo = ko + 4096 / g;   // this head's k and v in it
  const int64_t t0 = (int64_t)blockIdx.x * TB;
  // the 8 fp16 values of token TC's row at column COL
  auto ld8 = [&](int64_t tc, int64_t col) -> u32x4 {
    if constexpr (S == 0) {
      return *(const u32x4*)(qkv + tc * ld + col);
    } else {
      const float* p0 = part + tc * ld + col;
      f32x4 pa[S], pb[S];
#pragma unroll
      for (int z = 0; z < S; ++z) {
        pa[z] = *(const f32x4*)(p0 + (int64_t)z * n * ld);
        pb[z] = *(const f32x4*)(p0 + (int64_t)z * n * ld + 4);
      }
      f32x4 a = pa[0], b = pb[0];
#pragma unroll
      for (int z = 1; z < S; ++z) {
        a += pa[z];
        b += pb[z];
      }
      return u32x4{pack_f16x2(a[0], a[1]), pack_f16x2(a[2], a[3]), pack_f16x2(b[0], b[1]), pack_f16x2(b[2], b[3])};
    }
  };
  // q and k: 16 lanes a token, lane holding dims d8 .. d8+7 (its 4 rotation pairs) as one
  // 16-byte load and store; a wave takes 4 tokens a round, its TB / 4 tokens in RQ rounds whose
  // loads are all issued first.  The RMS sum is a reduction over the 16 lanes.
  const int sub = lane >> 4, d8 = (lane & 15) * 8;
  float wqv[8], wkv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    wqv[j] = wq[d8 + j];
    wkv[j] = wk[d8 + j];
  }
  u32x4 uq[RQ], uk[RQ];
  f32x4 ca[RQ], cb[RQ];
#pragma unroll
  for (int it = 0; it < RQ; ++it) {
    const int64_t tc = min(t0 + wave * (TB / 4) + it * 4 + sub, n - 1);   // rows past n: loaded, not stored
    uq[it] = ld8(tc, h * 128 + d8);
    uk[it] = ld8(tc, ko + d8);
    const float* cr = cs + (row0 + tc) * 128 + d8;   // cos, sin of pairs d8/2 .. d8/2 + 3
    ca[it] = *(const f32x4*)cr;
    cb[it] = *(const f32x4*)(cr + 4);
  }
#pragma unroll
  for (int it = 0; it < RQ; ++it) {
    const int64_t t = t0 + wave * (TB / 4) + it * 4 + sub;
    const float c[8] = {ca[it][0], ca[it][1], ca[it][2], ca[it][3], cb[it][0], cb[it][1], cb[it][2], cb[it][3]};
    float a[8], ssq = 0.f, ssk = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[2 * e] = f16_lo(uq[it][e]);
      a[2 * e + 1] = f16_hi(uq[it][e]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ssq += a[j] * a[j];
    float b[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[2 * e] = f16_lo(uk[it][e]);
      b[2 * e + 1] = f16_hi(uk[it][e]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ssk += b[j] * b[j];
    const float invq = rsqrtf(row16_sum(ssq) * (1.f / 128.f) + 1e-6f);
    const float invk = rsqrtf(row16_sum(ssk) * (1.f / 128.f) + 1e-6f);
    u32x4 oq, ok;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float cx = c[2 * e], cy = c[2 * e + 1];
      const float an = a[2 * e] * invq * wqv[2 * e], bn = a[2 * e + 1] * invq * wqv[2 * e + 1];
      oq[e] = pack_f16x2((an * cx - bn * cy) * qscale, (an * cy + bn * cx) * qscale);
      const float ak = b[2 * e] * invk * wkv[2 * e], bk = b[2 * e + 1] * invk * wkv[2 * e + 1];
      ok[e] = pack_f16x2(ak * cx - bk * cy, ak * cy + bk * cx);
    }
    if (t < n) {
      *(u32x4*)(q + ((int64_t)h * qld + t) * 128 + d8) = oq;
      *(u32x4*)(kc + ((int64_t)h * lcap + row0 + t) * 128 + d8) = ok;
    }
  }
  // v: TB tokens x 128 dims through LDS, out as 128 rows of TB consecutive keys
  for (int i = 0; i < TB / 16; ++i) {
    const int c = tid + 256 * i, tok = c >> 4, d8 = (c & 15) * 8;
    const int64_t t = t0 + tok;
    u32x4 v = u32x4{0, 0, 0, 0};
    if (t < n) v = ld8(t, vo + d8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      *(uint32_t*)&tile[tok][d8 + 2 * e] = v[e];
    }
  }
  __syncthreads();
  const int tok = tid % TB;
  const int64_t t = t0 + tok;
  if (t < n) {
    const int64_t col = vt_pos(row0 + t);
    for (int d = tid / TB; d < 128; d += 256 / TB) vt[((int64_t)h * 128 + d) * lcap + col] = tile[tok][d];
  }
}

hipError_t qkv_prep(hipStream_t s, const uint16_t* qkv, int64_t n, const float* wq, const float* wk, const float* cs,
                    uint16_t* q, uint16_t* k, uint16_t* vt, int64_t row0, int64_t lcap,
                    int64_t qld, int kv_group) {
  if (n == 0) return hipSuccess;
  if (kv_group != 1 && kv_group != 4) return hipErrorInvalidValue;
  // q is scaled by 1/sqrt(128) * log2(e): the attention's scores are then in log2 units
  const float qscale = QK_QSCALE;
  if (n <= 512)
    hipLaunchKernelGGL((k_qkv_prep<0, 32>), dim3(grid_of(n, 32), 32), dim3(256), 0, s, qkv, nullptr, n, wq, wk, cs,
                       qscale, q, k, vt, row0, lcap, qld, kv_group);
  else
    hipLaunchKernelGGL((k_qkv_prep<0, 64>), dim3(grid_of(n, 64), 32), dim3(256), 0, s, qkv, nullptr, n, wq, wk, cs,
                       qscale, q, k, vt, row0, lcap, qld, kv_group);
  return hipGetLastError();
}

hipError_t qkv_prep_part(hipStream_t s, const float* part, int S, int64_t n, const float* wq, const float* wk,
                         const float* cs, uint16_t* q, uint16_t* k_, uint16_t* vt, int64_t row0, int64_t lcap,
                         int64_t qld, int kv_group) {
  if (n == 0) return hipSuccess;
  if ((kv_group != 1 && kv_group != 4) || S < 1 || S > 8) return hipErrorInvalidValue;
  const bool t32 = n <= 512;   // 32 tokens a workgroup (as qkv_prep)
  const dim3 g(grid_of(n, t32 ? 32 : 64), 32);
  switch (S) {
#define EXN_PREP_S(k)                                                                                         \
  case k:                                                                                                     \
    if (t32)                                                                                                  \
      hipLaunchKernelGGL((k_qkv_prep<k, 32>), g, dim3(256), 0, s, nullptr, part, n, wq, wk, cs, QK_QSCALE, q, \
                         k_, vt, row0, lcap, qld, kv_group);                                                  \
    else                                                                                                      \
      hipLaunchKernelGGL((k_qkv_prep<k, 64>), g, dim3(256), 0, s, nullptr, part, n, wq, wk, cs, QK_QSCALE, q, \
                         k_, vt, row0, lcap, qld, kv_group);                                                  \
    break;
    EXN_PREP_S(1) EXN_PREP_S(2) EXN_PREP_S(3) EXN_PREP_S(4) EXN_PREP_S(5) EXN_PREP_S(6) EXN_PREP_S(7) EXN_PREP_S(8)
#undef EXN_PREP_S
  }
  return hipGetLastError();
}

// latent [64][nimg] fp32 -> rows [nimg][64] fp32
__global__ void k_latent_rows(const float* __restrict__ lat, int64_t nimg, float* __restrict__ rows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nimg * 64) return;
  const int64_t tok = i / 64, c = i % 64;
  rows[i] = lat[c * nimg + tok];
}

// rows [nimg][64] fp32 -> latent [64][nimg] fp32
__global__ void k_rows_latent(const float* __restrict__ rows, int64_t nimg, float* __restrict__ lat) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nimg * 64) return;
  const int64_t c = i / nimg, tok = i % nimg;
  lat[i] = rows[tok * 64 + c];
}

hipError_t latent_rows(hipStream_t s, const float* latent, int64_t nimg, float* rows) {
  hipLaunchKernelGGL(k_latent_rows, dim3(grid_of(nimg * 64, 256)), dim3(256), 0, s, latent, nimg, rows);
  return hipGetLastError();
}

hipError_t rows_to_latent(hipStream_t s, const float* rows, int64_t nimg, float* latent) {
  hipLaunchKernelGGL(k_rows_latent, dim3(grid_of(nimg * 64, 256)), dim3(256), 0, s, rows, nimg, latent);
  return hipGetLastError();
}

__global__ void k_euler(int64_t count, float* __restrict__ z, const float* __restrict__ v, float ds) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) z[i] = z[i] + ds * v[i];   // a product, then a sum: no fused multiply-add
}

hipError_t euler(hipStream_t s, int64_t count, float* z, const float* v, float ds) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(k_euler, dim3(grid_of(count, 256)), dim3(256), 0, s, count, z, v, ds);
  return hipGetLastError();
}

// *dit-trace*'s numbers (src/metal-dit.lisp:119-124) for COUNT values of X (fp32, or bf16 when
// BF16): the largest finite |x| into REC[0] (its bits: finite magnitudes order as unsigned
// integers) and the count of values that are not finite added to REC[2..3] (a 64-bit count).
// A grid of at most 1024 workgroups strides over X, 16 bytes a lane; one atomic of each kind
// a wave.
__global__ void __launch_bounds__(256)
k_stats(const void* __restrict__ x, int bf16, int64_t count, uint32_t* __restrict__ rec) {
  float mx = 0.f;
  uint32_t bad = 0;
  auto take = [&](float v) {
    const bool fin = (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u;
    mx = fin ? fmaxf(mx, fabsf(v)) : mx;
    bad += fin ? 0u : 1u;
  };
  const int64_t per = bf16 ? 8 : 4;   // values a 16-byte load
  const int64_t chunks = count / per, stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
    const u32x4 u = ((const u32x4*)x)[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (bf16) {
        take(bf16_lo(u[e]));
        take(bf16_hi(u[e]));
      } else {
        take(__uint_as_float(u[e]));
      }
    }
  }
  // the tail past whole 16-byte chunks, by the first threads
  const int64_t t = chunks * per + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < count)
    take(bf16 ? __uint_as_float((uint32_t)((const uint16_t*)x)[t] << 16) : ((const float*)x)[t]);
  mx = wave_max(mx);
  for (int o = 32; o >= 1; o >>= 1) bad += __shfl_xor(bad, o, 64);
  if ((threadIdx.x & 63) == 0) {
    atomicMax(rec, __float_as_uint(mx));
    if (bad) atomicAdd((unsigned long long*)(rec + 2), (unsigned long long)bad);
  }
}

__global__ void k_stats_clear(uint32_t* __restrict__ rec, int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < words) rec[i] = 0u;
}

hipError_t tensor_stats(hipStream_t s, const void* x, int bf16, int64_t count, uint32_t* rec) {
  if (count <= 0) return hipSuccess;
  const int64_t chunks = count / (bf16 ? 8 : 4);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(1024, (chunks + 255) / 256));
  hipLaunchKernelGGL(k_stats, dim3((unsigned)blocks), dim3(256), 0, s, x, bf16, count, rec);
  return hipGetLastError();
}

hipError_t tensor_stats_clear(hipStream_t s, uint32_t* rec, int64_t records) {
  if (records <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_stats_clear, dim3(grid_of(records * 4, 256)), dim3(256), 0, s, rec, records * 4);
  return hipGetLastError();
}

}  // namespace exn
