// attn.hip -- the DiT's joint attention on gfx950's MFMA, flash style: K and
// V tiles staged in LDS, an online softmax in fp32 (exp2 of scores in log2
// units), Q, K, V and P in fp16 (the reference's halves), fp32 sums.  The
// mask is the reference's xa_lim
// (src/cuda/dit.cu:60-66): sequence row g sees keys 0..lim(g), lim(g) = l-1
// for image rows (g >= p), b1-1 for a reference picture's rows b0..b1-1, g
// otherwise (the prompt is causal).  lim never decreases in g, so a query
// tile's last key is its last row's.  Replaces x_attend_mma
// (src/cuda/dit.cu:208-336).
//
// Layouts: Q [32 heads][n][128] (query t = sequence row q0 + t),
// K [32][lcap][128], V^T [32][128][lcap] (keys contiguous), all fp16;
// out [n][4096] bf16 (the next product's input).
//
// The products are taken transposed so that no register shuffles are needed:
// S^T = K Q^T puts one query in a lane's column (its 32 of a 64-key tile's
// scores in its registers, the other 32 in lane ^ 32), and O^T += V^T P^T
// takes that lane's P values straight as the B operand -- the contraction
// runs over the keys in the order the accumulator holds them, and V^T's A
// operand is read from LDS in the same order.
#include "exn_common.h"

namespace exn {

#define AQ 128          // queries a workgroup (32 a wave)
#define AK 64           // keys a tile
#define KS (128 + 8)    // LDS stride of a K row (fp16 values)
#define VS (AK + 8)     // LDS stride of a V^T row (fp16 values)

__device__ __forceinline__ int xa_lim(int g, int p, int l, int b0, int b1) {
  return g >= p ? l - 1 : (g >= b0 && g < b1 ? b1 - 1 : g);
}

// grid (ceil(n/128), 32 heads), block 256
__global__ void __launch_bounds__(256)
k_attend(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vt,
         uint16_t* __restrict__ O, int n, int q0, int p, int l, int64_t lcap, int b0, int b1, float scale) {
  __shared__ __align__(16) uint16_t ks[AK * KS];
  __shared__ __align__(16) uint16_t vs[128 * VS];
  const int h = blockIdx.y, t0 = blockIdx.x * AQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hi = lane >> 5, lo = lane & 31;
  const int tq = t0 + wave * 32 + lo;
  const int tqc = min(tq, n - 1);

  // Q^T as the B operand: 8 steps of 16 dims, this lane's query, dims 16s + 8*hi ..
  f16x8 qf[8];
  {
    const uint16_t* qr = Q + ((int64_t)h * n + tqc) * 128 + 8 * hi;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const f16x8*)(qr + 16 * s);
  }
  const int lim = xa_lim(q0 + tqc, p, l, b0, b1);
  const int last = xa_lim(q0 + min(n, t0 + AQ) - 1, p, l, b0, b1);
  const int minlim = xa_lim(q0 + t0, p, l, b0, b1);

  f32x16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x16{};
  float mrun = -INFINITY, lrun = 0.f;

  const uint16_t* kbase = Kc + (int64_t)h * lcap * 128;
  const uint16_t* vbase = Vt + (int64_t)h * 128 * lcap;

  for (int k0 = 0; k0 <= last; k0 += AK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int kr = c >> 4, k8 = (c & 15) * 8;
      *(u32x4*)(ks + kr * KS + k8) = *(const u32x4*)(kbase + (int64_t)(k0 + kr) * 128 + k8);
      const int vr = c >> 3, v8 = (c & 7) * 8;
      *(u32x4*)(vs + vr * VS + v8) = *(const u32x4*)(vbase + (int64_t)vr * lcap + k0 + v8);
    }
    __syncthreads();

    // S^T: two 32-key blocks x this wave's 32 queries
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const f16x8 a = *(const f16x8*)(ks + (32 * b + lo) * KS + 16 * kk + 8 * hi);
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[kk], s[b], 0, 0, 0);
      }
    }
    if (scale != 1.f) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[b][r] *= scale;
    }
    if (k0 + AK - 1 > minlim) {   // some key of this tile is hidden from some query
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * b + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (key > lim) s[b][r] = -INFINITY;
        }
    }
    float mx = s[0][0];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(mrun, mx);
    const float alpha = exp2f(mrun - mnew);
    float ls = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2f(s[b][r] - mnew);
        s[b][r] = e;
        ls += e;
      }
    lrun = lrun * alpha + ls;
    mrun = mnew;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] *= alpha;

    // O^T += V^T P^T over 4 steps of 16 keys; k-slot (hi, j) is key 16u + 8(j/4) + 4hi + j%4 of block b
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t p0 = pack_f16x2(s[b][8 * u + 0], s[b][8 * u + 1]);
        const uint32_t p1 = pack_f16x2(s[b][8 * u + 2], s[b][8 * u + 3]);
        const uint32_t p2 = pack_f16x2(s[b][8 * u + 4], s[b][8 * u + 5]);
        const uint32_t p3 = pack_f16x2(s[b][8 * u + 6], s[b][8 * u + 7]);
        const f16x8 pb = __builtin_bit_cast(f16x8, u32x4{p0, p1, p2, p3});
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint16_t* vp = vs + (32 * d + lo) * VS + 32 * b + 16 * u + 4 * hi;
          const u32x2 x0 = *(const u32x2*)vp, x1 = *(const u32x2*)(vp + 8);
          const f16x8 a = __builtin_bit_cast(f16x8, u32x4{x0[0], x0[1], x1[0], x1[1]});
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[d], 0, 0, 0);
        }
      }
  }

  const float ltot = lrun + __shfl_xor(lrun, 32, 64);
  const float inv = 1.f / ltot;
  if (tq < n) {
    uint16_t* orow = O + (int64_t)tq * 4096 + h * 128 + 4 * hi;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4;
        *(u32x2*)(orow + dim) = u32x2{pack_bf16x2(o[d][4 * r4] * inv, o[d][4 * r4 + 1] * inv),
                                      pack_bf16x2(o[d][4 * r4 + 2] * inv, o[d][4 * r4 + 3] * inv)};
      }
  }
}

hipError_t attend(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, uint16_t* out, int n,
                  int q0, int p, int l, int64_t lcap, int b0, int b1, float scale) {
  if (n <= 0) return hipSuccess;
  if (lcap % AK || l > lcap || l <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attend, dim3((unsigned)((n + AQ - 1) / AQ), 32), dim3(256), 0, s, q, k, vt, out, n, q0, p, l,
                     lcap, b0, b1, scale);
  return hipGetLastError();
}

}  // namespace exn
