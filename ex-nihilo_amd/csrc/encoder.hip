// encoder.hip -- the prompt encoder's own kernel (Qwen3-VL-8B's text model, read for its
// last block's states: src/encoder.lisp:143-183).  Its products, norms, q/k norm with the
// rotary, causal attention and SwiGLU run on the DiT's kernels (gemm.hip, attn.hip,
// eltwise.hip): the text model has the DiT block's widths (4096, 32 heads of 128, FFN 12288).
#include "exn_common.h"

namespace exn {

// one workgroup a token: row ids[t] of the token embedding, from Q8_0 codes and scales
// (fp32(d) x q, exact) or from fp32 rows; an id outside 0 .. vocab-1 gives a row of zeros (the
// host entry point rejects such ids before they get here)
__global__ void __launch_bounds__(256)
k_enc_embed(const int32_t* __restrict__ ids, int64_t vocab, const int8_t* __restrict__ qs,
            const uint16_t* __restrict__ d, const float* __restrict__ f32, int width, float* __restrict__ out) {
  const int t = blockIdx.x;
  const int64_t id = ids[t];
  float* o = out + (int64_t)t * width;
  const bool live = id >= 0 && id < vocab;
  for (int c = 4 * threadIdx.x; c < width; c += 1024) {
    if (!live) {
      *(f32x4*)(o + c) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else if (f32) {
      *(f32x4*)(o + c) = *(const f32x4*)(f32 + id * width + c);
    } else {
      const float sc = f16_to_f32(d[(id * width + c) / 32]);
      const uint32_t q = *(const uint32_t*)(qs + id * width + c);
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = sc * (float)(int8_t)(q >> (8 * e));
      *(f32x4*)(o + c) = v;
    }
  }
}

hipError_t enc_embed(hipStream_t s, const int32_t* ids, int n, int64_t vocab, const int8_t* qs, const uint16_t* d,
                     const float* f32, int width, float* out) {
  if (n <= 0) return hipSuccess;
  if (width % 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_enc_embed, dim3(n), dim3(256), 0, s, ids, vocab, qs, d, f32, width, out);
  return hipGetLastError();
}

}  // namespace exn
