// synth.hip -- the counter-based synthetic weights on the device, the Q8_0
// repack of GGUF block_q8_0 records, and the dequant test hook.
//
// Generator (the same definition as the host's, bit for bit; mod 2^64):
//   mix64 = SplitMix64's finaliser; key(s, t) = mix64(s*G + t + 1);
//   word(k, i) = mix64(k + (i + 1)*G), G = 0x9E3779B97F4A7C15.
//   Q8_0 block b: byte j = ((u*255 + 128) >> 8) - 127, u = byte j%8 of word(k, 5b + j/8);
//   d = fp16_rne(|fp32(2S - 262140) * 2.6428997921303017e-09f|), S = sum of the four
//   16-bit chunks of word(k, 5b + 4).
//   normal i = fp32(2S - 262140) * 1.3214498960651507e-05f, S from word(k, i).
#include "exn_common.h"

namespace exn {

#define G64 0x9E3779B97F4A7C15ull

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27; z *= 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t word(uint64_t k, uint64_t i) { return mix64(k + (i + 1) * G64); }

__device__ __forceinline__ int32_t sum2(uint64_t w) {
  const int32_t s = (int32_t)(w & 0xFFFF) + (int32_t)((w >> 16) & 0xFFFF) + (int32_t)((w >> 32) & 0xFFFF) +
                    (int32_t)((w >> 48) & 0xFFFF);
  return 2 * s - 262140;
}

// fp32 -> fp16 bits, round to nearest even, subnormals kept (integer arithmetic only)
__device__ __forceinline__ uint16_t f16_rne(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (ax >= 0x38800000u) return (uint16_t)(sign | ((ax + 0xFFFu + ((ax >> 13) & 1u) - 0x38000000u) >> 13));
  const uint32_t e = ax >> 23;
  if (e < 102) return (uint16_t)sign;
  const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u, shift = 126 - e;
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

// one thread a block of 32; output row r of the matrix goes to row row_map[r] (or r)
__global__ void k_synth_q8(uint64_t key, int64_t rows, int64_t kb, int64_t row_stride_blocks,
                           const int32_t* __restrict__ row_map, int8_t* __restrict__ qs, uint16_t* __restrict__ d) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= rows * kb) return;
  const int64_t r = b / kb, j = b % kb;
  const int64_t orow = row_map ? row_map[r] : r;
  const int64_t ob = orow * row_stride_blocks + j;
  uint32_t out[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint64_t x = word(key, 5 * (uint64_t)b + (uint64_t)w);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j8 = 0; j8 < 8; ++j8) {
      const uint32_t u = (uint32_t)((x >> (8 * j8)) & 0xFF);
      const uint32_t q = (uint32_t)((int32_t)((u * 255u + 128u) >> 8) - 127) & 0xFFu;
      if (j8 < 4) lo |= q << (8 * j8); else hi |= q << (8 * (j8 - 4));
    }
    out[2 * w] = lo; out[2 * w + 1] = hi;
  }
  u32x4* dst = (u32x4*)(qs + 32 * ob);
  dst[0] = u32x4{out[0], out[1], out[2], out[3]};
  dst[1] = u32x4{out[4], out[5], out[6], out[7]};
  const float z = __fmul_rn((float)sum2(word(key, 5 * (uint64_t)b + 4)), 2.6428997921303017e-09f);
  d[ob] = f16_rne(fabsf(z));
}

__global__ void k_synth_normal(uint64_t key, int64_t n, float base, float scale, int add_base, float* __restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // plain operators: under the pragma they stay a rounded product and a rounded sum (the
  // __fmul_rn / __fadd_rn intrinsics inline without it, and were fused into one v_fma_f32)
  const float z = (float)sum2(word(key, (uint64_t)i)) * 1.3214498960651507e-05f;
  const float v = scale * z;
  out[i] = add_base ? base + v : v;
}

// GGUF block_q8_0 rows (34 bytes a block) -> qs, d; row r to row_map[r]
__global__ void k_repack_q8(const uint8_t* __restrict__ blocks, int64_t kb, int64_t rows,
                            const int32_t* __restrict__ row_map, int8_t* __restrict__ qs, uint16_t* __restrict__ d) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= rows * kb) return;
  const int64_t r = b / kb, j = b % kb;
  const int64_t ob = (row_map ? (int64_t)row_map[r] : r) * kb + j;
  const uint8_t* src = blocks + 34 * b;                    // 2-byte aligned only
  const uint16_t* s16 = (const uint16_t*)src;
  d[ob] = s16[0];
  uint16_t* dst = (uint16_t*)(qs + 32 * ob);
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[i] = s16[1 + i];
}

__global__ void k_dequant(const int8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t n,
                          float* __restrict__ f32, uint16_t* __restrict__ bf) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = f16_to_f32(d[i / 32]) * (float)qs[i];    // exact in fp32
  if (f32) f32[i] = v;
  if (bf) bf[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
}

// each value to the nearest fp16 (even on ties, subnormals kept), back as fp32
__global__ void k_round_f16(int64_t n, float* __restrict__ x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = f16_to_f32(f16_rne(x[i]));
}

__global__ void k_f32_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  y[i] = (uint16_t)(pack_bf16x2(x[i], 0.f) & 0xFFFFu);
}

static inline unsigned grid_of(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

hipError_t synth_q8(hipStream_t s, uint64_t key, int64_t rows, int64_t cols, int64_t row_stride_blocks,
                    const int32_t* row_map, int8_t* qs, uint16_t* d) {
  const int64_t kb = cols / 32;
  hipLaunchKernelGGL(k_synth_q8, dim3(grid_of(rows * kb, 256)), dim3(256), 0, s, key, rows, kb, row_stride_blocks,
                     row_map, qs, d);
  return hipGetLastError();
}

hipError_t synth_normal(hipStream_t s, uint64_t key, int64_t n, float base, float scale, int add_base, float* out) {
  hipLaunchKernelGGL(k_synth_normal, dim3(grid_of(n, 256)), dim3(256), 0, s, key, n, base, scale, add_base, out);
  return hipGetLastError();
}

hipError_t repack_q8_blocks(hipStream_t s, const uint8_t* blocks, int64_t kb, int64_t rows, const int32_t* row_map,
                            int8_t* qs, uint16_t* d) {
  hipLaunchKernelGGL(k_repack_q8, dim3(grid_of(rows * kb, 256)), dim3(256), 0, s, blocks, kb, rows, row_map, qs, d);
  return hipGetLastError();
}

hipError_t dequant_q8(hipStream_t s, const int8_t* qs, const uint16_t* d, int64_t n, float* f32, uint16_t* bf16) {
  hipLaunchKernelGGL(k_dequant, dim3(grid_of(n, 256)), dim3(256), 0, s, qs, d, n, f32, bf16);
  return hipGetLastError();
}

hipError_t round_f16(hipStream_t s, int64_t n, float* x) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_round_f16, dim3(grid_of(n, 256)), dim3(256), 0, s, n, x);
  return hipGetLastError();
}

hipError_t f32_to_bf16(hipStream_t s, const float* x, uint16_t* y, int64_t n) {
  hipLaunchKernelGGL(k_f32_to_bf16, dim3(grid_of(n, 256)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

// QT (the tiled Q8_0 operand, exn_common.h) from the SoA codes and scales: a workgroup a chunk,
// 1024 16-byte units of codes (row u/4, bytes 16 (u%4) of the k-step) and 64 of scales (rows 4u' ..
// 4u'+3, both blocks of the k-step each)
__global__ void __launch_bounds__(256)
k_tile_q8(const int8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t N, int64_t K,
          uint8_t* __restrict__ qt) {
  const int64_t KT = K / 64, chunk = blockIdx.x, nb = chunk / KT, t = chunk % KT;
  uint8_t* dst = qt + chunk * QT_CHUNK;
  for (int u = threadIdx.x; u < QT_CHUNK / 16; u += 256) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (u < QT_SCALES / 16) {
      const int64_t row = nb * 256 + u / 4;
      if (row < N) v = *(const u32x4*)(qs + row * K + t * 64 + (u % 4) * 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = nb * 256 + 4 * (u - QT_SCALES / 16) + e;
        if (row < N) v[e] = *(const uint32_t*)(d + row * (K / 32) + 2 * t);
      }
    }
    *(u32x4*)(dst + (int64_t)u * 16) = v;
  }
}

hipError_t tile_q8(hipStream_t s, const int8_t* qs, const uint16_t* d, int64_t N, int64_t K, uint8_t* qt) {
  if (K % 64 || N <= 0) return hipErrorInvalidValue;
  const int64_t chunks = (N + 255) / 256 * (K / 64);
  hipLaunchKernelGGL(k_tile_q8, dim3((unsigned)chunks), dim3(256), 0, s, qs, d, N, K, qt);
  return hipGetLastError();
}

}  // namespace exn
