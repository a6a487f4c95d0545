/* synth.c -- the oracle's C restatement of the byte and integer arithmetic on
 * the DiT path.  TEST INFRASTRUCTURE ONLY: tests, the smoke check and the
 * CPU-baseline leg of the benchmark link it for the expected values; the product
 * (libexn-hip.so) never does.
 *
 * What it restates:
 *   - GGUF block_q8_0 (34 bytes: fp16 d, then 32 int8 qs) and its dequant
 *     value = fp32(d) * q.  The reference reads these blocks in
 *     src/cuda-dit.lisp:71-76 (raw upload, then repack to qs and d) and
 *     src/metal-dit.lisp:80-83 (34-byte blocks read in place); its numpy
 *     oracle dequantises them with gguf-py (inspect/ref_dit.py:28-30).
 *   - fp32 -> bf16 round-to-nearest-even, the rounding of a dequantised
 *     weight into a bf16 MFMA operand.
 *   - fp32 -> fp16 round-to-nearest-even (subnormals kept).
 *   - the accumulation of the int8 product (the reference's *int8* mode,
 *     src/cuda-dit.lisp:110-126; ggml's Q8_0 block product, compiled with a
 *     fused multiply-add): acc = fmaf(isum, dx * dw, acc), one rounding.
 *   - the counter-based synthetic generator that makes the same weights on
 *     the host and on the GPU.  It has no counterpart in the reference
 *     (whose weights come from a GGUF file); its definition is the one the
 *     HIP generator follows, and tests hold the two to bit equality.
 *
 * Generator definition (all arithmetic mod 2^64):
 *   mix64(z)  = SplitMix64's finaliser: z ^= z>>30; z *= 0xBF58476D1CE4E5B9;
 *               z ^= z>>27; z *= 0x94D049BB133111EB; z ^= z>>31
 *   key(s, t) = mix64(s * G + t + 1),  G = 0x9E3779B97F4A7C15
 *   word(k, i)= mix64(k + (i + 1) * G)
 *   normal(w) = fp32(2*S - 262140) * fp32(1.3214498960651507e-05), where S is
 *               the sum of w's four 16-bit chunks (Irwin-Hall of 4 uniforms,
 *               scaled to unit variance; exact integer, one fp32 product)
 *   Q8_0 block b of a rows x cols matrix (b = row * cols/32 + kblock):
 *     byte j of qs = ((u * 255 + 128) >> 8) - 127,  u = byte (j % 8) of word(k, 5b + j/8)
 *         (each of -127..127 once, +1 twice: mean 1/256)
 *     d = fp16_rne(|fp32(2*S - 262140) * fp32(2.6428997921303017e-09)|),
 *         S from word(k, 5b + 4)     (|N(0, 2e-4)|, some of it fp16-subnormal)
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

#define G64 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
  z ^= z >> 30; z *= 0xBF58476D1CE4E5B9ull;
  z ^= z >> 27; z *= 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t exo_key(uint64_t seed, uint64_t tensor) { return mix64(seed * G64 + tensor + 1); }
uint64_t exo_word(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * G64); }

static inline int32_t chunk_sum2(uint64_t w) {
  const int32_t s = (int32_t)(w & 0xFFFF) + (int32_t)((w >> 16) & 0xFFFF) +
                    (int32_t)((w >> 32) & 0xFFFF) + (int32_t)((w >> 48) & 0xFFFF);
  return 2 * s - 262140;
}

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> fp16 bits, round to nearest even, subnormals kept, overflow to inf */
uint16_t exo_f16_rne(float f) {
  const uint32_t x = f32_bits(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);          /* NaN */
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);         /* rounds to >= 65520: inf */
  if (ax >= 0x38800000u) {                                          /* normal fp16 */
    const uint32_t m = ax + 0xFFFu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | ((m - 0x38000000u) >> 13));
  }
  /* fp16 subnormal or zero: value = ax as real / 2^-24 units */
  const uint32_t e = ax >> 23;                                      /* biased fp32 exponent */
  if (e < 102) return (uint16_t)sign;                              /* below half of the least subnormal */
  const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
  const uint32_t shift = 126 - e;                                   /* 14 .. 24 */
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

float exo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  if (e == 0) {
    const float v = (float)m * 5.9604644775390625e-08f;            /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  if (e == 31) return bits_f32(sign | 0x7F800000u | (m << 13));
  return bits_f32(sign | ((e + 112) << 23) | (m << 13));
}

/* fp32 -> bf16 bits, round to nearest even (NaN kept quiet) */
uint16_t exo_bf16_rne(float f) {
  const uint32_t x = f32_bits(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

void exo_bf16_rne_n(const float* in, uint16_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = exo_bf16_rne(in[i]);
}

/* Q8_0 weights as SoA: qs[rows*cols] int8, d[rows*cols/32] fp16 bits */
void exo_q8_0_synth(uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, int8_t* qs, uint16_t* d) {
  const uint64_t k = exo_key(seed, tensor);
  const int64_t nb = rows * (cols / 32);
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    for (int w = 0; w < 4; ++w) {
      const uint64_t x = exo_word(k, 5 * (uint64_t)b + (uint64_t)w);
      for (int j = 0; j < 8; ++j) {
        const uint32_t u = (uint32_t)((x >> (8 * j)) & 0xFF);
        qs[32 * b + 8 * w + j] = (int8_t)((int32_t)((u * 255u + 128u) >> 8) - 127);
      }
    }
    const float z = (float)chunk_sum2(exo_word(k, 5 * (uint64_t)b + 4)) * 2.6428997921303017e-09f;
    d[b] = exo_f16_rne(fabsf(z));
  }
}

/* the same weights as GGUF block_q8_0 records: 34 bytes a block */
void exo_q8_0_synth_blocks(uint64_t seed, uint64_t tensor, int64_t rows, int64_t cols, uint8_t* blocks) {
  const uint64_t k = exo_key(seed, tensor);
  const int64_t nb = rows * (cols / 32);
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    uint8_t* r = blocks + 34 * b;
    const float z = (float)chunk_sum2(exo_word(k, 5 * (uint64_t)b + 4)) * 2.6428997921303017e-09f;
    const uint16_t h = exo_f16_rne(fabsf(z));
    r[0] = (uint8_t)(h & 0xFF); r[1] = (uint8_t)(h >> 8);
    for (int w = 0; w < 4; ++w) {
      const uint64_t x = exo_word(k, 5 * (uint64_t)b + (uint64_t)w);
      for (int j = 0; j < 8; ++j) {
        const uint32_t u = (uint32_t)((x >> (8 * j)) & 0xFF);
        r[2 + 8 * w + j] = (uint8_t)(int8_t)((int32_t)((u * 255u + 128u) >> 8) - 127);
      }
    }
  }
}

/* n unit normals (Irwin-Hall of 4), element i from word(key, i) */
void exo_normal(uint64_t seed, uint64_t tensor, int64_t n, float* out) {
  const uint64_t k = exo_key(seed, tensor);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = (float)chunk_sum2(exo_word(k, (uint64_t)i)) * 1.3214498960651507e-05f;
}

/* GGUF block_q8_0 records -> fp32: fp32(d) * q, exact */
void exo_dequant_q8_0_blocks(const uint8_t* blocks, int64_t nblocks, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* r = blocks + 34 * b;
    const float d = exo_f16_to_f32((uint16_t)(r[0] | (r[1] << 8)));
    for (int j = 0; j < 32; ++j) out[32 * b + j] = d * (float)(int8_t)r[2 + j];
  }
}

/* SoA Q8_0 -> fp32 */
void exo_dequant_q8_0(const int8_t* qs, const uint16_t* d, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = exo_f16_to_f32(d[i / 32]) * (float)qs[i];
}

/* the int8 product's accumulation over one 32-block: acc[i][j] = fmaf(isum[i][j], dx[i] * dw[j],
 * acc[i][j]) for an n x m tile of exact integer sums (held as floats), the scale product rounded
 * to fp32 and the fused multiply-add rounded once (C99's fmaf is exact) */
void exo_w8a8_fma(const float* isum, const float* dx, const float* dw, int64_t n, int64_t m, float* acc) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    for (int64_t j = 0; j < m; ++j) {
      const float sc = dx[i] * dw[j];
      acc[i * m + j] = fmaf(isum[i * m + j], sc, acc[i * m + j]);
    }
}
