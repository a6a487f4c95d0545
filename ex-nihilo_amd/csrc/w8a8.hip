// w8a8.hip -- the reference's default int8 products (src/cuda-dit.lisp:110-126, *int8*): a
// Q8_0 matrix times activations quantised to Q8_0 by blocks of 32 (quant_q8, :120-123), on
// the int8 MFMA.  illatio's kernels (quant_q8, MM_Q8_MMA2) are not in the reference tree; the
// arithmetic here follows ggml's CUDA forms, which the reference's note names as their model:
//
//   quant:   amax over the block, d = amax / 127 (kept as fp16), q = round(x / d) half away
//            from zero, 0 when amax is 0; the divisions correctly rounded;
//   product: per block the exact integer dot product, then y = fma(float(isum), dx * dw, y)
//            in fp32, blocks in order: the scale product rounded, the fused multiply-add
//            rounded once (ggml's sum += d * sumi as its CUDA compiler fuses it).
//
// On gfx950 the per-32 rescale, not the int8 MFMA, bounds the product: every 16x16x32 MFMA
// leaves 4 int32 sums a lane that each take a conversion, the scale product and a fused
// multiply-add.  k_gemm_w8a8_dma (below) is the product the model runs; k_gemm_w8a8, whose
// operands come straight from L2 into the MFMA registers, takes the shapes the DMA path does
// not (K not a multiple of 64, unaligned rows).
#include "exn_common.h"

namespace exn {

// rows of K values (fp32, or bf16 when XBF16; ldx apart) to Q8_0: codes [n][K], scales [n][K/32]
// fp16.  4 lanes a block, 8 values a lane.
__global__ void __launch_bounds__(256)
k_quant_q8(int64_t blocks, int kb, const void* __restrict__ x, int xbf16, int64_t ldx, int8_t* __restrict__ q,
           uint16_t* __restrict__ d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t blk = i >> 2;
  const bool live = blk < blocks;
  const int64_t row = live ? blk / kb : 0, col = live ? (blk % kb) * 32 + (i & 3) * 8 : 0;
  float v[8];
  if (xbf16) {
    const u32x4 u = *(const u32x4*)((const uint16_t*)x + row * ldx + col);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = bf16_lo(u[e]);
      v[2 * e + 1] = bf16_hi(u[e]);
    }
  } else {
    const f32x4 a = *(const f32x4*)((const float*)x + row * ldx + col);
    const f32x4 b = *(const f32x4*)((const float*)x + row * ldx + col + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  }
  float m = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
  m = fmaxf(m, __shfl_xor(m, 1, 64));   // the block's 4 lanes
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  const float dd = __fdiv_rn(m, 127.f);
  uint32_t w[2] = {0u, 0u};
  if (m != 0.f) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = (int)roundf(__fdiv_rn(v[e], dd));   // |c| <= 127
      w[e / 4] |= (uint32_t)(c & 0xFF) << (8 * (e % 4));
    }
  }
  if (live) {
    *(u32x2*)(q + row * (int64_t)kb * 32 + col) = u32x2{w[0], w[1]};
    if ((i & 3) == 0) d[row * kb + blk % kb] = __builtin_bit_cast(uint16_t, (_Float16)dd);
  }
}

hipError_t quant_q8(hipStream_t s, const void* x, int xbf16, int64_t ldx, int64_t n, int64_t K, int8_t* q,
                    uint16_t* d) {
  if (n <= 0) return hipSuccess;
  if (K % 32 || ldx % 8 || ((uintptr_t)x & 15) || ((uintptr_t)q & 7)) return hipErrorInvalidValue;
  const int64_t blocks = n * (K / 32);
  hipLaunchKernelGGL(k_quant_q8, dim3((unsigned)((blocks * 4 + 255) / 256)), dim3(256), 0, s, blocks, (int)(K / 32), x,
                     xbf16, ldx, q, d);
  return hipGetLastError();
}

// Y (M x N, ldy apart; fp32, or fp16 when F16OUT) from Q8_0 activations (xq [M][K], xd [M][K/32])
// and a Q8_0 matrix (wq [N][K], wd [N][K/32]).  128 x 128 tiles, 4 waves of 64 x 64, each 4 x 4
// tiles of v_mfma_i32_16x16x32_i8 (A: lane l holds row l%16, k = 8 (l/16) .. +7 of the block;
// D: lane l holds column l%16, rows 4 (l/16) + r).
template <bool F16OUT>
__global__ void __launch_bounds__(256)
k_gemm_w8a8(const int8_t* __restrict__ xq, const uint16_t* __restrict__ xd, const int8_t* __restrict__ wq,
            const uint16_t* __restrict__ wd, int64_t M, int64_t N, int64_t K, void* __restrict__ y, int64_t ldy) {
  __shared__ float sdx[8][128], sdw[8][128];   // the tile's scales of 8 blocks, fp32
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c16 = lane & 15, g = lane >> 4;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int64_t tm = (int64_t)blockIdx.y * 128, tn = (int64_t)blockIdx.x * 128;
  const int KB = (int)(K / 32);
  // the lane's operand rows (clamped: rows past M or N load a valid row and are never stored)
  int64_t ao[4], bo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ao[i] = min(tm + wm + 16 * i + c16, M - 1) * K + 8 * g;
    bo[i] = min(tn + wn + 16 * i + c16, N - 1) * K + 8 * g;
  }
  int32x4 zero = {0, 0, 0, 0};
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto load = [&](int b, int64_t (&a)[4], int64_t (&w)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = *(const int64_t*)(xq + ao[i] + 32 * b);
      w[i] = *(const int64_t*)(wq + bo[i] + 32 * b);
    }
  };
  // block bb (of the staged 8): 16 MFMAs and the rescale of their sums into the accumulators
  auto compute = [&](int bb, const int64_t (&a)[4], const int64_t (&w)[4]) {
    f32x4 dx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dx[i] = *(const f32x4*)&sdx[bb][wm + 16 * i + 4 * g];
    float dw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) dw[j] = sdw[bb][wn + 16 * j + c16];
    // the MFMAs of row tile i + 1 go out before row tile i's rescale, which then never waits on
    // the MFMA it reads
    int32x4 cur[4], nxt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cur[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[0], w[j], zero, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)   // the scale product rounded on its own, before the fused multiply-add
      if (i + 1 < 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) nxt[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i + 1], w[j], zero, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sc = dx[i][r] * dw[j];
          acc[i][j][r] = __builtin_fmaf((float)cur[j][r], sc, acc[i][j][r]);
        }
#pragma unroll
      for (int j = 0; j < 4; ++j) cur[j] = nxt[j];
    }
  };
  // the scales of blocks c0 .. c0 + 7 for this thread's row (threads 0..127) or column
  // (128..255) of the tile, 0 past the last block (such a block then adds exact zeros)
  const int sr = tid & 127;
  const uint16_t* ssrc = tid < 128 ? xd + min(tm + sr, M - 1) * KB : wd + min(tn + sr, N - 1) * KB;
  float* sdst = tid < 128 ? &sdx[0][sr] : &sdw[0][sr];
  auto fetch = [&](int c0, float (&v)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float f = f16_to_f32(ssrc[min(c0 + k, KB - 1)]);
      v[k] = c0 + k < KB ? f : 0.f;
    }
  };
  auto stage = [&](const float (&v)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) sdst[k * 128] = v[k];
  };
  // a chunk of 8 blocks is straight-line code: the operands of block b + 1 load while block b
  // computes (two register sets in turn), the next chunk's scales load into registers and go
  // to LDS at the chunk's end; loads past the last block re-read it, with zero scales
  int64_t A[2][4], W[2][4];
  float nsc[8];
  load(0, A[0], W[0]);
  fetch(0, nsc);
  stage(nsc);
  __syncthreads();
  for (int c0 = 0; c0 < KB; c0 += 8) {
    fetch(c0 + 8, nsc);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      load(min(c0 + k + 1, KB - 1), A[(k + 1) & 1], W[(k + 1) & 1]);
      compute(k, A[k & 1], W[k & 1]);
    }
    __syncthreads();   // every wave is done with this chunk's scales
    stage(nsc);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = tm + wm + 16 * i + 4 * g + r;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = tn + wn + 16 * j + c16;
        if (n >= N) continue;
        if constexpr (F16OUT)
          ((uint16_t*)y)[m * ldy + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
        else
          ((float*)y)[m * ldy + n] = acc[i][j][r];
      }
    }
}

typedef __attribute__((address_space(3))) void lds_void;

// one lane of a DMA into LDS: BYTES (4 or 16) from base + voff + soff, zeros where voff passes
// the extent (every offset here stays inside its row, so soff never carries a read past it)
__device__ __forceinline__ void dma16(const void* base, uint32_t extent, lds_void* dst, uint32_t voff, int soff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(const void* base, uint32_t extent, lds_void* dst, uint32_t voff, int soff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, voff, soff, 0, 0);
}

// The same product with its operands moved HBM/L2 -> LDS by the DMA path, NS stages of a chunk
// (2 blocks: 64 bytes of K) ahead (3 stages, 51 KB: three workgroups a CU; 4 stages, two
// workgroups, ran 17% slower, and loads straight from L2 into registers twice as slow again): per stage the tile's 128 code rows of X and of W (8 KB each,
// row r's 16-byte chunk c stored at c ^ (r / 4 % 4), so the fragment reads are conflict-free)
// and their fp16 scales of the two blocks (512 bytes each).  A wave's DMA a chunk is five
// instructions (2 X, 2 W, 1 scales), so waiting for chunk c while the NS - 2 after it are out
// is vmcnt(5 (NS - 2)).  Rows past M or N read as zeros (the buffer extents) and are not
// stored.  K a multiple of 64, ldx-free: X and W rows K bytes apart.
#define W8_NS 3
template <bool F16OUT>
__global__ void __launch_bounds__(256)
k_gemm_w8a8_dma(const int8_t* __restrict__ xq, const uint16_t* __restrict__ xd, const int8_t* __restrict__ wq,
                const uint16_t* __restrict__ wd, int64_t M, int64_t N, int64_t K, void* __restrict__ y, int64_t ldy) {
  // stage s: X codes at s * 17 KB, W codes + 8 KB, X scales + 16 KB, W scales + 16.5 KB
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int64_t tm = (int64_t)blockIdx.y * 128, tn = (int64_t)blockIdx.x * 128;
  const int KB = (int)(K / 32), KC = KB / 2;
  const uint32_t xext = (uint32_t)(max((int64_t)0, M - tm) * K), wext = (uint32_t)(max((int64_t)0, N - tn) * K);
  const uint32_t xsext = (uint32_t)(max((int64_t)0, M - tm) * KB * 2), wsext = (uint32_t)(max((int64_t)0, N - tn) * KB * 2);
  const int8_t* xbase = xq + tm * K;
  const int8_t* wbase = wq + tn * K;
  const uint16_t* xsbase = xd + tm * KB;
  const uint16_t* wsbase = wd + tn * KB;
  // code DMA: instruction i (0, 1) of wave w moves rows (2w + i) * 16 + l / 4, LDS chunk l % 4
  uint32_t coff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (2 * wave + i) * 16 + (lane >> 2);
    coff[i] = (uint32_t)(r * K + 16 * ((lane & 3) ^ ((r >> 2) & 3)));
  }
  // scale DMA: wave w moves 4 bytes (the chunk's two fp16 scales) of row (w & 1) * 64 + l, of X
  // (waves 0, 1) or W (waves 2, 3)
  const int srow = (wave & 1) * 64 + lane;
  const uint32_t soff = (uint32_t)(srow * KB * 2);
  auto issue = [&](int c) {
    uint8_t* st = smem + (c % W8_NS) * 17408;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma16(xbase, xext, (lds_void*)(st + (2 * wave + i) * 1024), coff[i], c * 64);
      dma16(wbase, wext, (lds_void*)(st + 8192 + (2 * wave + i) * 1024), coff[i], c * 64);
    }
    if (wave < 2) dma4(xsbase, xsext, (lds_void*)(st + 16384 + (wave & 1) * 256), soff, c * 4);
    else dma4(wsbase, wsext, (lds_void*)(st + 16896 + (wave & 1) * 256), soff, c * 4);
  };
  // fragment reads: row tile i (or column tile j) of the wave, block bb of the chunk: LDS row r,
  // chunk 2 bb + g / 2 at its swizzled place, 8 bytes at 8 (g % 2)
  int rdx[4], rdw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ra = wm + 16 * i + c16, rb = wn + 16 * i + c16;
    rdx[i] = ra * 64 + 8 * (g & 1) + ((ra >> 2) & 3) * 16;   // chunk index XORed in below
    rdw[i] = rb * 64 + 8 * (g & 1) + ((rb >> 2) & 3) * 16;
  }
  int32x4 zero = {0, 0, 0, 0};
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto frag = [&](const uint8_t* base, int rd, int chunk) {
    // rd holds row * 64 + 8 (g % 2) + 16 f(row); the place of chunk c is 16 (c ^ f(row))
    const int f16x = rd & 0x30;   // 16 f(row)
    return *(const int64_t*)(base + (rd & ~0x30) + ((chunk * 16) ^ f16x));
  };
  const int nc = KC;
  for (int c = 0; c < W8_NS - 1 && c < nc; ++c) issue(c);
  for (int c = 0; c < nc; ++c) {
    // chunk c has landed for every wave; every wave is done with chunk c - 1's stage
    asm volatile("" ::: "memory");
    constexpr int VM = 5 * (W8_NS - 2);   // the DMA of the chunks after c may stay out
    if (c + W8_NS - 2 < nc) __builtin_amdgcn_s_waitcnt((VM & 0xF) | (0x7 << 4) | (0x0 << 8) | ((VM >> 4) << 14));
    else __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));   // vmcnt(0): the last chunks
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + W8_NS - 1 < nc) issue(c + W8_NS - 1);
    const uint8_t* st = smem + (c % W8_NS) * 17408;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      int64_t a[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = frag(st, rdx[i], 2 * bb + (g >> 1));
        w[i] = frag(st + 8192, rdw[i], 2 * bb + (g >> 1));
      }
      f32x4 dx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 u = *(const u32x4*)(st + 16384 + (wm + 16 * i + 4 * g) * 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) dx[i][r] = f16_to_f32(bb ? u[r] >> 16 : u[r]);
      }
      float dw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t u = *(const uint32_t*)(st + 16896 + (wn + 16 * j + c16) * 4);
        dw[j] = f16_to_f32(bb ? u >> 16 : u);
      }
      int32x4 cur[4], nxt[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) cur[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[0], w[j], zero, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma clang fp contract(off)   // the scale product rounded on its own, before the fused multiply-add
        if (i + 1 < 4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) nxt[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i + 1], w[j], zero, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sc = dx[i][r] * dw[j];
            acc[i][j][r] = __builtin_fmaf((float)cur[j][r], sc, acc[i][j][r]);
          }
#pragma unroll
        for (int j = 0; j < 4; ++j) cur[j] = nxt[j];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = tm + wm + 16 * i + 4 * g + r;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = tn + wn + 16 * j + c16;
        if (n >= N) continue;
        if constexpr (F16OUT)
          ((uint16_t*)y)[m * ldy + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
        else
          ((float*)y)[m * ldy + n] = acc[i][j][r];
      }
    }
}

hipError_t gemm_w8a8(hipStream_t s, const int8_t* xq, const uint16_t* xd, int64_t M, const int8_t* wq,
                     const uint16_t* wd, int64_t N, int64_t K, void* y, int64_t ldy, int f16out) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (K % 32 || K <= 0 || ((uintptr_t)xq & 7) || ((uintptr_t)wq & 7) || ldy < N) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + 127) / 128));
  // the DMA path: 16-byte code chunks and 4-byte scale pairs, buffer extents within 32 bits
  const bool dma_ok = K % 64 == 0 && ((uintptr_t)xq & 15) == 0 && ((uintptr_t)wq & 15) == 0 &&
                      ((uintptr_t)xd & 3) == 0 && ((uintptr_t)wd & 3) == 0 && M * K < ((int64_t)1 << 31) &&
                      N * K < ((int64_t)1 << 31);
  if (dma_ok) {
    const size_t shm = W8_NS * 17408;
    {
      const hipError_t e = ensure_lds(f16out ? (const void*)k_gemm_w8a8_dma<true> : (const void*)k_gemm_w8a8_dma<false>,
                                      (int)shm);
      if (e != hipSuccess) return e;
    }
    if (f16out)
      hipLaunchKernelGGL(k_gemm_w8a8_dma<true>, grid, dim3(256), shm, s, xq, xd, wq, wd, M, N, K, y, ldy);
    else
      hipLaunchKernelGGL(k_gemm_w8a8_dma<false>, grid, dim3(256), shm, s, xq, xd, wq, wd, M, N, K, y, ldy);
  } else if (f16out) {
    hipLaunchKernelGGL(k_gemm_w8a8<true>, grid, dim3(256), 0, s, xq, xd, wq, wd, M, N, K, y, ldy);
  } else {
    hipLaunchKernelGGL(k_gemm_w8a8<false>, grid, dim3(256), 0, s, xq, xd, wq, wd, M, N, K, y, ldy);
  }
  return hipGetLastError();
}

}  // namespace exn
