// gemm.hip -- Y = X W^T for the DiT's weight products on gfx950's bf16 MFMA.
//
// X: bf16 rows (M x K, lda apart).  W: Q8_0 as SoA -- qs (N x K int8, a row's
// K/32 blocks of 32 contiguous) and d (N x K/32 fp16) -- or plain bf16 (N x K).
// A Q8_0 weight enters the MFMAs as bf16(fp32(d) * q): the product of an fp16
// and an int8 is exact in fp32 and is rounded once, to nearest even.
// This replaces the reference's mm dispatch (src/cuda-dit.lisp:115-130) and
// illatio's Q8_0 products behind it; the epilogues fuse the reference's
// x_gate_add (src/cuda/dit.cu:34-41), x_swiglu2 (:186-192) and x_gelu_tanh
// (:194-199) into the product's store.
//
// k_gemm_bt (below) is the block products' kernel, on bf16 rows or on Q8_0
// dequantised inside its LDS-DMA pipeline.  k_gemm is the fallback for shapes
// and alignments that pipeline does not take: BM x BN per workgroup, BK = 64
// (two Q8_0 blocks) per step, waves of WM x WN, each a grid of 32x32
// accumulators (v_mfma_f32_32x32x16_bf16); LDS is double-buffered, the next
// step's global loads are in registers while the current step's MFMAs run,
// and each thread dequantises one 32-value block on its way into LDS.
#include "exn_common.h"

#include <type_traits>

namespace exn {

#define BK 64
#define SA (BK + 8)   // LDS row stride in bf16: 144 bytes, conflict-free 16-byte fragment reads

// MFMA 32x32x16 bf16 operand/accumulator layout (wave64):
//   A (32 x 16): lane l holds row l%32, k = 8*(l/32) .. +7
//   B (16 x 32): lane l holds column l%32, k = 8*(l/32) .. +7
//   D (32 x 32): lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4 for r = 0..15

// The store of a wave's accumulators (rows wrow.., columns wcol..), fused with the
// reference's elementwise step that follows the product.
template <int EPI, int MI, int NI>
__device__ __forceinline__ void epilogue(const f32x16 (&acc)[MI][NI], int64_t wrow, int64_t wcol, int lane, int64_t M,
                                         int64_t N, const EpiArgs& ea) {
  if constexpr (EPI == EPI_SWIGLU) {
    // accumulator pairs (2jj, 2jj+1) hold matching gate and up columns (rows interleaved by 32 at load)
    uint16_t* y = (uint16_t*)ea.y;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int jj = 0; jj < NI / 2; ++jj) {
        const int64_t col = wcol / 2 + jj * 32 + (lane & 31);
        if (2 * (col - (lane & 31)) >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = wrow + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
          if (m < M) {
            const float g = acc[i][2 * jj][r], u = acc[i][2 * jj + 1][r];
            y[m * ea.ldy + col] = (uint16_t)(pack_bf16x2(silu_f(g) * u, 0.f) & 0xFFFF);
          }
        }
      }
  } else {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int64_t n = wcol + j * 32 + (lane & 31);
      if (n >= N) continue;
      float g0 = 0.f, g1 = 0.f;
      if constexpr (EPI == EPI_GATE_ADD) {
        g0 = tanh_f(ea.gate[n]);
        g1 = tanh_f(ea.gate[ea.mstride + n]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = wrow + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
          if (m >= M) continue;
          const float v = acc[i][j][r];
          if constexpr (EPI == EPI_F32) {
            ((float*)ea.y)[m * ea.ldy + n] = v;
          } else if constexpr (EPI == EPI_BF16) {
            ((uint16_t*)ea.y)[m * ea.ldy + n] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFF);
          } else if constexpr (EPI == EPI_F16) {
            ((uint16_t*)ea.y)[m * ea.ldy + n] = (uint16_t)(pack_f16x2(v, 0.f) & 0xFFFF);
          } else if constexpr (EPI == EPI_GELU_BF16) {
            ((uint16_t*)ea.y)[m * ea.ldy + n] = (uint16_t)(pack_bf16x2(gelu_tanh_f(v), 0.f) & 0xFFFF);
          } else if constexpr (EPI == EPI_GATE_ADD) {
            const float g = (ea.n0 + m < ea.p) ? g1 : g0;
            float* x = ea.resid + m * ea.ldy + n;
            *x = *x + g * v;
          }
        }
    }
  }
}

template <int BM, int BN, int WM, int WN, bool WBF16, int EPI>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
k_gemm(const uint16_t* __restrict__ X, int64_t lda, const int8_t* __restrict__ QS, const uint16_t* __restrict__ D,
       const uint16_t* __restrict__ WB, int64_t M, int64_t N, int64_t K, EpiArgs ea) {
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  constexpr int MI = WM / 32, NI = WN / 32;
  constexpr int A_CH = BM * (BK / 8) / NT;         // 16-byte X chunks per thread
  constexpr int B_PAIRS = BN * (BK / 32) / NT;     // Q8_0 blocks per thread
  constexpr int B_CH = BN * (BK / 8) / NT;         // 16-byte bf16 W chunks per thread
  static_assert(A_CH * NT == BM * (BK / 8), "A tile split");
  static_assert(WBF16 ? (B_CH * NT == BN * (BK / 8)) : (B_PAIRS * NT == BN * (BK / 32)), "B tile split");

  extern __shared__ __align__(16) uint16_t lds[];
  // buffer b: X tile at lds + b*(BM+BN)*SA, W tile right after it
#define As(b) (lds + (b) * (BM + BN) * SA)
#define Bs(b) (lds + (b) * (BM + BN) * SA + BM * SA)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / (BN / WN), wn = wave % (BN / WN);
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t kb = K / 32;

  u32x4 ra[A_CH];
  u32x4 rq[WBF16 ? B_CH : 2 * B_PAIRS];
  uint16_t rd[WBF16 ? 1 : B_PAIRS];

  auto load = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * NT, row = c >> 3, c8 = c & 7;
      const int64_t m = min(m0 + row, M - 1);
      ra[i] = *(const u32x4*)(X + m * lda + k0 + c8 * 8);
    }
    if constexpr (WBF16) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + i * NT, row = c >> 3, c8 = c & 7;
        const int64_t n = min(n0 + row, N - 1);
        rq[i] = *(const u32x4*)(WB + n * K + k0 + c8 * 8);
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_PAIRS; ++i) {
        const int c = tid + i * NT, row = c >> 1, blk = c & 1;
        const int64_t n = min(n0 + row, N - 1);
        const u32x4* src = (const u32x4*)(QS + n * K + k0 + 32 * blk);
        rq[2 * i] = src[0];
        rq[2 * i + 1] = src[1];
        rd[i] = D[n * kb + k0 / 32 + blk];
      }
    }
  };

  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * NT, row = c >> 3, c8 = c & 7;
      *(u32x4*)(As(buf) + row * SA + c8 * 8) = ra[i];
    }
    if constexpr (WBF16) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + i * NT, row = c >> 3, c8 = c & 7;
        *(u32x4*)(Bs(buf) + row * SA + c8 * 8) = rq[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_PAIRS; ++i) {
        const int c = tid + i * NT, row = c >> 1, blk = c & 1;
        const float dv = f16_to_f32(rd[i]);
        uint32_t o[16];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const uint32_t q = rq[2 * i + w / 4][w % 4];
          const float f0 = (float)(int8_t)(q & 0xFF) * dv, f1 = (float)(int8_t)((q >> 8) & 0xFF) * dv;
          const float f2 = (float)(int8_t)((q >> 16) & 0xFF) * dv, f3 = (float)(int8_t)(q >> 24) * dv;
          o[2 * w] = pack_bf16x2(f0, f1);
          o[2 * w + 1] = pack_bf16x2(f2, f3);
        }
        u32x4* dst = (u32x4*)(Bs(buf) + row * SA + 32 * blk);
        dst[0] = u32x4{o[0], o[1], o[2], o[3]};
        dst[1] = u32x4{o[4], o[5], o[6], o[7]};
        dst[2] = u32x4{o[8], o[9], o[10], o[11]};
        dst[3] = u32x4{o[12], o[13], o[14], o[15]};
      }
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

  const int KT = (int)(K / BK);
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load((int64_t)(kt + 1) * BK);
    const uint16_t* a_base = As(buf) + (wm * WM + (lane & 31)) * SA + 8 * (lane >> 5);
    const uint16_t* b_base = Bs(buf) + (wn * WN + (lane & 31)) * SA + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 a[MI], b[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) a[i] = *(const bf16x8*)(a_base + i * 32 * SA + kk * 16);
#pragma unroll
      for (int j = 0; j < NI; ++j) b[j] = *(const bf16x8*)(b_base + j * 32 * SA + kk * 16);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store(buf ^ 1);
    __syncthreads();
  }

  epilogue<EPI, MI, NI>(acc, m0 + wm * WM, n0 + wn * WN, lane, M, N, ea);
}

template <int BM, int BN, int WM, int WN, bool WBF16, int EPI>
static hipError_t launch(hipStream_t s, const uint16_t* x, int64_t lda, const int8_t* qs, const uint16_t* d,
                         const uint16_t* wb, int64_t M, int64_t N, int64_t K, const EpiArgs& ea) {
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  const size_t shm = 2 * (size_t)(BM + BN) * SA * sizeof(uint16_t);
  auto kern = k_gemm<BM, BN, WM, WN, WBF16, EPI>;
  {
    const hipError_t e = ensure_lds((const void*)kern, (int)shm);
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(kern, grid, dim3(NT), shm, s, x, lda, qs, d, wb, M, N, K, ea);
  return hipGetLastError();
}

template <bool WBF16>
static hipError_t dispatch(hipStream_t s, const uint16_t* x, int64_t lda, const int8_t* qs, const uint16_t* d,
                           const uint16_t* wb, int64_t M, int64_t N, int64_t K, Epi epi, const EpiArgs& ea) {
  switch (epi) {
    case EPI_F32: return launch<256, 256, 128, 64, WBF16, EPI_F32>(s, x, lda, qs, d, wb, M, N, K, ea);
    case EPI_BF16: return launch<256, 256, 128, 64, WBF16, EPI_BF16>(s, x, lda, qs, d, wb, M, N, K, ea);
    case EPI_GATE_ADD: return launch<256, 256, 128, 64, WBF16, EPI_GATE_ADD>(s, x, lda, qs, d, wb, M, N, K, ea);
    case EPI_SWIGLU: return launch<256, 256, 128, 64, WBF16, EPI_SWIGLU>(s, x, lda, qs, d, wb, M, N, K, ea);
    case EPI_GELU_BF16: return launch<256, 256, 128, 64, WBF16, EPI_GELU_BF16>(s, x, lda, qs, d, wb, M, N, K, ea);
    case EPI_F16: return launch<256, 256, 128, 64, WBF16, EPI_F16>(s, x, lda, qs, d, wb, M, N, K, ea);
    default: return hipErrorInvalidValue;   // the fused QKV and split sums run on k_gemm_bt only
  }
}

// --- bf16 weights: the pipelined kernel ----------------------------------------------
// 256 x 256 tiles, 8 waves of 128 x 64 (8 x 4 tiles of v_mfma_f32_16x16x32_bf16) or, for the
// QKV product's fused epilogue, 64 x 128 (one head a wave); BK = 64 in two slices of 32.
// Both tiles go HBM/L2 -> LDS by the LDS DMA path (buffer_load_dwordx4 ... lds: no VGPR
// staging, no ds_write), two stages, with the step schedule described at the kernel.
// LDS rows are 128 bytes with the 16-byte chunks XOR-swizzled by (row/2)%8: the
// fragment reads of 32 rows x 16 bytes are bank-conflict free.
typedef __attribute__((address_space(3))) void lds_void;
#define LDS_VMCNT0_BARRIER()                                     \
  do {                                                           \
    asm volatile("" ::: "memory");                               \
    __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));         \
    __builtin_amdgcn_s_barrier();                                \
    asm volatile("" ::: "memory");                               \
  } while (0)
#define SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)

__device__ __forceinline__ int chunk_swz(int r) { return (r >> 1) & 7; }

// The epilogue through LDS (free once the main loop is done): a wave's (16 MI) x (16 NI)
// accumulators go out 32 rows at a time into its own 32 x (16 NI + 8)-float LDS block, and
// come back as 4 consecutive columns a lane, so every global access is 16 bytes (8 for
// bf16/fp16) and a wave's instruction covers whole rows.  Needs N % 4 == 0, LDY % 4 == 0.
template <int EPI, int MI, int NI>
__device__ __forceinline__ void epilogue_lds(const f32x4 (&acc)[MI][NI], float* stage, int64_t wrow, int64_t wcol,
                                             int lane, int64_t M, int64_t N, const EpiArgs& ea) {
  constexpr int LS = 16 * NI + 8;
  // this lane's 4 columns (SwiGLU: 4 output columns, 8 NI / 4 lanes a row; others 16 NI / 4)
  constexpr int LPR = EPI == EPI_SWIGLU ? 2 * NI : 4 * NI;
  const int c4 = (lane % LPR) * 4;
  // the gated residual's rows are loaded two 32-row chunks at a time, before either is stored:
  // a wave waits out two round trips to HBM instead of one a row group (with loads and stores
  // both in flight the wait counter only tells when all have ended, so every load issued after
  // a store would be waited for alone).  The first pair goes out with the gate's loads.
  constexpr int IT = 32 * LPR / 64;
  f32x4 rb[2][IT];
  auto load_pair = [&](int i2) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int64_t m = wrow + 32 * (i2 + c) + it * (64 / LPR) + lane / LPR, n = wcol + c4;
        rb[c][it] = (i2 + c < MI / 2 && m < M && n < N) ? *(const f32x4*)(ea.resid + m * ea.ldy + n)
                                                         : f32x4{0.f, 0.f, 0.f, 0.f};
      }
  };
  // the gates' tanh is taken after the first pair's wait (below), so no wait of its own
  f32x4 g0 = {0.f, 0.f, 0.f, 0.f}, g1 = g0;
  if constexpr (EPI == EPI_GATE_ADD) {
    const int64_t n = wcol + c4;
    if (n < N) {
      g0 = *(const f32x4*)(ea.gate + n);
      g1 = *(const f32x4*)(ea.gate + ea.mstride + n);
    }
    load_pair(0);
  }
  // accumulators of v_mfma_f32_16x16x32: lane l holds column l%16, rows 4*(l/16) + r
  const int c16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int i2 = 0; i2 < MI / 2; ++i2) {
    if constexpr (EPI == EPI_GATE_ADD) {
      if (i2 % 2 == 0 && i2 > 0) load_pair(i2);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[(16 * h + 4 * q4 + r) * LS + 16 * j + c16] = acc[2 * i2 + h][j][r];
    if constexpr (EPI == EPI_GATE_ADD) {
      // the pair's residual loads have landed: one wait here, outside the per-row branches
      // (a wait inside one would be repeated at every row after it)
      if (i2 % 2 == 0) __builtin_amdgcn_s_waitcnt((0x0) | (0x7 << 4) | (0xF << 8) | (0x0 << 14));   // vmcnt(0)
      if (i2 == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g0[e] = tanh_f(g0[e]);
          g1[e] = tanh_f(g1[e]);
        }
      }
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = it * (64 / LPR) + lane / LPR;
      const int64_t m = wrow + 32 * i2 + row;
      if (m >= M) continue;
      if constexpr (EPI == EPI_SWIGLU) {
        // output column wcol/2 + c4: its gate at 64 (c4/32) + c4%32 of the LDS row, its up 32 on
        const int64_t col = wcol / 2 + c4;
        if (2 * (col - c4) >= N) continue;
        const int gc = 64 * (c4 >> 5) + (c4 & 31);
        const f32x4 v = *(const f32x4*)(stage + row * LS + gc);
        const f32x4 u = *(const f32x4*)(stage + row * LS + gc + 32);
        uint16_t* y = (uint16_t*)ea.y + m * ea.ldy + col;
        *(u32x2*)y = u32x2{pack_bf16x2(silu_bf16out(v[0]) * u[0], silu_bf16out(v[1]) * u[1]),
                           pack_bf16x2(silu_bf16out(v[2]) * u[2], silu_bf16out(v[3]) * u[3])};
      } else {
        const int64_t n = wcol + c4;
        if (n >= N) continue;
        const f32x4 v = *(const f32x4*)(stage + row * LS + c4);
        if constexpr (EPI == EPI_F32) {
          *(f32x4*)((float*)ea.y + m * ea.ldy + n) = v;
        } else if constexpr (EPI == EPI_PART) {
          *(f32x4*)((float*)ea.y + ((int64_t)blockIdx.z * M + m) * ea.ldy + n) = v;
        } else if constexpr (EPI == EPI_BF16) {
          *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + n) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        } else if constexpr (EPI == EPI_F16) {
          *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + n) = u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
        } else if constexpr (EPI == EPI_GELU_BF16) {
          *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + n) =
              u32x2{pack_bf16x2(gelu_tanh_f(v[0]), gelu_tanh_f(v[1])), pack_bf16x2(gelu_tanh_f(v[2]), gelu_tanh_f(v[3]))};
        } else if constexpr (EPI == EPI_GATE_ADD) {
          const f32x4 g = (ea.n0 + m < ea.p) ? g1 : g0;
          f32x4 xv = rb[i2 % 2][it];
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[e] = xv[e] + g[e] * v[e];
          *(f32x4*)(ea.resid + m * ea.ldy + n) = xv;
        }
      }
    }
  }
}

// The QKV product's epilogue (EPI_QKV): a wave's 64 rows x 128 columns are one head of q, k
// or v for 64 tokens (output row m is sequence row n0 + m).  q and k: the RMS of each row
// over the head from the accumulators (the lane's 8 values, then the 16 lanes that share the
// row), then rows through the wave's LDS block 16 at a time, each lane 4 consecutive
// columns: the norm weight, the rotation of its two pairs (one 16-byte cos/sin load), q's
// scale, and 8 bytes of fp16 into Q or the K cache.  v: 16 tokens of V^T at a time, 16 bytes
// (8 keys) a lane when the 16 keys are one aligned group of the V^T order, else key by key.
// The same arithmetic as qkv_prep (eltwise.hip) on the fp32 sums instead of their fp16
// rounding; V^T's values are the same fp16 roundings.
template <int MI, int NI>
__device__ __forceinline__ void epilogue_qkv(f32x4 (&acc)[MI][NI], float* stage, int64_t wrow, int64_t wcol,
                                             int lane, int64_t M, const EpiArgs& ea) {
  static_assert(MI == 4 && NI == 8, "a wave holds 64 rows of one head (128 columns)");
  constexpr int LS = 132;   // LDS row: 128 floats and 4 of padding
  const int part = (int)(wcol / EXN_W), h = (int)((wcol % EXN_W) / EXN_HD);   // part 0 q, 1 k, 2 v
  const int c16 = lane & 15, q4 = lane >> 4;
  const int c4 = (lane & 31) * 4;
  // the cos/sin of a 16-row block: 2 rows a wave instruction, 8 loads a lane.  Blocks 0 and 1
  // go out before the RMS; a buffer is refilled with block i + 2 once block i is stored, and
  // one wait before blocks 0 and 2 (outside the per-row branches) covers a pair: with loads
  // and stores both in flight the wait counter only tells when all have ended, so waits
  // inside the row loop would hold each store for the one before it
  auto cs_load = [&](f32x4 (&dst)[8], int i) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int64_t m = min(wrow + 16 * i + 2 * it + (lane >> 5), M - 1);   // rows past M: loaded, unused
      dst[it] = *(const f32x4*)(ea.cs + (ea.n0 + m) * EXN_HD + c4);
    }
  };
  // a wave's 64 x 128 accumulators through LDS 16 rows at a time
  auto stage_block = [&](int i) {
    // accumulators of v_mfma_f32_16x16x32: lane l holds column l%16, rows 4*(l/16) + r
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) stage[(4 * q4 + r) * LS + 16 * j + c16] = acc[i][j][r];
  };
  // q and k, and v, each in a loop of its own: the two paths meet only at the end, so the
  // wait counter's state is exact inside each
  if (part < 2) {
    f32x4 csa[8], csb[8];
    cs_load(csa, 0);
    if (MI > 1) cs_load(csb, 1);
    const f32x4 w = *(const f32x4*)((part == 0 ? ea.wq : ea.wk) + c4);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NI; ++j) ss += acc[i][j][r] * acc[i][j][r];
        const float inv = rsqrtf(row16_sum(ss) * (1.f / 128.f) + 1e-6f);
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j][r] *= inv;
      }
    const float sc = part == 0 ? ea.qscale : 1.f;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      stage_block(i);
      const int64_t mb = wrow + 16 * i;   // the output row of the 16 staged rows' first
      if (i % 2 == 0) __builtin_amdgcn_s_waitcnt((0x0) | (0x7 << 4) | (0xF << 8) | (0x0 << 14));   // vmcnt(0)
      f32x4(&csc)[8] = i % 2 == 0 ? csa : csb;
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int row = 2 * it + (lane >> 5);
        const int64_t m = mb + row;
        if (m >= M) continue;
        const f32x4 v = *(const f32x4*)(stage + row * LS + c4);
        const f32x4 cs = csc[it];   // cos, sin of the lane's 2 pairs
        const float a0 = v[0] * w[0], a1 = v[1] * w[1], a2 = v[2] * w[2], a3 = v[3] * w[3];
        const u32x2 o = {pack_f16x2((a0 * cs[0] - a1 * cs[1]) * sc, (a0 * cs[1] + a1 * cs[0]) * sc),
                         pack_f16x2((a2 * cs[2] - a3 * cs[3]) * sc, (a2 * cs[3] + a3 * cs[2]) * sc)};
        uint16_t* dst = part == 0 ? ea.q + ((int64_t)h * (ea.qld ? ea.qld : M) + m) * EXN_HD + c4
                                  : ea.kc + ((int64_t)h * ea.lcap + ea.n0 + m) * EXN_HD + c4;
        *(u32x2*)dst = o;
      }
      if (i + 2 < MI) cs_load(csc, i + 2);
    }
  } else {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      stage_block(i);
      const int64_t mb = wrow + 16 * i;
      const int64_t kb = ea.n0 + mb;   // the key of the first staged row
      if (kb % 16 == 0 && mb + 16 <= M) {
        // one aligned group of 16 keys: V^T column kb + c holds key kb + vt_pos(c); a lane
        // packs 8 columns of one dim, 4 times (128 dims x 2 halves)
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const int task = it * 64 + lane, d = task >> 1, hf = task & 1;
          uint32_t pk[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pk[e] = pack_f16x2(stage[vt_pos(8 * hf + 2 * e) * LS + d], stage[vt_pos(8 * hf + 2 * e + 1) * LS + d]);
          *(u32x4*)(ea.vt + ((int64_t)h * EXN_HD + d) * ea.lcap + kb + 8 * hf) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
      } else {
        for (int it = 0; it < 32; ++it) {
          const int task = it * 64 + lane, d = task & 127, k = task >> 7;
          if (mb + k < M)
            ea.vt[((int64_t)h * EXN_HD + d) * ea.lcap + vt_pos(kb + k)] = (uint16_t)(pack_f16x2(stage[k * LS + d], 0.f) & 0xFFFF);
        }
      }
    }
  }
}

// SwiGLU's epilogue, in registers first: a wave's 64 columns are 32 gate columns then their 32
// up columns (gate_up interleaved by 32), so the lane holding gate column block j holds its up
// block j + 2, and silu(gate) x up is computed on the accumulators.  Only the bf16 outputs
// (128 rows x 32 columns a wave, rows 40 halves apart) go through LDS, to come back as 8
// consecutive columns a lane for 16-byte stores.
template <int MI, int NI>
__device__ __forceinline__ void epilogue_swiglu(const f32x4 (&acc)[MI][NI], uint16_t* stage, int64_t wrow, int64_t wcol,
                                                int lane, int64_t M, int64_t N, const EpiArgs& ea) {
  static_assert(NI == 4, "a wave's 64 columns: one gate/up pair of 32");
  constexpr int LS = 40;
  const int c16 = lane & 15, q4 = lane >> 4;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float o = silu_bf16out(acc[i][j][r]) * acc[i][j + 2][r];
        stage[(16 * i + 4 * q4 + r) * LS + 16 * j + c16] = (uint16_t)(pack_bf16x2(o, 0.f) & 0xFFFF);
      }
  // rows of 32 outputs: 4 chunks of 8; 16 rows a wave instruction, 16 MI / 16 = MI instructions
  const int64_t col = wcol / 2 + 8 * (lane & 3);
  if (2 * (wcol / 2) >= N) return;
#pragma unroll
  for (int it = 0; it < MI; ++it) {
    const int row = 16 * it + (lane >> 2);
    const int64_t m = wrow + row;
    const u32x4 v = *(const u32x4*)(stage + row * LS + 8 * (lane & 3));
    if (m < M) *(u32x4*)((uint16_t*)ea.y + m * ea.ldy + col) = v;
  }
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// A buffer resource (V#) for the assembly load below: BASE, no stride, EXTENT bytes (offsets past it
// read as zeros), the flags the buffer builtins use
__device__ __forceinline__ i32x4 buffer_desc(const void* base, uint32_t extent) {
  const uint64_t a = (uint64_t)base;
  return i32x4{(int32_t)(uint32_t)a, (int32_t)(uint32_t)((a >> 32) & 0xFFFFu), (int32_t)extent, 0x00020000};
}

// A 4-byte buffer load the compiler does not see as one: it tracks no result for it, and so
// inserts no wait for it, where its model of the DMA counter is more careful than the schedule
// needs (the kernel's own vmcnt waits cover the value before its use).  The destination stays
// allocated to the value from the load to its last use; after the loop the kernel holds it
// live until every load has landed.  This is correct only while the register allocator neither
// reads nor copies that register between the load and the wait that covers it (a value carried
// round the loop in one register, as here, is not copied; two alternating registers selected by
// the step's parity were, before the wait, and that form is not used).  The bit-exact Q8_0 tests
// (the resident expansion against the in-pipeline dequantisation) are what catch a violation.
__device__ __forceinline__ uint32_t buffer_load_u32_untracked(i32x4 rsrc, uint32_t voff, uint32_t soff) {
  uint32_t v;
  asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rsrc), "s"(soff));
  return v;
}

// One 16-byte DMA lane of a tile: the buffer's extent makes rows past the matrix read as zeros.
__device__ __forceinline__ void tile_dma(const void* base, uint32_t extent, lds_void* dst, uint32_t voff, int soff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

// The vector memory operations a wait at position P of a step must leave out, when it waits for
// the one at position Q of K steps before: the rest of that step, the K - 1 steps between, and
// this step's before P (a step's operations at positions POS[0..N-1], one each, in issue order)
constexpr int ops_after(int Q, int K, int P, const int* pos, int n) {
  int c = (K - 1) * n;
  for (int i = 0; i < n; ++i) c += (pos[i] > Q) + (pos[i] < P);
  return c;
}

// NW waves of 128 x (512 / NW) a 256 x 256 tile.  The launch uses 8 waves of 128 x 64, two a
// SIMD.  4 waves of 128 x 128 (one a SIMD, a third less LDS read a FLOP) were slower under the
// one-barrier schedule and spill their 256 accumulators under this one.
//
// Q8: W is Q8_0 in the tiled layout QT (exn_common.h) and is dequantised inside the pipeline.
// A k-step of the tile is 17 KB in one run: its 16 KB of int8 codes go HBM -> LDS by the same
// DMA path into two raw stages (so the LDS holds 2 x 64 KB of bf16 stages + 2 x 16 KB of codes =
// 160 KB), each thread's two fp16 scales by a 4-byte load into a register (a wave's 64 loads one
// 128-byte line), and once a k-step the 512 threads turn one raw stage into the bf16 W stage the
// MFMAs read: thread t takes tile row t/2, Q8_0 block t%2 -- 32 codes, two 16-byte LDS reads --
// and writes bf16(fp32(d) q) as four swizzled 16-byte rows: a signed byte conversion and one
// multiply a value (q d has at most 18 significant bits, exact in fp32), rounded once, so the
// operand is bit for bit the resident expansion's value.
template <int EPI, int NW, bool Q8>
__global__ void __launch_bounds__(NW * 64)
k_gemm_bt(const uint16_t* __restrict__ X, int64_t lda, const uint16_t* __restrict__ WB,
          const uint8_t* __restrict__ QT, int64_t M, int64_t N, int64_t K, EpiArgs ea) {
  constexpr bool HEADS = EPI == EPI_QKV;   // a wave's columns one head of 128
  constexpr int WM = HEADS ? 64 : 128, WN = HEADS ? 128 : 512 / NW, MI = WM / 16, NI = WN / 16;
  constexpr int ROUNDS = 256 / (NW * 8);
  static_assert((256 / WM) * (256 / WN) == NW, "the waves tile 256 x 256");
  static_assert(!Q8 || NW == 8, "the Q8_0 dequantisation maps 512 threads to 256 rows x 2 blocks");
  // DMA instructions a k-step: X and W rounds (bf16), or X rounds only (Q8: the codes go apart)
  constexpr int NMF = MI * NI, NRD = MI + NI, NDMA = Q8 ? ROUNDS : 2 * ROUNDS;
  // 2 stages x (X tile 32 KB | W tile 32 KB), then (Q8) 2 raw code stages x 16 KB
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: LDS bases stay scalar
  const int wm = wave / (256 / WN), wn = wave % (256 / WN);
  // tile order: workgroups go to the 8 XCDs in turn, so XCD x takes the x-th eighth of a
  // tile order that walks 4 row tiles at a time -- its concurrent tiles share W and X in its L2
  int bm = blockIdx.y, bn = blockIdx.x;
  {
    const int gx = gridDim.x, gy = gridDim.y, G = gx * gy, b = blockIdx.y * gx + blockIdx.x;
    const int L = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    constexpr int GM = 4;
    const int grp = L / (GM * gx), first = grp * GM, sz = min(gy - first, GM), in = L % (GM * gx);
    bm = first + in % sz;
    bn = in / sz;
  }
  const int64_t m0 = (int64_t)bm * 256, n0 = (int64_t)bn * 256;
  // split K (EPI_PART): workgroup z of gridDim.z takes k-steps kt0 .. kt1-1, in pairs where the
  // step count is even (Q8 needs them, K % 128 == 0: the main loop runs whole pairs of steps and
  // no third copy of the step is live; the bf16 weights cut the same way, so that both give the
  // same partial sums)
  const int KTT = (int)(K / 64), SK = gridDim.z, zk = blockIdx.z;
  const bool pairs = Q8 || KTT % 2 == 0;
  const int kt0 = pairs ? 2 * (int)((int64_t)(KTT / 2) * zk / SK) : (int)((int64_t)KTT * zk / SK);
  const int kt1 = pairs ? 2 * (int)((int64_t)(KTT / 2) * (zk + 1) / SK) : (int)((int64_t)KTT * (zk + 1) / SK);
  // DMA: round i of wave w moves rows (i*8 + w)*8 .. +7 of a tile, lane l row +l/8, LDS chunk l%8
  // (global chunk (l%8) ^ swizzle); the k-step is the scalar offset
  const uint16_t* xbase = X + m0 * lda;
  const uint16_t* wbase = WB + n0 * K;
  const uint32_t xext = (uint32_t)((M - m0) * lda * 2);
  const uint32_t wext = Q8 ? 0u : (uint32_t)(max((int64_t)0, N - n0) * K * 2);
  uint32_t xoff[ROUNDS], woff[ROUNDS];
#pragma unroll
  for (int i = 0; i < ROUNDS; ++i) {
    const int row = (i * NW + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ chunk_swz(row);
    xoff[i] = (uint32_t)((row * lda + 8 * c) * 2);
    woff[i] = (uint32_t)((row * K + 8 * c) * 2);
  }
  auto dma_part = [&](int t, int stage, int p) {   // part p < ROUNDS: X round p, else W round p - ROUNDS
    uint8_t* dst = smem + stage * 65536 + (p < ROUNDS ? 0 : 32768) + ((p % ROUNDS) * NW + wave) * 1024;
    // Q8: round p's rows are round 0's plus p NW 8 (uniform): one offset register, not ROUNDS.  The
    // buffer's range check covers the vector offset only, never the scalar one, so the round's
    // rows move the base (and shrink the extent) rather than ride in the scalar offset: a row past
    // M is then past the extent and reads as zeros
    if constexpr (Q8) {
      const int64_t r0 = (int64_t)p * NW * 8;
      tile_dma(xbase + r0 * lda, (uint32_t)(max((int64_t)0, M - m0 - r0) * lda * 2), (lds_void*)dst, xoff[0], t * 128);
    } else if (p < ROUNDS) tile_dma(xbase, xext, (lds_void*)dst, xoff[p % ROUNDS], t * 128);
    else tile_dma(wbase, wext, (lds_void*)dst, woff[p % ROUNDS], t * 128);
  };
  // Q8: the tile's chunks of QT, one a k-step (QT_CHUNK bytes, every offset inside the buffer: rows
  // past N are zeros in it).  Raw round i of wave w moves 1 KB of codes, rows (i*8 + w)*16 ..
  // +15, lane l 16 bytes at 16 l of them, into the same place of the raw stage (row r at 64 r).
  // The scales of tile row tid/2, both blocks of the k-step in one dword -- a 32-bit value, so
  // that no widening of it is hoisted to the loop's head, where it would wait for the load before
  // its time
  const int64_t KT = K / 64;
  const i32x4 qrsrc = buffer_desc(QT + (int64_t)bn * KT * QT_CHUNK, Q8 ? (uint32_t)(KT * QT_CHUNK) : 0u);
  const uint32_t roff0 = (uint32_t)(wave * 1024 + lane * 16);
  const int dq_row = tid >> 1, dq_blk = tid & 1;
  const uint32_t doff = (uint32_t)(QT_SCALES + dq_row * 4);
  auto raw_dma = [&](int t, int stage, int i) {
    uint8_t* dst = smem + 131072 + stage * 16384 + (i * NW + wave) * 1024;
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(QT + (int64_t)bn * KT * QT_CHUNK), 0,
                                                                 (int)(KT * QT_CHUNK), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, roff0, t * QT_CHUNK + i * NW * 1024, 0, 0);
  };
  auto scale_load = [&](int t) -> uint32_t { return buffer_load_u32_untracked(qrsrc, doff, (uint32_t)(t * QT_CHUNK)); };
  // Q8: the thread's 32 codes of raw stage rs into bf16 W stage ws: two 16-code reads (dq_read,
  // halves 0 and 1), the block's fp16 scale from the half dq_blk of DPAIR (dq_scale), then four
  // conversions of 8 codes each, each storing its 16-byte chunk of bf16 (dq_convert).  The 16
  // lanes of a store quarter-wave (8 rows x 2 blocks) fill 16 distinct (row parity, chunk)
  // places, so the stores are free of bank conflicts (8-byte stores of half chunks met in pairs)
  u32x4 dq_q[2];
  float dq_d = 0.f;
  auto dq_read = [&](int h, int rs) { dq_q[h] = *(const u32x4*)(smem + 131072 + rs * 16384 + tid * 32 + 16 * h); };
  auto dq_scale = [&](uint32_t dpair) { dq_d = f16_to_f32((dpair >> (16 * dq_blk)) & 0xFFFFu); };
  auto dq_convert = [&](int j, int ws) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t u = dq_q[j >> 1][2 * (j & 1) + e];
      const float f0 = (float)(int8_t)(u & 0xFFu) * dq_d, f1 = (float)(int8_t)((u >> 8) & 0xFFu) * dq_d;
      const float f2 = (float)(int8_t)((u >> 16) & 0xFFu) * dq_d, f3 = (float)(int8_t)(u >> 24) * dq_d;
      o[2 * e] = pack_bf16x2(f0, f1);
      o[2 * e + 1] = pack_bf16x2(f2, f3);
    }
    const int c = (4 * dq_blk + j) ^ chunk_swz(dq_row);
    *(u32x4*)(smem + ws * 65536 + 32768 + dq_row * 128 + c * 16) = u32x4{o[0], o[1], o[2], o[3]};
  };
  auto dequant_all = [&](int rs, int ws, uint32_t dpair) {
    dq_read(0, rs);
    dq_read(1, rs);
    dq_scale(dpair);
#pragma unroll
    for (int j = 0; j < 4; ++j) dq_convert(j, ws);
  };
  // v_mfma_f32_16x16x32_bf16 operands: lane l holds row l%16, k = 8*(l/16) .. +7 of a slice of 32
  const int lo = lane & 15, q4 = lane >> 4, fs = chunk_swz(lo);
  const uint8_t* a_rd = smem + (wm * WM + lo) * 128;
  const uint8_t* b_rd = smem + 32768 + (wn * WN + lo) * 128;
  struct Frag {
    bf16x8 v[NRD];   // X fragments 0..MI-1, W fragments MI..
  };
  auto rd1 = [&](Frag& f, int stage, int kk, int q) {
    const int off = stage * 65536 + (((4 * kk + q4) ^ fs) << 4);
    if (q < MI) f.v[q] = *(const bf16x8*)(a_rd + off + q * 16 * 128);
    else f.v[q] = *(const bf16x8*)(b_rd + off + (q - MI) * 16 * 128);
  };
  f32x4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A step is 2 NMF MFMAs (two slices of 32 k) in a fixed order, with scheduling fences
  // between, so that reads, DMA and barriers never bunch up:
  //   MFMAs 0 .. NRD-1     read this step's second-slice fragments (stage cur) into F1;
  //   MFMA B1              barrier: every wave is done with stage cur, which is free;
  //   MFMAs B1 .. B1+DS-1  the DMA of step t+2 into stage cur, one part every DS/NDMA MFMAs;
  //   MFMA B2              barrier: step t+1's DMA, out since the step before, has landed;
  //   MFMAs B2 .. B2+NRD-1 read step t+1's first-slice fragments (stage cur^1) into F0.
  // The DMA then has from B1 of one step to B2 of the next to land (about 1.6 steps), and the
  // barrier before the DMA waits on no memory.
  // Q8 adds: after B1, the dequantisation of step t+2's codes (raw stage cur, landed: B1 waits
  // for them) into the freed W stage cur.  The thread's two 16-code reads go out at DQR0 and DQR1,
  // in registers of first-slice X fragments already dead, a dozen MFMAs before the first
  // conversion needs them; at DQ0 the scale's wait, then a conversion (8 codes to a 16-byte chunk
  // of bf16 in LDS) every DQS MFMAs through DQ0+3 DQS.  The step's vector memory operations: the X DMA
  // of step t+2 in four parts (XP0..XP3: at B1 and after the first conversions), then after B2 the
  // codes' DMA of step t+4 into raw stage cur (CP0, CP1; free: every wave's reads of it are behind
  // B2) and, between those, the load of step t+3's scales into the register the conversions have
  // read (SP; inside the conversions it cost 2-4% of every product).  The codes have about 1.5
  // steps to land, the scales about 0.7.  Each wait leaves out exactly the operations issued
  // after the one it waits for (ops_after, from the positions):
  //   B1 for the codes of step t+2 (issued at step t-2); DQ0 for the scales (step t-1); B2 for
  //   step t+1's X (step t-1).
  // The prologue issues the operations of the steps before kt0 in the same order, so the first
  // steps' waits count the same.  The scale load is invisible to the compiler (see
  // buffer_load_u32_untracked): DQ0's wait is what covers it.  The dequantisation's stores are
  // done (lgkmcnt 0) at the next B1, a step before anything reads them.
  constexpr int B1 = 14 * NMF / 32, B2 = 52 * NMF / 32, DSPREAD = NMF;
  constexpr int DQ0 = NMF, DQS = 4, DQR0 = B1 + 6, DQR1 = B1 + 8;
  constexpr int XP0 = B1, XP1 = DQ0 + 3, XP2 = DQ0 + 5, XP3 = DQ0 + 7, CP0 = B2 + 1, SP = B2 + 2, CP1 = B2 + 4;
  constexpr int QPOS[7] = {XP0, XP1, XP2, XP3, CP0, SP, CP1};
  constexpr int B1_VM = Q8 ? ops_after(CP1, 2, B1, QPOS, 7) : 63, B2_VM = Q8 ? ops_after(XP3, 1, B2, QPOS, 7) : NDMA,
                DQ_VM = ops_after(SP, 1, DQ0, QPOS, 7);
  // B2 lets this step's NDMA DMA parts stay outstanding, and no more: they must all be out
  static_assert(B1 >= NRD && B1 + DSPREAD <= B2 && B2 + NRD <= 2 * NMF, "step schedule");
  static_assert(!Q8 || (B1 < DQR0 && DQR0 < DQR1 && DQR1 < DQ0 && DQ0 + 3 * DQS < B2),
                "the dequantisation fits between the barriers");
  // the counts above take the codes' second part as a step's last operation, X's fourth as its
  // last X part, no operation at a wait's own position, and each wait under 16 (vmcnt's 6 bits
  // allow 63; the B1 / DQ0 / B2 order is what the schedule needs)
  static_assert(!Q8 || (XP0 < XP1 && XP1 < XP2 && XP2 < XP3 && XP3 < CP0 && CP0 < SP && SP < CP1 && CP1 < 2 * NMF &&
                        XP0 >= B1 && XP3 < B2 && SP > DQ0 && XP1 != DQ0 && B1_VM < 16 && B2_VM < 16 && DQ_VM < 16),
                "Q8 operation order");
  // Q8: the scales of the k-step the next dequantisation takes (both blocks of each tile row)
  uint32_t sc = 0;
  auto step = [&](Frag& F0, Frag& F1, int t) {
    const int cur = (t - kt0) & 1, nx = min(t + 2, kt1 - 1);
    // MFMA position x of the step: a lambda unrolled over two loops of NMF, each small
    // enough for the compiler to unroll whole (one loop of 2 NMF is past its limit once
    // anything is added to the body)
    auto pos = [&](const int x) {
      if (x == B1) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt((B1_VM & 15) | (0x7 << 4) | (0x0 << 8) | ((B1_VM >> 4) << 14));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      if (x == B2) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt((B2_VM & 15) | (0x7 << 4) | (0x0 << 8) | ((B2_VM >> 4) << 14));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      const int y = x % NMF;
      if (x < NMF)
        acc[y / NI][y % NI] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(F0.v[y / NI], F0.v[MI + y % NI], acc[y / NI][y % NI], 0, 0, 0);
      else
        acc[y / NI][y % NI] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(F1.v[y / NI], F1.v[MI + y % NI], acc[y / NI][y % NI], 0, 0, 0);
      if (x < NRD) rd1(F1, cur, 1, x);
      if (x >= B2 && x < B2 + NRD) rd1(F0, cur ^ 1, 0, x - B2);
      if constexpr (Q8) {
        static_assert(NDMA == 4, "X parts at XP0 .. XP3");
        if (x == XP0) dma_part(nx, cur, 0);
        if (x == XP1) dma_part(nx, cur, 1);
        if (x == XP2) dma_part(nx, cur, 2);
        if (x == XP3) dma_part(nx, cur, 3);
      } else if (x >= B1 && x < B1 + DSPREAD) {
#pragma unroll
        for (int p = ((x - B1) * NDMA) / DSPREAD; p < ((x - B1 + 1) * NDMA) / DSPREAD && p < NDMA; ++p)
          dma_part(nx, cur, p);
      }
      if constexpr (Q8) {
        if (x == DQR0) dq_read(0, cur);
        if (x == DQR1) dq_read(1, cur);
        if (x == DQ0) {
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_waitcnt((DQ_VM & 15) | (0x7 << 4) | (0xF << 8) | ((DQ_VM >> 4) << 14));
          // the scale load is invisible to the compiler; this marks its register as written here,
          // after the wait that covers it, so that no use of it moves above the wait
          asm volatile("" : "+v"(sc));
          dq_scale(sc);
        }
        if (x >= DQ0 && x <= DQ0 + 3 * DQS && (x - DQ0) % DQS == 0) dq_convert((x - DQ0) / DQS, cur);
        const int nq = min(t + 4, kt1 - 1);   // the codes' step
        if (x == CP0) raw_dma(nq, cur, 0);
        if (x == CP1) raw_dma(nq, cur, 1);
        // the next step's scales, into the register the conversions have read
        if (x == SP) sc = scale_load(min(t + 3, kt1 - 1));
      }
      __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int x = 0; x < NMF; ++x) pos(x);
#pragma unroll
    for (int x = NMF; x < 2 * NMF; ++x) pos(x);
  };
  Frag F0, F1;
  if constexpr (Q8) {
    // stages 0, 1 of steps kt0, kt0 + 1: codes, scales and X by DMA, then both dequantised
    const int t1 = min(kt0 + 1, kt1 - 1);
    raw_dma(kt0, 0, 0);
    raw_dma(kt0, 0, 1);
    raw_dma(t1, 1, 0);
    raw_dma(t1, 1, 1);
    uint32_t sa = scale_load(kt0), sb = scale_load(t1);
#pragma unroll
    for (int p = 0; p < NDMA; ++p) dma_part(kt0, 0, p);
    LDS_VMCNT0_BARRIER();
    asm volatile("" : "+v"(sa), "+v"(sb));   // the scales' uses stay after the wait (see DQ0)
    dequant_all(0, 0, sa);
    dequant_all(1, 1, sb);
    LDS_VMCNT0_BARRIER();   // the codes read, stages 0 and 1 of W written
    // the operations the loop's first waits count, as the steps before kt0 would have issued
    // them: step kt0 - 2's codes (of kt0 + 2), then step kt0 - 1's in position order (X of kt0 + 1,
    // the codes of kt0 + 3, the scales of kt0 + 2)
    raw_dma(min(kt0 + 2, kt1 - 1), 0, 0);
    raw_dma(min(kt0 + 2, kt1 - 1), 0, 1);
#pragma unroll
    for (int x = 0; x < 2 * NMF; ++x) {
      if (x == XP0) dma_part(t1, 1, 0);
      if (x == XP1) dma_part(t1, 1, 1);
      if (x == XP2) dma_part(t1, 1, 2);
      if (x == XP3) dma_part(t1, 1, 3);
      if (x == CP0) raw_dma(min(kt0 + 3, kt1 - 1), 1, 0);
      if (x == SP) sc = scale_load(min(kt0 + 2, kt1 - 1));
      if (x == CP1) raw_dma(min(kt0 + 3, kt1 - 1), 1, 1);
    }
#pragma unroll
    for (int q = 0; q < NRD; ++q) rd1(F0, 0, 0, q);
    for (int t = kt0; t < kt1; ++t) step(F0, F1, t);
  } else {
#pragma unroll
    for (int p = 0; p < NDMA; ++p) dma_part(kt0, 0, p);
    LDS_VMCNT0_BARRIER();
#pragma unroll
    for (int p = 0; p < NDMA; ++p) dma_part(min(kt0 + 1, kt1 - 1), 1, p);
#pragma unroll
    for (int q = 0; q < NRD; ++q) rd1(F0, 0, 0, q);
    // past the end the DMA re-reads the last step into the free stage, and nothing reads it:
    // no branch, so the order holds
    for (int t = kt0; t < kt1; ++t) step(F0, F1, t);
  }
  LDS_VMCNT0_BARRIER();   // the last DMA has landed before the epilogue takes the LDS over
  if constexpr (Q8) asm volatile("" ::"v"(sc));   // the last scale load has landed too
  if constexpr (HEADS)
    epilogue_qkv<MI, NI>(acc, (float*)smem + wave * (16 * 132), m0 + wm * WM, n0 + wn * WN, lane, M, ea);
  else if constexpr (EPI == EPI_SWIGLU)
    epilogue_swiglu<MI, NI>(acc, (uint16_t*)smem + wave * (WM * 40), m0 + wm * WM, n0 + wn * WN, lane, M, N, ea);
  else
    epilogue_lds<EPI, MI, NI>(acc, (float*)smem + wave * (32 * (WN + 8)), m0 + wm * WM, n0 + wn * WN, lane, M, N, ea);
}

// 16- and 4-byte buffer loads into V that the compiler does not see as loads (as
// buffer_load_u32_untracked), the destination tied to V's register (an in-out operand), so that
// the value keeps one register from the load to its use and no copy of it is made in between
__device__ __forceinline__ void buffer_load_u128_into(u32x4& v, i32x4 rsrc, uint32_t voff, uint32_t soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "+v"(v) : "v"(voff), "s"(rsrc), "s"(soff));
}
__device__ __forceinline__ void buffer_load_u32_into(uint32_t& v, i32x4 rsrc, uint32_t voff, uint32_t soff) {
  asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "+v"(v) : "v"(voff), "s"(rsrc), "s"(soff));
}

// The Q8_0 block products over many rows: 512 x 128 tiles, so that a tile dequantises 128 weight
// rows for 512 activation rows -- half the conversions an MFMA of k_gemm_bt's 256 x 256 tiles
// (whose exact conversion, a byte-to-float conversion, a multiply and half a pack a weight, is
// the Q8_0 path's largest cost).  8 waves of 128 x 64 (4 x 2; the QKV epilogue's 64 x 128, one
// head a wave: 8 x 1), BK = 64 in two slices of 32, the step schedule of k_gemm_bt:
//   a stage is the X tile (512 rows, 64 KB, by the LDS DMA) and the W tile (128 rows of bf16,
//   16 KB, written by the dequantisation); two stages fill the 160 KB of LDS, so the codes go to
//   registers: thread t loads the 16 codes of tile row t/4, k 16 (t%4) .. +15 (one 16-byte load,
//   a wave's 64 one contiguous KB of the tiled operand) and the dword of that row's two scales,
//   two steps ahead into one of two register sets (the step's parity: the loop runs steps in
//   pairs), and converts them into the W tile of step t+2 once B1 has freed it.
// The tiled operand's 256-row chunks hold two 128-row tiles: tile bn is chunk bn/2, rows
// 128 (bn%2) .. (codes at 8 KB (bn%2), scales at QT_SCALES + 512 (bn%2)).
// TR = 256: the products of 129 to 256 rows (a prompt's) on 256 x 128 tiles, 8 waves of 64 x 64:
// a weight row dequantised once a workgroup into LDS, where the few-row kernel's waves convert
// their own weight rows into registers twice a tile; a step of 32 MFMA positions, the same order
// of operations and the same waits counted from their positions.
template <int EPI, int TR = 512>
__global__ void __launch_bounds__(512)
k_gemm_q8_tall(const uint16_t* __restrict__ X, int64_t lda, const uint8_t* __restrict__ QT, int64_t M, int64_t N,
               int64_t K, EpiArgs ea) {
  constexpr bool HEADS = EPI == EPI_QKV;
  static_assert(TR == 512 || (TR == 256 && !HEADS), "512-row tiles, or 256-row tiles without the QKV epilogue");
  constexpr int WM = HEADS ? 64 : TR / 4, WN = HEADS ? 128 : 64, MI = WM / 16, NI = WN / 16;
  static_assert((TR / WM) * (128 / WN) == 8, "the waves tile TR x 128");
  constexpr int NMF = MI * NI, NRD = MI + NI, XPARTS = TR / 64, WOFF = TR * 128, STAGE = WOFF + 16384;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / (128 / WN), wn = wave % (128 / WN);
  // tile order: workgroups go to the 8 XCDs in turn, so XCD x takes the x-th eighth of a tile
  // order that walks 2 row tiles at a time -- its concurrent tiles share W and X in its L2
  int bm = blockIdx.y, bn = blockIdx.x;
  {
    const int gx = gridDim.x, gy = gridDim.y, G = gx * gy, b = blockIdx.y * gx + blockIdx.x;
    const int L = G % 8 == 0 ? (b % 8) * (G / 8) + b / 8 : b;
    constexpr int GM = 2;
    const int grp = L / (GM * gx), first = grp * GM, sz = min(gy - first, GM), in = L % (GM * gx);
    bm = first + in % sz;
    bn = in / sz;
  }
  const int64_t m0 = (int64_t)bm * TR, n0 = (int64_t)bn * 128;
  // split K (EPI_PART): workgroup z of gridDim.z takes k-steps kt0 .. kt1-1, cut in pairs as
  // k_gemm_bt cuts them (K % 128 == 0), so that both give the same partial sums
  const int KT = (int)(K / 64), SK = gridDim.z, zk = blockIdx.z;
  const int kt0 = 2 * (int)((int64_t)(KT / 2) * zk / SK), kt1 = 2 * (int)((int64_t)(KT / 2) * (zk + 1) / SK);
  // X DMA part p of wave w: tile rows (8p + w) 8 .. +7, lane l row +l/8, LDS chunk l%8 (global
  // chunk (l%8) ^ swizzle, the same for every part: 64 p rows keep (row/2)%8); the part's rows
  // move the buffer's base and shrink its extent (the range check covers the vector offset only)
  const uint16_t* xbase = X + m0 * lda;
  uint32_t xoff;
  {
    const int row = wave * 8 + (lane >> 3);
    xoff = (uint32_t)((row * lda + 8 * ((lane & 7) ^ chunk_swz(row))) * 2);
  }
  auto dma_part = [&](int t, int stage, int p) {
    uint8_t* dst = smem + stage * STAGE + (p * 8 + wave) * 1024;
    const int64_t r0 = (int64_t)p * 64;
    tile_dma(xbase + r0 * lda, (uint32_t)(max((int64_t)0, M - m0 - r0) * lda * 2), (lds_void*)dst, xoff, t * 128);
  };
  // the codes and scales of step t into registers (every offset inside the tile's chunks)
  const i32x4 qrsrc = buffer_desc(QT + (int64_t)(bn >> 1) * KT * QT_CHUNK, (uint32_t)((int64_t)KT * QT_CHUNK));
  const uint32_t coff = (uint32_t)((bn & 1) * 8192 + tid * 16);
  const uint32_t soff = (uint32_t)(QT_SCALES + (bn & 1) * 512 + (tid >> 2) * 4);
  const int dq_row = tid >> 2, dq_q = tid & 3;
  // two register sets, one for each step parity
  u32x4 cq0 = {0u, 0u, 0u, 0u}, cq1 = {0u, 0u, 0u, 0u};
  uint32_t sq0 = 0, sq1 = 0;
  auto code_load = [&](auto bc, int t) {
    if constexpr (decltype(bc)::value == 0) {
      buffer_load_u128_into(cq0, qrsrc, coff, (uint32_t)(t * QT_CHUNK));
      buffer_load_u32_into(sq0, qrsrc, soff, (uint32_t)(t * QT_CHUNK));
    } else {
      buffer_load_u128_into(cq1, qrsrc, coff, (uint32_t)(t * QT_CHUNK));
      buffer_load_u32_into(sq1, qrsrc, soff, (uint32_t)(t * QT_CHUNK));
    }
  };
  // conversion h (0, 1): codes 8h .. 8h+7 of the thread's 16 into the 16-byte chunk of bf16 at
  // k 16 q + 8h, one store a chunk: the 16 lanes of a store quarter-wave (4 rows x 4 quarters)
  // then fill 16 distinct (row parity, chunk) places, so the stores are free of bank conflicts
  // (8-byte stores of half chunks met in pairs and cost about 8% of the product)
  float dq_d = 0.f;
  auto dq_scale = [&](uint32_t sq) { dq_d = f16_to_f32((sq >> (16 * (dq_q >> 1))) & 0xFFFFu); };
  auto dq_convert = [&](const u32x4& cq, int h, int ws) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t u = cq[2 * h + e];
      const float f0 = (float)(int8_t)(u & 0xFFu) * dq_d, f1 = (float)(int8_t)((u >> 8) & 0xFFu) * dq_d;
      const float f2 = (float)(int8_t)((u >> 16) & 0xFFu) * dq_d, f3 = (float)(int8_t)(u >> 24) * dq_d;
      o[2 * e] = pack_bf16x2(f0, f1);
      o[2 * e + 1] = pack_bf16x2(f2, f3);
    }
    const int c = (2 * dq_q + h) ^ chunk_swz(dq_row);
    *(u32x4*)(smem + ws * STAGE + WOFF + dq_row * 128 + c * 16) = u32x4{o[0], o[1], o[2], o[3]};
  };
  // v_mfma_f32_16x16x32_bf16 operands: lane l holds row l%16, k = 8*(l/16) .. +7 of a slice of 32
  const int lo = lane & 15, q4 = lane >> 4, fs = chunk_swz(lo);
  const uint8_t* a_rd = smem + (wm * WM + lo) * 128;
  const uint8_t* b_rd = smem + WOFF + (wn * WN + lo) * 128;
  struct Frag {
    bf16x8 v[NRD];
  };
  auto rd1 = [&](Frag& f, int stage, int kk, int q) {
    const int off = stage * STAGE + (((4 * kk + q4) ^ fs) << 4);
    if (q < MI) f.v[q] = *(const bf16x8*)(a_rd + off + q * 16 * 128);
    else f.v[q] = *(const bf16x8*)(b_rd + off + (q - MI) * 16 * 128);
  };
  f32x4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // A step (k_gemm_bt's): MFMAs 0..NRD-1 read this step's second-slice fragments (stage cur);
  // B1: every wave is done with stage cur; the X DMA of step t+2 into it at XP0..XP7; at DQ0 the
  // codes' wait, then two conversions (DQ0, DQ0+4) of step t+2's codes into W stage cur;
  // at CLP the codes and scales of step t+4 into the register set just read (so they have two
  // steps to land: one was 0.7% slower, the loads waited on at DQ0); B2: step t+1's X has
  // landed (its W was written a step before, behind this step's B1); then step t+1's first-slice
  // fragments from stage cur^1.  The waits leave out what ops_after counts from the positions.
  // 512-row tiles (64 positions): X parts 0-3 at B1 + 4i, the codes at CLP, parts 4-7 after
  // them; 256-row tiles (32 positions): the 4 parts at B1 + 3i, the codes after the conversions
  constexpr bool T5 = TR == 512;
  constexpr int B1 = T5 ? 14 * NMF / 32 : 8, B2 = T5 ? 52 * NMF / 32 : 24, DQ0 = T5 ? B1 + 10 : 13,
                CLP = T5 ? DQ0 + 7 : 20, NQ = XPARTS + 2;
  constexpr int QPOS[10] = {B1,          B1 + (T5 ? 4 : 3),  B1 + (T5 ? 8 : 6),  B1 + (T5 ? 12 : 9), CLP,
                            CLP + 1,     B1 + 20,            B1 + 24,            B1 + 28,            B1 + 32};
  constexpr int XLAST = QPOS[T5 ? 9 : 3];   // the step's last X part
  constexpr int DQ_VM = ops_after(CLP + 1, 2, DQ0, QPOS, NQ), B2_VM = ops_after(XLAST, 1, B2, QPOS, NQ);
  static_assert(B1 >= NRD && XLAST < B2 && B2 + NRD <= 2 * NMF && DQ_VM < 64 && B2_VM < 64, "step schedule");
  static_assert(T5 ? (B1 + 32 < B2 && DQ0 > B1 + 8 && DQ0 + 6 < CLP && CLP + 1 < B1 + 20)
                   : (B2 == 2 * NMF - NRD && DQ0 > B1 + 3 && DQ0 + 4 < CLP && XLAST < CLP && CLP + 1 < B2 && B2 >= NMF),
                "step schedule");
  auto step = [&](Frag& F0, Frag& F1, int t, auto bc) {
    constexpr int P = decltype(bc)::value;
    u32x4& cq = P ? cq1 : cq0;
    uint32_t& sq = P ? sq1 : sq0;
    const int cur = (t - kt0) & 1, nx = min(t + 2, kt1 - 1);
    auto pos = [&](const int x) {
      if (x == B1) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt((63 & 15) | (0x7 << 4) | (0x0 << 8) | ((63 >> 4) << 14));   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      if (x == B2) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt((B2_VM & 15) | (0x7 << 4) | (0x0 << 8) | ((B2_VM >> 4) << 14));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      const int y = x % NMF;
      if (x < NMF)
        acc[y / NI][y % NI] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(F0.v[y / NI], F0.v[MI + y % NI], acc[y / NI][y % NI], 0, 0, 0);
      else
        acc[y / NI][y % NI] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(F1.v[y / NI], F1.v[MI + y % NI], acc[y / NI][y % NI], 0, 0, 0);
      if (x < NRD) rd1(F1, cur, 1, x);
      if (x >= B2 && x < B2 + NRD) rd1(F0, cur ^ 1, 0, x - B2);
#pragma unroll
      for (int p = 0; p < XPARTS; ++p)
        if (x == QPOS[p < 4 ? p : p + 2]) dma_part(nx, cur, p);
      if (x == DQ0) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt((DQ_VM & 15) | (0x7 << 4) | (0xF << 8) | ((DQ_VM >> 4) << 14));
        // the loads are invisible to the compiler; this marks their registers as written here,
        // after the wait that covers them, so that no use of them moves above the wait
        asm volatile("" : "+v"(cq), "+v"(sq));
        dq_scale(sq);
      }
      if (x == DQ0 || x == DQ0 + 4) dq_convert(cq, (x - DQ0) / 4, cur);
      if (x == CLP) code_load(bc, min(t + 4, kt1 - 1));
      __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int x = 0; x < NMF; ++x) pos(x);
#pragma unroll
    for (int x = NMF; x < 2 * NMF; ++x) pos(x);
  };
  Frag F0, F1;
  {
    // stages 0, 1: X of kt0 by DMA, the codes of kt0 and kt0 + 1 converted into both W tiles
    const int t1 = min(kt0 + 1, kt1 - 1);
#pragma unroll
    for (int p = 0; p < XPARTS; ++p) dma_part(kt0, 0, p);
    code_load(I0{}, kt0);
    LDS_VMCNT0_BARRIER();
    asm volatile("" : "+v"(cq0), "+v"(sq0));
    dq_scale(sq0);
#pragma unroll
    for (int h = 0; h < 2; ++h) dq_convert(cq0, h, 0);
    code_load(I1{}, t1);
    LDS_VMCNT0_BARRIER();
    asm volatile("" : "+v"(cq1), "+v"(sq1));
    dq_scale(sq1);
#pragma unroll
    for (int h = 0; h < 2; ++h) dq_convert(cq1, h, 1);
    // the codes of kt0 + 2 (step kt0 - 2's load) landed with the wait below; then step kt0 - 1's
    // operations in position order: X of kt0 + 1, the codes of kt0 + 3
    code_load(I0{}, min(kt0 + 2, kt1 - 1));
    LDS_VMCNT0_BARRIER();   // the codes read, stages 0 and 1 of W written, stage 0 of X landed
#pragma unroll
    for (int x = 0; x < 2 * NMF; ++x) {
#pragma unroll
      for (int p = 0; p < XPARTS; ++p)
        if (x == QPOS[p < 4 ? p : p + 2]) dma_part(t1, 1, p);
      if (x == CLP) code_load(I1{}, min(kt0 + 3, kt1 - 1));
    }
#pragma unroll
    for (int q = 0; q < NRD; ++q) rd1(F0, 0, 0, q);
  }
  for (int t = kt0; t < kt1; t += 2) {
    step(F0, F1, t, I0{});
    step(F0, F1, t + 1, I1{});
  }
  LDS_VMCNT0_BARRIER();   // the last DMA and loads have landed before the epilogue takes the LDS over
  asm volatile("" ::"v"(cq0), "v"(sq0), "v"(cq1), "v"(sq1));
  if constexpr (HEADS)
    epilogue_qkv<MI, NI>(acc, (float*)smem + wave * (16 * 132), m0 + wm * WM, n0 + wn * WN, lane, M, ea);
  else if constexpr (EPI == EPI_SWIGLU)
    epilogue_swiglu<MI, NI>(acc, (uint16_t*)smem + wave * (WM * 40), m0 + wm * WM, n0 + wn * WN, lane, M, N, ea);
  else
    epilogue_lds<EPI, MI, NI>(acc, (float*)smem + wave * (32 * (WN + 8)), m0 + wm * WM, n0 + wn * WN, lane, M, N, ea);
}

// bf16 weights WB, or (Q8) tiled Q8_0 weights QT dequantised in the pipeline
template <int EPI, bool Q8 = false>
static hipError_t launch_bt(hipStream_t s, const uint16_t* x, int64_t lda, const uint16_t* wb, int64_t M, int64_t N,
                            int64_t K, const EpiArgs& ea, int split = 1, const uint8_t* qt = nullptr) {
  const size_t shm = Q8 ? 2 * 65536 + 2 * 16384 : 2 * 65536;
  constexpr int NW = 8;
  auto kern = k_gemm_bt<EPI, NW, Q8>;
  {
    const hipError_t e = ensure_lds((const void*)kern, (int)shm);
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + 255) / 256), (unsigned)split);
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), shm, s, x, lda, wb, qt, M, N, K, ea);
  return hipGetLastError();
}

// the LDS-DMA pipeline's conditions on X and the output (16-byte chunks of X rows, 4-column
// stores, buffer extents within 31 bits) and on the weight (bf16 rows or tiled Q8_0)
static bool dma_fits(const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N, int64_t K,
                     const EpiArgs& ea) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  // tiled Q8_0: K % 128 == 0 (the kernel runs k-steps in pairs), a tile's chunks within 31 bits
  const bool wok = w.wb ? (a16(w.wb) && N * K < (int64_t)1 << 30)
                        : (w.qt && a16(w.qt) && K % 128 == 0 && (K / 64) * QT_CHUNK < (int64_t)1 << 31);
  return wok && K % 64 == 0 && lda % 8 == 0 && a16(x) && M * lda < (int64_t)1 << 30 && N % 4 == 0 &&
         ea.ldy % 4 == 0 && a16(ea.y) && a16(ea.resid) && a16(ea.gate) && ea.mstride % 4 == 0;
}

template <int EPI, int TR = 512>
static hipError_t launch_tall(hipStream_t s, const uint16_t* x, int64_t lda, const uint8_t* qt, int64_t M, int64_t N,
                              int64_t K, const EpiArgs& ea, int split) {
  const size_t shm = 2 * (TR * 128 + 16384);
  auto kern = k_gemm_q8_tall<EPI, TR>;
  {
    const hipError_t e = ensure_lds((const void*)kern, (int)shm);
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + TR - 1) / TR), (unsigned)split);
  hipLaunchKernelGGL(kern, grid, dim3(512), shm, s, x, lda, qt, M, N, K, ea);
  return hipGetLastError();
}

// Q8_0 products of at least 512 rows take the 512 x 128 tiles (half the conversions an MFMA);
// the same sums in the same order either way
template <int EPI>
static hipError_t launch_w(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                           int64_t K, const EpiArgs& ea, int split = 1) {
  if (w.wb) return launch_bt<EPI, false>(s, x, lda, w.wb, M, N, K, ea, split);
  if (M >= 512 && N % 128 == 0) return launch_tall<EPI>(s, x, lda, w.qt, M, N, K, ea, split);
  return launch_bt<EPI, true>(s, x, lda, nullptr, M, N, K, ea, split, w.qt);
}

// --- products over few rows -------------------------------------------------------------
// A product of at most 256 rows (a prompt's) reads each weight for only that many rows: the
// weights' stream and (at 256 rows) the MFMAs bound it, and the chip is covered by splitting N
// finely, not by 256 x 256 tiles with K cut 8 or 16 ways (whose fp32 partial sums then outweigh
// the weights).  Tiles of MT = 128 WMS rows x NT = 32 (8 / WMS) weight rows, 8 waves of 128 x 32
// (WMS along M, 8 / WMS along N, two a SIMD), K split over the tile's S workgroups where the
// tiles are fewer than the CUs:
//   X: the tile's MT rows x 64 k a step by the LDS DMA (buffer_load ... lds) a step ahead into
//      one of two LDS stages (rows of 128 bytes, the 16-byte chunks swizzled as k_gemm_bt's),
//      issued first in a step so that the wait for it leaves the later weight loads out; rows
//      past M read as zeros (the buffer's extent);
//   W: each wave's 32 weight rows go straight to registers, WD steps ahead: lane l takes row
//      l%16 of its fragments j = 0, 1 at k 16 (l/16) .. +15 of the step -- Q8_0: 16 codes (one
//      16-byte load from the tiled operand) and the dword of the row's two block scales; bf16: 32
//      bytes -- and makes the MFMA's B operand of them itself, a step ahead: bf16(fp32(d) q), the
//      resident expansion's value bit for bit, so bf16 and Q8_0 weights give the same sums.  A
//      wave's fragments are rows 32 wn .. +31, or with the SwiGLU epilogue the 16 gate rows and
//      their 16 up rows (gate_up interleaved by 32), so that a lane holds both of its column.
// v_mfma_f32_16x16x32_bf16 sums its 32 k in whatever order the two operands agree on: slice kk
// of a step holds, in lane l, k = 16 (l/16) + 8 kk .. +7, so that a lane's 16 codes are one load
// and lie in one Q8_0 block.  The WMS waves along M each convert a weight row's codes.
template <int EPI, int WMS, bool Q8>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_gemm_few(const uint16_t* __restrict__ X, int64_t lda, const uint16_t* __restrict__ WB,
           const uint8_t* __restrict__ QT, int64_t M, int64_t N, int64_t K, EpiArgs ea) {
  constexpr bool SWI = EPI == EPI_SWIGLU;
  constexpr int WNS = 8 / WMS, MT = 128 * WMS, NT = 32 * WNS, MI = 8, NI = 2;
  constexpr int XST = MT * 128;   // an X stage: MT rows of 64 bf16
  constexpr int XR = MT / 64;     // a thread's 16-byte loads of it
  constexpr int WD = 4;           // the weights' steps in flight
  static_assert(WMS == 1 || WMS == 2, "128 or 256 rows");
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNS, wn = wave % WNS, lo = lane & 15, q4 = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * MT, n0 = (int64_t)blockIdx.x * NT;
  // split K: workgroup z takes k-steps kt0 .. kt1-1, cut at whole groups of WD steps (K % 256 ==
  // 0), so that the main loop runs whole groups and keeps each weight set in its registers
  const int KT = (int)(K / 64), S = gridDim.z, z = blockIdx.z;
  const int kt0 = WD * (int)((int64_t)(KT / WD) * z / S), kt1 = WD * (int)((int64_t)(KT / WD) * (z + 1) / S);
  // X(t) into stage st by the LDS DMA: round i of thread t (wave w, lane l) moves 16 bytes of tile
  // row 64 i + t/8 (= 64 i + 8 w + l/8) into LDS chunk t%8 of that row, global chunk (t%8) ^
  // chunk_swz(row) (chunk_swz(64 i + t/8) = chunk_swz(t/8)): a wave's round is 1 KB at i 8192 +
  // 1024 w of the stage.  The row's offset rides in the vector offset, which the buffer's range
  // check covers, so rows past M read as zeros
  uint32_t xoff[XR];
#pragma unroll
  for (int i = 0; i < XR; ++i)
    xoff[i] = (uint32_t)(((64 * i + (tid >> 3)) * lda + 8 * ((tid & 7) ^ chunk_swz(tid >> 3))) * 2);
  const uint32_t xext = (uint32_t)(max((int64_t)0, M - m0) * lda * 2);
  auto x_dma = [&](int t, int st) {
#pragma unroll
    for (int i = 0; i < XR; ++i)
      tile_dma(X + m0 * lda, xext, (lds_void*)(smem + st * XST + i * 8192 + wave * 1024), xoff[i], t * 128);
  };
  // W: fragment j of the wave is tile rows f0 + JS j .. +15 (lane l: row + l%16)
  constexpr int JS = SWI ? 32 : 16;
  const int f0 = SWI ? 64 * (wn >> 1) + 16 * (wn & 1) : 32 * wn;
  const int wr = (int)(n0 % 256) + f0 + lo;   // Q8: the row of fragment 0 in its 256-row chunk
  const __amdgpu_buffer_rsrc_t wqs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(QT + (n0 / 256) * (int64_t)KT * QT_CHUNK), 0, Q8 ? KT * QT_CHUNK : 0, 0x00020000);
  const uint16_t* wrow = WB + (n0 + f0 + lo) * K + 16 * q4;
  u32x4 wc[WD][NI][Q8 ? 1 : 2];
  uint32_t wd[WD][NI];
  auto w_load = [&](auto sc, int t) {
    constexpr int s = decltype(sc)::value;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      if constexpr (Q8) {
        wc[s][j][0] = __builtin_amdgcn_raw_buffer_load_b128(wqs, (uint32_t)(wr * 64 + 16 * q4 + 64 * JS * j), t * QT_CHUNK, 0);
        wd[s][j] = __builtin_amdgcn_raw_buffer_load_b32(wqs, (uint32_t)(QT_SCALES + wr * 4 + 4 * JS * j), t * QT_CHUNK, 0);
      } else {
        const u32x4* p = (const u32x4*)(wrow + (int64_t)JS * j * K + t * 64);
        wc[s][j][0] = p[0];
        wc[s][j][1] = p[1];
      }
    }
  };
  // the B operands of two steps: the current one's and the next one's, converted meanwhile
  u32x4 bq[2][NI][2];
  float wsc[NI];   // the next step's block scales, a fragment each
  // piece q (0..3) of slice kk of the conversion of weight set S into bq[B]: fragment q/2, the
  // 4 codes of dword 2 kk + q%2 (the scale taken with the slice's first piece of the fragment)
  auto w_piece = [&](auto sc, auto bc, int kk, int q) {
    constexpr int s = decltype(sc)::value, b = decltype(bc)::value;
    const int j = q >> 1, e = q & 1;
    if constexpr (Q8) {
      if (kk == 0 && e == 0) wsc[j] = f16_to_f32((wd[s][j] >> (16 * (q4 >> 1))) & 0xFFFFu);
      const float d = wsc[j];
      const uint32_t u = wc[s][j][0][2 * kk + e];
      const float g0 = (float)(int8_t)(u & 0xFFu) * d, g1 = (float)(int8_t)((u >> 8) & 0xFFu) * d;
      const float g2 = (float)(int8_t)((u >> 16) & 0xFFu) * d, g3 = (float)(int8_t)(u >> 24) * d;
      bq[b][j][kk][2 * e] = pack_bf16x2(g0, g1);
      bq[b][j][kk][2 * e + 1] = pack_bf16x2(g2, g3);
    } else {
      bq[b][j][kk][2 * e] = wc[s][j][kk][2 * e];
      bq[b][j][kk][2 * e + 1] = wc[s][j][kk][2 * e + 1];
    }
  };
  f32x4 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fs = chunk_swz(lo);   // chunk_swz of the wave's fragment rows 16 i + l%16
  // X's fragments of slice kk: row 16 i + l%16 of the wave's 128 (i < MI), 16 bytes a lane
  bf16x8 af[MI];
  auto a_read = [&](int st, int kk, int i) {
    af[i] = *(const bf16x8*)(smem + st * XST + (wm * 128 + lo) * 128 + (((2 * q4 + kk) ^ fs) << 4) + i * 16 * 128);
  };
  // slice kk's MFMAs from bq[B], row by row, each row followed by its share of the other work (the
  // next slice's fragment i read, a piece of the next step's conversion into bq[NB]), fenced so
  // that the compiler keeps the order and with it the registers' lifetimes short
  auto mfma_slice = [&](auto bc, auto sc, auto nbc, int kk, int st) {
    constexpr int b = decltype(bc)::value;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int j = 0; j < NI; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], __builtin_bit_cast(bf16x8, bq[b][j][kk]), acc[i][j], 0, 0, 0);
      if (kk == 0) a_read(st, 1, i);
      if (i % 2 == 1) w_piece(sc, nbc, kk, i / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // step t (W(t) in register set t%4, its B operands in bq[t%2]): the wait for X(t)'s DMA and
  // the barrier (X(t) in its stage for every wave, the other stage free), X(t + 1)'s DMA into
  // that stage, W(t + 4) loaded into set t%4, X(t)'s fragments read, the MFMAs with W(t + 1)
  // converted between them.  The order is for the in-order wait counter: the wait for X(t)
  // leaves step t - 1's weight loads outstanding and forces only W(t + 2) and before.  Past the
  // end the loads repeat the last step and nothing reads them.
  auto step = [&](auto uc, int t) {
    constexpr int u = decltype(uc)::value;
    using Cur = std::integral_constant<int, u % 2>;
    using Nb = std::integral_constant<int, (u + 1) % 2>;
    using Ns = std::integral_constant<int, (u + 1) % WD>;
    // X(t)'s DMA (issued at step t - 1's start) has landed: only step t - 1's 4 weight loads
    // may be outstanding; then the barrier makes every wave's DMA visible
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((4 & 15) | (0x7 << 4) | (0xF << 8));
    __syncthreads();
    const int st = (t - kt0) & 1;
    x_dma(min(t + 1, kt1 - 1), st ^ 1);
    __builtin_amdgcn_sched_barrier(0);   // the DMA before the weight loads: the wait above counts on it
    w_load(uc, min(t + WD, kt1 - 1));
#pragma unroll
    for (int i = 0; i < MI; ++i) a_read(st, 0, i);
    mfma_slice(Cur{}, Ns{}, Nb{}, 0, st);
    mfma_slice(Cur{}, Ns{}, Nb{}, 1, st);
  };
  x_dma(kt0, 0);
  w_load(I0{}, kt0);
  w_load(I1{}, min(kt0 + 1, kt1 - 1));
  w_load(I2{}, min(kt0 + 2, kt1 - 1));
  w_load(I3{}, min(kt0 + 3, kt1 - 1));
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int q = 0; q < 4; ++q) w_piece(I0{}, I0{}, kk, q);
  static_assert(WD == 4, "a loop round is the four steps of the weight sets");
  for (int t = kt0; t < kt1; t += WD) {
    step(I0{}, t);
    step(I1{}, t + 1);
    step(I2{}, t + 2);
    step(I3{}, t + 3);
  }
  // every DMA landed (the last step's spare one too) and every wave done with the stages before
  // the epilogue takes the LDS
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));
  __syncthreads();
  const int64_t wrow0 = m0 + wm * 128;
  if constexpr (SWI) {
    // output column n0/2 + 32 (wn/2) + 16 (wn%2) + l%16 (gate row 64 (wn/2) + 16 (wn%2) + l%16 of
    // the tile is output column 32 (wn/2) + 16 (wn%2) + l%16) from gate fragment 0 and up fragment
    // 1: silu(gate) x up into bf16, through the wave's LDS block (128 rows of 16) so that each lane
    // stores 16-byte runs of 8 columns
    uint16_t* stg = (uint16_t*)smem + wave * (128 * 24);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float o = silu_bf16out(acc[i][0][r]) * acc[i][1][r];
        stg[(16 * i + 4 * q4 + r) * 24 + lo] = (uint16_t)(pack_bf16x2(o, 0.f) & 0xFFFF);
      }
    const int64_t col = n0 / 2 + 32 * (wn >> 1) + 16 * (wn & 1) + 8 * (lane & 1);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = 32 * it + (lane >> 1);
      const int64_t m = wrow0 + row;
      const u32x4 v = *(const u32x4*)(stg + row * 24 + 8 * (lane & 1));
      if (m < M) *(u32x4*)((uint16_t*)ea.y + m * ea.ldy + col) = v;
    }
  } else {
    epilogue_lds<EPI, MI, NI>(acc, (float*)smem + wave * (32 * 40), wrow0, n0 + f0, lane, M, N, ea);
  }
}

// the few-row kernel's conditions: at most 256 rows, whole tiles of N, 16-byte chunks of X and
// of the weights, 31-bit buffer extents
static bool few_fits(const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N, int64_t K,
                     const EpiArgs& ea) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const int64_t NT = M > 128 ? 128 : 256;
  const bool wok = w.wb ? a16(w.wb) : (w.qt && a16(w.qt) && (K / 64) * QT_CHUNK < ((int64_t)1 << 31));
  return M > 0 && M <= 256 && N % NT == 0 && K % 256 == 0 && wok && lda % 8 == 0 && a16(x) && 256 * lda < ((int64_t)1 << 30) &&
         ea.ldy % 4 == 0 && a16(ea.y) && a16(ea.resid) && a16(ea.gate) && ea.mstride % 4 == 0;
}

template <int EPI, bool Q8>
static hipError_t launch_few(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                             int64_t K, const EpiArgs& ea, int S) {
  const bool two = M > 128;
  auto kern = two ? k_gemm_few<EPI, 2, Q8> : k_gemm_few<EPI, 1, Q8>;
  // two X stages (64 or 32 KB), at least the epilogues' 48 KB (SwiGLU) and 40 KB
  const int shm = two ? 2 * 256 * 128 : 49152;
  const hipError_t e = ensure_lds((const void*)kern, shm);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)(N / (two ? 128 : 256)), 1, (unsigned)S);
  hipLaunchKernelGGL(kern, grid, dim3(512), shm, s, x, lda, w.wb, w.qt, M, N, K, ea);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_few_w(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                               int64_t K, const EpiArgs& ea, int S) {
  return w.wb ? launch_few<EPI, false>(s, x, lda, w, M, N, K, ea, S) : launch_few<EPI, true>(s, x, lda, w, M, N, K, ea, S);
}

// a few-row product with K whole (no partial sums), through epilogue EPI
static hipError_t few_direct(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                             int64_t K, Epi epi, const EpiArgs& ea) {
  switch (epi) {
    case EPI_F32: return launch_few_w<EPI_F32>(s, x, lda, w, M, N, K, ea, 1);
    case EPI_BF16: return launch_few_w<EPI_BF16>(s, x, lda, w, M, N, K, ea, 1);
    case EPI_GATE_ADD: return launch_few_w<EPI_GATE_ADD>(s, x, lda, w, M, N, K, ea, 1);
    case EPI_SWIGLU: return launch_few_w<EPI_SWIGLU>(s, x, lda, w, M, N, K, ea, 1);
    case EPI_GELU_BF16: return launch_few_w<EPI_GELU_BF16>(s, x, lda, w, M, N, K, ea, 1);
    case EPI_F16: return launch_few_w<EPI_F16>(s, x, lda, w, M, N, K, ea, 1);
    default: return hipErrorInvalidValue;
  }
}

// Q8_0 products of 129 to 256 rows: the tall kernel's 256 x 128 tiles, each weight row dequantised
// once a workgroup (the few-row kernel's waves convert theirs twice), where a workgroup's share of
// K (K / S) is at least 768: gate_up 67.8 -> 60.5 us at 256 rows, q | k | v 46.3 -> 43.0; with
// fewer k-steps its prologue outweighs that (to_out split 8 ways, 8 steps: 25.9 -> 26.7 us)
static bool tall256_fits(const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N, int64_t K, int64_t S,
                         const EpiArgs& ea) {
  return !w.wb && w.qt && M > 128 && M <= 256 && N % 128 == 0 && K / S >= 768 && dma_fits(x, lda, w, M, N, K, ea);
}

static hipError_t tall256(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                          int64_t K, Epi epi, const EpiArgs& ea, int S) {
  switch (epi) {
    case EPI_F32: return launch_tall<EPI_F32, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_BF16: return launch_tall<EPI_BF16, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_GATE_ADD: return launch_tall<EPI_GATE_ADD, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_SWIGLU: return launch_tall<EPI_SWIGLU, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_GELU_BF16: return launch_tall<EPI_GELU_BF16, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_F16: return launch_tall<EPI_F16, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    case EPI_PART: return launch_tall<EPI_PART, 256>(s, x, lda, w.qt, M, N, K, ea, S);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gemm_q8(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N, int64_t K,
                   Epi epi, const EpiArgs& ea) {
  if (tall256_fits(x, lda, w, M, N, K, 1, ea)) return tall256(s, x, lda, w, M, N, K, epi, ea, 1);
  if (few_fits(x, lda, w, M, N, K, ea)) return few_direct(s, x, lda, w, M, N, K, epi, ea);
  if (!dma_fits(x, lda, w, M, N, K, ea)) return dispatch<false>(s, x, lda, w.qs, w.qd, nullptr, M, N, K, epi, ea);
  switch (epi) {
    case EPI_F32: return launch_w<EPI_F32>(s, x, lda, w, M, N, K, ea);
    case EPI_BF16: return launch_w<EPI_BF16>(s, x, lda, w, M, N, K, ea);
    case EPI_GATE_ADD: return launch_w<EPI_GATE_ADD>(s, x, lda, w, M, N, K, ea);
    case EPI_SWIGLU: return launch_w<EPI_SWIGLU>(s, x, lda, w, M, N, K, ea);
    case EPI_GELU_BF16: return launch_w<EPI_GELU_BF16>(s, x, lda, w, M, N, K, ea);
    case EPI_F16: return launch_w<EPI_F16>(s, x, lda, w, M, N, K, ea);
    default: return hipErrorInvalidValue;
  }
}

// the S partial sums of a split product in order, through the epilogue: 4 output columns a
// thread (SwiGLU: 4 output columns from their gate and up columns, interleaved by 32)
template <int EPI>
__global__ void __launch_bounds__(256)
k_split_sum(int S, int64_t M, int64_t N, const float* __restrict__ part, EpiArgs ea) {
  constexpr int OC = EPI == EPI_SWIGLU ? 2 : 1;   // input columns an output column takes
  const int64_t NO = N / OC, i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * NO / 4) return;
  const int64_t m = i / (NO / 4), c = (i % (NO / 4)) * 4;   // output row, first output column
  auto sum = [&](int64_t col) {
    f32x4 v = *(const f32x4*)(part + m * N + col);
    for (int z = 1; z < S; ++z) v += *(const f32x4*)(part + ((int64_t)z * M + m) * N + col);
    return v;
  };
  if constexpr (EPI == EPI_SWIGLU) {
    const int64_t gc = 64 * (c >> 5) + (c & 31);   // the gate column of output column c; up is 32 on
    const f32x4 v = sum(gc), u = sum(gc + 32);
    *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + c) =
        u32x2{pack_bf16x2(silu_bf16out(v[0]) * u[0], silu_bf16out(v[1]) * u[1]),
              pack_bf16x2(silu_bf16out(v[2]) * u[2], silu_bf16out(v[3]) * u[3])};
  } else {
    const f32x4 v = sum(c);
    if constexpr (EPI == EPI_GATE_ADD) {
      const float* gr = ea.gate + (ea.n0 + m < ea.p ? ea.mstride : 0) + c;
      f32x4* x = (f32x4*)(ea.resid + m * ea.ldy + c);
      f32x4 xv = *x;
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[e] = xv[e] + tanh_f(gr[e]) * v[e];
      *x = xv;
    } else if constexpr (EPI == EPI_F32) {
      *(f32x4*)((float*)ea.y + m * ea.ldy + c) = v;
    } else if constexpr (EPI == EPI_BF16) {
      *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + c) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else if constexpr (EPI == EPI_F16) {
      *(u32x2*)((uint16_t*)ea.y + m * ea.ldy + c) = u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
    }
  }
}

// the S partial sums in PART (S x M x N floats) added in order through the epilogue EPI
static hipError_t split_sum(hipStream_t s, Epi epi, int S, int64_t M, int64_t N, const float* part, const EpiArgs& ea) {
  const int64_t threads = M * (epi == EPI_SWIGLU ? N / 2 : N) / 4;
  const dim3 g((unsigned)((threads + 255) / 256));
  switch (epi) {
    case EPI_GATE_ADD: hipLaunchKernelGGL(k_split_sum<EPI_GATE_ADD>, g, dim3(256), 0, s, (int)S, M, N, part, ea); break;
    case EPI_SWIGLU: hipLaunchKernelGGL(k_split_sum<EPI_SWIGLU>, g, dim3(256), 0, s, (int)S, M, N, part, ea); break;
    case EPI_F32: hipLaunchKernelGGL(k_split_sum<EPI_F32>, g, dim3(256), 0, s, (int)S, M, N, part, ea); break;
    case EPI_BF16: hipLaunchKernelGGL(k_split_sum<EPI_BF16>, g, dim3(256), 0, s, (int)S, M, N, part, ea); break;
    default: hipLaunchKernelGGL(k_split_sum<EPI_F16>, g, dim3(256), 0, s, (int)S, M, N, part, ea); break;
  }
  return hipGetLastError();
}

hipError_t gemm_split_rows(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t N,
                           int64_t K, Epi epi, const EpiArgs& ea, float* part, int64_t part_cap, int smax, int* nsum) {
  if (nsum) *nsum = 0;
  if (M == 0) return hipSuccess;
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool epi_ok = epi == EPI_GATE_ADD || epi == EPI_SWIGLU || epi == EPI_F32 || epi == EPI_BF16 || epi == EPI_F16;
  if (!epi_ok) return hipErrorNotSupported;
  if (few_fits(x, lda, w, M, N, K, ea) && a16(part)) {
    // at most 256 rows: the few-row tiles, K split so that the tiles' workgroups are about one a
    // CU, each at least 4 k-steps, at most SMAX ways and within PART_CAP
    const int64_t tiles = N / (M > 128 ? 128 : 256);
    int64_t S = 256 / tiles;
    if (S > K / 256) S = K / 256;
    if (S > smax) S = smax;
    if (S > part_cap / (M * N)) S = part_cap / (M * N);
    EpiArgs pa{};
    pa.y = part;
    pa.ldy = N;
    if (S <= 1)
      return tall256_fits(x, lda, w, M, N, K, 1, ea) ? tall256(s, x, lda, w, M, N, K, epi, ea, 1)
                                                     : few_direct(s, x, lda, w, M, N, K, epi, ea);
    const hipError_t e = tall256_fits(x, lda, w, M, N, K, S, pa)
                             ? tall256(s, x, lda, w, M, N, K, EPI_PART, pa, (int)S)
                             : launch_few_w<EPI_PART>(s, x, lda, w, M, N, K, pa, (int)S);
    if (e != hipSuccess) return e;
    if (nsum) {
      *nsum = (int)S;
      return hipSuccess;
    }
    return split_sum(s, epi, (int)S, M, N, part, ea);
  }
  // S workgroups a tile, about one wave in all, at least 4 k-steps each, at most SMAX (in a DiT
  // pass, past 8 the partial sums' traffic, S x M x N fp32 written and read back, outweighs the
  // wider spread: 256 prompt rows through to_out and down, 0.2 ms less a pass than at 16, 0.9 ms
  // less than at 4), and no more than PART_CAP holds
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  int64_t S = 256 / tiles;
  if (S > K / 64 / 4) S = K / 64 / 4;
  if (S > smax) S = smax;
  if (S > part_cap / (M * N)) S = part_cap / (M * N);
  if (S < 1) S = 1;
  EpiArgs pa{};
  pa.y = part;
  pa.ldy = N;
  const bool ok = N % 256 == 0 && a16(part) && S * M * N <= part_cap && dma_fits(x, lda, w, M, N, K, pa);
  if (!ok) return hipErrorNotSupported;
  hipError_t e = launch_w<EPI_PART>(s, x, lda, w, M, N, K, pa, (int)S);
  if (e != hipSuccess) return e;
  if (nsum) {
    *nsum = (int)S;
    return hipSuccess;
  }
  return split_sum(s, epi, (int)S, M, N, part, ea);
}

hipError_t gemm_qkv(hipStream_t s, const uint16_t* x, int64_t lda, const WOp& w, int64_t M, int64_t K,
                    const EpiArgs& ea) {
  const int64_t N = 3 * EXN_W;
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  // the DMA path's conditions, and 16-byte rows of q, k, V^T, the norm weights and the cos/sin table
  EpiArgs pa{};
  pa.ldy = 4;
  const bool ok = dma_fits(x, lda, w, M, N, K, pa) && a16(ea.q) && a16(ea.kc) && a16(ea.vt) && a16(ea.wq) &&
                  a16(ea.wk) && a16(ea.cs) && ea.lcap % 64 == 0 && ea.n0 >= 0 && ea.n0 + M <= ea.lcap;
  if (!ok) return hipErrorNotSupported;
  if (M == 0) return hipSuccess;
  return launch_w<EPI_QKV>(s, x, lda, w, M, N, K, ea);
}

hipError_t gemm_wbf16(hipStream_t s, const uint16_t* x, int64_t lda, const uint16_t* w, int64_t M, int64_t N,
                      int64_t K, Epi epi, const EpiArgs& ea) {
  const WOp wo{w, nullptr, nullptr, nullptr};
  if (few_fits(x, lda, wo, M, N, K, ea)) return few_direct(s, x, lda, wo, M, N, K, epi, ea);
  if (!dma_fits(x, lda, wo, M, N, K, ea)) return dispatch<true>(s, x, lda, nullptr, nullptr, w, M, N, K, epi, ea);
  switch (epi) {
    case EPI_F32: return launch_w<EPI_F32>(s, x, lda, wo, M, N, K, ea);
    case EPI_BF16: return launch_w<EPI_BF16>(s, x, lda, wo, M, N, K, ea);
    case EPI_GATE_ADD: return launch_w<EPI_GATE_ADD>(s, x, lda, wo, M, N, K, ea);
    case EPI_SWIGLU: return launch_w<EPI_SWIGLU>(s, x, lda, wo, M, N, K, ea);
    case EPI_GELU_BF16: return launch_w<EPI_GELU_BF16>(s, x, lda, wo, M, N, K, ea);
    case EPI_F16: return launch_w<EPI_F16>(s, x, lda, wo, M, N, K, ea);
    default: return hipErrorInvalidValue;
  }
}

// --- the edge products in fp32 -------------------------------------------------------
// img_in, txt_in and proj_out feed the residual stream and the velocity straight,
// and are 0.01% of a step's FLOPs: they run in fp32, the weights as they are stored --
// fp32 rows (the reference's d41_mm_f32, src/cuda-dit.lisp:127-130), bf16 rows, or
// Q8_0 dequantised exactly -- on v_mfma_f32_16x16x4_f32.  64 x 64 tiles, K 32 (a
// Q8_0 block) a step staged k-major in LDS as fp32; 4 waves of 32 x 32, each 2 x 2
// MFMA blocks (A: lane l holds row l % 16 at k l / 16, B: column l % 16 at k l / 16;
// D: lane l holds column l % 16, rows 4 (l / 16) + e), every k summed once.
__global__ void __launch_bounds__(256)
k_gemm_f32(const float* __restrict__ X, int64_t ldx, const int8_t* __restrict__ QS, const uint16_t* __restrict__ D,
           const uint16_t* __restrict__ WB, const float* __restrict__ WF, int64_t M, int64_t N, int64_t K,
           float* __restrict__ Y, int64_t ldy, int gelu) {
  __shared__ float xs[32][64 + 1];
  __shared__ float ws[32][64 + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32, c16 = lane & 15, g = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const int lr = tid >> 2, lk = (tid & 3) * 8;   // loader: row lr of the tile, k lk .. lk+7
  // split K: workgroup z of gridDim.z takes blocks of 32 kb0 .. kb1-1 and writes its raw sums
  // to Y + z M ldy (gelu then applies after the sum)
  const int64_t KB = K / 32, kb0 = KB * blockIdx.z / gridDim.z, kb1 = KB * (blockIdx.z + 1) / gridDim.z;
  if (gridDim.z > 1) Y += (int64_t)blockIdx.z * M * ldy;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 32 * kb0; k0 < 32 * kb1; k0 += 32) {
    {
      const int64_t m = min(m0 + lr, M - 1);
      const f32x4* src = (const f32x4*)(X + m * ldx + k0 + lk);
      const f32x4 a = src[0], b = src[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xs[lk + e][lr] = a[e];
        xs[lk + 4 + e][lr] = b[e];
      }
      const int64_t n = min(n0 + lr, N - 1);
      if (WF) {
        const f32x4* w = (const f32x4*)(WF + n * K + k0 + lk);
        const f32x4 w0 = w[0], w1 = w[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ws[lk + e][lr] = w0[e];
          ws[lk + 4 + e][lr] = w1[e];
        }
      } else if (WB) {
        const u32x4 w = *(const u32x4*)(WB + n * K + k0 + lk);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ws[lk + 2 * e][lr] = bf16_lo(w[e]);
          ws[lk + 2 * e + 1][lr] = bf16_hi(w[e]);
        }
      } else {
        const u32x2 q = *(const u32x2*)(QS + n * K + k0 + lk);
        const float dv = f16_to_f32(D[n * (K / 32) + k0 / 32]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ws[lk + e][lr] = (float)(int8_t)((q[e / 4] >> (8 * (e % 4))) & 0xFF) * dv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 32; kk += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = xs[kk + g][wm + 16 * i + c16];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = ws[kk + g][wn + 16 * j + c16];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn + 16 * j + c16;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm + 16 * i + 4 * g + e;
        if (m < M) Y[m * ldy + n] = gelu && gridDim.z == 1 ? gelu_tanh_f(acc[i][j][e]) : acc[i][j][e];
      }
    }
}

// Y = the S partial sums of a split edge product in order (M x N, ldy apart), GELU-tanh when asked
__global__ void __launch_bounds__(256)
k_f32_part_sum(int S, int64_t M, int64_t N, const float* __restrict__ part, float* __restrict__ Y, int64_t ldy,
               int gelu) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i - m * N;
  float v = part[i];
  for (int z = 1; z < S; ++z) v += part[(int64_t)z * M * N + i];
  Y[m * ldy + n] = gelu ? gelu_tanh_f(v) : v;
}

hipError_t gemm_f32(hipStream_t s, const float* x, int64_t ldx, const int8_t* qs, const uint16_t* d,
                    const uint16_t* wbf16, const float* wf32, int64_t M, int64_t N, int64_t K, float* y, int64_t ldy,
                    int gelu, float* part, int64_t part_cap) {
  if (K % 32 || M <= 0) return M == 0 ? hipSuccess : hipErrorInvalidValue;
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  // few tiles over a long K (proj_out: 64 tiles of 64 x 64 over 4096; txt_in over 256 prompt
  // rows: 256 tiles): K split over up to 16 workgroups a tile, about 1024 in all (four a CU: one
  // a CU leaves the loads' latency bare), at least 8 blocks of 32 each and no more than PART_CAP
  // holds, their sums added in order after
  const int64_t tiles = (int64_t)grid.x * grid.y;
  int64_t S = tiles < 512 ? 1024 / tiles : 1;
  if (S > 16) S = 16;
  if (S > K / 256) S = K / 256;
  if (part && S > part_cap / (M * N)) S = part_cap / (M * N);
  if (S >= 2 && part) {
    grid.z = (unsigned)S;
    hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, s, x, ldx, qs, d, wbf16, wf32, M, N, K, part, N, gelu);
    hipLaunchKernelGGL(k_f32_part_sum, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, s, (int)S, M, N, part, y,
                       ldy, gelu);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, s, x, ldx, qs, d, wbf16, wf32, M, N, K, y, ldy, gelu);
  return hipGetLastError();
}

// --- small M: a wave per output column, fp32 activations and sums ---------------------

__global__ void __launch_bounds__(256)
k_gemv(const float* __restrict__ X, int64_t ldx, const int8_t* __restrict__ QS, const uint16_t* __restrict__ D,
       const uint16_t* __restrict__ WB, const float* __restrict__ WF, int M, int64_t N, int64_t K,
       float* __restrict__ Y, int64_t ldy, int silu) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t c = lane; c < K / 16; c += 64) {
    const int64_t k = 16 * c;
    float w[16];
    if (WF) {
      const f32x4* src = (const f32x4*)(WF + n * K + k);
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const f32x4 v = src[e4];
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * e4 + e] = v[e];
      }
    } else if (WB) {
      const u32x4* src = (const u32x4*)(WB + n * K + k);
      const u32x4 a = src[0], b = src[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w[2 * e] = bf16_lo(a[e]); w[2 * e + 1] = bf16_hi(a[e]);
        w[8 + 2 * e] = bf16_lo(b[e]); w[8 + 2 * e + 1] = bf16_hi(b[e]);
      }
    } else {
      const u32x4 q = *(const u32x4*)(QS + n * K + k);
      const float dv = f16_to_f32(D[n * (K / 32) + k / 32]);
#pragma unroll
      for (int e = 0; e < 16; ++e) w[e] = (float)(int8_t)((q[e / 4] >> (8 * (e % 4))) & 0xFF) * dv;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < M) {
        const f32x4* xs = (const f32x4*)(X + m * ldx + k);
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const f32x4 xv = xs[e4];
          acc[m] = fmaf(w[4 * e4], xv[0], acc[m]);
          acc[m] = fmaf(w[4 * e4 + 1], xv[1], acc[m]);
          acc[m] = fmaf(w[4 * e4 + 2], xv[2], acc[m]);
          acc[m] = fmaf(w[4 * e4 + 3], xv[3], acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m < M) {
      const float v = wave_sum(acc[m]);
      if (lane == 0) Y[m * ldy + n] = silu ? silu_f(v) : v;
    }
  }
}

hipError_t gemv_q8(hipStream_t s, const float* x, int64_t ldx, const int8_t* qs, const uint16_t* d,
                   const uint16_t* wbf16, const float* wf32, int64_t M, int64_t N, int64_t K, float* y, int64_t ldy,
                   int silu) {
  if (M > 4 || K % 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gemv, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, s, x, ldx, qs, d, wbf16, wf32, (int)M, N, K,
                     y, ldy, silu);
  return hipGetLastError();
}

}  // namespace exn
