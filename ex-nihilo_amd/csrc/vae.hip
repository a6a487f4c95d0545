// vae.hip -- the VAE decoder's kernels on gfx950 (Qwen-Image-2.1's decoder,
// Wan 2.2's, on one frame): replaces src/cuda/vae.cu and the products and
// norms src/cuda-vae.lisp:94-136 takes from illatio.
//
// Activations are channels last: a picture of H x W pixels is H*W rows of C
// values, fp32 between blocks (the residual stream and the convolutions'
// outputs), bf16 where they feed a product.
//
// Convolutions (3 x 3 'same', and 1 x 1) are implicit products on the bf16
// MFMA, Y[pixel][o] = sum over k of A[pixel][k] Wt[o][k] with k = tap * C + c:
// the A tile is gathered straight from the input picture by LDS-DMA (buffer
// loads to LDS), each lane's 16 bytes (8 channels of one tap) from its
// pixel's neighbour, taps off the picture and K past 9C as out-of-range
// offsets, which the buffer load reads as zeros.  With UP the input is the
// half-size picture and the neighbour's pixel is halved: the nearest x2
// upsampling (x_up2) folded into the resample convolution's loads.
//
// Tiles: 256 pixels x 288 output channels a workgroup where 288 divides the
// width (1152, 576, 288), else 256 x 144 (144 divides every width of the
// decoder); 8 waves of 144 channels each, v_mfma_f32_16x16x32_bf16; K 64 a
// step, two LDS stages (72 KB each) at 288, three (50 KB each) at 144.  The
// epilogue stages each wave's accumulators through LDS 32 pixels at a time,
// so that bias, residual, DupUp3D and clamp are applied to 16-byte rows.
#include "exn_common.h"

namespace exn {

typedef __attribute__((address_space(3))) void lds_void;

static inline unsigned grid_of(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

// one 16-byte DMA lane; a byte offset at or past EXTENT reads as zeros
__device__ __forceinline__ void conv_dma(const void* base, uint32_t extent, lds_void* dst, uint32_t voff, int soff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

#define VOFF_NONE 0x80000000u   // past any extent: the load reads zeros

// Tiles of TM = 32 NW pixels x BN output channels, NW waves: BN = 144 (3 LDS stages), 288 (2
// stages; the widths that 288 divides), 96 (3 stages) and 192 (2 stages; the encoder's 96 ..
// 768) or 16 (3 stages; the head's 4 channels), NW 8 (256 pixels); or NW 4 (128 pixels, 2
// stages, under 80 KB of LDS so that two workgroups share a CU and one's epilogue runs under the
// other's products) at BN 96 and 144 on large pictures.  Waves of WM pixels x WNC channels (WNC
// = 144 where 144 divides BN, 96 where 96 does, else BN), each a (WM/16) x (WNC/16) grid of
// v_mfma_f32_16x16x32_bf16 -- 0.61 fragment reads an MFMA at BN 144, 0.36 at BN 288, 0.42 at
// BN 192.
template <int BN, int NW = 8>
struct ConvTile {
  static constexpr int WNC = BN % 144 == 0 ? 144 : BN % 96 == 0 ? 96 : BN, NJ = WNC / 16;
  static constexpr int NWN = BN / WNC, NWM = NW / NWN, TM = 32 * NW, WM = TM / NWM, MI = WM / 16;
  static constexpr int LS = WNC + 4, RC = WNC / 4, NCH = 32 * RC / 64;   // staging: row floats, chunks a row, a lane
  static constexpr int ABYTES = TM * 128;              // the A rows of a stage
  static constexpr int STAGE = ABYTES + BN * 128;      // A rows | B rows, 64 bf16 of K each
  static constexpr int NST = NW == 4 ? 2 : BN <= 144 ? 3 : 2;
  static constexpr int BFULL = BN * 8 / (64 * NW);     // full B DMA rounds a step
  static constexpr int BREM = (BN * 8 - 64 * NW * BFULL) / NW;   // lanes a wave in the partial round
  static constexpr int NDMA = 4 + BFULL + (BREM > 0);  // DMA instructions a wave a step
  static constexpr int EPI = NW * 32 * 148 * 4;        // the epilogue's staging: 32 pixels x 148 floats a wave
  static constexpr int LDS = NST * STAGE > EPI ? NST * STAGE : EPI;
  static_assert(BREM % 8 == 0 && BREM <= 64 && (NW == 8 || LDS <= 80 * 1024), "tile layout");
};

// UP: 0 a 'same' convolution of an H x W picture; 1 the same of the picture nearest-upsampled
// from H/2 x W/2 (the input); 2 stride 2 over a 2H x 2W input, padded with zeros below and to
// the right (src/cuda/vae.cu's x_conv3s2: output pixel (y, x) takes input rows 2y .. 2y + 2).
// OUT: VAE_F32 fp32 (+ bias, + res when given), VAE_BF16 bf16 (+ bias, + res when given),
// VAE_CLAMP fp32 (+ bias) clamped to -1 .. 1, VAE_DUPUP fp32 (+ bias, + DupUp3D of keep),
// VAE_PART the fp32 sums of k-steps kt0 .. kt1-1 only (workgroup z of a split K) into z's slice,
// VAE_RMS none (yr only).  GAM: the tile holds every output channel, and ep.yr gets
// silu(rms(output) x ep.gamma) in bf16.
template <int BN, int TAPS, int UP, int OUT, int GAM, int NW = 8>
__global__ void __launch_bounds__(NW * 64, NW == 4 ? 2 : 1)   // 4 waves: two workgroups a CU, 256 registers a lane
k_conv(const uint16_t* __restrict__ X, const uint16_t* __restrict__ Wt, const float* __restrict__ bias,
       VaeEpi ep, void* __restrict__ Y, int H, int W, int C, int cout, int Kp) {
  typedef ConvTile<BN, NW> T;
  extern __shared__ __align__(1024) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % T::NWM, wn = wave / T::NWM;
  const int P = H * W;
  const int m0 = blockIdx.x * T::TM, n0 = blockIdx.y * BN;
  // split K (VAE_PART): workgroup z of gridDim.z takes k-steps kt0 .. kt1-1
  const int KTT = Kp / 64, S = gridDim.z, z = blockIdx.z;
  const int kt0 = (int)((int64_t)KTT * z / S), kt1 = (int)((int64_t)KTT * (z + 1) / S);
  const int Hs = UP == 1 ? H >> 1 : UP == 2 ? 2 * H : H, Ws = UP == 1 ? W >> 1 : UP == 2 ? 2 * W : W;
  const uint32_t xext = (uint32_t)((int64_t)Hs * Ws * C * 2);
  const uint16_t* wbase = Wt + (int64_t)n0 * Kp;
  const uint32_t wext = (uint32_t)((int64_t)max(0, cout - n0) * Kp * 2);

  // A: round i moves tile rows (8i + wave) * 8 + lane / 8; LDS chunk lane % 8 of a row holds
  // K chunk (lane % 8) ^ swizzle(row).  The chunk's tap and channel move 64 K a step.
  int py[4], px[4], cc[4], tp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (NW * i + wave) * 8 + (lane >> 3);
    const int m = m0 + r;
    const int y = m / W;
    py[i] = m < P ? y : -0x40000000;   // a row past the picture: every neighbour off it
    px[i] = m - y * W;
    const int k = 64 * kt0 + 8 * ((lane & 7) ^ ((r >> 1) & 7));
    tp[i] = k / C;
    cc[i] = k - tp[i] * C;
  }
  // B: full rounds move rows 64 rd + 8 wave + lane / 8; the partial round rows
  // 64 BFULL + (BREM / 8) wave + lane / 8 for the first BREM lanes: every wave issues the same
  // number of DMA instructions
  uint32_t boff[T::BFULL + 1];
#pragma unroll
  for (int rd = 0; rd <= T::BFULL; ++rd) {
    int row = 8 * NW * rd + 8 * wave + (lane >> 3);
    if constexpr (T::BREM > 0)
      if (rd == T::BFULL) row = 8 * NW * T::BFULL + (T::BREM / 8) * wave + ((lane >> 3) % (T::BREM / 8));
    boff[rd] = (uint32_t)((row * Kp + 8 * ((lane & 7) ^ ((row >> 1) & 7))) * 2);
  }
  // issue the next k-step's tiles into stage s (the A chunks' positions then move on)
  auto dma = [&](int t, int s) {
    uint8_t* st = smem + s * T::STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tap = tp[i];
      int dy = 0, dx = 0;
      if constexpr (TAPS == 9) {
        const int q = (tap * 11) >> 5;   // tap / 3 for tap < 9
        dy = UP == 2 ? q : q - 1;
        dx = UP == 2 ? tap - 3 * q : tap - 3 * q - 1;
      }
      // UP 2: a row past the picture has py -2^30, so sy stays negative (-2^31 + dy at least)
      int sy = (UP == 2 ? 2 * py[i] : py[i]) + dy, sx = (UP == 2 ? 2 * px[i] : px[i]) + dx;
      const bool ok = tap < TAPS && sy >= 0 && sy < (UP == 2 ? Hs : H) && sx >= 0 && sx < (UP == 2 ? Ws : W);
      if constexpr (UP == 1) {
        sy >>= 1;
        sx >>= 1;
      }
      const uint32_t off = ok ? (uint32_t)(((sy * Ws + sx) * C + cc[i]) * 2) : VOFF_NONE;
      conv_dma(X, xext, (lds_void*)(st + (NW * i + wave) * 1024), off, 0);
      cc[i] += 64;
      if (cc[i] >= C) {   // C >= 64: one wrap at most
        cc[i] -= C;
        tp[i] += 1;
      }
    }
#pragma unroll
    for (int rd = 0; rd < T::BFULL; ++rd)
      conv_dma(wbase, wext, (lds_void*)(st + T::ABYTES + rd * (1024 * NW) + wave * 1024), boff[rd], t * 128);
    if constexpr (T::BREM > 0)
      if (lane < T::BREM)
        conv_dma(wbase, wext, (lds_void*)(st + T::ABYTES + T::BFULL * (1024 * NW) + wave * T::BREM * 16), boff[T::BFULL],
                 t * 128);
  };

  // fragments: lane holds row lo of a 16-row block, K 8 q4 .. of a slice of 32
  const int lo = lane & 15, q4 = lane >> 4, fs = (lo >> 1) & 7;
  const int a_rd = (T::WM * wm + lo) * 128, b_rd = T::ABYTES + (T::WNC * wn + lo) * 128;
  f32x4 acc[T::MI][T::NJ];
#pragma unroll
  for (int i = 0; i < T::MI; ++i)
#pragma unroll
    for (int j = 0; j < T::NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const uint8_t* st) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int co = ((4 * kk + q4) ^ fs) << 4;
      bf16x8 a[T::MI];
#pragma unroll
      for (int i = 0; i < T::MI; ++i) a[i] = *(const bf16x8*)(st + a_rd + i * 2048 + co);
#pragma unroll
      for (int j = 0; j < T::NJ; ++j) {
        const bf16x8 b = *(const bf16x8*)(st + b_rd + j * 2048 + co);
#pragma unroll
        for (int i = 0; i < T::MI; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b, acc[i][j], 0, 0, 0);
      }
    }
  };

  if constexpr (T::NST == 3) {
    dma(kt0, 0);
    dma(min(kt0 + 1, kt1 - 1), 1);   // every step issues NDMA instructions a wave, so vmcnt(NDMA) below
    int s = 0;
    for (int t = kt0; t < kt1; ++t) {
      // step t has landed for every wave, and every wave is done with stage (t + 2) % 3
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((T::NDMA & 0xF) | (0x7 << 4) | (0x0 << 8));   // vmcnt(NDMA) lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      dma(min(t + 2, kt1 - 1), s >= 1 ? s - 1 : 2);   // into (t + 2) % 3; past the end a reload, never read
      step(smem + s * T::STAGE);
      s = s == 2 ? 0 : s + 1;
    }
  } else {
    dma(kt0, 0);
    for (int t = kt0; t < kt1; ++t) {
      // step t has landed for every wave, and every wave is done with the other stage
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));   // vmcnt(0) lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      dma(min(t + 1, kt1 - 1), (t - kt0 + 1) & 1);   // past the end a reload, never read
      step(smem + ((t - kt0) & 1) * T::STAGE);
    }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));   // no DMA left in flight
  asm volatile("" ::: "memory");

  // The epilogue through LDS (free now), 32 of the wave's pixels at a time: the wave stages its
  // 32 x 144 block (row stride 148 floats), then moves it as 16-byte chunks, 4 channels of one
  // pixel a lane: bias, and the residual or the DupUp3D gather, summed into the staged rows
  // first, then the stores.
  float* stg = (float*)smem + wave * (32 * T::LS);
  const float winv = 1.f / (float)W;
  const int rsh = OUT == VAE_DUPUP ? __builtin_ctz((unsigned)(cout * ep.ft * 4 / ep.kcin)) : 0;
#pragma unroll
  for (int half = 0; half < T::MI / 2; ++half) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < T::NJ; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) stg[(16 * i + 4 * q4 + r) * T::LS + 16 * j + lo] = acc[2 * half + i][j][r];
    __syncthreads();
    // NCH chunks a lane (18 at WNC 144), 4 channels of one pixel each, in two passes.  Pass 1
    // adds bias and the residual or the DupUp3D gather in place in the staging rows, in batches
    // of 6 chunks (3 at BN 288, where half the accumulators are still live); with no stores
    // among them the loads of one batch can be in flight while the last is summed.  Pass 2
    // stores the rows: no load is left to wait for.  (Stores among the loads would make
    // every batch wait for the stores before it, a round trip to HBM each.)
    constexpr int CH = BN == 288 ? (OUT == VAE_DUPUP || GAM ? 2 : 3) : (T::NCH < 6 ? T::NCH : 6);
    static_assert(T::NCH % CH == 0, "whole batches");
    if constexpr (OUT != VAE_PART) {
#pragma unroll BN == 288 ? 2 : T::NCH / CH
      for (int bt = 0; bt < T::NCH / CH; ++bt) {
        f32x4 v[CH], add[CH];
#pragma unroll
        for (int q = 0; q < CH; ++q) {
          const int k = (bt * CH + q) * 64 + lane, row = k / T::RC, c4 = k - row * T::RC;
          const int m = m0 + T::WM * wm + 32 * half + row, n = n0 + T::WNC * wn + 4 * c4;
          const int mc = min(m, P - 1), nc = min(n, cout - 4);   // in bounds for the loads either way
          v[q] = *(const f32x4*)(stg + row * T::LS + 4 * c4);
          v[q] += *(const f32x4*)(bias + nc);
          add[q] = f32x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (OUT == VAE_DUPUP) {
            // channel c of pixel (yy, xx) adds keep's channel j / rep of pixel (yy/2, xx/2),
            // j = ((c ft + ft - 1) 2 + yy%2) 2 + xx%2, rep = cout ft 4 / kcin (a power of two)
            int yy = (int)(((float)mc + 0.5f) * winv);   // mc / W, corrected to exact below
            yy -= yy * W > mc;
            yy += (yy + 1) * W <= mc;
            const int xx = mc - yy * W;
            const float* kr = ep.keep + (((yy >> 1) * (W >> 1) + (xx >> 1)) * ep.kcin);
            const int j0 = ((nc * ep.ft + ep.ft - 1) * 2 + (yy & 1)) * 2 + (xx & 1);
            // keep channel of channel nc + e: (j0 >> rsh) + e * kstep, kstep = kcin / cout (rep
            // divides 4 ft then).  At kstep 1 that is channels nc .. nc + 3, at kstep 2 channels
            // 2 nc + d + 0, 2, 4, 6 (d = 0 or 1): one or two aligned 16-byte loads.
            const int kstep = (4 * ep.ft) >> rsh, k0 = j0 >> rsh;
            if (kstep == 1 && (4 * ep.ft) % (1 << rsh) == 0) {
              add[q] = *(const f32x4*)(kr + k0);
            } else if (kstep == 2 && (4 * ep.ft) % (1 << rsh) == 0) {
              const f32x4 t0 = *(const f32x4*)(kr + 2 * nc), t1 = *(const f32x4*)(kr + 2 * nc + 4);
              const int d = k0 - 2 * nc;
              add[q] = d ? f32x4{t0[1], t0[3], t1[1], t1[3]} : f32x4{t0[0], t0[2], t1[0], t1[2]};
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) add[q][e] = kr[(j0 + 4 * ep.ft * e) >> rsh];
            }
          } else if constexpr (OUT == VAE_F32 || OUT == VAE_BF16) {
            if (ep.res) add[q] = *(const f32x4*)(ep.res + (int64_t)mc * cout + nc);
          }
        }
#pragma unroll
        for (int q = 0; q < CH; ++q) {
          const int k = (bt * CH + q) * 64 + lane, row = k / T::RC, c4 = k - row * T::RC;
          *(f32x4*)(stg + row * T::LS + 4 * c4) = v[q] + add[q];
        }
      }
    }
#pragma unroll BN == 288 ? 3 : 6
    for (int q = 0; q < T::NCH; ++q) {
      const int k = q * 64 + lane, row = k / T::RC, c4 = k - row * T::RC;
      const int m = m0 + T::WM * wm + 32 * half + row, n = n0 + T::WNC * wn + 4 * c4;
      if (m >= P || n >= cout) continue;
      const int at = m * cout + n;
      const f32x4 o = *(const f32x4*)(stg + row * T::LS + 4 * c4);
      if constexpr (OUT == VAE_RMS) {
      } else if constexpr (OUT == VAE_BF16) {
        *(u32x2*)((uint16_t*)Y + at) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      } else if constexpr (OUT == VAE_PART) {
        *(f32x4*)((float*)Y + (int64_t)z * P * cout + at) = o;
      } else if constexpr (OUT == VAE_CLAMP) {
        f32x4 c;
#pragma unroll
        for (int e = 0; e < 4; ++e) c[e] = fminf(1.f, fmaxf(-1.f, o[e]));
        *(f32x4*)((float*)Y + at) = c;
      } else {
        if (OUT != VAE_DUPUP || Y) *(f32x4*)((float*)Y + at) = o;   // DupUp: no fp32 out when Y is null
        if constexpr (OUT == VAE_F32 || OUT == VAE_DUPUP) {
          if (ep.y2) *(u32x2*)(ep.y2 + at) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        }
      }
    }
    if constexpr (GAM) {
      static_assert(T::WNC == 144 || T::WNC == 96, "the norm's layout: rows of 144 or 96 a wave");
      // each staged row's sum of squares: lanes 2r and 2r + 1 take its two halves, then swap; at
      // BN 288 and 192 the row's other channels are the partner wave's (same pixels)
      constexpr int HALF4 = T::WNC / 8;   // 4-channel chunks in half a row
      const int rr = lane >> 1, hh = lane & 1;
      float ss = 0.f;
#pragma unroll 3
      for (int c = 0; c < HALF4; ++c) {
        const f32x4 t = *(const f32x4*)(stg + rr * T::LS + (T::WNC / 2) * hh + 4 * c);
        ss += (t[0] * t[0] + t[1] * t[1]) + (t[2] * t[2] + t[3] * t[3]);
      }
      ss += dpp_f<0xB1>(ss);   // quad_perm [1, 0, 3, 2]: lane ^ 1
      if constexpr (T::NWN == 2) {
        if (hh == 0) stg[rr * T::LS + T::WNC] = ss;
        __syncthreads();
        const int partner = wn ? wave - T::NWM : wave + T::NWM;
        ss += ((const float*)smem + partner * (32 * T::LS))[rr * T::LS + T::WNC];
      }
      const float inv = sqrtf((float)cout) / fmaxf(sqrtf(ss), 1e-12f);
      if (hh == 0) stg[rr * T::LS + T::WNC + 1] = inv;
      asm volatile("" ::: "memory");
#pragma unroll 2
      for (int q = 0; q < T::NCH; ++q) {
        const int k = q * 64 + lane, row = k / T::RC, c4 = k - row * T::RC;
        const int m = m0 + T::WM * wm + 32 * half + row, n = n0 + T::WNC * wn + 4 * c4;
        if (m >= P) continue;
        const f32x4 o = *(const f32x4*)(stg + row * T::LS + 4 * c4), g = *(const f32x4*)(ep.gamma + n);
        const float iv = stg[row * T::LS + T::WNC + 1];
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = silu_bf16out(o[j] * iv * g[j]);
        *(u32x2*)(ep.yr + (int64_t)m * cout + n) = u32x2{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3])};
      }
    }
  }
}

// y = the S partial sums of a split-K convolution in order, + bias, + res when given; fp32 or
// bf16 out; 4 channels a thread
template <int BF16OUT>
__global__ void __launch_bounds__(256)
k_part_sum(int S, int64_t n4, int cout, const float* __restrict__ part, const float* __restrict__ bias,
           const float* __restrict__ res, void* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  f32x4 v = ((const f32x4*)part)[i];
  for (int zz = 1; zz < S; ++zz) v += ((const f32x4*)part)[zz * n4 + i];
  v += *(const f32x4*)(bias + (4 * i) % cout);
  if (res) v += ((const f32x4*)res)[i];
  if constexpr (BF16OUT)
    ((u32x2*)y)[i] = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  else
    ((f32x4*)y)[i] = v;
}

static hipError_t part_sum(hipStream_t s, int S, int64_t n, int cout, const float* part, const float* bias,
                           const float* res, void* y, bool bf16out) {
  const int64_t n4 = n / 4;
  if (bf16out)
    hipLaunchKernelGGL(k_part_sum<1>, dim3(grid_of(n4, 256)), dim3(256), 0, s, S, n4, cout, part, bias, res, y);
  else
    hipLaunchKernelGGL(k_part_sum<0>, dim3(grid_of(n4, 256)), dim3(256), 0, s, S, n4, cout, part, bias, res, y);
  return hipGetLastError();
}

template <int BN, int TAPS, int UP, int OUT, int GAM = 0, int NW = 8>
static hipError_t launch_conv1(hipStream_t s, const uint16_t* x, const uint16_t* wt, const float* bias, const VaeEpi& ep,
                               void* y, int h, int w, int c, int cout, int kp, int split = 1) {
  auto kern = k_conv<BN, TAPS, UP, OUT, GAM, NW>;
  typedef ConvTile<BN, NW> T;
  {
    const hipError_t e = ensure_lds((const void*)kern, T::LDS);
    if (e != hipSuccess) return e;
  }
  dim3 grid(grid_of((int64_t)h * w, T::TM), grid_of(cout, BN), split);
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), T::LDS, s, x, wt, bias, ep, y, h, w, c, cout, kp);
  return hipGetLastError();
}

// 128-pixel tiles of 4 waves (two workgroups a CU) for the 96- and 144-wide convolutions of
// pictures of 2^18 pixels or more, where the output, residual and normed copy move as many bytes
// as the products take time; 256-pixel tiles otherwise
template <int BN, int TAPS, int UP, int OUT, int GAM = 0>
static hipError_t launch_conv(hipStream_t s, const uint16_t* x, const uint16_t* wt, const float* bias, const VaeEpi& ep,
                              void* y, int h, int w, int c, int cout, int kp, int split = 1) {
  if constexpr (BN == 96 || BN == 144) {
    if (split == 1 && !ep.wide_only && (int64_t)h * w >= (1 << 18))
      return launch_conv1<BN, TAPS, UP, OUT, GAM, 4>(s, x, wt, bias, ep, y, h, w, c, cout, kp, 1);
  }
  return launch_conv1<BN, TAPS, UP, OUT, GAM, 8>(s, x, wt, bias, ep, y, h, w, c, cout, kp, split);
}

// the decoder's tiles (BN 144, 288: waves of 144 channels) take the norm in the store, the
// clamp and the upsampling convolutions; the encoder's (BN 96, 192) the stride-2 ones
template <int BN>
static hipError_t conv_bn(hipStream_t s, int taps, int up, int out, const uint16_t* x, const uint16_t* wt,
                          const float* bias, const VaeEpi& ep, void* y, int h, int w, int c, int cout, int kp) {
  constexpr bool DEC = ConvTile<BN>::WNC == 144;
  // a 3 x 3 convolution of fewer tiles than the chip's CUs (the decoder's 64 x 64 stages: 64
  // tiles) splits its K over up to 4 workgroups a tile, each at least 16 k-steps, into fp32
  // partials; k_part_sum adds them in order with bias and res
  if (ep.gamma) {   // the output's norm too: one channel tile (cout == BN), never split
    if (taps == 9 && !up && out == VAE_F32) return launch_conv<BN, 9, 0, VAE_F32, 1>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    if (taps == 9 && !up && out == VAE_RMS) return launch_conv<BN, 9, 0, VAE_RMS, 1>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    if constexpr (DEC) {
      if (taps == 9 && up == 1 && out == VAE_DUPUP)
        return launch_conv<BN, 9, 1, VAE_DUPUP, 1>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    } else {
      // the encoder's first convolution (a 1 x 1 product over RGBA neighbourhoods) with the
      // first block's normed input
      if (taps == 1 && !up && out == VAE_F32) return launch_conv<BN, 1, 0, VAE_F32, 1>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    }
    return hipErrorInvalidValue;
  }
  const int64_t P = (int64_t)h * w, tiles = grid_of(P, ConvTile<BN>::TM) * (int64_t)grid_of(cout, BN);
  int64_t split = 256 / tiles < 4 ? 256 / tiles : 4;
  if (kp / 64 / 16 < split) split = kp / 64 / 16;
  if (taps == 9 && !up && (out == VAE_F32 || out == VAE_BF16) && !ep.y2 && ep.part && tiles < 192 && split >= 2 &&
      split * P * cout <= ep.part_cap) {
    hipError_t e = launch_conv<BN, 9, 0, VAE_PART>(s, x, wt, bias, ep, ep.part, h, w, c, cout, kp, (int)split);
    if (e != hipSuccess) return e;
    return part_sum(s, (int)split, P * cout, cout, ep.part, bias, ep.res, y, out == VAE_BF16);
  }
  if (taps == 9 && !up && out == VAE_F32) return launch_conv<BN, 9, 0, VAE_F32>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (taps == 9 && !up && out == VAE_BF16) return launch_conv<BN, 9, 0, VAE_BF16>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  if constexpr (DEC) {
    if (taps == 9 && !up && out == VAE_CLAMP) return launch_conv<BN, 9, 0, VAE_CLAMP>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    if (taps == 9 && up == 1 && out == VAE_F32) return launch_conv<BN, 9, 1, VAE_F32>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    if (taps == 9 && up == 1 && out == VAE_DUPUP)
      return launch_conv<BN, 9, 1, VAE_DUPUP>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  } else {
    if (taps == 9 && up == 2 && out == VAE_F32) return launch_conv<BN, 9, 2, VAE_F32>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  }
  if (taps == 1 && !up && out == VAE_F32) return launch_conv<BN, 1, 0, VAE_F32>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (taps == 1 && !up && out == VAE_BF16) return launch_conv<BN, 1, 0, VAE_BF16>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  return hipErrorInvalidValue;
}

hipError_t vae_conv(hipStream_t s, int taps, int up, int out, const uint16_t* x, const uint16_t* wt, const float* bias,
                    const VaeEpi& ep, void* y, int h, int w, int c, int cout, int kp) {
  // the loads move 8 channels at once and each k-step moves a chunk's tap at most once; the
  // epilogue moves 4 channels at once; every offset and extent fits 31 bits
  // (up 2: the input is 2h x 2w)
  const int64_t in_px = (int64_t)h * w * (up == 2 ? 4 : 1);
  if (c < 64 || c % 8 || kp % 64 || kp < taps * c || cout <= 0 || cout % 4 || h <= 0 || w <= 0 || up < 0 || up > 2 ||
      (up == 1 && (h % 2 || w % 2)) || (up == 2 && taps != 9) || ((uintptr_t)x & 15) || ((uintptr_t)wt & 15) || ((uintptr_t)y & 15) ||
      (!y && !(out == VAE_DUPUP && (ep.y2 || ep.yr)) && out != VAE_RMS) ||
      ((uintptr_t)bias & 15) || ((uintptr_t)ep.res & 15) || ((uintptr_t)ep.y2 & 7) || ((uintptr_t)ep.part & 15) ||
      (ep.gamma && (!ep.yr || ((uintptr_t)ep.yr & 7) || ((uintptr_t)ep.gamma & 15) ||
                    (cout != 144 && cout != 288 && cout != 96 && cout != 192))) ||
      (!ep.gamma && out == VAE_RMS) ||
      in_px * c * 2 >= ((int64_t)1 << 31) || (int64_t)cout * kp * 2 >= ((int64_t)1 << 31) ||
      (int64_t)h * w * cout >= ((int64_t)1 << 31) ||
      (out == VAE_DUPUP && (!ep.keep || ep.ft < 1 || ep.kcin <= 0 || (int64_t)cout * ep.ft * 4 % ep.kcin || h % 2 ||
                            w % 2 || ((cout * ep.ft * 4 / ep.kcin) & (cout * ep.ft * 4 / ep.kcin - 1)))))
    return hipErrorInvalidValue;
  // the wide tile where 288 divides the width (1152, 576, 288 and the 3456 of q|k|v); 144 for
  // the decoder's 144; 192 and 96 for the encoder's widths (96, 192, 384, 768); a narrow one
  // for a few channels (the head's 4): 16 columns of MFMA work instead of 144
  if (cout % 288 == 0) return conv_bn<288>(s, taps, up, out, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (cout % 144 != 0 && cout % 192 == 0) return conv_bn<192>(s, taps, up, out, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (cout % 144 != 0 && cout % 96 == 0) return conv_bn<96>(s, taps, up, out, x, wt, bias, ep, y, h, w, c, cout, kp);
  if (cout <= 16 && !ep.gamma) {
    if (taps == 9 && !up && out == VAE_CLAMP) return launch_conv<16, 9, 0, VAE_CLAMP>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
    if (taps == 9 && !up && out == VAE_F32) return launch_conv<16, 9, 0, VAE_F32>(s, x, wt, bias, ep, y, h, w, c, cout, kp);
  }
  return conv_bn<144>(s, taps, up, out, x, wt, bias, ep, y, h, w, c, cout, kp);
}

// --- the bandwidth kernels ----------------------------------------------------------

// y = x / max(|x|, 1e-12) * sqrt(C) * gamma over each pixel's C channels (src/cuda-vae.lisp's
// v_rms with eps 1e-12; inspect/ref_vae.py:50-52), then SiLU when SILU; bf16 out.  LP lanes a
// pixel, C a multiple of 4.
template <int LP, int SILU>
__global__ void __launch_bounds__(256)
k_rms_silu(int64_t P, int C, const float* __restrict__ x, const float* __restrict__ gamma, uint16_t* __restrict__ y) {
  const int64_t p = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LP;
  const int sub = threadIdx.x % LP;
  const bool live = p < P;
  const float* r = x + (live ? p : 0) * C;
  float ss = 0.f;
  for (int c = 4 * sub; c < C; c += 4 * LP) {
    const f32x4 v = *(const f32x4*)(r + c);
    ss += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
  }
  ss = LP == 64 ? wave_sum_dpp(ss) : row16_sum(ss);   // every lane of the group takes part
  const float inv = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
  if (!live) return;
  uint16_t* o = y + p * C;
  for (int c = 4 * sub; c < C; c += 4 * LP) {
    const f32x4 v = *(const f32x4*)(r + c), g = *(const f32x4*)(gamma + c);
    float e[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      e[q] = v[q] * inv * g[q];
      if constexpr (SILU) e[q] = silu_bf16out(e[q]);
    }
    *(u32x2*)(o + c) = u32x2{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3])};
  }
}

// the sum of v over each group of LP lanes (4, 8, 16 or 32 aligned lanes), in every lane of it
template <int LP>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);                       // pairs
  v += dpp_f<0x4E>(v);                       // quads
  if constexpr (LP >= 8) v += dpp_f<0x141>(v);   // the two quads of a half row
  if constexpr (LP >= 16) v += dpp_f<0x140>(v);  // the two halves of a row
  if constexpr (LP >= 32) {
    float a = v, b = v;
    xswap16(a, b);
    v = a + b;
  }
  return v;
}

// the decoder's widths, C = 36 LP (144, 288, 576, 1152): a lane holds 9 chunks of 4 channels in
// registers, so x is read once
template <int LP, int SILU>
__global__ void __launch_bounds__(256)
k_rms_silu9(int64_t P, const float* __restrict__ x, const float* __restrict__ gamma, uint16_t* __restrict__ y) {
  constexpr int C = 36 * LP;
  const int64_t p = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LP;
  const int sub = threadIdx.x % LP;
  const bool live = p < P;
  const float* r = x + (live ? p : 0) * C;
  f32x4 v[9];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    v[q] = *(const f32x4*)(r + 4 * (sub + LP * q));
    ss += (v[q][0] * v[q][0] + v[q][1] * v[q][1]) + (v[q][2] * v[q][2] + v[q][3] * v[q][3]);
  }
  ss = group_sum<LP>(ss);
  const float inv = sqrtf((float)C) / fmaxf(sqrtf(ss), 1e-12f);
  if (!live) return;
  uint16_t* o = y + p * C;
#pragma unroll
  for (int q = 0; q < 9; ++q) {
    const int c = 4 * (sub + LP * q);
    const f32x4 g = *(const f32x4*)(gamma + c);
    float e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      e[k] = v[q][k] * inv * g[k];
      if constexpr (SILU) e[k] = silu_bf16out(e[k]);
    }
    *(u32x2*)(o + c) = u32x2{pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3])};
  }
}

template <int LP>
static void launch_rms9(hipStream_t s, int64_t P, const float* x, const float* gamma, uint16_t* y, int silu) {
  const unsigned g = grid_of(P * LP, 256);
  if (silu) hipLaunchKernelGGL((k_rms_silu9<LP, 1>), dim3(g), dim3(256), 0, s, P, x, gamma, y);
  else hipLaunchKernelGGL((k_rms_silu9<LP, 0>), dim3(g), dim3(256), 0, s, P, x, gamma, y);
}

hipError_t vae_rms_silu(hipStream_t s, int64_t P, int C, const float* x, const float* gamma, uint16_t* y, int silu) {
  if (C % 4 || P <= 0) return P == 0 ? hipSuccess : hipErrorInvalidValue;
  switch (C) {
    case 144: launch_rms9<4>(s, P, x, gamma, y, silu); return hipGetLastError();
    case 288: launch_rms9<8>(s, P, x, gamma, y, silu); return hipGetLastError();
    case 576: launch_rms9<16>(s, P, x, gamma, y, silu); return hipGetLastError();
    case 1152: launch_rms9<32>(s, P, x, gamma, y, silu); return hipGetLastError();
  }
  if (C <= 512) {
    const unsigned g = grid_of(P * 16, 256);
    if (silu) hipLaunchKernelGGL((k_rms_silu<16, 1>), dim3(g), dim3(256), 0, s, P, C, x, gamma, y);
    else hipLaunchKernelGGL((k_rms_silu<16, 0>), dim3(g), dim3(256), 0, s, P, C, x, gamma, y);
  } else {
    const unsigned g = grid_of(P * 64, 256);
    if (silu) hipLaunchKernelGGL((k_rms_silu<64, 1>), dim3(g), dim3(256), 0, s, P, C, x, gamma, y);
    else hipLaunchKernelGGL((k_rms_silu<64, 0>), dim3(g), dim3(256), 0, s, P, C, x, gamma, y);
  }
  return hipGetLastError();
}

// y (2H x 2W x cout, fp32) += DupUp3D(x) (H x W x cin), frame ft - 1 of ft: channel c of pixel
// (Y, X) adds channel j / rep of pixel (Y/2, X/2), j = ((c ft + ft - 1) 2 + Y%2) 2 + X%2,
// rep = cout ft 4 / cin (src/cuda/vae.cu's x_dupup_add, the index of inspect/ref_vae.py:79-85)
__global__ void k_dupup_add(int cin, int cout, int ft, int H, int W, const float* __restrict__ x,
                            float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 4LL * H * W * cout) return;
  const int c = (int)(i % cout);
  const int64_t p = i / cout;
  const int yy = (int)(p / (2 * W)), xx = (int)(p % (2 * W));
  const int rep = cout * ft * 4 / cin;
  const int j = ((c * ft + ft - 1) * 2 + (yy & 1)) * 2 + (xx & 1);
  y[i] += x[((int64_t)(yy >> 1) * W + (xx >> 1)) * cin + j / rep];
}

hipError_t vae_dupup_add(hipStream_t s, int cin, int cout, int ft, int h, int w, const float* x, float* y) {
  if ((int64_t)cout * ft * 4 % cin) return hipErrorInvalidValue;
  const int64_t n = 4LL * h * w * cout;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_dupup_add, dim3(grid_of(n, 256)), dim3(256), 0, s, cin, cout, ft, h, w, x, y);
  return hipGetLastError();
}

// y (H/2 x W/2 x cout, fp32) += AvgDown3D(x) (H x W x cin) on one frame, padded in front to ft
// frames with zeros (src/cuda/vae.cu's x_avgdown_add): output channel o of pixel (Y, X) is the
// mean of the g = cin ft 4 / cout values j = o g .. o g + g - 1 of the view (cin, ft, 2, 2) of
// the 2 x 2 block at (2Y, 2X): channel j / (4 ft), frame (j / 4) % ft (zero but the last), row
// 2Y + (j / 2) % 2, column 2X + j % 2.  One thread an output value.
__global__ void k_avgdown_add(int cin, int cout, int ft, int H, int W, const float* __restrict__ x,
                              float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int ow = W / 2;
  if (i >= (int64_t)(H / 2) * ow * cout) return;
  const int o = (int)(i % cout);
  const int64_t p = i / cout;
  const int yy = (int)(p / ow), xx = (int)(p % ow);
  const int g = cin * ft * 4 / cout;
  float acc = 0.f;
  for (int k = 0; k < g; ++k) {
    const int j = o * g + k;
    if ((j >> 2) % ft != ft - 1) continue;   // a padding frame: zero
    acc += x[((int64_t)(2 * yy + ((j >> 1) & 1)) * W + 2 * xx + (j & 1)) * cin + j / (4 * ft)];
  }
  y[i] += acc / (float)g;
}

// the encoder's two cases, 4 output channels a thread: g = 4 with ft 1 (cout = cin: each
// channel's 2 x 2 mean, 16-byte loads) or ft 2 (cout = 2 cin: odd channel o takes channel
// o / 2's mean, even ones nothing; 8-byte loads)
template <int FT>
__global__ void k_avgdown_add4(int cin, int H, int W, const float* __restrict__ x, float* __restrict__ y) {
  const int cout = cin * FT, c4n = cout / 4, ow = W / 2;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)(H / 2) * ow * c4n) return;
  const int o = 4 * (int)(i % c4n);
  const int64_t p = i / c4n;
  const int yy = (int)(p / ow), xx = (int)(p % ow);
  const float* r0 = x + ((int64_t)(2 * yy) * W + 2 * xx) * cin;
  const float* r1 = r0 + (int64_t)W * cin;
  f32x4 add;
  if constexpr (FT == 1) {
    const f32x4 a = *(const f32x4*)(r0 + o), b = *(const f32x4*)(r0 + cin + o);
    const f32x4 c = *(const f32x4*)(r1 + o), d = *(const f32x4*)(r1 + cin + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) add[e] = (((a[e] + b[e]) + c[e]) + d[e]) / 4.f;
  } else {
    const int c0 = o / 2;
    const f32x2 a = *(const f32x2*)(r0 + c0), b = *(const f32x2*)(r0 + cin + c0);
    const f32x2 c = *(const f32x2*)(r1 + c0), d = *(const f32x2*)(r1 + cin + c0);
    add = f32x4{0.f, (((a[0] + b[0]) + c[0]) + d[0]) / 4.f, 0.f, (((a[1] + b[1]) + c[1]) + d[1]) / 4.f};
  }
  f32x4* yo = (f32x4*)(y + p * cout + o);
  *yo += add;
}

hipError_t vae_avgdown_add(hipStream_t s, int cin, int cout, int ft, int h, int w, const float* x, float* y) {
  if (cin <= 0 || cout <= 0 || ft < 1 || (int64_t)cin * ft * 4 % cout || h % 2 || w % 2) return hipErrorInvalidValue;
  const int64_t n = (int64_t)(h / 2) * (w / 2) * cout;
  if (n == 0) return hipSuccess;
  const bool al = ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && cin % 4 == 0;
  if (al && ft == 1 && cout == cin) {
    hipLaunchKernelGGL(k_avgdown_add4<1>, dim3(grid_of(n / 4, 256)), dim3(256), 0, s, cin, h, w, x, y);
  } else if (al && ft == 2 && cout == 2 * cin) {
    hipLaunchKernelGGL(k_avgdown_add4<2>, dim3(grid_of(n / 4, 256)), dim3(256), 0, s, cin, h, w, x, y);
  } else {
    hipLaunchKernelGGL(k_avgdown_add, dim3(grid_of(n, 256)), dim3(256), 0, s, cin, cout, ft, h, w, x, y);
  }
  return hipGetLastError();
}

// y += x over n floats (4 a thread; n a multiple of 4)
__global__ void k_add4(int64_t n4, const float* __restrict__ x, float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n4) ((f32x4*)y)[i] += ((const f32x4*)x)[i];
}

hipError_t vae_add(hipStream_t s, int64_t n, const float* x, float* y) {
  if (n % 4) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_add4, dim3(grid_of(n / 4, 256)), dim3(256), 0, s, n / 4, x, y);
  return hipGetLastError();
}

// the encoder's first convolution's input: each pixel's 3 x 3 neighbourhood of RGBA (x: H x W
// x 4 fp32) as one row of 64 bf16, k = tap 4 + channel for k < 36 (tap = 3 (dy + 1) + dx + 1,
// off the picture zero), zeros after -- a 1 x 1 product with the weights packed as (tap,
// channel) rows then is the 3 x 3 'same' convolution.  One thread 8 values of a row.
__global__ void k_rgba_taps(int H, int W, const float* __restrict__ x, uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)H * W * 8) return;
  const int64_t p = i >> 3;
  const int k0 = 8 * (int)(i & 7);
  const int py = (int)(p / W), px = (int)(p % W);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = k0 + e, tap = k >> 2, c = k & 3;
    const int sy = py + tap / 3 - 1, sx = px + tap % 3 - 1;
    v[e] = k < 36 && sy >= 0 && sy < H && sx >= 0 && sx < W ? x[((int64_t)sy * W + sx) * 4 + c] : 0.f;
  }
  *(u32x4*)(y + p * 64 + k0) =
      u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}

hipError_t vae_rgba_taps(hipStream_t s, int h, int w, const float* x, uint16_t* y) {
  const int64_t n = (int64_t)h * w * 8;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rgba_taps, dim3(grid_of(n, 256)), dim3(256), 0, s, h, w, x, y);
  return hipGetLastError();
}

// the first C of each pixel row's LD fp32 values, channel-major: z[c][p] = x[p][c] (the
// encoder's mean, out of its 2 z channels)
__global__ void k_pixels_latent(int64_t P, int C, int ld, const float* __restrict__ x, float* __restrict__ z) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P * C) return;
  const int c = (int)(i / P);
  const int64_t p = i % P;
  z[i] = x[p * ld + c];
}

hipError_t vae_pixels_latent(hipStream_t s, int64_t P, int C, int ld, const float* x, float* z) {
  if (C > ld) return hipErrorInvalidValue;
  if (P * C == 0) return hipSuccess;
  hipLaunchKernelGGL(k_pixels_latent, dim3(grid_of(P * C, 256)), dim3(256), 0, s, P, C, ld, x, z);
  return hipGetLastError();
}

// the latent (64 x P fp32, channel-major) as pixel rows of 64 bf16
__global__ void k_latent_pixels(int64_t P, int C, const float* __restrict__ z, uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= P * C) return;
  const int64_t p = i / C;
  const int c = (int)(i % C);
  y[i] = (uint16_t)(pack_bf16x2(z[c * P + p], 0.f) & 0xFFFFu);
}

hipError_t vae_latent_pixels(hipStream_t s, int64_t P, int C, const float* z, uint16_t* y) {
  if (P * C == 0) return hipSuccess;
  hipLaunchKernelGGL(k_latent_pixels, dim3(grid_of(P * C, 256)), dim3(256), 0, s, P, C, z, y);
  return hipGetLastError();
}

// the attention's q|k|v rows (n x 3c fp32) apart: q, k as n x c bf16 and v transposed, c x np
// bf16, columns n .. np - 1 zero (the second product's K is np, a multiple of 64)
__global__ void k_split_qkv(int64_t n, int64_t np, int c, const float* __restrict__ qkv, uint16_t* __restrict__ q,
                            uint16_t* __restrict__ k, uint16_t* __restrict__ vt) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= np * c) return;
  const int64_t t = i / c;
  const int j = (int)(i % c);
  if (t < n) {
    const float* r = qkv + t * 3 * c;
    q[i] = (uint16_t)(pack_bf16x2(r[j], 0.f) & 0xFFFFu);
    k[i] = (uint16_t)(pack_bf16x2(r[c + j], 0.f) & 0xFFFFu);
    vt[(int64_t)j * np + t] = (uint16_t)(pack_bf16x2(r[2 * c + j], 0.f) & 0xFFFFu);
  } else {
    vt[(int64_t)j * np + t] = 0;
  }
}

hipError_t vae_split_qkv(hipStream_t s, int64_t n, int64_t np, int c, const float* qkv, uint16_t* q, uint16_t* k,
                         uint16_t* vt) {
  if (np < n || np * c == 0) return np < n ? hipErrorInvalidValue : hipSuccess;
  hipLaunchKernelGGL(k_split_qkv, dim3(grid_of(np * c, 256)), dim3(256), 0, s, n, np, c, qkv, q, k, vt);
  return hipGetLastError();
}

// each row of S (n x np fp32, the first n columns the scores): softmax of the scores times
// SCALE as bf16 P, columns n .. np - 1 zero (src/cuda/vae.cu's x_softmax_rows)
__global__ void __launch_bounds__(256)
k_softmax_rows(int n, int np, float scale, const float* __restrict__ S, uint16_t* __restrict__ P) {
  __shared__ float red[8];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* r = S + (int64_t)row * np;
  uint16_t* o = P + (int64_t)row * np;
  float mx = -INFINITY;
  for (int c = tid; c < n; c += 256) mx = fmaxf(mx, r[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sum = 0.f;
  for (int c = tid; c < n; c += 256) sum += expf((r[c] - mx) * scale);
  sum = wave_sum_dpp(sum);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = sum;
  __syncthreads();
  const float inv = 1.f / (red[4] + red[5] + red[6] + red[7]);
  for (int c = tid; c < np; c += 256) {
    const float p = c < n ? expf((r[c] - mx) * scale) * inv : 0.f;
    o[c] = (uint16_t)(pack_bf16x2(p, 0.f) & 0xFFFFu);
  }
}

hipError_t vae_softmax_rows(hipStream_t s, int n, int np, float scale, const float* S, uint16_t* P) {
  if (n <= 0 || np < n) return n == 0 ? hipSuccess : hipErrorInvalidValue;
  hipLaunchKernelGGL(k_softmax_rows, dim3(n), dim3(256), 0, s, n, np, scale, S, P);
  return hipGetLastError();
}

// a tensor as the file holds it (fp32 values; a convolution (o, i, [1,] k, k)) -> the device
// form: a convolution's weights as bf16 rows of (tap, channel), K padded with zeros to kp
__global__ void k_pack_conv(int64_t o, int ci, int taps, int kp, const float* __restrict__ src,
                            uint16_t* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= o * kp) return;
  const int64_t r = i / kp;
  const int k = (int)(i % kp);
  float v = 0.f;
  if (k < taps * ci) {
    const int tap = k / ci, c = k % ci;
    v = src[(r * ci + c) * taps + tap];
  }
  dst[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
}

hipError_t vae_pack_conv(hipStream_t s, int64_t o, int ci, int taps, int kp, const float* src, uint16_t* dst) {
  if (kp < taps * ci || o * kp == 0) return kp < taps * ci ? hipErrorInvalidValue : hipSuccess;
  hipLaunchKernelGGL(k_pack_conv, dim3(grid_of(o * kp, 256)), dim3(256), 0, s, o, ci, taps, kp, src, dst);
  return hipGetLastError();
}

// fp32 values rounded through bf16 (a tensor the file ships as bf16, kept as fp32)
__global__ void k_round_bf16(int64_t n, float* __restrict__ x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = bf16_to_f32((uint16_t)(pack_bf16x2(x[i], 0.f) & 0xFFFFu));
}

hipError_t vae_round_bf16(hipStream_t s, int64_t n, float* x) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_round_bf16, dim3(grid_of(n, 256)), dim3(256), 0, s, n, x);
  return hipGetLastError();
}

}  // namespace exn
