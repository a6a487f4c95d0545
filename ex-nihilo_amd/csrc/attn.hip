// attn.hip -- the DiT's joint attention on gfx950's MFMA, flash style: K and
// V^T tiles moved HBM/L2 -> LDS by buffer loads to LDS (two rings of two
// stages, one barrier a tile), an online softmax in fp32 on scores in log2
// units, Q, K, V and P in fp16 (the reference's halves), fp32 sums.  Each
// wave's step is software-pipelined: the S product of the next tile runs on
// the MFMA pipe while the VALU takes this tile's exp2.  The mask is the
// reference's xa_lim (src/cuda/dit.cu:60-66): sequence row g sees keys
// 0..lim(g), lim(g) = l-1 for image rows (g >= p), b1-1 for a reference
// picture's rows b0..b1-1, g otherwise (the prompt is causal).  lim never
// decreases in g, so a query tile's last key is its last row's.  Replaces
// x_attend_mma (src/cuda/dit.cu:208-336).
//
// Layouts: Q [32 heads][n][128] (query t = sequence row q0 + t), pre-scaled
// so that scores come out in log2 units; K [32][lcap][128]; V^T [32][128][lcap]
// with the keys of every aligned group of 16 stored in the order of
// vt_pos() below; all fp16.  out [n][4096] bf16 (the next product's input), or fp32 (the
// int8 mode quantises it).
//
// The products are taken transposed so that no register shuffles are needed:
// S^T = K Q^T puts one query in a lane's column (its 32 of a 64-key tile's
// scores in its registers, the other 32 in lane ^ 32), and O^T += V^T P^T
// takes that lane's P values straight as the B operand.  The MFMA's k-slot
// 8*hi + j of a 16-key step u holds key 16u + 8(j/4) + 4hi + j%4 of the
// accumulator layout; V^T is stored so that those 8 keys are 16 contiguous
// bytes.
//
// Occupancy: at most 256 registers a lane and 64 KB of LDS a workgroup, so two
// workgroups share a CU and each SIMD interleaves one wave's softmax with
// another's MFMAs.  The running max moves only when a row's tile max exceeds
// it by more than 2^8 (P then stays <= 256, exact in fp16 to its 11 bits), so
// the O rescale is rare; the S product starts from -max, so the common tile
// needs no subtraction before exp2, and the row sums come from v_dot2 on the
// packed fp16 P.  The tile body is specialised per LDS stage, so every
// fragment read is a per-lane base plus an immediate offset.
#include "exn_common.h"

#include <type_traits>

namespace exn {

#define AQ 128          // queries a workgroup (32 a wave)
#define AK 64           // keys a tile
#define MAX_SLACK 8.f   // log2 units the running max may lag the true max by

typedef __attribute__((address_space(3))) void lds_void;

// one 16-byte DMA lane of a K or V^T tile
__device__ __forceinline__ void kv_dma(const void* base, uint32_t extent, lds_void* dst, uint32_t voff, int soff) {
  __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)extent, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ int xa_lim(int g, int p, int l, int b0, int b1) {
  return g >= p ? l - 1 : (g >= b0 && g < b1 ? b1 - 1 : g);
}

// max and sum over lanes l and l ^ 32 (xswap32 hands each lane its partner's value)
__device__ __forceinline__ float xmax32(float v) {
  float a = v, b = v;
  xswap32(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xsum32(float v) {
  float a = v, b = v;
  xswap32(a, b);
  return a + b;
}

// grid (ceil(n/128), 32 heads), block 256; O bf16, or fp32 when OF32; Q's heads QLD rows apart
template <bool OF32>
__global__ void __launch_bounds__(256, 2)
k_attend(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vt,
         void* __restrict__ O, int n, int q0, int p, int l, int64_t lcap, int b0, int b1, float scale, int64_t qld) {
  // Two rings, one tile apart: K stage s (64 keys x 256 B) at s * 16 KB, V^T stage s (128 dims x
  // 128 B) at 32 KB + s * 16 KB.  Step t reads K of tile t+1 and V^T of tile t, so the DMA of K
  // t+2 and V^T t+1 go into the stages step t-1 read.
  // K rows: 16-byte chunk c stored at c ^ (row % 16); V^T rows: chunk c at c ^ ((row / 2) % 8).
  __shared__ __align__(1024) uint8_t smem[4 * 16384];
  // Workgroups go to the 8 XCDs in turn (linear id mod 8).  XCD x takes whole heads x, x + 8,
  // .. in order, so the query tiles that stream one head's K and V^T share that XCD's L2:
  // two heads in flight an XCD, 4.4 MB at 4352 keys, instead of a sixteenth of each of 16.
  const int QT = gridDim.x, lin = blockIdx.y * QT + blockIdx.x, slot = lin / 8;
  const int h = lin % 8 + 8 * (slot / QT), t0 = slot % QT * AQ;
  const int tid = threadIdx.x, lane = tid & 63, hi = lane >> 5, lo = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: LDS bases stay scalar
  const int tq = t0 + wave * 32 + lo;
  const int tqc = min(tq, n - 1);

  // Q^T as the B operand: 8 steps of 16 dims, this lane's query, dims 16s + 8*hi ..
  f16x8 qf[8];
  {
    const uint16_t* qr = Q + ((int64_t)h * qld + tqc) * 128 + 8 * hi;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const f16x8*)(qr + 16 * s);
  }
  const int lim = xa_lim(q0 + tqc, p, l, b0, b1);
  const int last = xa_lim(q0 + min(n, t0 + AQ) - 1, p, l, b0, b1);
  const int minlim = xa_lim(q0 + t0, p, l, b0, b1);
  const int tiles = last / AK + 1;

  const uint16_t* kbase = Kc + (int64_t)h * lcap * 128;
  const uint16_t* vbase = Vt + (int64_t)h * 128 * lcap;
  const uint32_t kvext = (uint32_t)(lcap * 128 * 2);   // a head's K, and its V^T, in bytes
  // DMA: round i of wave w moves K rows (4i + w)*4 .. +3 (lane: row +l/16, LDS chunk l%16)
  // and V^T rows (4i + w)*8 .. +7 (lane: row +l/8, LDS chunk l%8); the lane's byte offsets
  // are fixed, the tile's key offset is scalar
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kr = (4 * i + wave) * 4 + (lane >> 4);
    koff[i] = (uint32_t)((kr * 128 + 8 * ((lane & 15) ^ (kr & 15))) * 2);
    const int vr = (4 * i + wave) * 8 + (lane >> 3);
    voff[i] = (uint32_t)((vr * lcap + 8 * ((lane & 7) ^ ((vr >> 1) & 7))) * 2);
  }
  auto dma_k = [&](int t) {
    uint8_t* ks = smem + (t & 1) * 16384;
#pragma unroll
    for (int i = 0; i < 4; ++i) kv_dma(kbase, kvext, (lds_void*)(ks + (4 * i + wave) * 1024), koff[i], t * AK * 256);
  };
  auto dma_v = [&](int t) {
    uint8_t* vs = smem + 32768 + (t & 1) * 16384;
#pragma unroll
    for (int i = 0; i < 4; ++i) kv_dma(vbase, kvext, (lds_void*)(vs + (4 * i + wave) * 1024), voff[i], t * AK * 2);
  };

  // per-lane LDS offsets: K row 32b + lo, chunk (2kk + hi) ^ (lo % 16); V^T row 32d + lo,
  // chunk (4b + 2u + hi) ^ ((lo / 2) % 8).  Stage, b and d are immediate offsets.
  int kofs[8], vofs[4];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kofs[kk] = lo * 256 + (((2 * kk + hi) ^ (lo & 15)) << 4);
#pragma unroll
  for (int bu = 0; bu < 4; ++bu) vofs[bu] = 32768 + lo * 128 + (((2 * bu + hi) ^ ((lo >> 1) & 7)) << 4);
  // S product i = 2kk + b: K fragment of 32-key block b, dims 16kk ..; O product j = 4bu + d:
  // V^T fragment of dims 32d .., keys 16bu ..
  auto kfrag = [&](auto ks_c, int i) {
    return *(const f16x8*)(smem + kofs[i / 2] + (decltype(ks_c)::value * 16384 + (i % 2) * 8192));
  };
  auto vfrag = [&](auto vs_c, int j) {
    return *(const f16x8*)(smem + vofs[j / 4] + (decltype(vs_c)::value * 16384 + (j % 4) * 4096));
  };

  f32x16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x16{};
  // mrun: the reference the scores are taken relative to (the row's running max, lagging
  // it by at most MAX_SLACK).  A tile's S product starts from -mrun (exact scale 1 only;
  // another scale multiplies first and subtracts after): it is issued after the previous
  // tile's max update, the last one before its own softmax.
  float mrun = 0.f, lrun = 0.f;
  const bool unit = scale == 1.f;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 ones = {(_Float16)1.f, (_Float16)1.f};
  f32x16 sc[2];   // S^T - mrun of the tile in hand: two 32-key blocks x this wave's 32 queries

  // Step t: the softmax of tile t, then the S product of tile t+1 interleaved with tile t's
  // exp2 (the VALU works while the MFMA pipe runs), then O^T += V^T P^T of tile t.
  auto step = [&](auto st_c, auto last_c, int t) {
    constexpr int ST = decltype(st_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    // K of tile t+1 and V^T of tile t have landed for every wave, and every wave is done
    // with K of tile t and V^T of tile t-1
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));   // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (!LAST) {
      if (t + 2 < tiles) dma_k(t + 2);
      dma_v(t + 1);
    }
    const int k0 = t * AK;
    if (!unit) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[b][r] = sc[b][r] * scale - mrun;
    }
    if (k0 + AK - 1 > minlim) {   // some key of this tile is hidden from some query
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * b + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (key > lim) sc[b][r] = -INFINITY;
        }
    }
    float m4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int b = c / 2, r0 = (c % 2) * 8;
      float m = fmaxf(fmaxf(sc[b][r0], sc[b][r0 + 1]), sc[b][r0 + 2]);
      m = fmaxf(fmaxf(m, sc[b][r0 + 3]), sc[b][r0 + 4]);
      m = fmaxf(fmaxf(m, sc[b][r0 + 5]), sc[b][r0 + 6]);
      m4[c] = fmaxf(m, sc[b][r0 + 7]);
    }
    const float mx = xmax32(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
    // the first tile always sets the reference (its key 0 is visible to every row)
    const bool move = t == 0 || mx > MAX_SLACK;
    if (__ballot(move)) {
      const float shift = move ? mx : 0.f;
      if (t > 0) {
        const float alpha = __builtin_amdgcn_exp2f(-shift);
        lrun *= alpha;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
      }
      mrun += shift;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[b][r] -= shift;
    }

    // S of tile t+1 from K stage ST^1, one MFMA a slot, with one pair of tile t's P values
    // (two exp2, an fp16 pack, and the row sum of the fp16 values the product uses) a slot
    // Fragment reads run KD MFMAs ahead of their use (an LDS read takes several 32-cycle MFMA
    // slots to return); the first KD V^T fragments of the O product go out in the last slots
    // of the S product, since V^T of tile t is in LDS since the step's barrier.
    constexpr int KD = 3;
    f32x16 sn[2];
    uint32_t pk[16];   // pair i: keys of S element (i / 8, 2 (i % 8)) and the next
    f16x8 kq[KD], vq[KD];
    if constexpr (!LAST) {
      const float c0 = unit ? -mrun : 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) sn[b][r] = c0;
#pragma unroll
      for (int i = 0; i < KD; ++i) kq[i] = kfrag(std::integral_constant<int, ST ^ 1>(), i);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (!LAST) {
        f16x8 kn = {};
        if (i + KD < 16) kn = kfrag(std::integral_constant<int, ST ^ 1>(), i + KD);
        sn[i % 2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kq[0], qf[i / 2], sn[i % 2], 0, 0, 0);
#pragma unroll
        for (int d = 0; d + 1 < KD; ++d) kq[d] = kq[d + 1];
        kq[KD - 1] = kn;
      }
      if (i >= 16 - KD) vq[i - (16 - KD)] = vfrag(std::integral_constant<int, ST>(), i - (16 - KD));
      const int b = i / 8, r = 2 * (i % 8);
      pk[i] = pack_f16x2(__builtin_amdgcn_exp2f(sc[b][r]), __builtin_amdgcn_exp2f(sc[b][r + 1]));
      lrun = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pk[i]), ones, lrun, false);
      __builtin_amdgcn_sched_barrier(0);
    }

    // O^T += V^T P^T of tile t over 4 steps of 16 keys (step bu: block bu / 2, rows 8 (bu % 2) ..)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      f16x8 vn = {};
      if (j + KD < 16) vn = vfrag(std::integral_constant<int, ST>(), j + KD);
      const int bu = j / 4;
      const f16x8 pb = __builtin_bit_cast(f16x8, u32x4{pk[4 * bu], pk[4 * bu + 1], pk[4 * bu + 2], pk[4 * bu + 3]});
      o[j % 4] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vq[0], pb, o[j % 4], 0, 0, 0);
#pragma unroll
      for (int d = 0; d + 1 < KD; ++d) vq[d] = vq[d + 1];
      vq[KD - 1] = vn;
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!LAST) {
      sc[0] = sn[0];
      sc[1] = sn[1];
    }
    // the row sum is complete here: its v_dot2 chain stays in the slots above instead of
    // sinking into the next step's max (its first use)
    asm volatile("" : "+v"(lrun));
  };

  // prologue: K of tile 0, then S of tile 0 (reference 0) while V^T 0 and K 1 move
  dma_k(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0x0 << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  dma_v(0);
  if (tiles > 1) dma_k(1);
#pragma unroll
  for (int b = 0; b < 2; ++b) sc[b] = f32x16{};
#pragma unroll
  for (int i = 0; i < 16; ++i)
    sc[i % 2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfrag(std::integral_constant<int, 0>(), i), qf[i / 2], sc[i % 2], 0, 0, 0);

  typedef std::integral_constant<int, 0> S0;
  typedef std::integral_constant<int, 1> S1;
  typedef std::integral_constant<bool, false> More;
  typedef std::integral_constant<bool, true> Last;
  int t = 0;
  for (; t + 2 < tiles; t += 2) {
    step(S0(), More(), t);
    step(S1(), More(), t + 1);
  }
  if (t + 1 < tiles) {
    step(S0(), More(), t);
    step(S1(), Last(), t + 1);
  } else {
    step(S0(), Last(), t);
  }

  const float inv = 1.f / xsum32(lrun);
  if (tq < n) {
    const int64_t o0 = (int64_t)tq * 4096 + h * 128 + 4 * hi;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int dim = 32 * d + 8 * r4;
        if constexpr (OF32)
          *(f32x4*)((float*)O + o0 + dim) = f32x4{o[d][4 * r4] * inv, o[d][4 * r4 + 1] * inv, o[d][4 * r4 + 2] * inv,
                                                  o[d][4 * r4 + 3] * inv};
        else
          *(u32x2*)((uint16_t*)O + o0 + dim) = u32x2{pack_bf16x2(o[d][4 * r4] * inv, o[d][4 * r4 + 1] * inv),
                                                     pack_bf16x2(o[d][4 * r4 + 2] * inv, o[d][4 * r4 + 3] * inv)};
      }
  }
}

hipError_t attend(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* vt, void* out, int n,
                  int q0, int p, int l, int64_t lcap, int b0, int b1, float scale, int of32, int64_t qld) {
  if (n <= 0) return hipSuccess;
  if (qld == 0) qld = n;
  if (qld < n) return hipErrorInvalidValue;
  // the DMA reads whole 64-key tiles: keys up to roundup(l, 64) - 1 must lie inside lcap
  // and a head's K (or V^T) is one buffer of lcap * 256 bytes
  if (lcap % AK || l > lcap || l <= 0 || lcap > (1 << 22)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((n + AQ - 1) / AQ), 32);
  if (of32)
    hipLaunchKernelGGL(k_attend<true>, grid, dim3(256), 0, s, q, k, vt, out, n, q0, p, l, lcap, b0, b1, scale, qld);
  else
    hipLaunchKernelGGL(k_attend<false>, grid, dim3(256), 0, s, q, k, vt, out, n, q0, p, l, lcap, b0, b1, scale, qld);
  return hipGetLastError();
}

}  // namespace exn
