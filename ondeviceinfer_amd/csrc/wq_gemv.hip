// Decode / small-batch kernels (M <= 64): HBM-streaming MFMA GEMV.
//
// Work unit: one 16-row tile x one 128-k block = one 1 KiB coalesced load
// (W4 tile layout) or two 16 B-per-lane loads (INT8 row-major).  A workgroup
// owns TPW tiles; its KSW waves split the k blocks, so each wave keeps
// U blocks of loads in flight and the waves' partial sums meet in LDS.
//
// Arithmetic: the weights are the MFMA A operand (16 rows), the activations
// the B operand (16 columns = 16 activation rows m, zero beyond M).  For W4
// each (tile, group) block accumulates sum_k (q - z) * x exactly in fp32
// (the fp16 (q - z) and the products are exact), then adds
// scale[n, g] * block_sum into the running fp32 result.  INT8 accumulates
// sum_k q * x and applies the row scale once at the end.
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

template <int MC>
__device__ __forceinline__ void load_x_w4(const half_t* __restrict__ x, int M, int K, int blk, int lane,
                                          half8_t (&xv)[MC][4]) {
  const int i = lane & 15, kb = lane >> 4;
#pragma unroll
  for (int mc = 0; mc < MC; ++mc) {
    const int m = mc * 16 + i;
    if (m < M) {
      const half_t* p = x + (size_t)m * K + blk * kW4BlockK + kb * 32;
#pragma unroll
      for (int w = 0; w < 4; ++w) xv[mc][w] = ld_h8(p + 8 * w);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) xv[mc][w] = half8_t{};
    }
  }
}

// Sum the per-wave partials (through LDS when KSW > 1) and hand each
// (m chunk, tile, lane) accumulator to `store`.  Register arrays are only
// indexed with compile-time indices.
template <int MC, int TPW, int KSW, typename Store>
__device__ __forceinline__ void skinny_epilogue(float4_t (&acc)[MC][TPW], int lane, int wave, Store store) {
  if constexpr (KSW == 1) {
#pragma unroll
    for (int mc = 0; mc < MC; ++mc)
#pragma unroll
      for (int t = 0; t < TPW; ++t) store(mc, t, lane, acc[mc][t]);
  } else {
    __shared__ float4_t red[KSW][MC * TPW][64];
#pragma unroll
    for (int mc = 0; mc < MC; ++mc)
#pragma unroll
      for (int t = 0; t < TPW; ++t) red[wave][mc * TPW + t][lane] = acc[mc][t];
    __syncthreads();
    for (int idx = threadIdx.x; idx < MC * TPW * 64; idx += 64 * KSW) {
      const int mt = idx >> 6, l = idx & 63;
      float4_t s = red[0][mt][l];
#pragma unroll
      for (int w2 = 1; w2 < KSW; ++w2) s += red[w2][mt][l];
      store(mt / TPW, mt % TPW, l, s);
    }
  }
}

// W4A16, M <= 16*MC.  grid.x = ceil(ntile / TPW); block = 64*KSW threads.
template <int MC, int TPW, int KSW, int U>
__global__ __launch_bounds__(64 * KSW) void w4_skinny_kernel(const half_t* __restrict__ x, int M, int K,
                                                             const uint4_t* __restrict__ tiles,
                                                             const uint8_t* __restrict__ meta, int N, int G,
                                                             half_t* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK, ngrp = K / G, bpg = G / kW4BlockK;
  const int b_lo = (wave * nblk) / KSW, b_hi = ((wave + 1) * nblk) / KSW;

  int tile[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) tile[t] = min((int)blockIdx.x * TPW + t, ntile - 1);

  float4_t acc[MC][TPW];
#pragma unroll
  for (int mc = 0; mc < MC; ++mc)
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[mc][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int b0 = b_lo; b0 < b_hi; b0 += U) {
    uint4_t wv[U][TPW];
    uint2_t sc[U][TPW];
    uint32_t zw[U][TPW];
    half8_t xv[U][MC][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int blk = b0 + u;
      if (blk < b_hi) {
        const int g = blk / bpg;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          wv[u][t] = tiles[((size_t)tile[t] * nblk + blk) * 64 + lane];
          const uint8_t* mp = meta + ((size_t)tile[t] * ngrp + g) * kW4MetaBytes;
          sc[u][t] = *reinterpret_cast<const uint2_t*>(mp + 8 * kb);
          zw[u][t] = *reinterpret_cast<const uint32_t*>(mp + 32 + 4 * (i >> 3));
        }
        load_x_w4<MC>(x, M, K, blk, lane, xv[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (b0 + u < b_hi) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          uint32_t c_lo, c_hi;
          w4_zero_consts((zw[u][t] >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
          float4_t cg[MC];
#pragma unroll
          for (int mc = 0; mc < MC; ++mc) cg[mc] = float4_t{0.f, 0.f, 0.f, 0.f};
          const uint32_t words[4] = {wv[u][t].x, wv[u][t].y, wv[u][t].z, wv[u][t].w};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const half8_t a = w4_word_to_h8(words[w], c_lo, c_hi);
#pragma unroll
            for (int mc = 0; mc < MC; ++mc) cg[mc] = mfma16(a, xv[u][mc][w], cg[mc]);
          }
          const half4_t s4 = __builtin_bit_cast(half4_t, sc[u][t]);
#pragma unroll
          for (int mc = 0; mc < MC; ++mc)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[mc][t][v] += (float)s4[v] * cg[mc][v];
        }
      }
    }
  }

  // Accumulator lane l holds rows 4*(l/16)+v of the tile, column m = mc*16 + l%16.
  skinny_epilogue<MC, TPW, KSW>(acc, lane, wave, [&](int mc, int t, int l, float4_t s) {
    const int m = mc * 16 + (l & 15);
    const int t_out = (int)blockIdx.x * TPW + t;
    const int n0 = t_out * 16 + 4 * (l >> 4);
    if (m < M && t_out < ntile && n0 < N) {
      half4_t o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (half_t)s[v];
      *reinterpret_cast<half4_t*>(y + (size_t)m * N + n0) = o;
    }
  });
}

// W4A16, M <= 16*MC, as a continuous load ring: each wave keeps its next U
// k blocks (the TPW tiles' weights and scale/zero records and the MC
// activation fragments) in flight and refills a slot as soon as it is
// consumed.  Every load goes through a buffer resource whose range ends at
// the wave's last block (weights), the tile's last group (records) or row M
// (activations), so loads past an end are unconditional and read zeros
// without touching memory; the per-block math and its order are those of
// w4_skinny_kernel.  Used for K <= 2^25, where the 32-bit lane offsets
// (up to 15 rows of x plus K) and the per-tile weight ranges fit.
template <int MC, int TPW>
struct SkinnySlot {
  uint4_t w[TPW];
  uint2_t sc[TPW];
  uint32_t zw[TPW];
  half8_t xv[MC][4];
};

template <int MC, int TPW, int KSW, int U>
__global__ __launch_bounds__(64 * KSW) void w4_skinny_ring_kernel(const half_t* __restrict__ x, int M, int K,
                                                                  const uint4_t* __restrict__ tiles,
                                                                  const uint8_t* __restrict__ meta, int N, int G,
                                                                  half_t* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK, ngrp = K / G, bpg = G / kW4BlockK;
  const int b_lo = (wave * nblk) / KSW, nb = ((wave + 1) * nblk) / KSW - b_lo;

  __amdgpu_buffer_rsrc_t rw[TPW], rm[TPW], rx[MC];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tile = min((int)blockIdx.x * TPW + t, ntile - 1);
    rw[t] = buf_rsrc(tiles + ((size_t)tile * nblk + b_lo) * 64, (int64_t)nb * 1024);
    rm[t] = buf_rsrc(meta + (size_t)tile * ngrp * kW4MetaBytes, (int64_t)ngrp * kW4MetaBytes);
  }
#pragma unroll
  for (int mc = 0; mc < MC; ++mc)
    rx[mc] = buf_rsrc(x + (size_t)mc * 16 * K, (int64_t)min(max(M - mc * 16, 0), 16) * K * 2);
  const uint32_t xo = (uint32_t)((i * K + kb * 32) * 2);

  auto load = [&](SkinnySlot<MC, TPW>& s, int r) {
    // r: block index relative to b_lo; past the wave's range every load is out of bounds.
    const bool in = r < nb;
    const uint32_t wo = (uint32_t)r * 1024;
    const uint32_t mo = in ? (uint32_t)(((b_lo + r) / bpg) * kW4MetaBytes) : 0x7ffff000u;
    const uint32_t xs = in ? (uint32_t)(b_lo + r) * kW4BlockK * 2 : 0x7ffff000u;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      s.w[t] = __builtin_amdgcn_raw_buffer_load_b128(rw[t], (uint32_t)lane * 16, wo, kNtPolicy);
      s.sc[t] = __builtin_bit_cast(uint2_t, __builtin_amdgcn_raw_buffer_load_b64(rm[t], (uint32_t)kb * 8, mo, 0));
      s.zw[t] = __builtin_amdgcn_raw_buffer_load_b32(rm[t], 32 + (uint32_t)(i >> 3) * 4, mo, 0);
    }
#pragma unroll
    for (int mc = 0; mc < MC; ++mc)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        s.xv[mc][w] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rx[mc], xo + 16 * w, xs, 0));
  };

  float4_t acc[MC][TPW];
#pragma unroll
  for (int mc = 0; mc < MC; ++mc)
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[mc][t] = float4_t{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](const SkinnySlot<MC, TPW>& s) {
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      uint32_t c_lo, c_hi;
      w4_zero_consts((s.zw[t] >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
      float4_t cg[MC];
#pragma unroll
      for (int mc = 0; mc < MC; ++mc) cg[mc] = float4_t{0.f, 0.f, 0.f, 0.f};
      const uint32_t words[4] = {s.w[t].x, s.w[t].y, s.w[t].z, s.w[t].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const half8_t a = w4_word_to_h8(words[w], c_lo, c_hi);
#pragma unroll
        for (int mc = 0; mc < MC; ++mc) cg[mc] = mfma16(a, s.xv[mc][w], cg[mc]);
      }
      const half4_t s4 = __builtin_bit_cast(half4_t, s.sc[t]);
#pragma unroll
      for (int mc = 0; mc < MC; ++mc)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[mc][t][v] += (float)s4[v] * cg[mc][v];
    }
  };

  SkinnySlot<MC, TPW> ring[U];
#pragma unroll
  for (int u = 0; u < U; ++u) load(ring[u], u);
  for (int r0 = 0; r0 < nb; r0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (r0 + u < nb) consume(ring[u]);
      load(ring[u], r0 + u + U);
    }
  }

  skinny_epilogue<MC, TPW, KSW>(acc, lane, wave, [&](int mc, int t, int l, float4_t s) {
    const int m = mc * 16 + (l & 15);
    const int t_out = (int)blockIdx.x * TPW + t;
    const int n0 = t_out * 16 + 4 * (l >> 4);
    if (m < M && t_out < ntile && n0 < N) {
      half4_t o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (half_t)s[v];
      *reinterpret_cast<half4_t*>(y + (size_t)m * N + n0) = o;
    }
  });
}

// INT8 x fp16, M <= 16*MC, weights [N, K] row-major int8, fp16 row scale.
// Lane (i, kb) of block blk reads row 16t+i at k = 128*blk + 16*kb + [0,16)
// and 128*blk + 64 + 16*kb + [0,16); each 16 B feeds two MFMA k-steps.
template <int MC, int TPW, int KSW, int U>
__global__ __launch_bounds__(64 * KSW) void w8_skinny_kernel(const half_t* __restrict__ x, int M, int K,
                                                             const int8_t* __restrict__ q,
                                                             const half_t* __restrict__ scale,
                                                             const half_t* __restrict__ bias, int N,
                                                             half_t* __restrict__ y, W8Layout wl8) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW8BlockK;
  const int b_lo = (wave * nblk) / KSW, b_hi = ((wave + 1) * nblk) / KSW;
  const int blk_bytes = wl8.block_bytes(), p1 = wl8.piece1();

  const int8_t* rowp[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tt = min((int)blockIdx.x * TPW + t, ntile - 1);   // tiles (rows) past the end: read, never stored
    rowp[t] = q + wl8.lane_base(tt, lane, N, K);
  }

  float4_t acc[MC][TPW];
#pragma unroll
  for (int mc = 0; mc < MC; ++mc)
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[mc][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int b0 = b_lo; b0 < b_hi; b0 += U) {
    uint4_t wa[U][TPW], wb[U][TPW];
    half8_t xv[U][MC][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int blk = b0 + u;
      if (blk < b_hi) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          wa[u][t] = *reinterpret_cast<const uint4_t*>(rowp[t] + (size_t)blk * blk_bytes);
          wb[u][t] = *reinterpret_cast<const uint4_t*>(rowp[t] + (size_t)blk * blk_bytes + p1);
        }
#pragma unroll
        for (int mc = 0; mc < MC; ++mc) {
          const int m = mc * 16 + i;
          if (m < M) {
            const half_t* p = x + (size_t)m * K + blk * kW8BlockK + 16 * kb;
            xv[u][mc][0] = ld_h8(p);
            xv[u][mc][1] = ld_h8(p + 8);
            xv[u][mc][2] = ld_h8(p + 64);
            xv[u][mc][3] = ld_h8(p + 72);
          } else {
#pragma unroll
            for (int w = 0; w < 4; ++w) xv[u][mc][w] = half8_t{};
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (b0 + u < b_hi) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          const half8_t a0 = i8x8_to_h8(wa[u][t].x, wa[u][t].y);
          const half8_t a1 = i8x8_to_h8(wa[u][t].z, wa[u][t].w);
          const half8_t a2 = i8x8_to_h8(wb[u][t].x, wb[u][t].y);
          const half8_t a3 = i8x8_to_h8(wb[u][t].z, wb[u][t].w);
#pragma unroll
          for (int mc = 0; mc < MC; ++mc) {
            acc[mc][t] = mfma16(a0, xv[u][mc][0], acc[mc][t]);
            acc[mc][t] = mfma16(a1, xv[u][mc][1], acc[mc][t]);
            acc[mc][t] = mfma16(a2, xv[u][mc][2], acc[mc][t]);
            acc[mc][t] = mfma16(a3, xv[u][mc][3], acc[mc][t]);
          }
        }
      }
    }
  }

  skinny_epilogue<MC, TPW, KSW>(acc, lane, wave, [&](int mc, int t, int l, float4_t s) {
    const int m = mc * 16 + (l & 15);
    const int t_out = (int)blockIdx.x * TPW + t;
    const int n0 = t_out * 16 + 4 * (l >> 4);
    if (m < M && t_out < ntile && n0 < N) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = n0 + v;
        if (n < N) {
          float r = s[v] * (float)scale[n];
          if (bias) r += (float)bias[n];
          y[(size_t)m * N + n] = (half_t)r;
        }
      }
    }
  });
}

// Decode GEMV for M <= MM (MM = 1 or 4), W4 tiles or INT8 row-major weights.
//
// One workgroup per 16-row tile; its ksw waves split the tile's K/128
// blocks: every wave owns NB consecutive blocks and the first `extra` waves
// one more (NB is a template parameter, so the bulk of the loads is
// straight-line code).  A wave first loads its slice of x[M, K] and (W4) the
// scale/zero records of its groups, then keeps D ~ NB/2 weight blocks in
// flight (non-temporal loads in a compile-time ring, each consumed behind an
// exact vmcnt and refilled at once), so the math of the first blocks overlaps
// the arrival of the rest.  x and the records go to a wave-private LDS region,
// so the only workgroup barrier is the final cross-wave sum.
//
// W4 arithmetic here differs from the skinny kernels: the weights enter the
// MFMA as 1024+q / 1024+16q (four VALU ops per word, against x with the
// 16q positions pre-divided by 16), and four more MFMAs per block with the
// row's zero fragment take off (1024 + z) / (1024 + 16z).  The block sum is
// then sum_k (q - z) x up to fp32 rounding of terms ~1024|x| (relative error
// ~1e-6 of the block), and the matrix pipe, idle at M = 1, absorbs the work
// that would otherwise cost two more VALU ops per word.  INT8 likewise feeds
// 1152+q and takes 1152 * x off with a constant fragment.  Rows m >= M read row M-1
// (in bounds) and are never stored; reads past the end of x are clamped.
enum class WFmt { W4, W8 };
// The flat kernel's fmt_arg: W4 = log2 of the 128-k blocks per group; W8 =
// the weight layout (W8Layout::tiled: 1 INT8 tiles, 0 row-major [N, K]).

// Widest workgroup (in waves) each instantiation is compiled for: the
// register budget of a 1024-thread group (128 VGPRs) holds about 12 W4 or 8
// INT8 blocks per wave.
template <int NB, WFmt F>
constexpr int flat_max_ksw() { return NB <= (F == WFmt::W4 ? 12 : 8) ? 16 : 8; }

// Waves per SIMD each instantiation must reach: the wide-N plans launch
// about 4.25 waves per SIMD (e.g. 1088 four-wave workgroups for 5120->17408),
// so NB <= 10 is held to 96 VGPRs (five waves per SIMD) and the whole grid is
// resident at once instead of leaving a second launch wave.  The fused
// RMSNorm / SiLU·up prologues fit in the same budget (no scratch).
template <int NB, WFmt F>
constexpr int flat_min_waves() { return NB <= (F == WFmt::W4 ? 10 : 6) ? 5 : 1; }

template <WFmt F>
struct BlockRegs;
template <>
struct BlockRegs<WFmt::W4> { uint4_t w; };
template <>
struct BlockRegs<WFmt::W8> { uint4_t a, b; };

// k offset (in halves, inside one 128-k block) of MFMA step w for lane slot kb.
template <WFmt F>
__device__ __forceinline__ int blk_kcol(int kb, int w) {
  return F == WFmt::W4 ? kb * 32 + 8 * w : kb * 16 + 8 * (w & 1) + 64 * (w >> 1);
}

// Decode-step fusions of the flat GEMV (M = 1, W4 and INT8): how x is formed while it
// is staged, and the residual / sum-of-squares epilogue.
enum class XMode {
  Plain,     // x as given
  RmsNorm,   // x <- w * fp16(x * rsqrt(sum(sumsq_in) / K + eps)): the next RMSNorm
  SiluMul,   // x is [gate | up] of length 2K: x <- fp16(fp16(silu(gate)) * up)
};

struct FuseArgs {
  const half_t* norm_w;    // RmsNorm: weight [K]
  const float* sumsq_in;   // RmsNorm: sums of squares of x, one per 16-row tile of its producer (<= 512)
  int sumsq_count;
  float eps;
  const half_t* residual;  // y = residual + x.W^T (fp16 add); may alias y
  float* sumsq_out;        // per-16-row tile sum of squares of y (for the next RmsNorm)
};

// Eight (gate, up) pairs -> fp16(fp16(silu(gate)) * up), as F.silu on an
// fp16 tensor followed by an fp16 product (silu in fp32, see silu_f).
__device__ __forceinline__ uint4_t silu_mul8(uint4_t gv, uint4_t uv) {
  const half8_t gh = __builtin_bit_cast(half8_t, gv), uh = __builtin_bit_cast(half8_t, uv);
  half8_t o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] = (half_t)silu_f((float)gh[e]) * uh[e];
  }
  return __builtin_bit_cast(uint4_t, o);
}

template <int NB, int MM, WFmt F, XMode XM = XMode::Plain>
__global__ __launch_bounds__((64 * flat_max_ksw<NB, F>()), (flat_min_waves<NB, F>())) void gemv_flat_kernel(
    const half_t* __restrict__ x, int M, int K, const void* __restrict__ wsrc, const void* __restrict__ wmeta,
    const half_t* __restrict__ bias, int N, int fmt_arg, half_t* y, int S,
    float4_t* __restrict__ ws_part, uint32_t* __restrict__ ws_cnt, FuseArgs fz) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int NBX = NB + 1;                                // staged slice length (blocks)
  constexpr int D = NB <= 3 ? NB : ((NB + 1) / 2 < 3 ? 3 : (NB + 1) / 2);   // weight blocks in flight
  constexpr int kXChunks = MM * NBX * 16;                    // 16 B chunks of the x slice
  constexpr int kXPerLane = (kXChunks + 63) / 64;
  constexpr int kXBytes = kXPerLane * 64 * 16;
  constexpr int kMetaChunks = F == WFmt::W4 ? (NBX + 1) * kW4MetaBytes / 8 : 0;
  constexpr int kMPerLane = (kMetaChunks + 63) / 64;
  constexpr int kWaveBytes = kXBytes + kMPerLane * 64 * 8;
  const int ksw = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x;
  const int nblk = K / kW4BlockK;
  const int split = blockIdx.y;                               // k range [base, base + nblk_s) of S
  const int base = (split * nblk) / S;
  const int nblk_s = ((split + 1) * nblk) / S - base;
  const int extra = nblk_s - NB * ksw;                        // 0 <= extra <= ksw
  const bool more = wave < extra;
  const int b0 = base + wave * NB + min(wave, extra);
  uint8_t* wl = smem + wave * kWaveBytes;
  half_t* xl = reinterpret_cast<half_t*>(wl);
  uint8_t* ml = wl + kXBytes;

  // 1) x slice (and the W4 records): small, mostly L2 hits.  The fused
  //    modes (M = 1 only) also fetch what they transform x with: RmsNorm the
  //    norm weight and the producer's per-tile sums of squares, SiluMul the
  //    up half of a [2K] x.  The transform itself waits until the weight
  //    loads below are in flight.
  uint4_t xr[kXPerLane];
  uint4_t xa[XM == XMode::Plain ? 1 : kXPerLane];   // up half (SiluMul) or norm weight (RmsNorm)
  // The producer's sums of squares (<= 512): 16-byte loads of the first
  // count & ~3 (two per lane) and one load of the remainder.
  constexpr int kSqPerLane = 2;
  float4_t sq[XM == XMode::RmsNorm ? kSqPerLane : 1];
  float sqt = 0.f;
  auto x_offset = [&](int j) { return min(b0 * kW4BlockK + (min(lane + 64 * j, kXChunks - 1) % (NBX * 16)) * 8, K - 8); };
#pragma unroll
  for (int j = 0; j < kXPerLane; ++j) {
    const int m = min(min(lane + 64 * j, kXChunks - 1) / (NBX * 16), M - 1);
    const int off = x_offset(j);
    xr[j] = *reinterpret_cast<const uint4_t*>(x + (size_t)m * K + off);
    if constexpr (XM == XMode::SiluMul) xa[j] = *reinterpret_cast<const uint4_t*>(x + K + off);
    if constexpr (XM == XMode::RmsNorm) xa[j] = *reinterpret_cast<const uint4_t*>(fz.norm_w + off);
  }
  if constexpr (XM == XMode::RmsNorm) {
    // Clamped loads; entries past the count are dropped when summed.  With
    // fewer than 4 sums there is no whole float4 to read (a uniform branch).
#pragma unroll
    for (int u = 0; u < kSqPerLane; ++u)
      sq[u] = fz.sumsq_count >= 4
                  ? reinterpret_cast<const float4_t*>(fz.sumsq_in)[min(lane + 64 * u, fz.sumsq_count / 4 - 1)]
                  : float4_t{0.f, 0.f, 0.f, 0.f};
    sqt = fz.sumsq_in[min((fz.sumsq_count & ~3) + (lane & 3), fz.sumsq_count - 1)];
  }
  // The fused residual (M = 1; wave 0 stores the tile) is fetched now so
  // that its latency is not added after the reduction (for NB <= 8, where the
  // two registers are free).  Every split reads it before it counts in, so
  // an aliased y still holds the old value here.
  constexpr bool kEarlyResidual = NB <= 8;
  const bool has_x = i < M;
  const int n0 = tile * 16 + 4 * kb;
  half4_t res = {};
  if (kEarlyResidual && fz.residual && wave == 0 && has_x && n0 < N)
    res = *reinterpret_cast<const half4_t*>(fz.residual + n0);
  int g_lo = 0;
  uint2_t mr[kMPerLane > 0 ? kMPerLane : 1];
  if constexpr (F == WFmt::W4) {
    const int ngrp = nblk >> fmt_arg;
    g_lo = b0 >> fmt_arg;
    const int g_hi = min((b0 + NB) >> fmt_arg, ngrp - 1);
    const int meta_chunks = (g_hi - g_lo + 1) * (kW4MetaBytes / 8);
    const uint2_t* mg = reinterpret_cast<const uint2_t*>(reinterpret_cast<const uint8_t*>(wmeta) +
                                                         ((size_t)tile * ngrp + g_lo) * kW4MetaBytes);
#pragma unroll
    for (int j = 0; j < kMPerLane; ++j) mr[j] = mg[min(lane + 64 * j, meta_chunks - 1)];
  }

  // 2) the first D weight blocks (and the optional extra one) in flight
  //    before anything is used; the rest refill the ring as it drains.
  const uint4_t* wp;
  if constexpr (F == WFmt::W4) {
    wp = reinterpret_cast<const uint4_t*>(wsrc) + ((size_t)tile * nblk + b0) * 64 + lane;
  } else {
    const W8Layout wl8{fmt_arg};
    wp = reinterpret_cast<const uint4_t*>(reinterpret_cast<const int8_t*>(wsrc) + wl8.lane_base(tile, lane, N, K) +
                                          (size_t)b0 * wl8.block_bytes());
  }
  // INT8: a block and piece 1 in 16-byte units (row-major 8 / 4, tiles 128 / 64).
  const int w8_blk = F == WFmt::W8 ? W8Layout{fmt_arg}.block_bytes() / 16 : 0;
  const int w8_p1 = F == WFmt::W8 ? W8Layout{fmt_arg}.piece1() / 16 : 0;
  auto load_block = [&](BlockRegs<F>& r, int s2) {
    if constexpr (F == WFmt::W4) {
      r.w = __builtin_nontemporal_load(wp + s2 * 64);
    } else {
      r.a = __builtin_nontemporal_load(wp + s2 * w8_blk);
      r.b = __builtin_nontemporal_load(wp + s2 * w8_blk + w8_p1);
    }
  };
  BlockRegs<F> ring[D], xtra;
#pragma unroll
  for (int s2 = 0; s2 < D; ++s2) load_block(ring[s2], s2);
  if (more) load_block(xtra, NB);

  // 3) transform x for the fused modes, then park x and the records in this
  //    wave's LDS region (every lane stores, so the loads above stay ahead of
  //    the weight loads).
  if constexpr (XM == XMode::SiluMul) {
#pragma unroll
    for (int j = 0; j < kXPerLane; ++j) xr[j] = silu_mul8(xr[j], xa[j]);
  }
  if constexpr (XM == XMode::RmsNorm) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kSqPerLane; ++u)
      ss += lane + 64 * u < fz.sumsq_count / 4 ? (sq[u][0] + sq[u][1]) + (sq[u][2] + sq[u][3]) : 0.f;
    ss += lane < (fz.sumsq_count & 3) ? sqt : 0.f;
    const float r = rsqrtf(wave_sum_rl(ss) / (float)K + fz.eps);
#pragma unroll
    for (int j = 0; j < kXPerLane; ++j) xr[j] = rms_scale8(xr[j], xa[j], r);
  }
#pragma unroll
  for (int j = 0; j < kXPerLane; ++j)
    reinterpret_cast<uint4_t*>(xl)[lane + 64 * j] = F == WFmt::W4 ? w4_prescale_x(xr[j]) : xr[j];
  if constexpr (F == WFmt::W4) {
#pragma unroll
    for (int j = 0; j < kMPerLane; ++j) reinterpret_cast<uint2_t*>(ml)[lane + 64 * j] = mr[j];
  }

  half8_t xv[4] = {half8_t{}, half8_t{}, half8_t{}, half8_t{}};   // columns m >= M stay zero
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  auto consume = [&](const BlockRegs<F>& wb, int s2) {
    if (has_x) {
      const half_t* xp = xl + (i * NBX + s2) * kW4BlockK;
#pragma unroll
      for (int w = 0; w < 4; ++w) xv[w] = ld_h8(xp + blk_kcol<F>(kb, w));
    }
    if constexpr (F == WFmt::W4) {
      const uint8_t* rec = ml + (((b0 + s2) >> fmt_arg) - g_lo) * kW4MetaBytes;
      const uint2_t sc = *reinterpret_cast<const uint2_t*>(rec + 8 * kb);
      const uint32_t zw = *reinterpret_cast<const uint32_t*>(rec + 32 + 4 * (i >> 3));
      // The zero-point terms go through the matrix pipe (they need only x
      // and z, so they issue before the weights land); the weights take four
      // VALU ops per word.
      const half8_t zf = w4_zero_frag((zw >> (4 * (i & 7))) & 0xFu);
      float4_t cg = {0.f, 0.f, 0.f, 0.f};
      cg = mfma16(zf, xv[0], cg);
      cg = mfma16(zf, xv[1], cg);
      cg = mfma16(zf, xv[2], cg);
      cg = mfma16(zf, xv[3], cg);
      cg = mfma16(w4_word_to_h8_raw(wb.w.x), xv[0], cg);
      cg = mfma16(w4_word_to_h8_raw(wb.w.y), xv[1], cg);
      cg = mfma16(w4_word_to_h8_raw(wb.w.z), xv[2], cg);
      cg = mfma16(w4_word_to_h8_raw(wb.w.w), xv[3], cg);
      const half4_t s4 = __builtin_bit_cast(half4_t, sc);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[v] = __builtin_fmaf((float)s4[v], cg[v], acc[v]);
    } else {
      const half8_t bf = i8_bias_frag();
#pragma unroll
      for (int w = 0; w < 4; ++w) acc = mfma16(bf, xv[w], acc);
      acc = mfma16(i8x8_to_h8_raw(wb.a.x, wb.a.y), xv[0], acc);
      acc = mfma16(i8x8_to_h8_raw(wb.a.z, wb.a.w), xv[1], acc);
      acc = mfma16(i8x8_to_h8_raw(wb.b.x, wb.b.y), xv[2], acc);
      acc = mfma16(i8x8_to_h8_raw(wb.b.z, wb.b.w), xv[3], acc);
    }
  };
#pragma unroll
  for (int s2 = 0; s2 < NB; ++s2) {
    consume(ring[s2 % D], s2);
    if (s2 + D < NB) load_block(ring[s2 % D], s2 + D);   // compile-time condition
  }
  if (more) consume(xtra, NB);

  float4_t* red = reinterpret_cast<float4_t*>(smem + ksw * kWaveBytes);
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  float4_t sum = red[lane];
  for (int w2 = 1; w2 < ksw; ++w2) sum += red[w2 * 64 + lane];
  if (S > 1) {
    // Cross-workgroup sum over the S k-splits of this tile: every split
    // publishes its partial, the last to arrive adds them in split order (so
    // the result does not depend on arrival order) and re-arms the counter.
    // Partials move with 16-byte sc1 (device-coherent) buffer accesses and
    // the counter with a device-scope atomic; the vmcnt(0) wait orders this
    // lane's partial before the increment.  A fence here would write back
    // and invalidate the whole L2 in every workgroup.
    coherent_store16(ws_part, (uint32_t)((((size_t)tile * S + split) * 64 + lane) * 16),
                     __builtin_bit_cast(uint4_t, sum));
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    uint32_t prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(&ws_cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != (uint32_t)(S - 1)) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t base = (uint32_t)(((size_t)tile * S * 64 + lane) * 16);
    sum = __builtin_bit_cast(float4_t, coherent_load16(ws_part, base));
    for (int s2 = 1; s2 < S; ++s2) sum += __builtin_bit_cast(float4_t, coherent_load16(ws_part, base + s2 * 1024));
    if (lane == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (has_x) {
    // Lane (i, kb) holds outputs n0 .. n0 + 3 of row i.  W4 applies the
    // group scales per block; INT8 applies the row scale (and bias) here.
    half4_t o;
    if constexpr (F == WFmt::W4) {
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (half_t)sum[v];
    } else {
      const half_t* scale = reinterpret_cast<const half_t*>(wmeta);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = min(n0 + v, N - 1);
        float r = sum[v] * (float)scale[n];
        if (bias) r += (float)bias[n];
        o[v] = (half_t)r;
      }
    }
    // W4 rows come in whole 16-row tiles; INT8 stores a quad at once when
    // every row of y keeps 8-byte alignment, else element-wise.
    const bool quad = F == WFmt::W4 || ((N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0);
    if (quad && n0 < N) {
      // Fused residual (M = 1): y = residual + fp16(x.W^T), as the
      // reference adds the rounded projection to the fp16 residual.
      if (fz.residual) o = (kEarlyResidual ? res : *reinterpret_cast<const half4_t*>(fz.residual + n0)) + o;
      *reinterpret_cast<half4_t*>(y + (size_t)i * N + n0) = o;
    } else if (!quad) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (n0 + v < N) y[(size_t)i * N + n0 + v] = o[v];
    }
    if (fz.sumsq_out) {
      // Lanes 0, 16, 32, 48 hold the tile's 16 outputs (M = 1).
      float q = 0.f;
      if (n0 < N) {
#pragma unroll
        for (int v = 0; v < 4; ++v) q += (float)o[v] * (float)o[v];
      }
      q = (lane_f(q, 0) + lane_f(q, 16)) + (lane_f(q, 32) + lane_f(q, 48));
      if (lane == 0) fz.sumsq_out[tile] = q;
    }
  }
}

// Any-shape INT8 x fp16 linear: one wavefront per output (m, n), lanes
// stride over k, fp32 accumulation, row scale applied at the end.  Serves
// shapes the tiled kernels do not take (k % 128 != 0 or unaligned operands).
__global__ __launch_bounds__(256) void w8_generic_kernel(const half_t* __restrict__ x, int M, int K,
                                                         const int8_t* __restrict__ q,
                                                         const half_t* __restrict__ scale,
                                                         const half_t* __restrict__ bias, int N,
                                                         half_t* __restrict__ y) {
  const int64_t out = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (out >= (int64_t)M * N) return;
  const int m = (int)(out / N), n = (int)(out % N);
  float acc = 0.0f;
  for (int c = lane; c < K; c += 64) acc += (float)x[(size_t)m * K + c] * (float)q[(size_t)n * K + c];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    float r = acc * (float)scale[n];
    if (bias) r += (float)bias[n];
    y[(size_t)m * N + n] = (half_t)r;
  }
}

struct SkinnyCfg {
  int tpw, ksw;
};

// Prefetch depth (k blocks in flight per wave): deep for M <= 16, where the
// activation fragments are tiny; shallower when several 16-row chunks of
// activations share the registers.
template <int MC>
constexpr int skinny_unroll() { return MC == 1 ? 4 : 2; }

// Largest k-split per workgroup: 16 waves for M <= 16 with one tile per
// wave, 8 with more tiles (their registers exceed a 1024-thread group's
// 128 VGPRs); 4 above M = 16.
template <int MC, int TPW>
constexpr int skinny_max_ksw() { return MC == 1 ? (TPW == 1 ? 16 : 8) : 4; }

// Enough waves to cover the machine (256 CUs) several times over while each
// wave keeps at least two k blocks.  W4 waves take 2 tiles (4 from 1024
// tiles on) so that each activation fragment read from L2 feeds 2 or 4
// tiles' MFMAs, and at least 2 waves split k: from sweeps of the fused
// QKV, gate_up and lm_head shapes at M = 8 .. 64 on MI355X (gate_up M = 8:
// 42 -> 33 us, lm_head M = 32: 229 -> 155 us against one tile per wave).
SkinnyCfg pick_skinny(int ntile, int nblk, int mc, bool w4) {
  SkinnyCfg c{mc >= 2 ? 2 : 1, 1};
  if (w4) c.tpw = ntile >= 1024 ? 4 : 2;
  const int max_ksw = mc == 1 ? (c.tpw == 1 ? 16 : 8) : 4;
  const int groups = (ntile + c.tpw - 1) / c.tpw;
  int ksw = 1;
  while (ksw < max_ksw && groups * ksw < 2048 && nblk / (ksw * 2) >= 2) ksw *= 2;
  if (w4 && ksw == 1 && nblk >= 4) ksw = 2;
  c.ksw = ksw;
  return c;
}

// The load ring pays where a wave streams many blocks per tile group: wide N
// (>= 1024 tiles, four tiles per wave) or long K at M <= 16, and at
// 33 <= M <= 48.  The batch form stays ahead on the fused QKV shape at
// M <= 16, at 17 <= M <= 32 and at M > 48 (MI355X, same box: gate_up M = 8
// 31.5 -> 26.9 us, lm_head M = 8 98.6 -> 84.4 us, 17408->5120 M = 8
// 21.4 -> 19.8 us, gate_up M = 33 67.7 -> 54.0 us; QKV M = 8 9.0 against
// 9.5 us, gate_up M = 32 46.6 against 49.9 us, lm_head M = 64 235 against
// 238 us).  Both give the same bits.
bool skinny_use_ring(int mc, int ntile, int nblk, int K) {
  if (K > (1 << 25)) return false;   // the ring's lane offsets are 32-bit
  if (mc == 1) return ntile >= 1024 || nblk >= 64;
  return mc == 3;
}

template <int MC, int TPW, int KSW>
int launch_w4_skinny_cfg(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         half_t* y, hipStream_t s) {
  const int ntile = (N + 15) / 16;
  const unsigned grid = (unsigned)((ntile + TPW - 1) / TPW);
  if (skinny_use_ring(MC, ntile, K / kW4BlockK, K))
    hipLaunchKernelGGL((w4_skinny_ring_kernel<MC, TPW, KSW, 2>), dim3(grid), dim3(64 * KSW), 0, s, x, M, K, tiles,
                       meta, N, G, y);
  else
    hipLaunchKernelGGL((w4_skinny_kernel<MC, TPW, KSW, skinny_unroll<MC>()>), dim3(grid), dim3(64 * KSW), 0, s, x, M,
                       K, tiles, meta, N, G, y);
  return check_launch("w4_skinny");
}

template <int MC, int TPW>
int launch_w4_skinny_k(int ksw, const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N,
                       int G, half_t* y, hipStream_t s) {
  switch (ksw) {
    case 1: return launch_w4_skinny_cfg<MC, TPW, 1>(x, M, K, tiles, meta, N, G, y, s);
    case 2: return launch_w4_skinny_cfg<MC, TPW, 2>(x, M, K, tiles, meta, N, G, y, s);
    case 4: return launch_w4_skinny_cfg<MC, TPW, 4>(x, M, K, tiles, meta, N, G, y, s);
    default:
      if constexpr (skinny_max_ksw<MC, TPW>() >= 16) {
        if (ksw == 8) return launch_w4_skinny_cfg<MC, TPW, 8>(x, M, K, tiles, meta, N, G, y, s);
        return launch_w4_skinny_cfg<MC, TPW, 16>(x, M, K, tiles, meta, N, G, y, s);
      } else if constexpr (skinny_max_ksw<MC, TPW>() >= 8) {
        return launch_w4_skinny_cfg<MC, TPW, 8>(x, M, K, tiles, meta, N, G, y, s);
      } else {
        return launch_w4_skinny_cfg<MC, TPW, 4>(x, M, K, tiles, meta, N, G, y, s);
      }
  }
}

template <int MC, int TPW, int KSW>
int launch_w8_skinny_cfg(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias,
                         int N, half_t* y, hipStream_t s, int tiled) {
  const int ntile = (N + 15) / 16;
  const unsigned grid = (unsigned)((ntile + TPW - 1) / TPW);
  hipLaunchKernelGGL((w8_skinny_kernel<MC, TPW, KSW, skinny_unroll<MC>()>), dim3(grid), dim3(64 * KSW), 0, s, x, M, K,
                     q, scale, bias, N, y, W8Layout{tiled});
  return check_launch("w8_skinny");
}

template <int MC, int TPW>
int launch_w8_skinny_k(int ksw, const half_t* x, int M, int K, const int8_t* q, const half_t* scale,
                       const half_t* bias, int N, half_t* y, hipStream_t s, int tiled) {
  switch (ksw) {
    case 1: return launch_w8_skinny_cfg<MC, TPW, 1>(x, M, K, q, scale, bias, N, y, s, tiled);
    case 2: return launch_w8_skinny_cfg<MC, TPW, 2>(x, M, K, q, scale, bias, N, y, s, tiled);
    case 4: return launch_w8_skinny_cfg<MC, TPW, 4>(x, M, K, q, scale, bias, N, y, s, tiled);
    default:
      if constexpr (skinny_max_ksw<MC, TPW>() >= 16) {
        if (ksw == 8) return launch_w8_skinny_cfg<MC, TPW, 8>(x, M, K, q, scale, bias, N, y, s, tiled);
        return launch_w8_skinny_cfg<MC, TPW, 16>(x, M, K, q, scale, bias, N, y, s, tiled);
      } else {
        return launch_w8_skinny_cfg<MC, TPW, 4>(x, M, K, q, scale, bias, N, y, s, tiled);
      }
  }
}

constexpr int kGemvFlatMaxM = 4;
constexpr int kGemvMaxBytes = 64 * 1024;
constexpr int kNotApplicable = -1;
constexpr int kFlatMaxNB = 16;

template <int NB, int MM, WFmt F>
constexpr int flat_lds_bytes(int ksw) {
  const int x = ((MM * (NB + 1) * 16 + 63) / 64) * 64 * 16;
  const int m = F == WFmt::W4 ? (((NB + 2) * kW4MetaBytes / 8 + 63) / 64) * 64 * 8 : 0;
  return ksw * (x + m) + ksw * 1024;
}

struct FlatPlan {
  int split, ksw;
};

// Work split for the flat GEMV, from sweeps of the Qwen3-14B shapes on
// MI355X.  Long-K, short-N shapes (17408 -> 5120: 320 tiles x 136 blocks)
// split each tile's k range over four 4-wave workgroups, so the 1280
// workgroups are all resident at once (five per CU) and every CU streams the
// same share; one 12-wave workgroup per tile fits only once per CU at that
// register count and leaves a second launch wave.  Otherwise one workgroup
// per tile: 12 waves for N < 1024 tiles (enough loads in flight), 4 for wide
// N.
constexpr int kFlatSplitMaxTiles = 512;   // only shapes with fewer tiles split their k range

// Split workspace layout: one uint32 arrival counter per tile in a fixed
// region sized for the largest split shape, then the fp32 partials.  The
// counter region does not depend on the shape, so one buffer shared by
// several shapes (the allocation-free entry point's scratch) never has one
// shape's partials written over another shape's counters.
constexpr size_t kFlatCounterBytes = kSplitCounterBytes;
static_assert(kFlatSplitMaxTiles <= kSplitMaxCounters, "one counter per split tile");

template <WFmt F>
FlatPlan plan_flat(int ntile, int nblk, bool may_split = true) {
  FlatPlan p{1, 1};
  if (ntile < kFlatSplitMaxTiles && nblk >= 64) p.split = 4;
  if (p.split > nblk || !may_split) p.split = 1;
  const int per = nblk / p.split;
  int ksw = p.split > 1 || ntile >= 1024 ? 4 : 12;
  if (ksw > per) ksw = per;
  if (ksw < 1) ksw = 1;
  const int limit = per / ksw <= (F == WFmt::W4 ? 12 : 8) ? 16 : 8;
  p.ksw = ksw > limit ? limit : ksw;
  return p;
}

size_t flat_workspace_bytes(int ntile, int split) {
  if (split <= 1) return 0;
  return kFlatCounterBytes + (size_t)ntile * split * 64 * sizeof(float4_t);
}

template <int NB, int MM, WFmt F, XMode XM>
int launch_flat(const half_t* x, int M, int K, const void* w, const void* meta, const half_t* bias, int N,
                int fmt_arg, half_t* y, FlatPlan p, void* ws, const FuseArgs& fz, hipStream_t s) {
  if (p.ksw > flat_max_ksw<NB, F>()) return kNotApplicable;
  const int lds = flat_lds_bytes<NB, MM, F>(p.ksw);
  if (lds > kGemvMaxBytes) return kNotApplicable;
  const int ntile = (N + 15) / 16;
  uint32_t* cnt = reinterpret_cast<uint32_t*>(ws);
  float4_t* part = p.split > 1 ? reinterpret_cast<float4_t*>(reinterpret_cast<uint8_t*>(ws) + kFlatCounterBytes)
                               : nullptr;
  hipLaunchKernelGGL((gemv_flat_kernel<NB, MM, F, XM>), dim3((unsigned)ntile, (unsigned)p.split), dim3(64 * p.ksw),
                     lds, s, x, M, K, w, meta, bias, N, fmt_arg, y, p.split, part, cnt, fz);
  return check_launch(F == WFmt::W4 ? "w4_gemv_flat" : "w8_gemv_flat");
}

template <int MM, WFmt F, XMode XM, int NB = 1>
int launch_flat_nb(int nb, const half_t* x, int M, int K, const void* w, const void* meta, const half_t* bias,
                   int N, int fmt_arg, half_t* y, FlatPlan p, void* ws, const FuseArgs& fz, hipStream_t s) {
  if constexpr (NB > kFlatMaxNB) {
    return kNotApplicable;
  } else {
    if (nb == NB) return launch_flat<NB, MM, F, XM>(x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
    return launch_flat_nb<MM, F, XM, NB + 1>(nb, x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
  }
}

template <WFmt F>
int launch_gemv_flat(const half_t* x, int M, int K, const void* w, const void* meta, const half_t* bias, int N,
                     int fmt_arg, half_t* y, void* ws, size_t ws_bytes, hipStream_t s,
                     XMode xm = XMode::Plain, const FuseArgs& fz = FuseArgs{}) {
  const int nblk = K / kW4BlockK, ntile = (N + 15) / 16;
  FlatPlan p = plan_flat<F>(ntile, nblk);
  // Without enough workspace the tile's k range stays in one workgroup.
  if (p.split > 1 && (ws == nullptr || ws_bytes < flat_workspace_bytes(ntile, p.split)))
    p = plan_flat<F>(ntile, nblk, false);
  const int nb = (nblk / p.split) / p.ksw;
  if (nb < 1 || nb > kFlatMaxNB) return kNotApplicable;
  if (xm == XMode::RmsNorm) return launch_flat_nb<1, F, XMode::RmsNorm>(nb, x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
  if (xm == XMode::SiluMul) return launch_flat_nb<1, F, XMode::SiluMul>(nb, x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
  if (M == 1) return launch_flat_nb<1, F, XMode::Plain>(nb, x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
  return launch_flat_nb<4, F, XMode::Plain>(nb, x, M, K, w, meta, bias, N, fmt_arg, y, p, ws, fz, s);
}

int launch_w4_gemv_flat(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                        half_t* y, void* ws, size_t ws_bytes, hipStream_t s) {
  const int bpg = G / kW4BlockK;
  if (bpg & (bpg - 1)) return kNotApplicable;     // group must be 128 * 2^j
  return launch_gemv_flat<WFmt::W4>(x, M, K, tiles, meta, nullptr, N, __builtin_ctz(bpg), y, ws, ws_bytes, s);
}

}  // namespace

int launch_w4_batch(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G, half_t* y,
                    void* ws, size_t ws_bytes, hipStream_t st);

int launch_w4_gemv_fused(const half_t* x, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         int x_mode, const half_t* norm_w, const float* sumsq_in, int sumsq_count, float eps,
                         const half_t* residual, float* sumsq_out, half_t* y, void* ws, size_t ws_bytes,
                         hipStream_t s) {
  const int bpg = G / kW4BlockK;
  if (bpg & (bpg - 1)) return fail(WQ_ERR_UNSUPPORTED, "fused decode linear needs group size 128 * 2^j");
  const FuseArgs fz{norm_w, sumsq_in, sumsq_count, eps, residual, sumsq_out};
  const XMode xm = x_mode == 1 ? XMode::RmsNorm : x_mode == 2 ? XMode::SiluMul : XMode::Plain;
  const int rc = launch_gemv_flat<WFmt::W4>(x, 1, K, tiles, meta, nullptr, N, __builtin_ctz(bpg), y, ws, ws_bytes, s,
                                            xm, fz);
  if (rc == kNotApplicable)
    return fail(WQ_ERR_UNSUPPORTED, "fused decode linear: this k is beyond the decode kernel's blocks per wave");
  return rc;
}

int launch_w8_gemv_fused(const half_t* x, int K, const int8_t* q, const half_t* scale, int N, int x_mode,
                         const half_t* norm_w, const float* sumsq_in, int sumsq_count, float eps,
                         const half_t* residual, float* sumsq_out, half_t* y, void* ws, size_t ws_bytes,
                         hipStream_t s, int tiled) {
  const FuseArgs fz{norm_w, sumsq_in, sumsq_count, eps, residual, sumsq_out};
  const XMode xm = x_mode == 1 ? XMode::RmsNorm : x_mode == 2 ? XMode::SiluMul : XMode::Plain;
  const int rc = launch_gemv_flat<WFmt::W8>(x, 1, K, q, scale, nullptr, N, tiled, y, ws, ws_bytes, s, xm, fz);
  if (rc == kNotApplicable)
    return fail(WQ_ERR_UNSUPPORTED, "fused decode linear: this k is beyond the decode kernel's blocks per wave");
  return rc;
}

size_t gemv_workspace_bytes(bool w4, int64_t m, int64_t n, int64_t k) {
  if (m > kGemvFlatMaxM) return 0;
  const int ntile = (int)((n + 15) / 16), nblk = (int)(k / kW4BlockK);
  const FlatPlan p = w4 ? plan_flat<WFmt::W4>(ntile, nblk) : plan_flat<WFmt::W8>(ntile, nblk);
  return flat_workspace_bytes(ntile, p.split);
}

int launch_w4_skinny(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                     half_t* y, void* ws, size_t ws_bytes, hipStream_t s) {
  if (M <= kGemvFlatMaxM) {
    int rc = launch_w4_gemv_flat(x, M, K, tiles, meta, N, G, y, ws, ws_bytes, s);
    if (rc != kNotApplicable) return rc;
  } else {
    // 12 <= M <= 32 on narrow N: activations shared in LDS (wq_batch.hip).
    int rc = launch_w4_batch(x, M, K, tiles, meta, N, G, y, ws, ws_bytes, s);
    if (rc != kNotApplicable) return rc;
  }
  const int mc = (M + 15) / 16;
  const SkinnyCfg c = pick_skinny((N + 15) / 16, K / kW4BlockK, mc, true);
  const bool t4 = c.tpw == 4;
  switch (mc) {
    case 1: return t4 ? launch_w4_skinny_k<1, 4>(c.ksw, x, M, K, tiles, meta, N, G, y, s)
                      : launch_w4_skinny_k<1, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    case 2: return t4 ? launch_w4_skinny_k<2, 4>(c.ksw, x, M, K, tiles, meta, N, G, y, s)
                      : launch_w4_skinny_k<2, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    case 3: return t4 ? launch_w4_skinny_k<3, 4>(c.ksw, x, M, K, tiles, meta, N, G, y, s)
                      : launch_w4_skinny_k<3, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    default: return t4 ? launch_w4_skinny_k<4, 4>(c.ksw, x, M, K, tiles, meta, N, G, y, s)
                       : launch_w4_skinny_k<4, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
  }
}

int launch_w8_skinny(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                     half_t* y, void* ws, size_t ws_bytes, hipStream_t s, int tiled) {
  if (M <= kGemvFlatMaxM) {
    int rc = launch_gemv_flat<WFmt::W8>(x, M, K, q, scale, bias, N, tiled, y, ws, ws_bytes, s);
    if (rc != kNotApplicable) return rc;
  }
  const int mc = (M + 15) / 16;
  const SkinnyCfg c = pick_skinny((N + 15) / 16, K / kW8BlockK, mc, false);
  switch (mc) {
    case 1: return launch_w8_skinny_k<1, 1>(c.ksw, x, M, K, q, scale, bias, N, y, s, tiled);
    case 2: return launch_w8_skinny_k<2, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s, tiled);
    case 3: return launch_w8_skinny_k<3, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s, tiled);
    default: return launch_w8_skinny_k<4, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s, tiled);
  }
}

int launch_w8_generic(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                      half_t* y, hipStream_t s) {
  const int64_t waves = (int64_t)M * N;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7FFFFFFF) return fail(WQ_ERR_UNSUPPORTED, "w8 generic grid too large");
  hipLaunchKernelGGL(w8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, q, scale, bias, N, y);
  return check_launch("w8_generic");
}

}  // namespace wq
