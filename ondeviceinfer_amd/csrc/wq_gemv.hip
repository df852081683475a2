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

// INT8 x fp16, M <= 16*MC, weights [N, K] row-major int8, fp16 row scale.
// Lane (i, kb) of block blk reads row 16t+i at k = 128*blk + 16*kb + [0,16)
// and 128*blk + 64 + 16*kb + [0,16); each 16 B feeds two MFMA k-steps.
template <int MC, int TPW, int KSW, int U>
__global__ __launch_bounds__(64 * KSW) void w8_skinny_kernel(const half_t* __restrict__ x, int M, int K,
                                                             const int8_t* __restrict__ q,
                                                             const half_t* __restrict__ scale,
                                                             const half_t* __restrict__ bias, int N,
                                                             half_t* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW8BlockK;
  const int b_lo = (wave * nblk) / KSW, b_hi = ((wave + 1) * nblk) / KSW;

  const int8_t* rowp[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int tt = min((int)blockIdx.x * TPW + t, ntile - 1);
    const int row = min(tt * 16 + i, N - 1);   // rows past N read a valid row; never stored
    rowp[t] = q + (size_t)row * K + 16 * kb;
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
          wa[u][t] = *reinterpret_cast<const uint4_t*>(rowp[t] + blk * kW8BlockK);
          wb[u][t] = *reinterpret_cast<const uint4_t*>(rowp[t] + blk * kW8BlockK + 64);
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

// Largest k-split per workgroup: 16 waves for M <= 16; 4 above, where a
// wave needs more than 128 VGPRs and 1024-thread groups would spill.
template <int MC>
constexpr int skinny_max_ksw() { return MC == 1 ? 16 : 4; }

// Enough waves to cover the machine (256 CUs) several times over while each
// wave keeps at least two k blocks.
SkinnyCfg pick_skinny(int ntile, int nblk, int mc) {
  SkinnyCfg c{mc >= 2 ? 2 : 1, 1};
  const int max_ksw = mc == 1 ? 16 : 4;
  const int groups = (ntile + c.tpw - 1) / c.tpw;
  int ksw = 1;
  while (ksw < max_ksw && groups * ksw < 2048 && nblk / (ksw * 2) >= 2) ksw *= 2;
  c.ksw = ksw;
  return c;
}

template <int MC, int TPW, int KSW>
int launch_w4_skinny_cfg(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         half_t* y, hipStream_t s) {
  const int ntile = (N + 15) / 16;
  const unsigned grid = (unsigned)((ntile + TPW - 1) / TPW);
  hipLaunchKernelGGL((w4_skinny_kernel<MC, TPW, KSW, skinny_unroll<MC>()>), dim3(grid), dim3(64 * KSW), 0, s, x, M, K, tiles, meta, N,
                     G, y);
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
      if constexpr (skinny_max_ksw<MC>() >= 16) {
        if (ksw == 8) return launch_w4_skinny_cfg<MC, TPW, 8>(x, M, K, tiles, meta, N, G, y, s);
        return launch_w4_skinny_cfg<MC, TPW, 16>(x, M, K, tiles, meta, N, G, y, s);
      } else {
        return launch_w4_skinny_cfg<MC, TPW, 4>(x, M, K, tiles, meta, N, G, y, s);
      }
  }
}

template <int MC, int TPW, int KSW>
int launch_w8_skinny_cfg(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias,
                         int N, half_t* y, hipStream_t s) {
  const int ntile = (N + 15) / 16;
  const unsigned grid = (unsigned)((ntile + TPW - 1) / TPW);
  hipLaunchKernelGGL((w8_skinny_kernel<MC, TPW, KSW, skinny_unroll<MC>()>), dim3(grid), dim3(64 * KSW), 0, s, x, M, K, q, scale, bias,
                     N, y);
  return check_launch("w8_skinny");
}

template <int MC, int TPW>
int launch_w8_skinny_k(int ksw, const half_t* x, int M, int K, const int8_t* q, const half_t* scale,
                       const half_t* bias, int N, half_t* y, hipStream_t s) {
  switch (ksw) {
    case 1: return launch_w8_skinny_cfg<MC, TPW, 1>(x, M, K, q, scale, bias, N, y, s);
    case 2: return launch_w8_skinny_cfg<MC, TPW, 2>(x, M, K, q, scale, bias, N, y, s);
    case 4: return launch_w8_skinny_cfg<MC, TPW, 4>(x, M, K, q, scale, bias, N, y, s);
    default:
      if constexpr (skinny_max_ksw<MC>() >= 16) {
        if (ksw == 8) return launch_w8_skinny_cfg<MC, TPW, 8>(x, M, K, q, scale, bias, N, y, s);
        return launch_w8_skinny_cfg<MC, TPW, 16>(x, M, K, q, scale, bias, N, y, s);
      } else {
        return launch_w8_skinny_cfg<MC, TPW, 4>(x, M, K, q, scale, bias, N, y, s);
      }
  }
}

}  // namespace

int launch_w4_skinny(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                     half_t* y, hipStream_t s) {
  const int mc = (M + 15) / 16;
  const SkinnyCfg c = pick_skinny((N + 15) / 16, K / kW4BlockK, mc);
  switch (mc) {
    case 1: return launch_w4_skinny_k<1, 1>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    case 2: return launch_w4_skinny_k<2, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    case 3: return launch_w4_skinny_k<3, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
    default: return launch_w4_skinny_k<4, 2>(c.ksw, x, M, K, tiles, meta, N, G, y, s);
  }
}

int launch_w8_skinny(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                     half_t* y, hipStream_t s) {
  const int mc = (M + 15) / 16;
  const SkinnyCfg c = pick_skinny((N + 15) / 16, K / kW8BlockK, mc);
  switch (mc) {
    case 1: return launch_w8_skinny_k<1, 1>(c.ksw, x, M, K, q, scale, bias, N, y, s);
    case 2: return launch_w8_skinny_k<2, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s);
    case 3: return launch_w8_skinny_k<3, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s);
    default: return launch_w8_skinny_k<4, 2>(c.ksw, x, M, K, q, scale, bias, N, y, s);
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
