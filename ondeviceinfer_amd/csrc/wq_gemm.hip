// Prefill GEMM (large M): y[M, N] = x[M, K] . dequant(W)^T on fp16 MFMA.
//
// Workgroup = 4 waves.  Each wave owns NT 16-row weight tiles (a 16*NT
// slice of N, disjoint between waves, so no weight is dequantized twice in a
// workgroup); all four waves share a BM = 16*MT slice of M.  Per 128-k block:
//  * the activation tile x[BM, 128] is staged in LDS (double buffered, rows
//    padded by 16 B against bank conflicts) and read back as MFMA B
//    fragments;
//  * each wave loads its weight tiles straight from HBM (one 16 B load per
//    lane per tile: the W4 tile layout already is the MFMA A-fragment order),
//    and dequantizes them in registers;
//  * NT x MT x 4 MFMA v_mfma_f32_16x16x32_f16 accumulate in fp32.
// W4 weights are dequantized with their group scale, fp16((q - z) * s): the
// oracle's fp16 weight bit for bit.  INT8 weights enter as exact fp16 q and
// the per-row scale multiplies the fp32 sum in the epilogue.
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

constexpr int kXPad = 8;                    // halves of padding per LDS row
constexpr int kXStride = kW4BlockK + kXPad; // 136 halves = 272 B

enum class WFmt { W4, W8 };

template <WFmt F, int NT>
struct WFrag;

template <int NT>
struct WFrag<WFmt::W4, NT> {
  uint4_t wv[NT];
  uint32_t zw[NT];
  uint16_t sb[NT];
};

template <int NT>
struct WFrag<WFmt::W8, NT> {
  uint4_t wa[NT], wb[NT];
};

template <WFmt F, int NT, int MT>
__global__ __launch_bounds__(256) void wq_gemm_kernel(const half_t* __restrict__ x, int M, int K,
                                                      const void* __restrict__ wsrc, const void* __restrict__ wmeta,
                                                      int N, int G, const half_t* __restrict__ bias,
                                                      half_t* __restrict__ y) {
  constexpr int BM = MT * 16;
  constexpr int XCH = BM * 16 / 256;  // 16 B chunks of the x tile per thread
  __shared__ __attribute__((aligned(16))) half_t xs[2][BM][kXStride];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK;
  const int m0 = blockIdx.y * BM;
  const int tile0 = ((int)blockIdx.x * 4 + wave) * NT;

  int tile[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) tile[t] = min(tile0 + t, ntile - 1);

  // ---- weight fetch for one 128-k block
  auto fetch_w = [&](int blk, WFrag<F, NT>& f) {
    if constexpr (F == WFmt::W4) {
      const uint4_t* tiles = reinterpret_cast<const uint4_t*>(wsrc);
      const uint8_t* meta = reinterpret_cast<const uint8_t*>(wmeta);
      const int ngrp = K / G, g = blk * kW4BlockK / G;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f.wv[t] = tiles[((size_t)tile[t] * nblk + blk) * 64 + lane];
        const uint8_t* mp = meta + ((size_t)tile[t] * ngrp + g) * kW4MetaBytes;
        f.sb[t] = reinterpret_cast<const uint16_t*>(mp)[i];
        f.zw[t] = reinterpret_cast<const uint32_t*>(mp + 32)[i >> 3];
      }
    } else {
      const int8_t* q = reinterpret_cast<const int8_t*>(wsrc);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = min(tile[t] * 16 + i, N - 1);
        const int8_t* p = q + (size_t)row * K + blk * kW8BlockK + 16 * kb;
        f.wa[t] = *reinterpret_cast<const uint4_t*>(p);
        f.wb[t] = *reinterpret_cast<const uint4_t*>(p + 64);
      }
    }
  };

  // ---- activation tile: chunk c = tid + 256*j -> row c/16, 8 halves at (c%16)*8
  uint4_t xr[XCH];
  auto fetch_x = [&](int blk) {
#pragma unroll
    for (int j = 0; j < XCH; ++j) {
      const int c = tid + 256 * j;
      const int row = min(m0 + (c >> 4), M - 1);
      xr[j] = *reinterpret_cast<const uint4_t*>(x + (size_t)row * K + blk * kW4BlockK + (c & 15) * 8);
    }
  };
  auto stage_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < XCH; ++j) {
      const int c = tid + 256 * j;
      *reinterpret_cast<uint4_t*>(&xs[buf][c >> 4][(c & 15) * 8]) = xr[j];
    }
  };

  float4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  WFrag<F, NT> cur, nxt;
  fetch_x(0);
  fetch_w(0, cur);
  stage_x(0);
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    const bool more = blk + 1 < nblk;
    if (more) {
      fetch_x(blk + 1);
      fetch_w(blk + 1, nxt);
    }
    // Dequantize this block's weight fragments (A operands, 4 k-steps).
    half8_t a[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (F == WFmt::W4) {
        uint32_t c_lo, c_hi;
        w4_zero_consts((cur.zw[t] >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
        const half2_t s2 = as_h2((uint32_t)cur.sb[t] * 0x00010001u);
        a[t][0] = w4_word_to_h8_scaled(cur.wv[t].x, c_lo, c_hi, s2);
        a[t][1] = w4_word_to_h8_scaled(cur.wv[t].y, c_lo, c_hi, s2);
        a[t][2] = w4_word_to_h8_scaled(cur.wv[t].z, c_lo, c_hi, s2);
        a[t][3] = w4_word_to_h8_scaled(cur.wv[t].w, c_lo, c_hi, s2);
      } else {
        a[t][0] = i8x8_to_h8(cur.wa[t].x, cur.wa[t].y);
        a[t][1] = i8x8_to_h8(cur.wa[t].z, cur.wa[t].w);
        a[t][2] = i8x8_to_h8(cur.wb[t].x, cur.wb[t].y);
        a[t][3] = i8x8_to_h8(cur.wb[t].z, cur.wb[t].w);
      }
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      // k offset of step w inside the block, matching the weight fragment.
      const int kcol = (F == WFmt::W4) ? (kb * 32 + 8 * w) : (kb * 16 + 8 * (w & 1) + 64 * (w >> 1));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const half8_t b = *reinterpret_cast<const half8_t*>(&xs[buf][mt * 16 + i][kcol]);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][mt] = mfma16(a[t][w], b, acc[t][mt]);
      }
    }
    if (more) {
      stage_x(buf ^ 1);
      cur = nxt;
    }
    __syncthreads();
  }

  // Epilogue: lane holds D[n = 4*kb + v][m = i] of every (tile, m-subtile).
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n0 = (tile0 + t) * 16 + 4 * kb;
    if (tile0 + t >= ntile || n0 >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 16 + i;
      if (m >= M) continue;
      half4_t o;
      if constexpr (F == WFmt::W4) {
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] = (half_t)acc[t][mt][v];
        *reinterpret_cast<half4_t*>(y + (size_t)m * N + n0) = o;
      } else {
        const half_t* scale = reinterpret_cast<const half_t*>(wmeta);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int n = n0 + v;
          if (n < N) {
            float r = acc[t][mt][v] * (float)scale[n];
            if (bias) r += (float)bias[n];
            y[(size_t)m * N + n] = (half_t)r;
          }
        }
      }
    }
  }
}

template <WFmt F, int NT, int MT>
int launch_gemm(const half_t* x, int M, int K, const void* w, const void* meta, int N, int G, const half_t* bias,
                half_t* y, hipStream_t s) {
  const int ntile = (N + 15) / 16;
  const dim3 grid((unsigned)((ntile + 4 * NT - 1) / (4 * NT)), (unsigned)((M + MT * 16 - 1) / (MT * 16)));
  hipLaunchKernelGGL((wq_gemm_kernel<F, NT, MT>), grid, dim3(256), 0, s, x, M, K, w, meta, N, G, bias, y);
  return check_launch(F == WFmt::W4 ? "w4_gemm" : "w8_gemm");
}

}  // namespace

int launch_w4_gemm(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G, half_t* y,
                   hipStream_t s) {
  const int ntile = (N + 15) / 16;
  // Prefer 256-wide n slices; fall back to narrower ones when N is small so
  // the grid still spreads over the machine.
  if ((long)((ntile + 15) / 16) * ((M + 127) / 128) >= 256)
    return launch_gemm<WFmt::W4, 4, 8>(x, M, K, tiles, meta, N, G, nullptr, y, s);
  return launch_gemm<WFmt::W4, 1, 8>(x, M, K, tiles, meta, N, G, nullptr, y, s);
}

int launch_w8_gemm(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                   half_t* y, hipStream_t s) {
  const int ntile = (N + 15) / 16;
  if ((long)((ntile + 15) / 16) * ((M + 127) / 128) >= 256)
    return launch_gemm<WFmt::W8, 4, 8>(x, M, K, q, scale, N, 128, bias, y, s);
  return launch_gemm<WFmt::W8, 1, 8>(x, M, K, q, scale, N, 128, bias, y, s);
}

}  // namespace wq
