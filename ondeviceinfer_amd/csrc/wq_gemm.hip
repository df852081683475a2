// Prefill GEMM (large M): y[M, N] = x[M, K] . dequant(W)^T on fp16 MFMA.
//
// Workgroup = 4 waves.  Each wave owns NT 16-row weight tiles (a 16*NT slice
// of N, disjoint between waves, so no weight is dequantized twice in a
// workgroup); all four waves share a BM = 16*MT slice of M.  Per 128-k block:
//  * the activation tile x[BM, 128] is copied buffer -> LDS with
//    buffer_load_dwordx4 ... lds (no register staging) into a two-stage ring;
//    16-byte chunk c of row r sits at slot c ^ (r & 15), so the sixteen rows
//    a B-fragment read touches fall in sixteen different bank groups;
//  * each wave loads its weight tiles straight from HBM into registers one
//    block ahead (the W4 tile layout already is the MFMA A-fragment order)
//    and dequantizes them there, one tile at a time;
//  * NT x MT x 4 MFMA v_mfma_f32_16x16x32_f16 accumulate in fp32.
// Every load goes through a buffer resource with a wave-uniform base and a
// 32-bit lane offset, so no 64-bit per-lane address stays live and the
// accumulators fit without spills; rows past M and tiles past N fall
// outside the buffers and read as zero.
// W4 weights are dequantized with their group scale, fp16((q - z) * s): the
// oracle's fp16 weight bit for bit.  INT8 weights enter as exact fp16 q and
// the per-row scale multiplies the fp32 sum in the epilogue.
// The tile shape follows the grid size (launch_gemm_auto); grids whose
// blocks are too short to hide a load run a deep-ring form with several
// blocks in flight (wq_gemm_deep_kernel), with the same block math; from
// M = 4096 on, W4 row blocks are assigned to XCDs (gemm_coords).  The W4
// kernel can also finish the Qwen3 MLP's elementwise ops in its epilogue
// (Epi: silu(gate) * up over a fused [gate | up] weight, or a residual add).
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

constexpr int kRowBytes = kW4BlockK * 2;   // one activation row of a 128-k block

enum class GFmt { W4, W8 };

// Epilogue of the prefill GEMM.  SiluPair: the weight is a fused [gate | up]
// of 2 * nh tiles and each wave's NT tiles are NT/2 gate tiles and the NT/2
// up tiles of the same columns, so the wave writes fp16(fp16(silu(g)) * u)
// (g, u the fp16-rounded sums) to an [M, N/2] output.  Residual:
// y = fp16(residual + fp16(sum)).  Both equal the separate elementwise
// kernel after a plain GEMM bit for bit.
enum class Epi { Plain, SiluPair, Residual };

template <GFmt F, int NT>
struct WRegs;
template <int NT>
struct WRegs<GFmt::W4, NT> {
  uint4_t w[NT];
  uint32_t z[NT];
  uint16_t s[NT];
};
template <int NT>
struct WRegs<GFmt::W8, NT> {
  uint4_t a[NT], b[NT];
};

// LDS slot (16-byte chunk index inside a 256-byte row) of chunk c in row r.
__device__ __forceinline__ int swz(int r, int c) { return c ^ (r & 15); }

// The MT B-fragments of one k-step: fragment mt is row mt*16 + i of the
// stage, so its address is a per-lane base plus the immediate mt*16 rows
// (no address arithmetic per read).  Inline asm for the reason given at
// lds_read16_asm.
template <int OFF>
__device__ __forceinline__ uint4_t lds_read16_off(uint32_t a) {
  uint4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int MT, int MTI = 0>
__device__ __forceinline__ void lds_read_frags(uint4_t (&b)[MT], uint32_t a) {
  if constexpr (MTI < MT) {
    b[MTI] = lds_read16_off<MTI * 16 * kRowBytes>(a);
    lds_read_frags<MT, MTI + 1>(b, a);
  }
}

// One 128-k block of a wave's NT x MT tile: per 32-k step, MT B-fragments
// from the LDS stage and NT A-fragments dequantized from the block's weight
// registers, tile-outer so that tile t+1 is dequantized (VALU) while tile t's
// MT MFMAs run; tile 0's first half of m-subtiles starts while the second
// half of the fragments is still in flight.  The wave runs the block at
// raised issue priority and drops it for the loads, waits and barrier
// between blocks, so a SIMD's other wave (another workgroup) that is inside
// its block math wins issue over one that is setting up its next block
// (M = 4096, same box: fused QKV 281.8 -> 275.2 us, gate 656 -> 644 us,
// k_proj 54.3 -> 49.6 us together with the load order of wq_gemm_kernel).
template <GFmt F, int NT, int MT>
__device__ __forceinline__ void gemm_block(const uint8_t* stage, const WRegs<F, NT>& cur, int i, int kb,
                                           float4_t (&acc)[NT][MT]) {
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    // chunk of this k-step inside the 128-k block, matching the fragment
    const int c = F == GFmt::W4 ? 4 * kb + w : 2 * kb + (w & 1) + 8 * (w >> 1);
    // row r = mt*16 + i holds chunk c at slot c ^ (r & 15) = c ^ i
    uint4_t b[MT];
    lds_read_frags<MT>(b, (uint32_t)(size_t)((const __attribute__((address_space(3))) uint8_t*)stage) +
                              (uint32_t)(i * kRowBytes + (c ^ i) * 16));
    auto dequant = [&](int t) -> half8_t {
      if constexpr (F == GFmt::W4) {
        uint32_t c_lo, c_hi;
        w4_zero_consts((cur.z[t] >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
        const half2_t s2 = as_h2((uint32_t)cur.s[t] * 0x00010001u);
        const uint32_t word = w == 0 ? cur.w[t].x : w == 1 ? cur.w[t].y : w == 2 ? cur.w[t].z : cur.w[t].w;
        return w4_word_to_h8_scaled(word, c_lo, c_hi, s2);
      } else {
        return w == 0 ? i8x8_to_h8(cur.a[t].x, cur.a[t].y)
             : w == 1 ? i8x8_to_h8(cur.a[t].z, cur.a[t].w)
             : w == 2 ? i8x8_to_h8(cur.b[t].x, cur.b[t].y)
                      : i8x8_to_h8(cur.b[t].z, cur.b[t].w);
      }
    };
    half8_t a = dequant(0);
    lds_wait_first_half<MT>(b);
#pragma unroll
    for (int mt = 0; mt < MT / 2; ++mt) acc[0][mt] = mfma16(a, __builtin_bit_cast(half8_t, b[mt]), acc[0][mt]);
    lds_wait_rest<MT>(b);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const half8_t a_next = t + 1 < NT ? dequant(t + 1) : a;
#pragma unroll
      for (int mt = t == 0 ? MT / 2 : 0; mt < MT; ++mt)
        acc[t][mt] = mfma16(a, __builtin_bit_cast(half8_t, b[mt]), acc[t][mt]);
      a = a_next;
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// Epilogue: lane holds D[n = 4*kb + v][m = i] of every (tile, m-subtile).
template <GFmt F, int NT, int MT>
__device__ __forceinline__ void gemm_store(const float4_t (&acc)[NT][MT], int tile0, int ntile, int m0, int M,
                                           int N, int i, int kb, const void* __restrict__ wmeta,
                                           const half_t* __restrict__ bias, half_t* __restrict__ y) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n0 = (tile0 + t) * 16 + 4 * kb;
    if (tile0 + t >= ntile || n0 >= N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 16 + i;
      if (m >= M) continue;
      if constexpr (F == GFmt::W4) {
        half4_t o;
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
            // A plain fp32 result, then one conversion: left alone, hipcc may
            // fold the product and the conversion into one mixed-precision
            // FMA that rounds straight to fp16, which the fused epilogues
            // (gemm_store_epi) could not match bit for bit.
            asm("" : "+v"(r));
            y[(size_t)m * N + n] = (half_t)r;
          }
        }
      }
    }
  }
}

// Epilogue of the fused modes: lane holds D[n = 4*kb + v][m = i] as above;
// the linear's fp16 output is the sum rounded (W4) or the sum times the
// channel scale rounded (INT8, as gemm_store).  y may alias res (an in-place
// residual add): each element is read and then written by the same lane, so
// neither pointer is restrict.
template <GFmt F, Epi EP, int NT, int MT>
__device__ __forceinline__ void gemm_store_epi(const float4_t (&acc)[NT][MT], int tile0, int ntile, int m0, int M,
                                               int N, int i, int kb, const void* wmeta, const half_t* res,
                                               half_t* y) {
  auto out16 = [&](float a, int n) -> half_t {
    if constexpr (F == GFmt::W4) return (half_t)a;
    else {
      float r = a * (float)reinterpret_cast<const half_t*>(wmeta)[n];
      asm("" : "+v"(r));   // as gemm_store: one fp32 product, then one conversion
      return (half_t)r;
    }
  };
  constexpr int NO = EP == Epi::SiluPair ? NT / 2 : NT;   // output tiles per wave
  const int nout = EP == Epi::SiluPair ? N / 2 : N;
  const int nt_out = EP == Epi::SiluPair ? ntile / 2 : ntile;
#pragma unroll
  for (int t = 0; t < NO; ++t) {
    const int n0 = (tile0 + t) * 16 + 4 * kb;
    if (tile0 + t >= nt_out || n0 >= nout) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 16 + i;
      if (m >= M) continue;
      half4_t o;
      if constexpr (EP == Epi::SiluPair) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const half_t g = out16(acc[t][mt][v], n0 + v), u = out16(acc[t + NO][mt][v], nout + n0 + v);
          o[v] = (half_t)silu_f((float)g) * u;
        }
      } else {
        const half4_t r = *reinterpret_cast<const half4_t*>(res + (size_t)m * N + n0);
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] = (half_t)((float)out16(acc[t][mt][v], n0 + v) + (float)r[v]);
      }
      *reinterpret_cast<half4_t*>(y + (size_t)m * nout + n0) = o;
    }
  }
}

// Workgroup -> (n slice bx, row block by).  Workgroups go to the 8 XCDs
// round-robin by flat id.  With rpx > 0 (the host sets it when the row blocks
// divide by 8: rpx = row blocks / 8), XCD x takes row blocks
// [x*rpx, (x+1)*rpx) with every n slice, row block fastest, so the
// workgroups resident on one XCD at a time share a few activation row blocks
// and a few weight slices in that XCD's L2.
__device__ __forceinline__ void gemm_coords(int rpx, int& bx, int& by) {
  if (rpx > 0) {
    const int b = blockIdx.x + gridDim.x * blockIdx.y;
    const int local = b >> 3;
    by = (b & 7) * rpx + local % rpx;
    bx = local / rpx;
  } else {
    bx = blockIdx.x;
    by = blockIdx.y;
  }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  // s_waitcnt simm16: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt
  // 11:8 left at their maxima.  The builtin (not inline asm) lets the
  // compiler's own wait insertion count it.
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <GFmt F, int NT, int MT, Epi EP = Epi::Plain>
__global__ __launch_bounds__(256, 2) void wq_gemm_kernel(const half_t* __restrict__ x, int M, int K,
                                                         const void* __restrict__ wsrc,
                                                         const void* __restrict__ wmeta, int N, int bpg,
                                                         const half_t* __restrict__ bias, half_t* y, int rpx,
                                                         int w8_tiled, const half_t* res) {
  static_assert(EP != Epi::SiluPair || NT % 2 == 0, "SiluPair pairs gate and up tiles");
  constexpr int BM = MT * 16;
  constexpr int kStageBytes = BM * kRowBytes;
  constexpr int kInstrPerWave = BM * 16 / 64 / 4;   // 1 KiB direct loads per wave per stage
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2 * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK;
  int bx, by;
  gemm_coords(rpx, bx, by);
  const int m0 = by * BM;
  // First tile of this wave (SiluPair: its first gate tile; the up tiles of
  // the same columns sit nh tiles further on).
  const int tile0 = (bx * 4 + wave) * (EP == Epi::SiluPair ? NT / 2 : NT);
  const int nh = ntile / 2;
  auto toff = [&](int t) { return EP == Epi::SiluPair && t >= NT / 2 ? nh + t - NT / 2 : t; };

  // Activation copy for block `blk` into stage `st`: instruction J of the
  // workgroup fills rows 4J..4J+3; lane L lands in row 4J + L/16, slot L%16,
  // so it fetches chunk (L%16) ^ (row & 15) of that row.  The buffer ends at
  // row M, so rows past it land as zeros.  With kInstrPerWave a multiple of
  // 4, row & 15 depends only on j & 3 and the lane: four lane offsets.
  static_assert(kInstrPerWave % 4 == 0, "x copy layout");
  uint32_t xvo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rl = 4 * q + (lane >> 4);   // row & 15 of instruction j with j & 3 == q
    xvo[q] = (uint32_t)((lane >> 4) * K * 2 + swz(rl, lane & 15) * 16);
  }
  const half_t* xw = x + (size_t)m0 * K;
  const int64_t x_bytes = (int64_t)(M - m0) * K * 2;
  auto copy_x = [&](int blk, int st) {
    // The block after the last (the loop's run-out) reads nothing: an empty range.
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(xw + (size_t)blk * kW4BlockK,
                                              blk < nblk ? x_bytes - (int64_t)blk * kRowBytes : 0);
#pragma unroll
    for (int j = 0; j < kInstrPerWave; ++j) {
      const int J = wave * kInstrPerWave + j;
      lds_load16(r, xvo[j & 3], (uint32_t)(4 * J * K * 2), xs + st * kStageBytes + J * 1024);
    }
  };

  // This wave's NT weight tiles from tile0 on; tiles past the last read as zero.
  // The weight loads keep the default cache policy: every weight block is read
  // again by the other row blocks resident on the same XCD, and the
  // non-temporal hint cost 4-5 % on the W4 shapes at M = 4096 (gate_up
  // 1302 vs 1367 us), 7-15 % on INT8 tiles (gate_up 1498 vs 1754 us) and
  // 9-11 % at M = 512.
  __amdgpu_buffer_rsrc_t rw, rm;
  if constexpr (F == GFmt::W4) {
    const int ngrp = nblk / bpg;
    rw = buf_rsrc(reinterpret_cast<const uint8_t*>(wsrc) + (size_t)tile0 * nblk * 1024,
                  (int64_t)(ntile - tile0) * nblk * 1024);
    rm = buf_rsrc(reinterpret_cast<const uint8_t*>(wmeta) + (size_t)tile0 * ngrp * kW4MetaBytes,
                  (int64_t)(ntile - tile0) * ngrp * kW4MetaBytes);
  } else {
    // INT8: row-major rows from tile0 * 16 on, or the tiles from tile0 on
    // (W8Layout); rows / tiles past the end fall outside the buffer (zeros).
    rw = w8_tiled ? buf_rsrc(reinterpret_cast<const int8_t*>(wsrc) + (size_t)tile0 * nblk * kW8TileBlockBytes,
                             (int64_t)(ntile - tile0) * nblk * kW8TileBlockBytes)
                  : buf_rsrc(reinterpret_cast<const int8_t*>(wsrc) + (size_t)tile0 * 16 * K, (int64_t)(N - tile0 * 16) * K);
  }
  // The block after the last takes an offset beyond every buffer's range, so
  // it reads zeros without touching memory.
  constexpr uint32_t kPastEnd = 0x80000000u;
  auto fetch_w = [&](int blk, WRegs<F, NT>& r) {
    const bool live = blk < nblk;
    if constexpr (F == GFmt::W4) {
      const int ngrp = nblk / bpg, g = blk / bpg;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        r.w[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)lane * 16,
                                                       live ? (uint32_t)((toff(t) * nblk + blk) * 1024) : kPastEnd, 0);
        const uint32_t mo = live ? (uint32_t)((toff(t) * ngrp + g) * kW4MetaBytes) : kPastEnd;
        r.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rm, (uint32_t)i * 2, mo, 0);
        r.z[t] = __builtin_amdgcn_raw_buffer_load_b32(rm, 32 + (uint32_t)(i >> 3) * 4, mo, 0);
      }
    } else {
      const uint32_t vo = w8_tiled ? (uint32_t)lane * 16 : (uint32_t)(i * K + 16 * kb);
      const uint32_t p1 = w8_tiled ? kW8TileBlockBytes / 2 : 64;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t so = !live ? kPastEnd
                            : w8_tiled ? (uint32_t)((toff(t) * nblk + blk) * kW8TileBlockBytes)
                                       : (uint32_t)(t * 16 * K + blk * kW8BlockK);
        r.a[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo, so, 0);
        r.b[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo + p1, so, 0);
      }
    }
  };

  float4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Pipeline: block b+1's activations (LDS stage (b+1) & 1) and weights
  // (register set (b+1) & 1) are requested before block b's math.  The loop
  // is unrolled by two so both register sets are fixed (no copy, which would
  // wait for the loads), and every step issues its loads (the run-out block
  // reads nothing), so the per-block wait is an exact count: only the
  // activation copy, issued before the weights, must have landed for the
  // barrier; the weights may arrive during the next block's first LDS reads,
  // where the compiler waits for them.
  constexpr int kWLoads = (F == GFmt::W4 ? 3 : 2) * NT;   // weight loads per block per wave
  WRegs<F, NT> wr[2];
  copy_x(0, 0);
  fetch_w(0, wr[0]);
  __builtin_amdgcn_s_waitcnt(0);   // vmcnt(0) lgkmcnt(0): stage 0 landed
  __syncthreads();
  // nblk >= 1 (K >= 128 is checked by the host), so the loop runs at least once.
  int base = 0;
  do {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = base + u;
      copy_x(b + 1, u ^ 1);   // stage u ^ 1 was read in block b - 1, before the barrier that ended it
      fetch_w(b + 1, wr[u ^ 1]);
      __builtin_amdgcn_sched_barrier(0);   // keep the loads in this order: the wait below counts them
      if (b < nblk) gemm_block<F, NT, MT>(xs + u * kStageBytes, wr[u], i, kb, acc);
      wait_vmcnt<kWLoads>();           // this wave's part of stage u ^ 1 landed
      __builtin_amdgcn_s_barrier();    // ... and everyone's
    }
    base += 2;
  } while (base < nblk);
  wait_vmcnt<0>();   // the run-out block's empty loads, before the stores

  if constexpr (EP == Epi::Plain)
    gemm_store<F, NT, MT>(acc, tile0, ntile, m0, M, N, i, kb, wmeta, bias, y);
  else
    gemm_store_epi<F, EP, NT, MT>(acc, tile0, ntile, m0, M, N, i, kb, wmeta, res, y);
}

// Deep-ring form, for grids whose per-block math is short (wide N at
// 16 < M <= 64, and the smallest prefill grids on 32-row tiles): the same
// tiles and block math, so bit-identical results, with D - 1 blocks of
// activations (an LDS ring of D stages) and weights (D register sets) in
// flight instead of one, so the math does not wait out each block's load
// latency.  The
// block loop is unrolled by D so every stage and register set is a constant;
// the loads of blocks past the last (the ring's run-out) are empty and never
// used.  Per block: wait until block b+1's loads have landed (vmcnt = the
// loads of the D-2 younger blocks, counted in issue order) and a barrier
// without a memory fence, which would wait for every outstanding load.
// With gridDim.z = S > 1 (W4, small grids) the K/128 blocks are split in S
// ranges, one per z: each workgroup publishes its fp32 partial tile through
// the workspace (device-coherent stores, then a device-scope arrival count on
// its (bx, by) tile) and the last to arrive adds the S partials in split
// order and stores y, so the result does not depend on arrival order.  The
// counters sit in a fixed region at the start of the workspace and are back
// at zero after every call.
constexpr int kDeepMaxTiles = kSplitMaxCounters;          // (bx, by) tiles with a counter
constexpr size_t kDeepCounterBytes = kSplitCounterBytes;

template <GFmt F, int NT, int MT, int D>
__global__ __launch_bounds__(256) void wq_gemm_deep_kernel(const half_t* __restrict__ x, int M, int K,
                                                           const void* __restrict__ wsrc,
                                                           const void* __restrict__ wmeta, int N, int bpg,
                                                           const half_t* __restrict__ bias, half_t* __restrict__ y,
                                                           int rpx, int w8_tiled, float4_t* ws_part,
                                                           uint32_t* ws_cnt) {
  constexpr int BM = MT * 16;
  constexpr int kStageBytes = BM * kRowBytes;
  constexpr int kInstrPerWave = BM * 16 / 64 / 4;   // 1 KiB direct loads per wave per stage
  constexpr int kLoadsPerBlock = kInstrPerWave + (F == GFmt::W4 ? 3 : 2) * NT;
  static_assert(D >= 3 && (D - 2) * kLoadsPerBlock <= 63, "ring depth");
  __shared__ __attribute__((aligned(1024))) uint8_t xs[D * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK;
  // This workgroup's k range [b_lo, b_lo + nloc) of the S splits; block
  // indices below are relative to b_lo.
  const int S = gridDim.z, split = blockIdx.z;
  const int b_lo = (split * nblk) / S, nloc = ((split + 1) * nblk) / S - b_lo;
  int bx, by;
  gemm_coords(rpx, bx, by);
  const int m0 = by * BM;
  const int tile0 = (bx * 4 + wave) * NT;

  // Activation copy as in wq_gemm_kernel: instruction J of the workgroup
  // fills rows 4J..4J+3 with lane L in row 4J + L/16, slot L%16.
  uint32_t xvo[kInstrPerWave];
#pragma unroll
  for (int j = 0; j < kInstrPerWave; ++j) {
    const int J = wave * kInstrPerWave + j;
    xvo[j] = (uint32_t)((lane >> 4) * K * 2 + swz(4 * J + (lane >> 4), lane & 15) * 16);
  }
  const half_t* xw = x + (size_t)m0 * K;
  const int64_t x_bytes = (int64_t)(M - m0) * K * 2;
  auto copy_x = [&](int blk, int st) {
    // Blocks past the range (the ring's tail) read nothing: an empty range.
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(xw + (size_t)(b_lo + blk) * kW4BlockK,
                                              blk < nloc ? x_bytes - (int64_t)(b_lo + blk) * kRowBytes : 0);
#pragma unroll
    for (int j = 0; j < kInstrPerWave; ++j) {
      const int J = wave * kInstrPerWave + j;
      lds_load16(r, xvo[j], (uint32_t)(4 * J * K * 2), xs + st * kStageBytes + J * 1024);
    }
  };
  __amdgpu_buffer_rsrc_t rw, rm;
  if constexpr (F == GFmt::W4) {
    const int ngrp = nblk / bpg;
    rw = buf_rsrc(reinterpret_cast<const uint8_t*>(wsrc) + (size_t)tile0 * nblk * 1024,
                  (int64_t)(ntile - tile0) * nblk * 1024);
    rm = buf_rsrc(reinterpret_cast<const uint8_t*>(wmeta) + (size_t)tile0 * ngrp * kW4MetaBytes,
                  (int64_t)(ntile - tile0) * ngrp * kW4MetaBytes);
  } else {
    // INT8: row-major rows from tile0 * 16 on, or the tiles from tile0 on
    // (W8Layout); rows / tiles past the end fall outside the buffer (zeros).
    rw = w8_tiled ? buf_rsrc(reinterpret_cast<const int8_t*>(wsrc) + (size_t)tile0 * nblk * kW8TileBlockBytes,
                             (int64_t)(ntile - tile0) * nblk * kW8TileBlockBytes)
                  : buf_rsrc(reinterpret_cast<const int8_t*>(wsrc) + (size_t)tile0 * 16 * K, (int64_t)(N - tile0 * 16) * K);
  }
  // Blocks past the end take an offset beyond every buffer's range, so they
  // read zeros without touching memory.
  constexpr uint32_t kPastEnd = 0x80000000u;
  auto fetch_w = [&](int lblk, WRegs<F, NT>& r) {
    const bool live = lblk < nloc;
    const int blk = b_lo + lblk;
    if constexpr (F == GFmt::W4) {
      const int ngrp = nblk / bpg, g = blk / bpg;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        r.w[t] = __builtin_amdgcn_raw_buffer_load_b128(
            rw, (uint32_t)lane * 16, live ? (uint32_t)((t * nblk + blk) * 1024) : kPastEnd, kNtPolicy);
        const uint32_t mo = live ? (uint32_t)((t * ngrp + g) * kW4MetaBytes) : kPastEnd;
        r.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rm, (uint32_t)i * 2, mo, 0);
        r.z[t] = __builtin_amdgcn_raw_buffer_load_b32(rm, 32 + (uint32_t)(i >> 3) * 4, mo, 0);
      }
    } else {
      const uint32_t vo = w8_tiled ? (uint32_t)lane * 16 : (uint32_t)(i * K + 16 * kb);
      const uint32_t p1 = w8_tiled ? kW8TileBlockBytes / 2 : 64;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t so = !live ? kPastEnd
                            : w8_tiled ? (uint32_t)((t * nblk + blk) * kW8TileBlockBytes)
                                       : (uint32_t)(t * 16 * K + blk * kW8BlockK);
        r.a[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo, so, kNtPolicy);
        r.b[t] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo + p1, so, kNtPolicy);
      }
    }
  };

  float4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  WRegs<F, NT> wr[D];
#pragma unroll
  for (int j = 0; j < D - 1; ++j) {
    copy_x(j, j);
    fetch_w(j, wr[j]);
    __builtin_amdgcn_sched_barrier(0);   // keep the loads in block order: the vmcnt waits count them
  }
  wait_vmcnt<(D - 2) * kLoadsPerBlock>();   // block 0 landed (this wave's part)
  __builtin_amdgcn_s_barrier();             // ... and every wave's
  // nblk >= 1 (K >= 128 is checked by the host), so the loop runs at least
  // once; as a do-while it has no guard block for the prologue's weight loads
  // to sink into, which would reorder them behind the x copies.
  int base = 0;
  do {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      // Stage and registers (u - 1) mod D were consumed in the previous step,
      // before the barrier that ended it.
      copy_x(base + u + D - 1, (u + D - 1) % D);
      fetch_w(base + u + D - 1, wr[(u + D - 1) % D]);
      __builtin_amdgcn_sched_barrier(0);
      if (base + u < nloc) gemm_block<F, NT, MT>(xs + u * kStageBytes, wr[u], i, kb, acc);
      wait_vmcnt<(D - 2) * kLoadsPerBlock>();
      __builtin_amdgcn_s_barrier();
    }
    base += D;
  } while (base < nloc);
  wait_vmcnt<0>();   // the tail's empty loads, before the waves end

  if (S > 1) {
    // Partial (tile, split, wave, t, mt) at 1 KiB granules, lane l at +16l.
    const int tile_id = by * (int)gridDim.x + bx;
    auto part_off = [&](int s2, int t, int mt) {
      return (uint32_t)((((((size_t)tile_id * S + s2) * 4 + wave) * NT + t) * MT + mt) * 1024 + lane * 16);
    };
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        coherent_store16(ws_part, part_off(split, t, mt), __builtin_bit_cast(uint4_t, acc[t][mt]));
    __builtin_amdgcn_s_waitcnt(0);   // this wave's partials are acknowledged
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();    // ... and every wave's
    // The arrival count goes through the first word of the activation ring,
    // dead once every wave has passed the barrier above (its run-out copies
    // landed before each wave's vmcnt(0)): a separate LDS word would push
    // the five-stage 64-row ring (80 KiB) past half of the CU's LDS and halve
    // its occupancy.
    uint32_t* arrival = reinterpret_cast<uint32_t*>(xs);
    if (tid == 0) *arrival = __hip_atomic_fetch_add(&ws_cnt[tile_id], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*arrival != (uint32_t)(S - 1)) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float4_t sum = split == 0 ? acc[t][mt]
                                  : __builtin_bit_cast(float4_t, coherent_load16(ws_part, part_off(0, t, mt)));
        for (int s2 = 1; s2 < S; ++s2)
          sum += s2 == split ? acc[t][mt]
                             : __builtin_bit_cast(float4_t, coherent_load16(ws_part, part_off(s2, t, mt)));
        acc[t][mt] = sum;
      }
    if (tid == 0) __hip_atomic_store(&ws_cnt[tile_id], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  gemm_store<F, NT, MT>(acc, tile0, ntile, m0, M, N, i, kb, wmeta, bias, y);
}

// Row blocks owned per XCD (gemm_coords) from M = 4096 on, for W4 (M = 4096:
// fused gate_up 1274 -> 1241 us, down 681 -> 665 us; at M = 2048 it slows the
// down projection, and the W8 GEMM gains nothing); 0 = launch order.
template <GFmt F>
int xcd_rows(int M, unsigned grid_y) {
  return F == GFmt::W4 && M >= 4096 && grid_y % 8 == 0 ? (int)grid_y / 8 : 0;
}

template <GFmt F, int NT, int MT, Epi EP = Epi::Plain>
int launch_gemm(const half_t* x, int M, int K, const void* w, const void* meta, int N, int bpg,
                const half_t* bias, half_t* y, hipStream_t s, int w8_tiled, const half_t* res = nullptr) {
  // SiluPair: N counts gate and up columns; a wave covers NT/2 of each, so
  // the grid has the same number of n slices.
  const int ntile = (N + 15) / 16;
  const dim3 grid((unsigned)((ntile + 4 * NT - 1) / (4 * NT)), (unsigned)((M + MT * 16 - 1) / (MT * 16)));
  hipLaunchKernelGGL((wq_gemm_kernel<F, NT, MT, EP>), grid, dim3(256), 0, s, x, M, K, w, meta, N, bpg, bias, y,
                     xcd_rows<F>(M, grid.y), w8_tiled, res);
  return check_launch(F == GFmt::W4 ? "w4_gemm" : "w8_gemm");
}

// k splits of the deep-ring grid (W4) for grids of at most 384 workgroups
// (640 on long k chains):
// enough workgroups to cover the machine several times (at most 2048 with
// the splits) while every split keeps at least 8 blocks; 1 when the
// workspace is missing or too small.  MI355X, µs, whole k -> split: k/v
// (5120->1024) M = 65 / 128 / 300 22.8 / 22.5 / 23.1 -> 11.4 / 11.8 / 16.2;
// q/o M = 65 / 128 22.9 / 27.0 -> 20.6 / 24.9; down (17408->5120) M = 65 /
// 128 68.7 / 79.9 -> 49.0 / 59.5.  Larger grids lost: fused QKV M = 128
// (448 workgroups) 29.2 -> 32.8, q/o M = 256 35.5 -> 37.6; up to 384 gained
// (320 before): fused QKV M = 65 / 96 (336 workgroups) 24.5 / 25.2 -> 23.2 /
// 24.1, k/v M = 700 / 760 25.5 / 25.8 -> 23.9 / 24.7.  Long k chains
// (at least 64 blocks) split up to 640 workgroups: down at M = 256 (640
// workgroups, two splits of 68 blocks) 101.6 -> 94.9.
constexpr long kDeepSplitMaxGrid = 384;
constexpr long kDeepSplitMaxGridLongK = 640;
constexpr int kDeepLongKBlocks = 64;

template <int NT, int MT>
int deep_splits(int M, int N, int K) {
  const long tiles = (long)(((N + 15) / 16 + 4 * NT - 1) / (4 * NT)) * ((M + MT * 16 - 1) / (MT * 16));
  if (tiles > (K / kW4BlockK >= kDeepLongKBlocks ? kDeepSplitMaxGridLongK : kDeepSplitMaxGrid)) return 1;
  int S = 1;
  while (S < 8 && (K / kW4BlockK) / (2 * S) >= 8 && tiles * 2 * S <= 2048 &&
         kDeepCounterBytes + (size_t)tiles * 2 * S * 4 * NT * MT * 1024 <= kSplitWorkspaceMaxBytes)
    S *= 2;
  return S;
}

template <int NT, int MT>
size_t deep_ws_bytes(int M, int N, int K) {
  const int S = deep_splits<NT, MT>(M, N, K);
  if (S <= 1) return 0;
  const size_t tiles = (size_t)(((N + 15) / 16 + 4 * NT - 1) / (4 * NT)) * ((M + MT * 16 - 1) / (MT * 16));
  return kDeepCounterBytes + tiles * S * 4 * NT * MT * 1024;
}

template <GFmt F, int NT, int MT, int D>
int launch_gemm_deep(const half_t* x, int M, int K, const void* w, const void* meta, int N, int bpg,
                     const half_t* bias, half_t* y, hipStream_t s, int w8_tiled, void* ws = nullptr,
                     size_t ws_bytes = 0) {
  const int ntile = (N + 15) / 16;
  int S = 1;
  if (F == GFmt::W4 && bias == nullptr && ws != nullptr && ws_bytes >= deep_ws_bytes<NT, MT>(M, N, K))
    S = deep_splits<NT, MT>(M, N, K);
  const dim3 grid((unsigned)((ntile + 4 * NT - 1) / (4 * NT)), (unsigned)((M + MT * 16 - 1) / (MT * 16)),
                  (unsigned)S);
  float4_t* part = S > 1 ? reinterpret_cast<float4_t*>(reinterpret_cast<uint8_t*>(ws) + kDeepCounterBytes) : nullptr;
  hipLaunchKernelGGL((wq_gemm_deep_kernel<F, NT, MT, D>), grid, dim3(256), 0, s, x, M, K, w, meta, N, bpg, bias, y,
                     xcd_rows<F>(M, grid.y), w8_tiled, part, reinterpret_cast<uint32_t*>(ws));
  return check_launch(F == GFmt::W4 ? "w4_gemm_deep" : "w8_gemm_deep");
}

// Workgroups from which the prefill GEMM takes 256-wide n slices of 128-row
// tiles (NT = 4, MT = 8): 384, three quarters of the 512 resident slots (the
// 128-row grid at 448 workgroups ran the fused QKV at M = 2048 in 137 us
// against 155 us for 64-row tiles, 5120^2 at M = 3072 (480) in 143 against
// 171 us, down 458 against 565 us; at 320, 5120^2 at M = 2048, the 64-row
// grid stays ahead, 118 against 129 us; same bits on every grid).
constexpr long kWideGrid = 384;

// Grids: 256-wide n slices of 128-row tiles (NT = 4, MT = 8) from kWideGrid
// workgroups on.  Otherwise W4 takes the most work per
// workgroup that still gives at least 384 workgroups: 128-wide slices of
// 64-row tiles (NT = 2, MT = 4), then 64-wide slices (NT = 1), then 64-wide
// slices of 32-row tiles on the deep ring (NT = 1, MT = 2, D = 4: three
// blocks in flight; D = 6 was 2-15 % slower once the block math ran at raised
// priority, e.g. 5120^2 at M = 65 17.4 against 20.4 us, q/o at M = 128 23.5
// against 25.0 us, same bits).  The
// narrow shapes gain most (k_proj 5120->1024: M = 2048 46.7 -> 38.0 us,
// M = 512 37.4 -> 21.8 us; down 17408->5120 at M = 128 101 -> 77 us; 5120^2
// at M = 2048 155 -> 127 us).  INT8 tiles take the same grids (5120^2 at
// M = 2048 190 -> 159 us, k_proj at M = 512 48 -> 22 us); row-major INT8,
// whose weight loads are 16 rows x 64 B, loses from two tiles per wave and
// keeps 64-wide slices of 64-row (M <= 256) or 128-row tiles.
// Whether launch_gemm_auto runs the deep ring on 32-row tiles for this shape.
bool gemm_takes_deep(long M, long N, bool w4_or_tiles) {
  const long ntile = (N + 15) / 16, mblk = (M + 127) / 128, mb64 = (M + 63) / 64;
  if (((ntile + 15) / 16) * mblk >= kWideGrid || !w4_or_tiles) return false;
  constexpr long kMinGrid = 384;
  return ((ntile + 7) / 8) * mb64 < kMinGrid && ((ntile + 3) / 4) * mb64 < kMinGrid;
}

template <GFmt F>
int launch_gemm_auto(const half_t* x, int M, int K, const void* w, const void* meta, int N, int bpg,
                     const half_t* bias, half_t* y, hipStream_t s, int w8_tiled, void* ws = nullptr,
                     size_t ws_bytes = 0) {
  const long ntile = (N + 15) / 16, mblk = (M + 127) / 128;
  if (((ntile + 15) / 16) * mblk >= kWideGrid) return launch_gemm<F, 4, 8>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled);
  if (F == GFmt::W4 || w8_tiled) {
    constexpr long kMinGrid = 384;
    const long mb64 = (M + 63) / 64;
    if (((ntile + 7) / 8) * mb64 >= kMinGrid)
      return launch_gemm<F, 2, 4>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled);
    if (((ntile + 3) / 4) * mb64 >= kMinGrid)
      return launch_gemm<F, 1, 4>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled);
    return launch_gemm_deep<F, 1, 2, 4>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled, ws, ws_bytes);
  } else {
    if (M <= 256) return launch_gemm<F, 1, 4>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled);
    return launch_gemm<F, 1, 8>(x, M, K, w, meta, N, bpg, bias, y, s, w8_tiled);
  }
}

}  // namespace

int launch_w4_gemm(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G, half_t* y,
                   hipStream_t s, void* ws, size_t ws_bytes) {
  return launch_gemm_auto<GFmt::W4>(x, M, K, tiles, meta, N, G / kW4BlockK, nullptr, y, s, 0, ws, ws_bytes);
}

// Workspace the W4 GEMM can use at this shape: the deep ring's k splits on
// the smallest grids (0 when the shape takes another grid).
size_t w4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < kW4BlockK || !gemm_takes_deep(M, N, true)) return 0;
  return deep_ws_bytes<1, 2>((int)M, (int)N, (int)K);
}

// The grid launch_gemm_auto picks for a W4 (or INT8-tile) shape, when it is a wq_gemm_kernel
// grid that can carry a fused epilogue: 1 = NT 4 / MT 8, 2 = NT 2 / MT 4,
// 3 = NT 1 / MT 4 (Residual only: SiluPair pairs tiles within a wave); 0
// otherwise.  SiluPair also needs the up tiles' offsets (nh + NT tiles of
// block_bytes per 128-k block from a wave's first tile) inside the 31-bit
// buffer range.
int gemm_epi_plan(int64_t M, int64_t N, int64_t K, int mode, int64_t block_bytes) {
  const long ntile = (N + 15) / 16, mblk = (M + 127) / 128, mb64 = (M + 63) / 64;
  int plan = 0;
  if (((ntile + 15) / 16) * mblk >= kWideGrid) plan = 1;
  else if (((ntile + 7) / 8) * mb64 >= 384) plan = 2;
  else if (((ntile + 3) / 4) * mb64 >= 384) plan = 3;
  if (mode == 1) {
    if (plan == 3 || N % 32 != 0) return 0;
    if ((ntile / 2 + 4) * (K / kW4BlockK) * block_bytes > 0x7fffffffL) return 0;
  }
  return plan;
}

// W4 prefill GEMM with a fused epilogue (mode 1 SiluPair, 2 Residual); the
// caller has checked w4_gemm_epi_plan.
int launch_w4_gemm_epi(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                       int mode, const half_t* res, half_t* y, hipStream_t s) {
  const int bpg = G / kW4BlockK;
  switch (gemm_epi_plan(M, N, K, mode, 1024) * 2 + (mode == 1 ? 0 : 1)) {
    case 2: return launch_gemm<GFmt::W4, 4, 8, Epi::SiluPair>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0);
    case 3: return launch_gemm<GFmt::W4, 4, 8, Epi::Residual>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0, res);
    case 4: return launch_gemm<GFmt::W4, 2, 4, Epi::SiluPair>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0);
    case 5: return launch_gemm<GFmt::W4, 2, 4, Epi::Residual>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0, res);
    case 7: return launch_gemm<GFmt::W4, 1, 4, Epi::Residual>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0, res);
    default: return fail(WQ_ERR_UNSUPPORTED, "w4 GEMM epilogue: shape has no fused-epilogue grid");
  }
}

// The same for INT8 tiles (scale: fp16 per output row).
int launch_w8_gemm_epi(const half_t* x, int M, int K, const int8_t* tiles, const half_t* scale, int N, int mode,
                       const half_t* res, half_t* y, hipStream_t s) {
  switch (gemm_epi_plan(M, N, K, mode, kW8TileBlockBytes) * 2 + (mode == 1 ? 0 : 1)) {
    case 2: return launch_gemm<GFmt::W8, 4, 8, Epi::SiluPair>(x, M, K, tiles, scale, N, 1, nullptr, y, s, 1);
    case 3: return launch_gemm<GFmt::W8, 4, 8, Epi::Residual>(x, M, K, tiles, scale, N, 1, nullptr, y, s, 1, res);
    case 4: return launch_gemm<GFmt::W8, 2, 4, Epi::SiluPair>(x, M, K, tiles, scale, N, 1, nullptr, y, s, 1);
    case 5: return launch_gemm<GFmt::W8, 2, 4, Epi::Residual>(x, M, K, tiles, scale, N, 1, nullptr, y, s, 1, res);
    case 7: return launch_gemm<GFmt::W8, 1, 4, Epi::Residual>(x, M, K, tiles, scale, N, 1, nullptr, y, s, 1, res);
    default: return fail(WQ_ERR_UNSUPPORTED, "INT8 GEMM epilogue: shape has no fused-epilogue grid");
  }
}

// Wide N at 16 < M <= 64: the deep ring keeps three weight blocks per wave in
// flight where the prefill GEMM keeps one (at M <= 32 a ring of five measured
// 4-5 % slower on the fused gate_up and 1-3 % on the LM head; at M = 40 and 64
// four stages of 64-row tiles (64 KiB) run 45.6 / 48.4 us on the fused gate_up
// where five (80 KiB) fit only one workgroup per CU, same bits).  Two tiles per wave when that still
// leaves more than 1024 workgroups (the LM head), else one (the fused
// gate_up).  Measured at K = 5120: gate_up 46.8 -> 39.9 us (M = 32) and
// 85.1 -> 50.2 us (M = 64), LM head 153.7 -> 106.8 us and 242.7 -> 148.8 us.
bool w4_gemm_small_fits(int64_t M, int64_t N) { return M > 16 && M <= 64 && (N + 15) / 16 >= 2048; }

int launch_w4_gemm_small(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         half_t* y, hipStream_t s) {
  const int bpg = G / kW4BlockK;
  const int ntile = (N + 15) / 16;
  if (M <= 32) {
    if (ntile >= 4096) return launch_gemm_deep<GFmt::W4, 2, 2, 4>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0);
    return launch_gemm_deep<GFmt::W4, 1, 2, 4>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0);
  }
  return launch_gemm_deep<GFmt::W4, 2, 4, 4>(x, M, K, tiles, meta, N, bpg, nullptr, y, s, 0);
}

int launch_w8_gemm(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                   half_t* y, hipStream_t s, int tiled) {
  return launch_gemm_auto<GFmt::W8>(x, M, K, q, scale, N, 1, bias, y, s, tiled);
}

}  // namespace wq
