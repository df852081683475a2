// W8A8: dynamic per-token symmetric INT8 activations times per-output-channel
// INT8 weights, accumulated exactly in int32 on the int8 matrix cores
// (v_mfma_i32_16x16x64_i8) and scaled once per output in fp32.
//
// Fragment convention of v_mfma_i32_16x16x64_i8: lane l supplies 16 bytes of
// A row l%16 and 16 bytes of B column l%16 taken from k-slot l/16; A and B
// use the same (lane, byte) -> k map, which is all the dot product needs, so
// both are loaded as 16 consecutive bytes at k = 64s + 16(l/16).  The
// accumulator lane l holds D[row = 4(l/16) + v][column = l%16].  Weights are
// the A operand (rows n), activations the B operand (columns m).
#include "ondeviceinfer_wq.h"
#include "wq_common.h"
#include "wq_status.h"

#include <math.h>

namespace wq {
namespace {

typedef int32_t int4v_t __attribute__((ext_vector_type(4)));

constexpr int kI8Step = 64;   // k per int8 MFMA

__device__ __forceinline__ int4v_t mfma_i8(uint4_t a, uint4_t b, int4v_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int4v_t, a), __builtin_bit_cast(int4v_t, b), c, 0,
                                               0, 0);
}

__device__ __forceinline__ float wave_max_abs(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// One workgroup per row of x [M, K] (K % 8 == 0): absmax in fp32,
// scale = max(absmax, 1e-12) / 127, q = clamp(rint(x / scale), -127, 127)
// with an IEEE divide and round-half-even, as the reference's W8A8 oracle
// (backend.py:258-261).
__global__ __launch_bounds__(256) void w8a8_quantize_kernel(const half_t* __restrict__ x, int K,
                                                            int8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float part[4];
  const size_t base = (size_t)blockIdx.x * K;
  const int nc = K >> 3;
  float mx = 0.f;
  for (int c = threadIdx.x; c < nc; c += 256) {
    const half8_t v = ld_h8(x + base + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf((float)v[e]));
  }
  mx = wave_max_abs(mx);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float s = fmaxf(mx, 1e-12f) / 127.0f;
  if (threadIdx.x == 0) scale[blockIdx.x] = s;
  for (int c = threadIdx.x; c < nc; c += 256) {
    const half8_t v = ld_h8(x + base + 8 * c);
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float r = fminf(fmaxf(rintf((float)v[e] / s), -127.0f), 127.0f);
      w[e >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * (e & 3));
    }
    *reinterpret_cast<uint2_t*>(q + base + 8 * c) = uint2_t{w[0], w[1]};
  }
}

// y = fp16(float(acc) * sx[m] * sw[n] (+ bias[n])), the scaling of the
// int32 sum in that order, each operation rounded on its own (no fma).
__device__ __forceinline__ void w8a8_store(int32_t acc, int m, int n, const float* __restrict__ sx,
                                           const float* __restrict__ sw, const half_t* __restrict__ bias, int N,
                                           half_t* __restrict__ y) {
#pragma clang fp contract(off)
  float r = (float)acc * sx[m] * sw[n];
  if (bias) r += (float)bias[n];
  y[(size_t)m * N + n] = (half_t)r;
}

// Decode (M <= 16): grid = 16-row tiles of the weight, 64*ksw threads.  The
// tile's K/64 steps are split evenly over the ksw waves; a wave requests
// eight steps' weight fragments (non-temporal, 16 B per lane) and x
// fragments (row min(l%16, M-1)) at once, then issues eight MFMAs (a step
// past its range repeats the last one and is skipped).  The waves' int32
// sums meet in LDS (exact, order-free); wave 0 scales and stores.
__global__ __launch_bounds__(1024) void w8a8_gemv_kernel(const int8_t* __restrict__ qx, const float* __restrict__ sx,
                                                         int M, int K, const int8_t* __restrict__ qw,
                                                         const float* __restrict__ sw, const half_t* __restrict__ bias,
                                                         int N, half_t* __restrict__ y, W8Layout wl8) {
  __shared__ int4v_t red[16][64];
  const int ksw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x;
  const int nsteps = K / kI8Step;
  const int s_lo = (wave * nsteps) / ksw, s_hi = ((wave + 1) * nsteps) / ksw;
  const int8_t* wp = qw + wl8.lane_base(tile, lane, N, K);
  const int8_t* xp = qx + (size_t)min(i, M - 1) * K + 16 * kb;
  const int blk_bytes = wl8.block_bytes(), p1 = wl8.piece1();
  int4v_t acc = {0, 0, 0, 0};
  for (int s0 = s_lo; s0 < s_hi; s0 += 8) {
    uint4_t a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int st = min(s0 + j, s_hi - 1);   // 64-k step: block st / 2, piece st % 2
      a[j] = __builtin_nontemporal_load(
          reinterpret_cast<const uint4_t*>(wp + (size_t)(st >> 1) * blk_bytes + (st & 1) * p1));
      b[j] = *reinterpret_cast<const uint4_t*>(xp + (size_t)kI8Step * st);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < s_hi) acc = mfma_i8(a[j], b[j], acc);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  int4v_t sum = red[0][lane];
  for (int w2 = 1; w2 < ksw; ++w2) sum += red[w2][lane];
  if (i < M) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int n = tile * 16 + 4 * kb + v;
      if (n < N) w8a8_store(sum[v], i, n, sx, sw, bias, N, y);
    }
  }
}

// LDS slot of 16-byte chunk c (0..7) in row r of a 128-byte stage row: rows
// 2 apart share banks, so the slot is permuted by r / 2; the sixteen rows a
// B-fragment read touches then hit sixteen distinct 16-byte bank groups.
__device__ __forceinline__ int i8_swz(int r, int c) { return c ^ ((r >> 1) & 7); }

constexpr int kI8Blk = 128;              // k per GEMM stage (two int8 MFMA steps)
constexpr int kI8RowBytes = kI8Blk;      // one int8 x row per stage

// The MT B-fragments of one 64-k step, fragment mt from row mt*16 + i of the
// stage: a per-lane address plus the immediate mt * 16 rows.  Inline asm,
// as in the W4 GEMM: a read the compiler can see makes it wait for every
// outstanding buffer -> LDS copy (vmcnt(0)) first, the next stage's included,
// which serializes the copies with the math; these reads are completed by
// lds_wait_first_half / lds_wait_rest.
template <int OFF>
__device__ __forceinline__ uint4_t i8_lds_read_off(uint32_t a) {
  uint4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}
template <int MT, int MTI = 0>
__device__ __forceinline__ void i8_read_frags(uint4_t (&b)[MT], uint32_t a) {
  if constexpr (MTI < MT) {
    b[MTI] = i8_lds_read_off<MTI * 16 * kI8RowBytes>(a);
    i8_read_frags<MT, MTI + 1>(b, a);
  }
}

// M > 16: grid = (ceil(tiles / (4 NT)), ceil(M / BM)), 256 threads, BM = 16 MT.
// Wave w owns the NT 16-row weight tiles (4 bx + w) NT .. +NT-1 (disjoint
// between waves); all four share the BM x rows of the workgroup.  Per 128-k
// stage the x tile goes global -> LDS with global_load_lds_dwordx4 into a
// two-stage ring (row r's chunk c at slot i8_swz(r, c)); each wave's weight
// fragments come straight from memory into registers one stage ahead.  Per
// 64-k step a wave reads MT x fragments from LDS and issues NT x MT int8
// MFMAs.  Two workgroups per CU (the accumulators then live in VGPRs, not
// AGPRs: 236 registers, no scratch), so one workgroup's load wait overlaps
// the other's math: 1.4-1.8x the throughput of one per CU.  K % 128 == 0.
template <int NT, int MT>
__global__ __launch_bounds__(256, 2) void w8a8_gemm_kernel(const int8_t* __restrict__ qx,
                                                           const float* __restrict__ sx, int M, int K,
                                                           const int8_t* __restrict__ qw,
                                                           const float* __restrict__ sw,
                                                           const half_t* __restrict__ bias, int N,
                                                           half_t* __restrict__ y, W8Layout wl8) {
  constexpr int BM = MT * 16;
  constexpr int kStageBytes = BM * kI8RowBytes;
  constexpr int kInstrPerWave = kStageBytes / 1024 / 4;   // 1 KiB per wave-wide DMA instruction
  static_assert(kInstrPerWave >= 1, "stage too small for four waves");
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2 * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kI8Blk;
  const int m0 = blockIdx.y * BM;
  const int tile0 = ((int)blockIdx.x * 4 + wave) * NT;
  // Every load goes through a buffer resource with a wave-uniform base and
  // 32-bit offsets (K <= 2^23, checked by the host): rows past M and tiles
  // past N fall outside the buffers and read as zero (never stored).  With
  // plain global loads of the weights the compiler put a vmcnt(0) before
  // each block's first MFMA, waiting for the next block's loads as well.
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(qx + (size_t)m0 * K, (int64_t)(M - m0) * K);
  const __amdgpu_buffer_rsrc_t rw =
      wl8.tiled ? buf_rsrc(qw + (size_t)tile0 * nblk * kW8TileBlockBytes, (int64_t)(ntile - tile0) * nblk * kW8TileBlockBytes)
                : buf_rsrc(qw + (size_t)tile0 * 16 * K, (int64_t)(N - tile0 * 16) * K);
  const uint32_t w_voff = wl8.tiled ? (uint32_t)lane * 16 : (uint32_t)(i * K + 16 * kb);
  const uint32_t w_p1 = (uint32_t)wl8.piece1();

  // Stage `st` <- x rows m0 .. m0+BM-1, k block `blk`: instruction J of the
  // workgroup fills bytes [1024 J, 1024 J + 1024), i.e. rows 8J .. 8J+7;
  // lane L lands in row 8J + L/8, slot L%8, so it fetches chunk
  // i8_swz(row, L%8) of that row.
  auto copy_x = [&](int blk, int st) {
#pragma unroll
    for (int j = 0; j < kInstrPerWave; ++j) {
      const int J = wave * kInstrPerWave + j;
      const int r = 8 * J + (lane >> 3);
      const int c = i8_swz(r, lane & 7);
      lds_load16(rx, (uint32_t)(r * K + 16 * c), (uint32_t)(blk * kI8Blk), xs + st * kStageBytes + J * 1024);
    }
  };
  auto fetch_w = [&](int blk, uint4_t (&r)[NT][2]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t so = wl8.tiled ? (uint32_t)((t * nblk + blk) * kW8TileBlockBytes)
                                    : (uint32_t)(t * 16 * K + blk * kI8Blk);
      r[t][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff, so, 0);          // k + 16 kb .. +15
      r[t][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff + w_p1, so, 0);   // k + 64 + 16 kb .. +15
    }
  };

  int4v_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = int4v_t{0, 0, 0, 0};

  const uint32_t xs_lds = (uint32_t)(size_t)((const __attribute__((address_space(3))) uint8_t*)xs);
  // The one-tile path's block math: two 64-k MFMA steps of stage `st` with
  // the weight registers w (the same steps as the loop of the wider grids).
  auto block_math = [&](int st, const uint4_t (&w)[NT][2]) {
    // Row r = mt*16 + i of the stage holds chunk c at slot i8_swz(r, c) =
    // c ^ ((i >> 1) & 7): one lane address per step, mt in the offset.
    const uint32_t stage = xs_lds + (uint32_t)(st * kStageBytes + i * kI8RowBytes);
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      const int c = 4 * step + kb;   // 16-byte chunk of this lane's k range
      uint4_t b[MT];
      i8_read_frags<MT>(b, stage + (uint32_t)(i8_swz(i, c) * 16));
      lds_wait_first_half<MT>(b);
#pragma unroll
      for (int mt = 0; mt < (MT + 1) / 2; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][mt] = mfma_i8(w[t][step], b[mt], acc[t][mt]);
      lds_wait_rest<MT>(b);
#pragma unroll
      for (int mt = (MT + 1) / 2; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][mt] = mfma_i8(w[t][step], b[mt], acc[t][mt]);
    }
  };
  if constexpr (NT == 1) {
    // One weight tile per wave (grids of at most one round of workgroups):
    // the loop is unrolled by two over two fixed register sets, every step
    // issues its loads (the block after the last reads nothing: a
    // past-the-end offset), and the per-block wait covers only the x copy,
    // issued before the weights, so the next block's weights may still be in
    // flight across the barrier (M = 512, same box, same bits: 17408->5120
    // 116.7 -> 84.1 us, 5120^2 38.8 -> 33.7 us; M = 4096 k_proj 43.0 ->
    // 40.2 us).  The larger grids keep the loop below: this form cost them
    // 1-2 %.
    constexpr uint32_t kPastEnd = 0x80000000u;
    constexpr int kWLoads = 2 * NT;   // weight loads per block per wave
    uint4_t wr[2][NT][2];
    copy_x(0, 0);
    fetch_w(0, wr[0]);
    __builtin_amdgcn_s_waitcnt(0);   // stage 0 landed
    __syncthreads();
    int base = 0;
    do {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int blk = base + u;
#pragma unroll
        for (int j = 0; j < kInstrPerWave; ++j) {   // copy_x(blk + 1, u ^ 1), empty past the end
          const int J = wave * kInstrPerWave + j;
          const int r = 8 * J + (lane >> 3);
          lds_load16(rx, (uint32_t)(r * K + 16 * i8_swz(r, lane & 7)),
                     blk + 1 < nblk ? (uint32_t)((blk + 1) * kI8Blk) : kPastEnd, xs + (u ^ 1) * kStageBytes + J * 1024);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {               // fetch_w(blk + 1, wr[u ^ 1]), empty past the end
          const uint32_t so = blk + 1 >= nblk ? kPastEnd
                              : wl8.tiled ? (uint32_t)((t * nblk + blk + 1) * kW8TileBlockBytes)
                                          : (uint32_t)(t * 16 * K + (blk + 1) * kI8Blk);
          wr[u ^ 1][t][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff, so, 0);
          wr[u ^ 1][t][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff + w_p1, so, 0);
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the loads in this order: the wait below counts them
        if (blk < nblk) block_math(u, wr[u]);
        __builtin_amdgcn_s_waitcnt((kWLoads & 0xF) | ((kWLoads >> 4) << 14) | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();   // every wave's part of stage u ^ 1 landed
      }
      base += 2;
    } while (base < nblk);
    __builtin_amdgcn_s_waitcnt(0);   // the run-out block's empty loads, before the stores
  } else {
    uint4_t cur[NT][2], nxt[NT][2];
    copy_x(0, 0);
    fetch_w(0, cur);
    __builtin_amdgcn_s_waitcnt(0);   // stage 0 landed
    __syncthreads();
    for (int blk = 0; blk < nblk; ++blk) {
      const int st = blk & 1;
      const bool more = blk + 1 < nblk;
      if (more) {
        copy_x(blk + 1, st ^ 1);
        fetch_w(blk + 1, nxt);
      }
      // Row r = mt*16 + i of the stage holds chunk c at slot i8_swz(r, c) =
      // c ^ ((i >> 1) & 7): one lane address per step, mt in the offset.
      const uint32_t stage = xs_lds + (uint32_t)(st * kStageBytes + i * kI8RowBytes);
#pragma unroll
      for (int step = 0; step < 2; ++step) {
        const int c = 4 * step + kb;   // 16-byte chunk of this lane's k range
        uint4_t b[MT];
        i8_read_frags<MT>(b, stage + (uint32_t)(i8_swz(i, c) * 16));
        lds_wait_first_half<MT>(b);
#pragma unroll
        for (int mt = 0; mt < (MT + 1) / 2; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t][mt] = mfma_i8(cur[t][step], b[mt], acc[t][mt]);
        lds_wait_rest<MT>(b);
#pragma unroll
        for (int mt = (MT + 1) / 2; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[t][mt] = mfma_i8(cur[t][step], b[mt], acc[t][mt]);
      }
      if (more) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          cur[t][0] = nxt[t][0];
          cur[t][1] = nxt[t][1];
        }
      }
      __builtin_amdgcn_s_waitcnt(0);   // this wave's part of the next stage landed
      __syncthreads();                  // ... and everyone's; stage st may be overwritten next
    }
  }

#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (tile0 + t >= ntile) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 16 + i;
      if (m >= M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = (tile0 + t) * 16 + 4 * kb + v;
        if (n < N) w8a8_store(acc[t][mt][v], m, n, sx, sw, bias, N, y);
      }
    }
  }
}

constexpr int kW8A8GemvMaxM = 16;
// Largest k of the W8A8 GEMM: its x and weight offsets are 32-bit (127 rows
// of k bytes, 64 weight rows of k bytes); longer rows run the GEMV kernel 16
// rows at a time.
constexpr int64_t kW8A8GemmMaxK = 1 << 23;

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_w8a8_quantize(const uint16_t* x, int64_t m, int64_t k, int8_t* qx, float* x_scale, void* stream) {
  if (m == 0) return WQ_OK;
  WQ_REQUIRE(x && qx && x_scale, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(m > 0 && m <= 0x7fffffff && k > 0 && k % 8 == 0 && k <= (1 << 26), WQ_ERR_INVALID_ARGUMENT,
             "need m >= 0 and 0 < k, k %% 8 == 0 (k = %lld)", (long long)k);
  WQ_REQUIRE(((uintptr_t)x | (uintptr_t)qx) % 16 == 0, WQ_ERR_INVALID_ARGUMENT, "x and qx must be 16-byte aligned");
  hipLaunchKernelGGL(w8a8_quantize_kernel, dim3((unsigned)m), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const half_t*>(x), (int)k, qx, x_scale);
  return check_launch("w8a8_quantize");
}

namespace {

int w8a8_linear_impl(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const int8_t* qweight,
                     const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream, int tiled) {
  if (m == 0 || n == 0) return WQ_OK;
  WQ_REQUIRE(qx && x_scale && qweight && w_scale && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(m > 0 && n > 0 && k > 0 && m <= 0x7fffffff && n <= 0x7fffffff && k <= (1 << 26),
             WQ_ERR_INVALID_ARGUMENT, "m, n, k out of range");
  WQ_REQUIRE(k % (tiled ? kI8Blk : kI8Step) == 0, WQ_ERR_UNSUPPORTED, "W8A8 linear needs k %% %d == 0 (got %lld)",
             tiled ? kI8Blk : kI8Step, (long long)k);
  const W8Layout wl8{tiled};
  WQ_REQUIRE(((uintptr_t)qx | (uintptr_t)qweight) % 16 == 0, WQ_ERR_INVALID_ARGUMENT,
             "qx and qweight must be 16-byte aligned");
  const half_t* b = reinterpret_cast<const half_t*>(bias);
  half_t* yy = reinterpret_cast<half_t*>(y);
  const int64_t nsteps = k / kI8Step, ntile = (n + 15) / 16;
  if (m > kW8A8GemvMaxM && k % kI8Blk == 0 && k <= kW8A8GemmMaxK) {
    // GEMM: 128-row x tiles for long batches, 32-row ones otherwise; four
    // weight tiles per wave while that still leaves a full machine of
    // workgroups, else one.  Over INT8 tiles, long batches take two tiles
    // per wave while that gives 512 workgroups (M = 4096: 5120^2 197 ->
    // 159 us, 5120->17408 513 -> 454 us, 17408->5120 466 -> 410 us).
    const bool big_m = m >= 256;
    const int64_t mblocks = big_m ? (m + 127) / 128 : (m + 31) / 32;
    const bool two_tiles = tiled && big_m && (ntile + 7) / 8 * mblocks >= 512;
    const int nt = two_tiles ? 2 : (ntile + 15) / 16 * mblocks >= 256 ? 4 : 1;
    WQ_REQUIRE(mblocks <= 65535, WQ_ERR_UNSUPPORTED, "too many rows for the W8A8 GEMM grid");
    const dim3 grid((unsigned)((ntile + 4 * nt - 1) / (4 * nt)), (unsigned)mblocks);
    auto launch = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(256), 0, as_stream(stream), qx, x_scale, (int)m, (int)k, qweight,
                         w_scale, b, (int)n, yy, wl8);
    };
    if (big_m) {
      if (nt == 4) launch(w8a8_gemm_kernel<4, 8>);
      else if (nt == 2) launch(w8a8_gemm_kernel<2, 8>);
      else launch(w8a8_gemm_kernel<1, 8>);
    } else {
      if (nt == 4) launch(w8a8_gemm_kernel<4, 2>); else launch(w8a8_gemm_kernel<1, 2>);
    }
    return check_launch("w8a8_gemm");
  }
  // Decode kernel: about eight 64-k steps per wave (one round of loads).
  int ksw = (int)((nsteps + 7) / 8);
  ksw = ksw < 1 ? 1 : (ksw > 16 ? 16 : ksw);
  for (int64_t r = 0; r < m; r += kW8A8GemvMaxM) {   // batches beyond 16 rows only when k % 128 != 0 or k > 2^23
    const int64_t mr = m - r < kW8A8GemvMaxM ? m - r : kW8A8GemvMaxM;
    hipLaunchKernelGGL(w8a8_gemv_kernel, dim3((unsigned)ntile), dim3(64 * ksw), 0, as_stream(stream), qx + r * k,
                       x_scale + r, (int)mr, (int)k, qweight, w_scale, b, (int)n, yy + r * n, wl8);
    const int rc = check_launch("w8a8_gemv");
    if (rc != WQ_OK) return rc;
  }
  return WQ_OK;
}

}  // namespace

extern "C" int wq_w8a8_linear(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const int8_t* qweight,
                              const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream) {
  return w8a8_linear_impl(qx, x_scale, m, k, qweight, w_scale, n, bias, y, stream, 0);
}

extern "C" int wq_w8a8_linear_tiled(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const void* tiles,
                                    const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream) {
  return w8a8_linear_impl(qx, x_scale, m, k, reinterpret_cast<const int8_t*>(tiles), w_scale, n, bias, y, stream, 1);
}
