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
                                                         int N, half_t* __restrict__ y) {
  __shared__ int4v_t red[16][64];
  const int ksw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x;
  const int nsteps = K / kI8Step;
  const int s_lo = (wave * nsteps) / ksw, s_hi = ((wave + 1) * nsteps) / ksw;
  const int8_t* wp = qw + (size_t)min(tile * 16 + i, N - 1) * K + 16 * kb;
  const int8_t* xp = qx + (size_t)min(i, M - 1) * K + 16 * kb;
  int4v_t acc = {0, 0, 0, 0};
  for (int s0 = s_lo; s0 < s_hi; s0 += 8) {
    uint4_t a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const size_t off = (size_t)kI8Step * min(s0 + j, s_hi - 1);
      a[j] = __builtin_nontemporal_load(reinterpret_cast<const uint4_t*>(wp + off));
      b[j] = *reinterpret_cast<const uint4_t*>(xp + off);
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

// M > 16: grid = (ceil(N / 64), ceil(M / 64)), 256 threads.  Wave w owns the
// 16 weight rows 64*bx + 16w .. +15; the four waves share the 64 x rows
// 64*by .. +63 (four 16-column blocks, so every weight fragment feeds four
// MFMAs; the x fragments are L1 hits for three of the four waves).  K is
// walked in chunks of four 64-k steps, the next chunk requested before the
// current one is multiplied.
constexpr int kGemmChunk = 4;

__global__ __launch_bounds__(256, 2) void w8a8_gemm_kernel(const int8_t* __restrict__ qx,
                                                           const float* __restrict__ sx, int M, int K,
                                                           const int8_t* __restrict__ qw,
                                                           const float* __restrict__ sw,
                                                           const half_t* __restrict__ bias, int N,
                                                           half_t* __restrict__ y) {
  constexpr int CH = kGemmChunk;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * 64 + wave * 16, m0 = blockIdx.y * 64;
  const int nsteps = K / kI8Step;   // a multiple of CH (checked by the host)
  const int8_t* wp = qw + (size_t)min(n0 + i, N - 1) * K + 16 * kb;
  const int8_t* xp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xp[j] = qx + (size_t)min(m0 + 16 * j + i, M - 1) * K + 16 * kb;
  int4v_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = int4v_t{0, 0, 0, 0};

  uint4_t a[CH], b[CH][4];
  auto load_chunk = [&](int c, uint4_t (&aa)[CH], uint4_t (&bb)[CH][4]) {
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      const size_t off = (size_t)kI8Step * (c * CH + t);
      aa[t] = *reinterpret_cast<const uint4_t*>(wp + off);   // cached: every 64 rows of x reread it
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[t][j] = *reinterpret_cast<const uint4_t*>(xp[j] + off);
    }
  };
  const int nchunks = nsteps / CH;
  load_chunk(0, a, b);
  for (int c = 0; c < nchunks; ++c) {
    uint4_t an[CH], bn[CH][4];
    if (c + 1 < nchunks) load_chunk(c + 1, an, bn);
#pragma unroll
    for (int t = 0; t < CH; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = mfma_i8(a[t], b[t][j], acc[j]);
    if (c + 1 < nchunks) {
#pragma unroll
      for (int t = 0; t < CH; ++t) {
        a[t] = an[t];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[t][j] = bn[t][j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 16 * j + i;
    if (m < M) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int n = n0 + 4 * kb + v;
        if (n < N) w8a8_store(acc[j][v], m, n, sx, sw, bias, N, y);
      }
    }
  }
}

constexpr int kW8A8GemvMaxM = 16;

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

extern "C" int wq_w8a8_linear(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const int8_t* qweight,
                              const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream) {
  if (m == 0 || n == 0) return WQ_OK;
  WQ_REQUIRE(qx && x_scale && qweight && w_scale && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(m > 0 && n > 0 && k > 0 && m <= 0x7fffffff && n <= 0x7fffffff && k <= (1 << 26),
             WQ_ERR_INVALID_ARGUMENT, "m, n, k out of range");
  WQ_REQUIRE(k % kI8Step == 0, WQ_ERR_UNSUPPORTED, "W8A8 linear needs k %% 64 == 0 (got %lld)", (long long)k);
  WQ_REQUIRE(((uintptr_t)qx | (uintptr_t)qweight) % 16 == 0, WQ_ERR_INVALID_ARGUMENT,
             "qx and qweight must be 16-byte aligned");
  const half_t* b = reinterpret_cast<const half_t*>(bias);
  half_t* yy = reinterpret_cast<half_t*>(y);
  if (m <= kW8A8GemvMaxM || (k / kI8Step) % kGemmChunk != 0) {
    const int64_t nsteps = k / kI8Step, ntile = (n + 15) / 16;
    int ksw = (int)((nsteps + 9) / 10);
    ksw = ksw < 1 ? 1 : (ksw > 16 ? 16 : ksw);
    if (m > kW8A8GemvMaxM) {
      // k/64 not a multiple of the GEMM chunk: run the decode kernel per 16 rows of x.
      for (int64_t r = 0; r < m; r += kW8A8GemvMaxM) {
        const int64_t mr = m - r < kW8A8GemvMaxM ? m - r : kW8A8GemvMaxM;
        hipLaunchKernelGGL(w8a8_gemv_kernel, dim3((unsigned)ntile), dim3(64 * ksw), 0, as_stream(stream),
                           qx + r * k, x_scale + r, (int)mr, (int)k, qweight, w_scale, b, (int)n, yy + r * n);
        const int rc = check_launch("w8a8_gemv");
        if (rc != WQ_OK) return rc;
      }
      return WQ_OK;
    }
    hipLaunchKernelGGL(w8a8_gemv_kernel, dim3((unsigned)ntile), dim3(64 * ksw), 0, as_stream(stream), qx, x_scale,
                       (int)m, (int)k, qweight, w_scale, b, (int)n, yy);
    return check_launch("w8a8_gemv");
  }
  WQ_REQUIRE((m + 63) / 64 <= 65535, WQ_ERR_UNSUPPORTED, "too many rows for the W8A8 GEMM grid");
  hipLaunchKernelGGL(w8a8_gemm_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)((m + 63) / 64)), dim3(256), 0,
                     as_stream(stream), qx, x_scale, (int)m, (int)k, qweight, w_scale, b, (int)n, yy);
  return check_launch("w8a8_gemm");
}
