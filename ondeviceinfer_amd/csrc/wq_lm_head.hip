// fp16 LM head of the batch-1 decode step with the greedy token picked in
// the same pass: logits[v] = fp16(sum_k W[v, k] x[k]) over the row-major fp16
// weight [vocab, k] (the reference keeps lm_head unquantized), and
// token = argmax_v logits[v] with torch.argmax's rules (first index among
// equal values; NaN counts as the largest value).
//
// The weight is read exactly once (1.56 GB for Qwen3-14B: the largest single
// read of the decode step), so the kernel is a pure HBM stream: x lives in
// registers, each wave walks rows with a grid stride and keeps two rows of
// loads in flight, and the row dot products run on v_dot2_f32_f16 (fp32
// accumulation) with a DPP + lane-read wave sum.
#include "ondeviceinfer_decode.h"
#include "wq_common.h"
#include "wq_status.h"

#include <limits.h>
#include <math.h>

namespace wq {
namespace {

constexpr int kLmChunk = 64 * 8;       // k covered by one 16-byte load of every lane
constexpr int kLmMaxCh = 16;           // k <= 8192
constexpr int kLmGroupsPerCu = 3;      // resident workgroups per CU at ~140 VGPRs
constexpr int kLmCus = 256;

// a beats b: NaN first, then the larger value, then the smaller index.
__device__ __forceinline__ bool lm_better(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}

// grid = lm_head_grid(V) workgroups of 4 waves; wave g of nw walks rows
// g, g + nw, ... (at most 64 of them).  Lane l holds x[8 (l + 64 j) .. + 7]
// for j < CH and reads the same k of every row (one 16-byte load per chunk,
// 1 KiB per wave-load).  Rows past V are read clamped to row V - 1 and
// ignored, so every load of the two-row pipeline is unconditional.  The
// q-th row's logit waits in lane q and all are stored after the loop: a store
// inside it would leave loads and stores pending together, which forces a
// full vmcnt wait at every row.  Each wave leaves its best (value, index) in
// cand[g] for lm_head_pick_kernel.
// With norm_w, x is the final residual stream and every wave first forms
// the model's final RMSNorm itself, w * fp16(x * rsqrt(sum(sumsq) / K + eps)),
// from the per-16-element sums of squares of x that its producer (the last
// down projection) left in sumsq (count <= 1024): the norm kernel's launch
// before the LM head is folded in.
template <int CH>
__global__ __launch_bounds__(256) void lm_head_kernel(const half_t* __restrict__ x, const half_t* __restrict__ w,
                                                      int V, half_t* __restrict__ logits,
                                                      float2_t* __restrict__ cand, const half_t* __restrict__ norm_w,
                                                      const float* __restrict__ sumsq, int sumsq_count, float eps) {
  constexpr int K = CH * kLmChunk;
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6), nw = gridDim.x * 4;
  uint4_t xr[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) xr[j] = reinterpret_cast<const uint4_t*>(x)[lane + 64 * j];
  if (norm_w != nullptr) {
    uint4_t nr[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) nr[j] = reinterpret_cast<const uint4_t*>(norm_w)[lane + 64 * j];
    float ss = 0.f;
    for (int c = lane; c < sumsq_count; c += 64) ss += sumsq[c];
    const float r = rsqrtf(wave_sum_rl(ss) / (float)K + eps);
#pragma unroll
    for (int j = 0; j < CH; ++j) xr[j] = rms_scale8(xr[j], nr[j], r);
  }
  uint4_t ra[CH], rb[CH];
  auto load = [&](uint4_t (&r)[CH], int row) {
    const uint4_t* p = reinterpret_cast<const uint4_t*>(w + (size_t)min(row, V - 1) * K) + lane;
#pragma unroll
    for (int j = 0; j < CH; ++j) r[j] = __builtin_nontemporal_load(p + 64 * j);
  };
  auto dot = [&](const uint4_t (&r)[CH]) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      a0 = __builtin_amdgcn_fdot2(as_h2(r[j].x), as_h2(xr[j].x), a0, false);
      a1 = __builtin_amdgcn_fdot2(as_h2(r[j].y), as_h2(xr[j].y), a1, false);
      a0 = __builtin_amdgcn_fdot2(as_h2(r[j].z), as_h2(xr[j].z), a0, false);
      a1 = __builtin_amdgcn_fdot2(as_h2(r[j].w), as_h2(xr[j].w), a1, false);
    }
    return wave_sum_rl(a0 + a1);
  };
  float best = -INFINITY;
  int bidx = INT_MAX;
  half_t lg = 0;   // lane q: logit of this wave's row q
  int q = 0;
  auto take = [&](float logit, int row) {
    if (row < V) {
      const half_t lh = (half_t)logit;
      lg = lane == q ? lh : lg;
      ++q;
      const float v = (float)lh;
      if (lm_better(v, row, best, bidx)) {
        best = v;
        bidx = row;
      }
    }
  };
  // Two-row pipeline: the next row is requested before the current one is
  // used, and only one row is in flight where the loop is entered, so every
  // wait leaves exactly one row (CH loads) outstanding.
  int r = g;
  load(ra, r);
  while (true) {
    load(rb, r + nw);
    take(dot(ra), r);
    r += nw;
    if (r >= V) break;
    load(ra, r + nw);
    take(dot(rb), r);
    r += nw;
    if (r >= V) break;
  }
  if (logits != nullptr && lane < q) logits[g + (size_t)lane * nw] = lg;
  if (cand != nullptr && lane == 0) cand[g] = float2_t{best, __builtin_bit_cast(float, bidx)};
}

// One workgroup: the best of the n wave candidates (lm_better order) -> token.
__global__ __launch_bounds__(256) void lm_head_pick_kernel(const float2_t* __restrict__ cand, int n,
                                                           int64_t* __restrict__ token) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int t = threadIdx.x;
  float best = -INFINITY;
  int bidx = INT_MAX;
  for (int c = t; c < n; c += 256) {
    const float2_t e = cand[c];
    // Through a scalar: hipcc's __builtin_bit_cast of a vector component
    // (e.y) reads component 0.
    const float ey = e.y;
    const int ei = __builtin_bit_cast(int, ey);
    if (lm_better(e.x, ei, best, bidx)) {
      best = e.x;
      bidx = ei;
    }
  }
  sv[t] = best;
  si[t] = bidx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s && lm_better(sv[t + s], si[t + s], sv[t], si[t])) {
      sv[t] = sv[t + s];
      si[t] = si[t + s];
    }
    __syncthreads();
  }
  if (t == 0) *token = si[0];
}

// argmax of n fp16 values with the same rules (for logits that a separate
// kernel produced, e.g. a quantized LM head): each wave keeps the best of a
// grid-stride walk over 8-value chunks, reduces it over its lanes and leaves
// one candidate; lm_head_pick_kernel then picks the token.
constexpr int kArgmaxMaxGroups = 512;   // at most 2048 candidates for the pick

int argmax_grid(int64_t n) {
  const int64_t g = (n + 256 * 8 - 1) / (256 * 8);
  return (int)(g < kArgmaxMaxGroups ? g : kArgmaxMaxGroups);
}

__global__ __launch_bounds__(256) void argmax_f16_kernel(const half_t* __restrict__ x, int64_t n,
                                                         float2_t* __restrict__ cand) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float best = -INFINITY;
  int bidx = INT_MAX;
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i0 < n; i0 += stride) {
    if (i0 + 8 <= n) {
      const half8_t v = ld_h8(x + i0);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = (float)v[e];
        if (lm_better(f, (int)i0 + e, best, bidx)) {
          best = f;
          bidx = (int)i0 + e;
        }
      }
    } else {
      for (int64_t i = i0; i < n; ++i) {
        const float f = (float)x[i];
        if (lm_better(f, (int)i, best, bidx)) {
          best = f;
          bidx = (int)i;
        }
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bidx, o);
    if (lm_better(ov, oi, best, bidx)) {
      best = ov;
      bidx = oi;
    }
  }
  if (lane == 0) cand[blockIdx.x * 4 + wave] = float2_t{best, __builtin_bit_cast(float, bidx)};
}

// Enough workgroups to fill the machine once (fewer for a small vocab), and
// never more than 64 rows per wave.
int lm_head_grid(int64_t vocab) {
  const int64_t full = (int64_t)kLmCus * kLmGroupsPerCu;
  const int64_t need = (vocab + 3) / 4;
  const int64_t cap = (vocab + 4 * 64 - 1) / (4 * 64);
  const int64_t g = need < full ? need : full;
  return (int)(g > cap ? g : cap);
}

int lm_head_check(int64_t k, int64_t vocab) {
  WQ_REQUIRE(vocab > 0 && vocab <= INT_MAX / 2, WQ_ERR_INVALID_ARGUMENT, "vocab must be in [1, 2^30] (got %lld)",
             (long long)vocab);
  WQ_REQUIRE(k > 0 && k % kLmChunk == 0 && k / kLmChunk <= kLmMaxCh, WQ_ERR_UNSUPPORTED,
             "LM head needs k %% %d == 0 and k <= %d (got %lld)", kLmChunk, kLmChunk * kLmMaxCh, (long long)k);
  return WQ_OK;
}

struct LmNorm {
  const half_t* weight;   // nullptr: x is used as given
  const float* sumsq;
  int count;
  float eps;
};

template <int CH>
void launch_lm_head(const half_t* x, const half_t* w, int V, half_t* logits, float2_t* cand, int grid,
                    const LmNorm& nm, hipStream_t s) {
  hipLaunchKernelGGL(lm_head_kernel<CH>, dim3((unsigned)grid), dim3(256), 0, s, x, w, V, logits, cand, nm.weight,
                     nm.sumsq, nm.count, nm.eps);
}

int lm_head_run(const uint16_t* x, int64_t k, const uint16_t* weight, int64_t vocab, uint16_t* logits,
                int64_t* token, void* workspace, size_t workspace_bytes, const LmNorm& nm, void* stream) {
  const int rc = lm_head_check(k, vocab);
  if (rc != WQ_OK) return rc;
  WQ_REQUIRE(x && weight, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(logits || token, WQ_ERR_INVALID_ARGUMENT, "nothing to compute: logits and token are both NULL");
  WQ_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)nm.weight) % 16 == 0 && (uintptr_t)logits % 2 == 0,
             WQ_ERR_INVALID_ARGUMENT, "x, weight and the norm weight must be 16-byte aligned");
  const int grid = lm_head_grid(vocab);
  const size_t need = token ? (size_t)grid * 4 * sizeof(float2_t) : 0;
  WQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need && (uintptr_t)workspace % 8 == 0), WQ_ERR_WORKSPACE,
             "LM head argmax needs an 8-byte aligned workspace of %zu bytes (got %zu)", need, workspace_bytes);
  const half_t* xh = reinterpret_cast<const half_t*>(x);
  const half_t* wh = reinterpret_cast<const half_t*>(weight);
  half_t* lh = reinterpret_cast<half_t*>(logits);
  float2_t* cand = token ? reinterpret_cast<float2_t*>(workspace) : nullptr;
  const hipStream_t s = as_stream(stream);
  const int V = (int)vocab;
  switch (k / kLmChunk) {
    case 1: launch_lm_head<1>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 2: launch_lm_head<2>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 3: launch_lm_head<3>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 4: launch_lm_head<4>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 5: launch_lm_head<5>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 6: launch_lm_head<6>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 7: launch_lm_head<7>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 8: launch_lm_head<8>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 9: launch_lm_head<9>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 10: launch_lm_head<10>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 11: launch_lm_head<11>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 12: launch_lm_head<12>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 13: launch_lm_head<13>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 14: launch_lm_head<14>(xh, wh, V, lh, cand, grid, nm, s); break;
    case 15: launch_lm_head<15>(xh, wh, V, lh, cand, grid, nm, s); break;
    default: launch_lm_head<16>(xh, wh, V, lh, cand, grid, nm, s); break;
  }
  const int rc1 = check_launch("lm_head");
  if (rc1 != WQ_OK || !token) return rc1;
  hipLaunchKernelGGL(lm_head_pick_kernel, dim3(1), dim3(256), 0, s, cand, grid * 4, token);
  return check_launch("lm_head_pick");
}

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_lm_head_workspace_size(int64_t k, int64_t vocab, size_t* bytes) {
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int rc = lm_head_check(k, vocab);
  if (rc != WQ_OK) return rc;
  *bytes = (size_t)lm_head_grid(vocab) * 4 * sizeof(float2_t);
  return WQ_OK;
}

extern "C" int wq_lm_head(const uint16_t* x, int64_t k, const uint16_t* weight, int64_t vocab, uint16_t* logits,
                          int64_t* token, void* workspace, size_t workspace_bytes, void* stream) {
  return lm_head_run(x, k, weight, vocab, logits, token, workspace, workspace_bytes, LmNorm{nullptr, nullptr, 0, 0.f},
                     stream);
}

extern "C" int wq_lm_head_rmsnorm(const uint16_t* x, int64_t k, const uint16_t* norm_weight, const float* sumsq_in,
                                  int64_t sumsq_count, float eps, const uint16_t* weight, int64_t vocab,
                                  uint16_t* logits, int64_t* token, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  WQ_REQUIRE(norm_weight && sumsq_in, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(sumsq_count > 0 && sumsq_count <= 1024 && (uintptr_t)sumsq_in % 4 == 0, WQ_ERR_INVALID_ARGUMENT,
             "need 0 < sumsq_count <= 1024 (got %lld)", (long long)sumsq_count);
  return lm_head_run(x, k, weight, vocab, logits, token, workspace, workspace_bytes,
                     LmNorm{reinterpret_cast<const half_t*>(norm_weight), sumsq_in, (int)sumsq_count, eps}, stream);
}

extern "C" int wq_argmax_f16_workspace_size(int64_t n, size_t* bytes) {
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(n > 0 && n <= INT_MAX / 2, WQ_ERR_INVALID_ARGUMENT, "argmax needs 1 <= n <= 2^30 (got %lld)",
             (long long)n);
  *bytes = (size_t)argmax_grid(n) * 4 * sizeof(float2_t);
  return WQ_OK;
}

extern "C" int wq_argmax_f16(const uint16_t* x, int64_t n, int64_t* token, void* workspace, size_t workspace_bytes,
                             void* stream) {
  WQ_REQUIRE(n > 0 && n <= INT_MAX / 2, WQ_ERR_INVALID_ARGUMENT, "argmax needs 1 <= n <= 2^30 (got %lld)",
             (long long)n);
  WQ_REQUIRE(x && token, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE((uintptr_t)x % 16 == 0, WQ_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
  const int grid = argmax_grid(n);
  const size_t need = (size_t)grid * 4 * sizeof(float2_t);
  WQ_REQUIRE(workspace && workspace_bytes >= need && (uintptr_t)workspace % 8 == 0, WQ_ERR_WORKSPACE,
             "argmax needs an 8-byte aligned workspace of %zu bytes (got %zu)", need, workspace_bytes);
  const hipStream_t s = as_stream(stream);
  float2_t* cand = reinterpret_cast<float2_t*>(workspace);
  hipLaunchKernelGGL(argmax_f16_kernel, dim3((unsigned)grid), dim3(256), 0, s, reinterpret_cast<const half_t*>(x), n,
                     cand);
  const int rc = check_launch("argmax_f16");
  if (rc != WQ_OK) return rc;
  hipLaunchKernelGGL(lm_head_pick_kernel, dim3(1), dim3(256), 0, s, cand, grid * 4, token);
  return check_launch("argmax_pick");
}
