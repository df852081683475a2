// Decode-step operators around the quantized linears (batch-1 Qwen3 decode):
// residual add + RMSNorm, SiLU(gate) * up, and single-token grouped-query
// attention over the resident fp16 KV cache with Qwen3's per-head q/k
// RMSNorm, RoPE and the cache append folded into the same launch.
//
// Numerics follow the reference's fp16 operation order where it rounds:
// the residual add, the normalized value and its product with the norm
// weight, and each product and the sum of the rotary embedding round to fp16
// (ondeviceinfer/functional.py:17-22, layers.py:64-80); reductions, softmax and
// the attention sums run in fp32.
#include "ondeviceinfer_decode.h"
#include "wq_common.h"
#include "wq_status.h"

#include <math.h>

namespace wq {
namespace {

constexpr int kHeadDim = 128;     // Qwen3 head_dim; one lane holds two elements
constexpr int kChunk = 64;        // KV positions per attention workgroup
constexpr int kMaxGroup = 8;      // q heads per kv head
constexpr int kMaxChunks = 256;   // so the combine's staging fits the reduction buffer

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// ------------------------------------------------------------------ RMSNorm
// One workgroup per row, eight elements per thread per step.  out_sum may
// alias x: each thread rereads only what it wrote itself.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const half_t* x, const half_t* delta,
                                                          const half_t* __restrict__ w, int n, float eps,
                                                          half_t* __restrict__ out_norm, half_t* out_sum) {
  __shared__ float part[4];
  const size_t base = (size_t)blockIdx.x * n;
  const int nc = n >> 3;
  float ss = 0.f;
  for (int c = threadIdx.x; c < nc; c += 256) {
    half8_t a = ld_h8(x + base + 8 * c);
    if (delta) a = a + ld_h8(delta + base + 8 * c);
    if (out_sum) *reinterpret_cast<half8_t*>(out_sum + base + 8 * c) = a;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = (float)a[e];
      ss += f * f;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
  for (int c = threadIdx.x; c < nc; c += 256) {
    half8_t a;
    if (out_sum) {
      a = ld_h8(out_sum + base + 8 * c);
    } else {
      a = ld_h8(x + base + 8 * c);
      if (delta) a = a + ld_h8(delta + base + 8 * c);
    }
    const half8_t wv = ld_h8(w + 8 * c);
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = wv[e] * (half_t)((float)a[e] * r);
    *reinterpret_cast<half8_t*>(out_norm + base + 8 * c) = o;
  }
}

// ---------------------------------------------------------------- SiLU * up
__global__ __launch_bounds__(256) void silu_mul_kernel(const half_t* __restrict__ gu, int rows, int n,
                                                       half_t* __restrict__ out) {
  const int nc = n >> 3;
  const size_t total = (size_t)rows * nc;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const size_t r = idx / nc;
    const int c = (int)(idx % nc);
    const half8_t g = ld_h8(gu + r * 2 * n + 8 * c);
    const half8_t u = ld_h8(gu + r * 2 * n + n + 8 * c);
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gf = (float)g[e];
      o[e] = (half_t)(gf / (1.0f + expf(-gf))) * u[e];
    }
    *reinterpret_cast<half8_t*>(out + r * n + 8 * c) = o;
  }
}

// ---------------------------------------------------------------- attention
// Per-head RMSNorm and RoPE of one 128-vector held two elements per lane
// (lane l: elements 2l, 2l+1).  rotate_half pairs element d with d +- 64,
// i.e. lane l with lane l ^ 32.  Every product and the sum round to fp16, as
// in `q * cos + rotate_half(q) * sin` on fp16 tensors.
__device__ __forceinline__ half2_t norm_rope_pair(half2_t v, const half_t* nw, float eps, const half_t* cs,
                                                  const half_t* sn, int lane) {
#pragma clang fp contract(off)
  if (nw) {
    const float a = (float)v[0], b = (float)v[1];
    const float r = rsqrtf(wave_sum(a * a + b * b) * (1.0f / kHeadDim) + eps);
    v[0] = nw[2 * lane] * (half_t)(a * r);
    v[1] = nw[2 * lane + 1] * (half_t)(b * r);
  }
  half2_t p = as_h2(__shfl_xor(as_u32(v), 32));
  if (lane < 32) p = -p;
  const half2_t c2 = {cs[2 * lane], cs[2 * lane + 1]};
  const half2_t s2 = {sn[2 * lane], sn[2 * lane + 1]};
  const half2_t t1 = v * c2;
  const half2_t t2 = p * s2;
  return t1 + t2;
}

// grid = (kv_heads, chunks of 64 positions over max_seq); 256 threads.
// Chunk c of kv head h scores its positions against the head's G query
// heads, keeps its softmax partial (max, sum, unnormalized output) and the
// last chunk to finish merges all partials in chunk order.  The workgroup
// whose chunk holds `pos` also normalizes, rotates and appends the new key
// and value, and uses them from LDS.
__global__ __launch_bounds__(256) void decode_attention_kernel(
    const half_t* __restrict__ qkv, int H, int KV, const half_t* __restrict__ qn_w,
    const half_t* __restrict__ kn_w, float eps, const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
    const int32_t* __restrict__ position, half_t* kc, half_t* vc, int max_seq, float scale,
    half_t* __restrict__ out, float* ws_o, float* ws_ml, uint32_t* ws_cnt) {
  constexpr int D = kHeadDim, C = kChunk, GM = kMaxGroup;
  __shared__ float qs[GM][D];
  __shared__ __attribute__((aligned(16))) half_t knew[D];
  __shared__ __attribute__((aligned(16))) half_t vnew[D];
  __shared__ float sc[GM][C];
  __shared__ float red[4 * GM * D];   // P.V partials per position group; later the combine's staging
  __shared__ float mls[GM][2];
  __shared__ uint32_t s_prev;

  const int h = blockIdx.x, chunk = blockIdx.y, NC = gridDim.y;
  const int G = H / KV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = *position;
  if (pos < 0 || pos >= max_seq) {
    if (h == 0 && chunk == 0)
      for (int i = tid; i < H * D; i += 256) out[i] = (half_t)__builtin_nanf("");
    return;
  }
  const int L = pos + 1;
  const int p0 = chunk * C;
  const bool active = p0 < L;
  const bool owner = pos >= p0 && pos < p0 + C;
  const size_t head_base = (size_t)h * max_seq * D;

  // Issue this chunk's K and V loads first (row pos is produced below).
  const int pl = tid >> 2, part = tid & 3;   // scores: position p0 + pl, elements [32 part, 32 part + 32)
  const int pk = p0 + pl;
  uint4_t kr[4] = {};
  if (active && pk < L && pk != pos) {
    const uint4_t* src = reinterpret_cast<const uint4_t*>(kc + head_base + (size_t)pk * D + part * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) kr[j] = src[j];
  }
  const int dp = tid & 63, pg = tid >> 6;    // P.V: elements 2dp, 2dp+1 of positions p0 + 16 pg + j
  uint32_t vr[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int p = p0 + 16 * pg + j;
    vr[j] = (active && p < L && p != pos)
                ? reinterpret_cast<const uint32_t*>(vc + head_base + (size_t)p * D)[dp]
                : 0u;
  }

  if (active) {
    const half_t* cs = cos_t + (size_t)pos * D;
    const half_t* sn = sin_t + (size_t)pos * D;
    for (int g = wave; g < G; g += 4) {
      const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(h * G + g) * D)[lane];
      const half2_t r = norm_rope_pair(v, qn_w, eps, cs, sn, lane);
      qs[g][2 * lane] = (float)r[0];
      qs[g][2 * lane + 1] = (float)r[1];
    }
    if (owner && wave == 0) {
      const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + h) * D)[lane];
      const half2_t r = norm_rope_pair(v, kn_w, eps, cs, sn, lane);
      reinterpret_cast<half2_t*>(knew)[lane] = r;
      reinterpret_cast<half2_t*>(kc + head_base + (size_t)pos * D)[lane] = r;
    }
    if (owner && wave == 1) {
      const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + KV + h) * D)[lane];
      reinterpret_cast<half2_t*>(vnew)[lane] = v;
      reinterpret_cast<half2_t*>(vc + head_base + (size_t)pos * D)[lane] = v;
    }
  }
  __syncthreads();

  if (active) {
    float s[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) s[g] = 0.f;
    if (pk < L) {
      half8_t kv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        kv[j] = pk == pos ? reinterpret_cast<const half8_t*>(knew + part * 32)[j] : __builtin_bit_cast(half8_t, kr[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float kf = (float)kv[j][e];
#pragma unroll
          for (int g = 0; g < GM; ++g)
            if (g < G) s[g] += qs[g][part * 32 + 8 * j + e] * kf;
        }
    }
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      s[g] += __shfl_xor(s[g], 1);
      s[g] += __shfl_xor(s[g], 2);
    }
    if (part == 0)
      for (int g = 0; g < G; ++g) sc[g][pl] = pk < L ? s[g] * scale : -INFINITY;
  }
  __syncthreads();

  if (active) {
    // An active chunk holds position p0 < L, so every row max is finite.
    for (int g = wave; g < G; g += 4) {
      const float v = sc[g][lane];
      const float m = wave_max(v);
      const float e = v == -INFINITY ? 0.f : expf(v - m);
      const float l = wave_sum(e);
      sc[g][lane] = e;
      if (lane == 0) {
        mls[g][0] = m;
        mls[g][1] = l;
      }
    }
  }
  __syncthreads();

  if (active) {
    float a0[GM], a1[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) a0[g] = a1[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int q = 16 * pg + j;
      if (p0 + q < L) {
        const half2_t v2 = p0 + q == pos ? reinterpret_cast<const half2_t*>(vnew)[dp] : as_h2(vr[j]);
        const float v0 = (float)v2[0], v1 = (float)v2[1];
#pragma unroll
        for (int g = 0; g < GM; ++g)
          if (g < G) {
            const float pr = sc[g][q];
            a0[g] += pr * v0;
            a1[g] += pr * v1;
          }
      }
    }
    for (int g = 0; g < G; ++g) {
      red[(pg * GM + g) * D + 2 * dp] = a0[g];
      red[(pg * GM + g) * D + 2 * dp + 1] = a1[g];
    }
  }
  __syncthreads();

  if (NC == 1) {
    for (int i = tid; i < G * D; i += 256) {
      const int g = i / D, d = i % D;
      const float o = red[g * D + d] + red[(GM + g) * D + d] + red[(2 * GM + g) * D + d] + red[(3 * GM + g) * D + d];
      out[(size_t)(h * G + g) * D + d] = (half_t)(o / mls[g][1]);
    }
    return;
  }

  // Publish this chunk's partial (device-coherent stores), then count it.
  if (active) {
    float* po = ws_o + ((size_t)(h * NC + chunk) * G) * D;
    for (int i = tid; i < G * D; i += 256) {
      const int g = i / D, d = i % D;
      const float o = red[g * D + d] + red[(GM + g) * D + d] + red[(2 * GM + g) * D + d] + red[(3 * GM + g) * D + d];
      __hip_atomic_store(po + i, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < 2 * G)
      __hip_atomic_store(ws_ml + ((size_t)(h * NC + chunk) * G) * 2 + tid, mls[tid >> 1][tid & 1], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) s_prev = __hip_atomic_fetch_add(&ws_cnt[h], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_prev != (uint32_t)(NC - 1)) return;

  // Last chunk to arrive: merge the active chunks' partials in chunk order.
  const int NA = (L + C - 1) / C;
  float* stm = red;                     // [NA][G] maxima
  float* stl = red + kMaxChunks * GM;   // [NA][G] sums
  for (int i = tid; i < NA * G; i += 256) {
    const float* src = ws_ml + ((size_t)h * NC * G + i) * 2;
    stm[i] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    stl[i] = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += 256) {
    const int g = i / D;
    float M = -INFINITY;
    for (int c = 0; c < NA; ++c) M = fmaxf(M, stm[c * G + g]);
    float num = 0.f, den = 0.f;
    for (int c = 0; c < NA; ++c) {
      const float wgt = expf(stm[c * G + g] - M);
      num += wgt * __hip_atomic_load(ws_o + ((size_t)(h * NC + c) * G) * D + i, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
      den += wgt * stl[c * G + g];
    }
    out[(size_t)h * G * D + i] = (half_t)(num / den);
  }
  if (tid == 0) __hip_atomic_store(&ws_cnt[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t attention_workspace_bytes(int64_t H, int64_t KV, int64_t max_seq) {
  const int64_t nc = (max_seq + kChunk - 1) / kChunk;
  const int64_t g = H / KV;
  return nc <= 1 ? 0 : align256((size_t)KV * 4) + align256((size_t)KV * nc * g * 2 * 4) + (size_t)KV * nc * g * kHeadDim * 4;
}

int attention_shape_check(int64_t H, int64_t KV, int64_t head_dim, int64_t max_seq) {
  WQ_REQUIRE(H > 0 && KV > 0 && max_seq > 0, WQ_ERR_INVALID_ARGUMENT, "q_heads, kv_heads and max_seq must be positive");
  WQ_REQUIRE(head_dim == kHeadDim, WQ_ERR_UNSUPPORTED, "decode attention is built for head_dim 128 (got %lld)",
             (long long)head_dim);
  WQ_REQUIRE(H % KV == 0, WQ_ERR_INVALID_ARGUMENT, "q_heads (%lld) must be a multiple of kv_heads (%lld)",
             (long long)H, (long long)KV);
  WQ_REQUIRE(H / KV <= kMaxGroup, WQ_ERR_UNSUPPORTED, "at most %d query heads per kv head", kMaxGroup);
  WQ_REQUIRE(max_seq <= (int64_t)kMaxChunks * kChunk, WQ_ERR_UNSUPPORTED, "max_seq must be <= %d",
             kMaxChunks * kChunk);
  WQ_REQUIRE(KV <= 65535, WQ_ERR_UNSUPPORTED, "too many kv heads");
  return WQ_OK;
}

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_add_rmsnorm(const uint16_t* x, const uint16_t* delta, const uint16_t* weight, int64_t rows,
                              int64_t n, float eps, uint16_t* out_norm, uint16_t* out_sum, void* stream) {
  if (rows == 0) return WQ_OK;
  WQ_REQUIRE(x && weight && out_norm, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && n <= (1 << 24) && rows <= 0x7fffffff, WQ_ERR_INVALID_ARGUMENT,
             "need rows >= 0 and 0 < n, n %% 8 == 0 (n = %lld)", (long long)n);
  WQ_REQUIRE(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out_norm | (uintptr_t)delta | (uintptr_t)out_sum) % 16 == 0,
             WQ_ERR_INVALID_ARGUMENT, "operands must be 16-byte aligned");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const half_t*>(x), reinterpret_cast<const half_t*>(delta),
                     reinterpret_cast<const half_t*>(weight), (int)n, eps, reinterpret_cast<half_t*>(out_norm),
                     reinterpret_cast<half_t*>(out_sum));
  return check_launch("add_rmsnorm");
}

extern "C" int wq_silu_mul(const uint16_t* gate_up, int64_t rows, int64_t n, uint16_t* out, void* stream) {
  if (rows == 0) return WQ_OK;
  WQ_REQUIRE(gate_up && out, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(rows > 0 && n > 0 && n % 8 == 0 && n <= (1 << 26), WQ_ERR_INVALID_ARGUMENT,
             "need rows >= 0 and 0 < n, n %% 8 == 0 (n = %lld)", (long long)n);
  WQ_REQUIRE(((uintptr_t)gate_up | (uintptr_t)out) % 16 == 0, WQ_ERR_INVALID_ARGUMENT, "operands must be 16-byte aligned");
  const size_t chunks = (size_t)rows * (size_t)(n / 8);
  const unsigned grid = (unsigned)((chunks + 255) / 256 < 4096 ? (chunks + 255) / 256 : 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const half_t*>(gate_up), (int)rows, (int)n, reinterpret_cast<half_t*>(out));
  return check_launch("silu_mul");
}

extern "C" int wq_decode_attention_workspace_size(int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                                  size_t* bytes) {
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int rc = attention_shape_check(q_heads, kv_heads, head_dim, max_seq);
  if (rc != WQ_OK) return rc;
  *bytes = attention_workspace_bytes(q_heads, kv_heads, max_seq);
  return WQ_OK;
}

extern "C" int wq_decode_attention(const uint16_t* qkv, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                   const uint16_t* q_norm_weight, const uint16_t* k_norm_weight, float eps,
                                   const uint16_t* cos_table, const uint16_t* sin_table, const int32_t* position,
                                   uint16_t* key_cache, uint16_t* value_cache, int64_t max_seq, float scale,
                                   uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  const int rc = attention_shape_check(q_heads, kv_heads, head_dim, max_seq);
  if (rc != WQ_OK) return rc;
  WQ_REQUIRE(qkv && cos_table && sin_table && position && key_cache && value_cache && out, WQ_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  WQ_REQUIRE(((uintptr_t)qkv | (uintptr_t)key_cache | (uintptr_t)value_cache) % 16 == 0, WQ_ERR_INVALID_ARGUMENT,
             "qkv and the caches must be 16-byte aligned");
  const int64_t nc = (max_seq + kChunk - 1) / kChunk;
  const size_t need = attention_workspace_bytes(q_heads, kv_heads, max_seq);
  WQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), WQ_ERR_WORKSPACE,
             "decode attention needs a zero-filled workspace of %zu bytes (got %zu)", need, workspace_bytes);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(workspace);
  float* ml = need ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + align256((size_t)kv_heads * 4))
                   : nullptr;
  float* po = need ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ml) +
                                              align256((size_t)kv_heads * nc * (q_heads / kv_heads) * 2 * 4))
                   : nullptr;
  hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)kv_heads, (unsigned)nc), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const half_t*>(qkv), (int)q_heads, (int)kv_heads,
                     reinterpret_cast<const half_t*>(q_norm_weight), reinterpret_cast<const half_t*>(k_norm_weight), eps,
                     reinterpret_cast<const half_t*>(cos_table), reinterpret_cast<const half_t*>(sin_table), position,
                     reinterpret_cast<half_t*>(key_cache), reinterpret_cast<half_t*>(value_cache), (int)max_seq, scale,
                     reinterpret_cast<half_t*>(out), po, ml, cnt);
  return check_launch("decode_attention");
}
