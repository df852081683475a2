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
constexpr int kSub = 64;          // KV positions per attention sub-chunk (one per lane of a softmax wave)
constexpr int kMaxGroup = 8;      // q heads per kv head
constexpr int kMaxChunks = 64;    // attention workgroups per kv head
constexpr int kMaxSpc = 2;        // sub-chunks per workgroup
constexpr int kMaxSeq = kMaxChunks * kMaxSpc * kSub;

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

// Reductions over the 16 lanes of a DPP row (every lane gets the result):
// quad swaps, then the half-row and row mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_f<0xb1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4e>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
  return fmaxf(v, dpp_f<0x140>(v));  // row_mirror
}

__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<0xb1>(v);
  v += dpp_f<0x4e>(v);
  v += dpp_f<0x141>(v);
  return v + dpp_f<0x140>(v);
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

// Split of a kv head's positions over workgroups: `spc` (1 or 2) sub-chunks
// of 64 positions per workgroup, so that no head has more than kMaxChunks
// workgroups (the merge reads one partial per workgroup).
struct AttnSplit {
  int spc, nc;
};

AttnSplit attn_split(int64_t max_seq) {
  const int64_t subs = (max_seq + kSub - 1) / kSub;
  const int spc = (int)((subs + kMaxChunks - 1) / kMaxChunks);
  return {spc, (int)((subs + spc - 1) / spc)};
}

// grid = (kv_heads, chunks); 256 threads = 4 waves.  Workgroup c of kv head
// h covers positions [c * SPC * 64, (c + 1) * SPC * 64) in sub-chunks of 64,
// with an online softmax over the head's G <= 8 query heads:
//   loads   every K fragment and V row this workgroup needs is requested
//           before the q/k prologue (rows clamped into the cache; rows past
//           L or at `pos` are replaced below);
//   scores  S[g][p] = q_g . k_p on the matrix cores: A = the query heads
//           (rows g, zero past G), B = 16 key rows per wave (each lane 16
//           bytes of one row), four k-steps of 32 elements;
//   softmax DPP row r (16 lanes x 4 positions) of wave w owns query head
//           4w + r: running max / sum and the rescale factor;
//   P.V     lane (dg, q) of wave w: elements 8dg .. 8dg+7 of positions
//           4(q + 4w) .. +3, one 16-byte V load per position, one float4
//           of P per head; the four position quads of a wave are summed
//           with shuffles at the end.
// The workgroup whose chunk holds `pos` also normalizes, rotates and
// appends the new key and value, and takes them from LDS.  With one chunk
// per head the workgroup writes the output; otherwise each chunk writes its
// (max, sum, unnormalized output) to the workspace and
// decode_attention_merge_kernel, launched next, combines them.
template <int G, int SPC>
__global__ __launch_bounds__(256, 2) void decode_attention_kernel(
    const half_t* __restrict__ qkv, int H, int KV, const half_t* __restrict__ qn_w,
    const half_t* __restrict__ kn_w, float eps, const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
    const int32_t* __restrict__ position, half_t* kc, half_t* vc, int max_seq, float scale,
    half_t* __restrict__ out, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  constexpr int D = kHeadDim, C = kSub, GM = kMaxGroup;
  __shared__ __attribute__((aligned(16))) half_t qh[GM][D];
  __shared__ __attribute__((aligned(16))) half_t knew[D];
  __shared__ __attribute__((aligned(16))) half_t vnew[D];
  __shared__ __attribute__((aligned(16))) float sc[GM][C];
  __shared__ float alph[GM];
  __shared__ __attribute__((aligned(16))) float red[4 * GM * D];   // per-wave P.V partials; later the merge's staging
  __shared__ float mls[GM][2];

  const int h = blockIdx.x, chunk = blockIdx.y, NC = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, kb = lane >> 4;
  const int pos = *position;
  if (pos < 0 || pos >= max_seq) {
    if (h == 0 && chunk == 0)
      for (int j = tid; j < H * D; j += 256) out[j] = (half_t)__builtin_nanf("");
    return;
  }
  const int L = pos + 1;
  const int p0 = chunk * SPC * C;
  const bool active = p0 < L;
  const bool owner = pos >= p0 && pos < p0 + SPC * C;
  const half_t* kh = kc + (size_t)h * max_seq * D;
  const half_t* vh = vc + (size_t)h * max_seq * D;
  const int dg = lane & 15, pq = (lane >> 4) + 4 * wave;   // P.V: elements 8dg.., positions 4pq..4pq+3

  uint4_t kr[SPC][4], vr[SPC][4];
  if (active) {
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
      const int rk = min(p0 + s * C + 16 * wave + i, max_seq - 1);
      const uint4_t* ks_src = reinterpret_cast<const uint4_t*>(kh + (size_t)rk * D + 8 * kb);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kr[s][ks] = ks_src[4 * ks];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rv = min(p0 + s * C + 4 * pq + e, max_seq - 1);
        vr[s][e] = *reinterpret_cast<const uint4_t*>(vh + (size_t)rv * D + 8 * dg);
      }
    }
  }

  if (active) {
    const half_t* cs = cos_t + (size_t)pos * D;
    const half_t* sn = sin_t + (size_t)pos * D;
    for (int g = wave; g < GM; g += 4) {
      half2_t r = {};
      if (g < G) {
        const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(h * G + g) * D)[lane];
        r = norm_rope_pair(v, qn_w, eps, cs, sn, lane);
      }
      reinterpret_cast<half2_t*>(qh[g])[lane] = r;
    }
    if (owner && wave == 0) {
      const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + h) * D)[lane];
      const half2_t r = norm_rope_pair(v, kn_w, eps, cs, sn, lane);
      reinterpret_cast<half2_t*>(knew)[lane] = r;
      reinterpret_cast<half2_t*>(kc + (size_t)h * max_seq * D + (size_t)pos * D)[lane] = r;
    }
    if (owner && wave == 1) {
      const half2_t v = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + KV + h) * D)[lane];
      reinterpret_cast<half2_t*>(vnew)[lane] = v;
      reinterpret_cast<half2_t*>(vc + (size_t)h * max_seq * D + (size_t)pos * D)[lane] = v;
    }
  }
  __syncthreads();

  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int k = 0; k < 8; ++k) o[g][k] = 0.f;
  const int srow = lane >> 4, sj = lane & 15, sg = 4 * wave + srow;
  float m_run = -INFINITY, l_run = 0.f;

  if (active) {
    half8_t qa[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qa[ks] = i < GM ? *reinterpret_cast<const half8_t*>(&qh[i < GM ? i : 0][32 * ks + 8 * kb]) : half8_t{};
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
      const int ps = p0 + s * C;
      if (ps < L) {
        const int pk = ps + 16 * wave + i;
        if (pk == pos) {
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) kr[s][ks] = *reinterpret_cast<const uint4_t*>(knew + 32 * ks + 8 * kb);
        }
        float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16(qa[ks], __builtin_bit_cast(half8_t, kr[s][ks]), acc);
        if (kb < 2) {
#pragma unroll
          for (int v = 0; v < 4; ++v) sc[4 * kb + v][16 * wave + i] = pk < L ? acc[v] * scale : -INFINITY;
        }
        __syncthreads();
        if (sg < G) {
          float4_t x = *reinterpret_cast<const float4_t*>(&sc[sg][4 * sj]);
          const float m_new = fmaxf(m_run, row_max16(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]))));   // finite
          float es = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[e] = x[e] == -INFINITY ? 0.f : expf(x[e] - m_new);
            es += x[e];
          }
          const float a = expf(m_run - m_new);   // 0 on the first sub-chunk
          l_run = l_run * a + row_sum16(es);
          m_run = m_new;
          *reinterpret_cast<float4_t*>(&sc[sg][4 * sj]) = x;
          if (sj == 0) alph[sg] = a;
        }
        __syncthreads();
        // Rows past L carry P = 0; row `pos` comes from LDS, clamped or stale
        // rows are zeroed so that 0 * garbage cannot produce NaN.
        half8_t v8[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int p = ps + 4 * pq + e;
          v8[e] = p == pos ? *reinterpret_cast<const half8_t*>(vnew + 8 * dg)
                           : (p < L ? __builtin_bit_cast(half8_t, vr[s][e]) : half8_t{});
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float a = alph[g];
          const float4_t pr = *reinterpret_cast<const float4_t*>(&sc[g][4 * pq]);
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            float t = o[g][k] * a;
#pragma unroll
            for (int e = 0; e < 4; ++e) t += pr[e] * (float)v8[e][k];
            o[g][k] = t;
          }
        }
        __syncthreads();
      }
    }
    if (sg < G && sj == 0) {
      mls[sg][0] = m_run;
      mls[sg][1] = l_run;
    }
    // Sum the four position quads of this wave (lanes dg, dg+16, dg+32, dg+48).
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float t = o[g][k];
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        o[g][k] = t;
      }
    if (lane < 16) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float* dst = red + (wave * GM + g) * D + 8 * dg;
        *reinterpret_cast<float4_t*>(dst) = float4_t{o[g][0], o[g][1], o[g][2], o[g][3]};
        *reinterpret_cast<float4_t*>(dst + 4) = float4_t{o[g][4], o[g][5], o[g][6], o[g][7]};
      }
    }
  }
  __syncthreads();

  if (NC == 1) {
    for (int j = tid; j < G * D; j += 256) {
      const int g = j / D, d = j % D;
      const float o = red[g * D + d] + red[(GM + g) * D + d] + red[(2 * GM + g) * D + d] + red[(3 * GM + g) * D + d];
      out[(size_t)(h * G + g) * D + d] = (half_t)(o / mls[g][1]);
    }
    return;
  }
  // Several chunks: publish this chunk's partial for decode_attention_merge
  // (the next launch on the stream).
  if (active) {
    if (tid < G * (D / 4)) {
      const int g = tid / (D / 4), d = 4 * (tid % (D / 4));
      float4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = red[g * D + d + e] + red[(GM + g) * D + d + e] + red[(2 * GM + g) * D + d + e] +
               red[(3 * GM + g) * D + d + e];
      *reinterpret_cast<float4_t*>(ws_o + (((size_t)(h * NC + chunk) * G + g) * D + d)) = o;
    }
    if (tid < 2 * G) ws_ml[((size_t)(h * NC + chunk) * G) * 2 + tid] = mls[tid >> 1][tid & 1];
  }
}

// Merge of the chunk partials of one query head: grid = q_heads, 128 threads
// (one output element each).  All of the head's partial outputs are
// requested before the maxima are known, then combined in chunk order:
// out = sum_c exp(m_c - M) O_c / sum_c exp(m_c - M) l_c.
__global__ __launch_bounds__(128) void decode_attention_merge_kernel(const int32_t* __restrict__ position, int G,
                                                                     int NC, int chunk_positions, int max_seq,
                                                                     const float* __restrict__ ws_o,
                                                                     const float* __restrict__ ws_ml,
                                                                     half_t* __restrict__ out) {
  constexpr int D = kHeadDim;
  __shared__ float ms[kMaxChunks], ls[kMaxChunks];
  const int qh = blockIdx.x, h = qh / G, g = qh % G, d = threadIdx.x;
  const int pos = *position;
  if (pos < 0 || pos >= max_seq) return;   // the attention launch already wrote NaN
  const int NA = min((pos + chunk_positions) / chunk_positions, NC);   // chunks holding positions 0..pos
  float part[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c)
    part[c] = c < NA ? ws_o[((size_t)(h * NC + c) * G + g) * D + d] : 0.f;
  if (d < NA) {
    ms[d] = ws_ml[((size_t)(h * NC + d) * G + g) * 2];
    ls[d] = ws_ml[((size_t)(h * NC + d) * G + g) * 2 + 1];
  }
  __syncthreads();
  float M = -INFINITY;
  for (int c = 0; c < NA; ++c) M = fmaxf(M, ms[c]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c)
    if (c < NA) {
      const float w = expf(ms[c] - M);
      num += w * part[c];
      den += w * ls[c];
    }
  out[(size_t)qh * D + d] = (half_t)(num / den);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t attention_workspace_bytes(int64_t H, int64_t KV, int64_t max_seq) {
  const int64_t nc = attn_split(max_seq).nc;
  const int64_t g = H / KV;
  return nc <= 1 ? 0 : align256((size_t)KV * nc * g * 2 * 4) + (size_t)KV * nc * g * kHeadDim * 4;
}

int attention_shape_check(int64_t H, int64_t KV, int64_t head_dim, int64_t max_seq) {
  WQ_REQUIRE(H > 0 && KV > 0 && max_seq > 0, WQ_ERR_INVALID_ARGUMENT, "q_heads, kv_heads and max_seq must be positive");
  WQ_REQUIRE(head_dim == kHeadDim, WQ_ERR_UNSUPPORTED, "decode attention is built for head_dim 128 (got %lld)",
             (long long)head_dim);
  WQ_REQUIRE(H % KV == 0, WQ_ERR_INVALID_ARGUMENT, "q_heads (%lld) must be a multiple of kv_heads (%lld)",
             (long long)H, (long long)KV);
  WQ_REQUIRE(H / KV <= kMaxGroup, WQ_ERR_UNSUPPORTED, "at most %d query heads per kv head", kMaxGroup);
  WQ_REQUIRE(max_seq <= kMaxSeq, WQ_ERR_UNSUPPORTED, "max_seq must be <= %d", kMaxSeq);
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
  const AttnSplit split = attn_split(max_seq);
  const int64_t nc = split.nc;
  const size_t need = attention_workspace_bytes(q_heads, kv_heads, max_seq);
  WQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), WQ_ERR_WORKSPACE,
             "decode attention needs a zero-filled workspace of %zu bytes (got %zu)", need, workspace_bytes);
  float* ml = need ? reinterpret_cast<float*>(workspace) : nullptr;
  float* po = need ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) +
                                              align256((size_t)kv_heads * nc * (q_heads / kv_heads) * 2 * 4))
                   : nullptr;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)kv_heads, (unsigned)nc), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const half_t*>(qkv), (int)q_heads, (int)kv_heads,
                       reinterpret_cast<const half_t*>(q_norm_weight), reinterpret_cast<const half_t*>(k_norm_weight),
                       eps, reinterpret_cast<const half_t*>(cos_table), reinterpret_cast<const half_t*>(sin_table),
                       position, reinterpret_cast<half_t*>(key_cache), reinterpret_cast<half_t*>(value_cache),
                       (int)max_seq, scale, reinterpret_cast<half_t*>(out), po, ml);
  };
  const int g = (int)(q_heads / kv_heads);
#define WQ_ATTN_CASE(GG)                                                                     \
  case GG:                                                                                   \
    if (split.spc == 1) launch(decode_attention_kernel<GG, 1>); else launch(decode_attention_kernel<GG, 2>); \
    break;
  switch (g) {
    WQ_ATTN_CASE(1) WQ_ATTN_CASE(2) WQ_ATTN_CASE(3) WQ_ATTN_CASE(4)
    WQ_ATTN_CASE(5) WQ_ATTN_CASE(6) WQ_ATTN_CASE(7) WQ_ATTN_CASE(8)
    default: return fail(WQ_ERR_UNSUPPORTED, "query heads per kv head out of range");
  }
#undef WQ_ATTN_CASE
  if (nc > 1) {
    const int rc2 = check_launch("decode_attention");
    if (rc2 != WQ_OK) return rc2;
    hipLaunchKernelGGL(decode_attention_merge_kernel, dim3((unsigned)q_heads), dim3(kHeadDim), 0, as_stream(stream),
                       position, g, (int)nc, split.spc * kSub, (int)max_seq, po, ml, reinterpret_cast<half_t*>(out));
    return check_launch("decode_attention_merge");
  }
  return check_launch("decode_attention");
}
