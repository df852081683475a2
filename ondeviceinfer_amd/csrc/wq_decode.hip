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
constexpr int kBlock = 16;        // KV positions per attention block (one wave's matrix tile)
constexpr int kMaxGroup = 8;      // q heads per kv head
constexpr int kMaxBlocksPerWave = 4;
constexpr int kMaxChunks = 64;    // attention workgroups per kv head (one merge lane each)
constexpr int kMaxSeq = 16384;    // positions of the cache (the API's limit)
static_assert(kMaxSeq <= kMaxChunks * 4 * kMaxBlocksPerWave * kBlock, "the four-wave split covers the largest cache");


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
  ss = wave_sum_rl(ss);
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
    for (int e = 0; e < 8; ++e) o[e] = (half_t)silu_f((float)g[e]) * u[e];
    *reinterpret_cast<half8_t*>(out + r * n + 8 * c) = o;
  }
}

// ---------------------------------------------------------------- attention
// Per-head RMSNorm and RoPE of one 128-vector held two elements per lane
// (lane l: elements 2l, 2l+1), with the lane's norm weights, cos and sin
// already loaded.  rotate_half pairs element d with d +- 64, i.e. lane l
// with lane l ^ 32.  Every product and the sum round to fp16, as in
// `q * cos + rotate_half(q) * sin` on fp16 tensors.
__device__ __forceinline__ half2_t norm_rope_pair(half2_t v, bool norm, half2_t nw, float eps, half2_t c2,
                                                  half2_t s2, int lane) {
#pragma clang fp contract(off)
  if (norm) {
    const float a = (float)v[0], b = (float)v[1];
    const float r = rsqrtf(wave_sum_rl(a * a + b * b) * (1.0f / kHeadDim) + eps);
    v[0] = nw[0] * (half_t)(a * r);
    v[1] = nw[1] * (half_t)(b * r);
  }
  half2_t p = as_h2(__shfl_xor(as_u32(v), 32));
  if (lane < 32) p = -p;
  const half2_t t1 = v * c2;
  const half2_t t2 = p * s2;
  return t1 + t2;
}

// Work split of the attention: a kv head's cache is cut into `nc` chunks of
// `nbc` 16-position blocks, one workgroup of `sw` waves each; wave w takes
// blocks w, w + sw, ...  Five waves when about one workgroup per compute unit
// over the whole grid (256 / kv_heads chunks per kv head) leaves each wave
// at most two blocks, the chunk rounded up to whole rounds of the five waves:
// at the Qwen3-14B geometry with a 4229-position cache, 27 chunks of 10
// blocks per kv head, 216 workgroups.  Longer caches take four-wave
// workgroups of 4, 8, 12 or 16 blocks, as few as keep nc <= 64 (at 16384
// positions 64 chunks of 16 blocks, two workgroups per compute unit; five
// waves of four blocks need 174 registers, one workgroup per unit).
// Measured on MI355X (40 layers, 4229 positions, position 4101): 7.4 us for
// the attention launch against 7.9 for four-wave workgroups of 8 blocks (272
// workgroups, 16 of them sharing a compute unit), 8.6 for four waves of 9
// blocks (the third block of wave 0 costs more than the shared units did),
// 7.7 for six waves of 12, 8.8 for eight of 16.  With 8 kv heads the chunks
// of kv head h are workgroups h, h + 8, ..., all on XCD h.
struct AttnSplit {
  int nbc, nc, bpw, sw;   // blocks per chunk, chunks per kv head, blocks per wave, waves per workgroup
};

AttnSplit attn_split(int64_t kv_heads, int64_t max_seq) {
  const int64_t blocks = (max_seq + kBlock - 1) / kBlock;
  int64_t target = 256 / kv_heads;
  target = target < 1 ? 1 : (target > kMaxChunks ? kMaxChunks : target);
  int64_t nbc = ((blocks + target - 1) / target + 4) / 5 * 5;
  int sw = 5;
  if (nbc > 2 * 5) {
    sw = 4;
    const int64_t subs = (blocks + 3) / 4;                     // four-block sub-chunks
    nbc = 4 * ((subs + kMaxChunks - 1) / kMaxChunks);
  }
  const int64_t nc = (blocks + nbc - 1) / nbc;
  return {(int)nbc, (int)nc, (int)((nbc + sw - 1) / sw), sw};
}

// Orders this wave's LDS accesses around a wave-private exchange (the
// compiler reasons per lane and could otherwise move a lane's read of another
// lane's value above the write; the hardware keeps one wave's LDS operations
// in order).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// grid = kv_heads * nc workgroups (flat id f: kv head f % kv_heads, chunk
// f / kv_heads); SW = 5 or 4 waves.  Chunk c covers positions
// [c * nbc * 16, (c + 1) * nbc * 16); wave w owns blocks w, w + SW, ... (16
// positions each, BPW at most) and runs its own online softmax over them for
// the head's G <= 8 query heads, so the block loop has no workgroup barrier.
// Lane l is (r, i) = (l / 16, l % 16).
//   loads   the position, then the prologue's operands (q heads w and w + SW,
//           cos/sin rows, norm weights, the new k/v), then every K fragment
//           and V row of the wave's blocks (rows clamped into the cache; rows
//           past L or at `pos` are replaced below), so the q/k prologue runs
//           while the
//           cache streams in (issuing the stream itself takes the wave about
//           1.5 us: the memory pipeline accepts the requests only as fast as
//           it drains them);
//   prologue q/k RMSNorm + RoPE, q and (in the chunk that holds `pos`) the
//           new key / value to LDS, the new key / value appended to the cache;
//   scores  S[g][p] = q_g . k_p on the matrix cores (16x16x32): A = the query
//           heads (rows g, zero past G), B = the block's 16 key rows (each
//           lane 16 bytes of one row); lane (r, i) gets heads 4r .. 4r+3 at
//           position i, in log2 units (scale * log2 e);
//   softmax the 16 lanes of DPP row r reduce max and sum for heads 4r + v;
//   P.V     on the matrix cores (16x16x16): A = P as fp16 [head][position],
//           B = V^T [d][position], both through wave-private LDS (the V rows
//           arrive 16 bytes of d per lane and are written transposed), one
//           MFMA per 16 values of d; the accumulator rows are the heads 4r+v
//           of the lane's own softmax row, so the online rescale is local.
// The waves' (max, sum, output) are combined through LDS.  Rows past L
// and row `pos` (fetched before it was written) are replaced: P = 0 and
// zeroed V past L, the LDS copies at `pos`.  With one workgroup per head the
// workgroup writes the output; otherwise every workgroup, active or not,
// writes its (max, sum) pair and unnormalized output to the workspace, and
// decode_attention_merge_kernel (the next launch) combines them without
// reading the position: an empty chunk writes (-inf, 0) and zeros and
// weighs nothing, and an invalid position leaves every max at -inf, which
// the merge turns into NaN.
template <int G, int BPW, int SW>
__global__ __launch_bounds__(64 * SW, 2) void decode_attention_kernel(
    const half_t* __restrict__ qkv, int H, int KV, const half_t* __restrict__ qn_w,
    const half_t* __restrict__ kn_w, float eps, const half_t* __restrict__ cos_t, const half_t* __restrict__ sin_t,
    const int32_t* __restrict__ position, half_t* kc, half_t* vc, int max_seq, float scale_log2, int nbc,
    half_t* __restrict__ out, float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  constexpr int D = kHeadDim, GM = kMaxGroup;
  constexpr int VTS = 20;   // V^T row stride in halves (40 bytes: the 16 B-fragment reads hit distinct banks)
  __shared__ __attribute__((aligned(16))) half_t qh[GM][D];
  __shared__ __attribute__((aligned(16))) half_t knew[D];
  __shared__ __attribute__((aligned(16))) half_t vnew[D];
  __shared__ __attribute__((aligned(16))) half_t pl[SW][16][16];    // per-wave P, [head][position]
  __shared__ __attribute__((aligned(16))) half_t vt[SW][D][VTS];    // per-wave V^T, [d][position]
  __shared__ __attribute__((aligned(16))) float red[SW][GM][D];    // per-wave unnormalized outputs
  __shared__ float mlw[SW][GM][2];                                 // per-wave (max, sum)

  const int h = blockIdx.x % KV, chunk = blockIdx.x / KV, NC = gridDim.x / KV;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int p0 = chunk * nbc * kBlock;
  const half_t* kh = kc + (size_t)h * max_seq * D;
  const half_t* vh = vc + (size_t)h * max_seq * D;
  const int dg = lane & 15, q4 = lane >> 4;   // V rows: elements 8dg.., the block's positions 4q4 .. 4q4+3

  // 1) The position, then the prologue's operands: query heads wave and
  //    wave + SW, the new key (owner wave 0) or value (owner wave 1), norm
  //    weights, cos / sin at the position.
  const int pos = *position;
  const bool valid = pos >= 0 && pos < max_seq;
  const int L = valid ? pos + 1 : 0;
  const bool owner = valid && pos >= p0 && pos < p0 + nbc * kBlock;
  const int prow = valid ? pos : 0;
  const half2_t c2 = reinterpret_cast<const half2_t*>(cos_t + (size_t)prow * D)[lane];
  const half2_t s2 = reinterpret_cast<const half2_t*>(sin_t + (size_t)prow * D)[lane];
  static_assert(SW >= kMaxGroup / 2, "two query heads per wave at most");
  half2_t qv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int g = wave + SW * j;
    qv[j] = g < G ? reinterpret_cast<const half2_t*>(qkv + (size_t)(h * G + g) * D)[lane] : half2_t{};
  }
  const half2_t nq = qn_w ? reinterpret_cast<const half2_t*>(qn_w)[lane] : half2_t{};
  half2_t nv = {}, nk = {};
  if (owner && wave == 0) {
    nv = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + h) * D)[lane];
    if (kn_w) nk = reinterpret_cast<const half2_t*>(kn_w)[lane];
  }
  if (owner && wave == 1) nv = reinterpret_cast<const half2_t*>(qkv + (size_t)(H + KV + h) * D)[lane];

  // 2) The cache stream: this wave's blocks w, w + SW, ... of the chunk.
  //    Every slot issues its loads (a slot past the chunk's blocks rereads
  //    the chunk's last block, a cache hit, and is never used), so the
  //    prologue's wait counts only the requests issued after its own.
  uint4_t kr[BPW][4], vr[BPW][4];
#pragma unroll
  for (int b = 0; b < BPW; ++b) {
    const int pb = p0 + min(wave + SW * b, nbc - 1) * kBlock;
    const int rk = min(pb + i, max_seq - 1);
    const uint4_t* ks_src = reinterpret_cast<const uint4_t*>(kh + (size_t)rk * D + 8 * kb);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kr[b][ks] = ks_src[4 * ks];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rv = min(pb + 4 * q4 + e, max_seq - 1);
      vr[b][e] = *reinterpret_cast<const uint4_t*>(vh + (size_t)rv * D + 8 * dg);
    }
  }

  // 3) q / k RMSNorm + RoPE; the new key and value go to LDS and are
  //    appended to the cache (this workgroup's loads of row `pos` were
  //    issued before and are replaced by the LDS copies).
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int g = wave + SW * j;
    const half2_t r = g < G ? norm_rope_pair(qv[j], qn_w != nullptr, nq, eps, c2, s2, lane) : half2_t{};
    if (g < GM) reinterpret_cast<half2_t*>(qh[g])[lane] = r;
  }
  if (owner && wave == 0) {
    const half2_t r = norm_rope_pair(nv, kn_w != nullptr, nk, eps, c2, s2, lane);
    reinterpret_cast<half2_t*>(knew)[lane] = r;
    reinterpret_cast<half2_t*>(kc + (size_t)h * max_seq * D + (size_t)pos * D)[lane] = r;
  }
  if (owner && wave == 1) {
    reinterpret_cast<half2_t*>(vnew)[lane] = nv;
    reinterpret_cast<half2_t*>(vc + (size_t)h * max_seq * D + (size_t)pos * D)[lane] = nv;
  }
  __syncthreads();

  if (p0 >= L) {
    // Nothing to attend in this chunk (in any chunk when the position is
    // invalid; chunk 0 is active whenever it is valid).
    if (NC == 1) {
      for (int j = tid; j < G * D; j += 64 * SW) out[(size_t)h * G * D + j] = (half_t)__builtin_nanf("");
    } else {
      for (int j = tid; j < G * (D / 4); j += 64 * SW) {
        const size_t slot = (size_t)(h * G + j / (D / 4)) * NC + chunk;
        *reinterpret_cast<float4_t*>(ws_o + slot * D + 4 * (j % (D / 4))) = float4_t{0.f, 0.f, 0.f, 0.f};
      }
      if (tid < G) {
        ws_ml[((size_t)(h * G + tid) * NC + chunk) * 2] = -INFINITY;
        ws_ml[((size_t)(h * G + tid) * NC + chunk) * 2 + 1] = 0.f;
      }
    }
    return;
  }

  half8_t qa[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qa[ks] = i < GM ? *reinterpret_cast<const half8_t*>(&qh[i < GM ? i : 0][32 * ks + 8 * kb]) : half8_t{};
  float4_t oacc[D / 16];
#pragma unroll
  for (int t = 0; t < D / 16; ++t) oacc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[4], l_run[4];   // heads 4kb + v, the same in all 16 lanes of the row
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    m_run[v] = -INFINITY;
    l_run[v] = 0.f;
  }

#pragma unroll
  for (int b = 0; b < BPW; ++b) {
    const int ps = p0 + (wave + SW * b) * kBlock;   // the block's first position (wave-uniform)
    if (wave + SW * b < nbc && ps < L) {
      const int pk = ps + i;
      if (pk == pos) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) kr[b][ks] = *reinterpret_cast<const uint4_t*>(knew + 32 * ks + 8 * kb);
      }
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16(qa[ks], __builtin_bit_cast(half8_t, kr[b][ks]), acc);
      // Position ps < L is in every row, so each row max is finite.
      float pv[4], alpha[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float sv = pk < L ? acc[v] * scale_log2 : -INFINITY;
        const float mn = fmaxf(m_run[v], row_max16(sv));
        pv[v] = exp2_hw(sv - mn);           // -inf -> 0
        alpha[v] = exp2_hw(m_run[v] - mn);  // 0 on the wave's first block
        l_run[v] = l_run[v] * alpha[v] + row_sum16(pv[v]);
        m_run[v] = mn;
      }
      // Rows past L carry P = 0 and are zeroed (0 * NaN would poison the
      // sum); row `pos` comes from LDS.
      half8_t v8[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int p = ps + 4 * q4 + e;
        v8[e] = p == pos ? *reinterpret_cast<const half8_t*>(vnew + 8 * dg)
                         : (p < L ? __builtin_bit_cast(half8_t, vr[b][e]) : half8_t{});
      }
      wave_lds_sync();   // the previous block's fragment reads are done
#pragma unroll
      for (int v = 0; v < 4; ++v) pl[wave][4 * kb + v][i] = (half_t)pv[v];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        *reinterpret_cast<half4_t*>(&vt[wave][8 * dg + k][4 * q4]) = half4_t{v8[0][k], v8[1][k], v8[2][k], v8[3][k]};
      wave_lds_sync();
      const half4_t pa = *reinterpret_cast<const half4_t*>(&pl[wave][i][4 * kb]);
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        const half4_t vb = *reinterpret_cast<const half4_t*>(&vt[wave][16 * t + i][4 * kb]);
        float4_t o = oacc[t];
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] *= alpha[v];
        oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vb, o, 0, 0, 0);
      }
    }
  }

  // oacc[t][v] = this wave's unnormalized output of head 4kb + v at
  // d = 16t + i (a wave with no block holds zeros, max -inf).
  if (kb < 2) {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (4 * kb + v < G) {
#pragma unroll
        for (int t = 0; t < D / 16; ++t) red[wave][4 * kb + v][16 * t + i] = oacc[t][v];
      }
  }
  if (i == 0 && kb < 2) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      mlw[wave][4 * kb + v][0] = m_run[v];
      mlw[wave][4 * kb + v][1] = l_run[v];
    }
  }
  __syncthreads();

  // Combine the waves (a wave with no position below L has max -inf,
  // sum 0 and output 0; wave 0 always has one, so M is finite).
  for (int j = tid; j < G * (D / 4); j += 64 * SW) {
    const int g = j / (D / 4), d = 4 * (j % (D / 4));
    float M = mlw[0][g][0];
#pragma unroll
    for (int w = 1; w < SW; ++w) M = fmaxf(M, mlw[w][g][0]);
    float4_t num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int w = 0; w < SW; ++w) {
      const float wt = exp2_hw(mlw[w][g][0] - M);
      num += wt * *reinterpret_cast<const float4_t*>(&red[w][g][d]);
      den += wt * mlw[w][g][1];
    }
    if (NC == 1) {
      half4_t r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = (half_t)(num[e] / den);
      *reinterpret_cast<half4_t*>(out + (size_t)(h * G + g) * D + d) = r;
    } else {
      const size_t slot = (size_t)(h * G + g) * NC + chunk;
      *reinterpret_cast<float4_t*>(ws_o + slot * D + d) = num;
      if (d == 0) {
        ws_ml[slot * 2] = M;
        ws_ml[slot * 2 + 1] = den;
      }
    }
  }
}

// Merge of the workgroup partials of one query head: grid = q_heads, 128
// threads (one output element each).  The NC <= NCM partial outputs are
// requested at once (at chunk indices clamped below NC, which weigh 0).
// Each wave holds the chunks' (max, sum) pairs one per lane and turns them
// into weights w_c = 2^(m_c - M) (0 for an empty chunk, whose output slot
// holds zeros) and sum_c w_c l_c with DPP row reductions and lane reads, so
// the merge needs no LDS and no barrier; lane c's weight is read out with
// v_readlane.  out = sum_c w_c O_c / sum_c w_c l_c, summed in chunk order.
// With no non-empty chunk (invalid position) the result is 0 / 0 = NaN.
template <int NCM>
__global__ __launch_bounds__(128) void decode_attention_merge_kernel(int NC, const float* __restrict__ ws_o,
                                                                     const float2_t* __restrict__ ws_ml,
                                                                     half_t* __restrict__ out, int xcd_group) {
  constexpr int D = kHeadDim;
  static_assert(NCM <= kMaxChunks && kMaxChunks <= 64, "one chunk per lane");
  // With 8 kv heads the attention's workgroups of kv head h all run on XCD h
  // (workgroups are dealt to the 8 XCDs round-robin by flat id h + 8c), so
  // its partials sit in that XCD's L2; xcd_group = query heads per kv head
  // then maps workgroup b to query head (b % 8) * xcd_group + b / 8, which
  // lands on the same XCD.  0 = launch order.
  const int b = blockIdx.x;
  const int qh = xcd_group > 0 ? (b & 7) * xcd_group + (b >> 3) : b;
  const int d = threadIdx.x, lane = d & 63;
  const float* po = ws_o + (size_t)qh * NC * D + d;
  float part[NCM];
#pragma unroll
  for (int c = 0; c < NCM; ++c) part[c] = po[(size_t)min(c, NC - 1) * D];
  const float2_t ml = lane < NC ? ws_ml[(size_t)qh * NC + lane] : float2_t{-INFINITY, 0.f};
  const float M = wave_max_rl(ml.x);
  const float w = ml.x == -INFINITY ? 0.f : exp2_hw(ml.x - M);
  const float den = wave_sum_rl(w * ml.y);
  float num = 0.f;
#pragma unroll
  for (int c = 0; c < NCM; ++c) num += lane_f(w, c) * part[c];
  out[(size_t)qh * D + d] = (half_t)(num / den);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t attention_workspace_bytes(int64_t H, int64_t KV, int64_t max_seq) {
  const int64_t nc = attn_split(KV, max_seq).nc;
  const int64_t g = H / KV;
  return nc <= 1 ? 0 : align256((size_t)KV * nc * g * 2 * 4) + (size_t)KV * nc * g * kHeadDim * 4;
}

// Prefill counterpart of the decode kernel's prologue, for `tokens` rows of
// a fused [q | k | v] projection at positions start .. start + tokens - 1:
// for each (token, head) a wave (lane l holds d = 2l, 2l+1) applies the
// head's RMSNorm and RoPE with norm_rope_pair (q and k), writes q token-major as
// [token][head][d], the layout prefill_attention_kernel reads (and torch's
// SDPA as a strided [head][token][d] view), and appends k and v to the cache
// rows.
// grid = tokens, 256 threads: wave w of token t's workgroup takes heads w,
// w + 4, ... with four head rows in flight (one workgroup per (token, four
// heads) left the waves too little to keep in flight).
__global__ __launch_bounds__(256) void prefill_qk_rope_kernel(const half_t* __restrict__ qkv, int T, int H, int KV,
                                                              const half_t* __restrict__ qn_w,
                                                              const half_t* __restrict__ kn_w, float eps,
                                                              const half_t* __restrict__ cos_t,
                                                              const half_t* __restrict__ sin_t, int start,
                                                              half_t* __restrict__ kc, half_t* __restrict__ vc,
                                                              int max_seq, half_t* __restrict__ q_out) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t = blockIdx.x;
  const int NH = H + 2 * KV;
  const half_t* src = qkv + (size_t)t * NH * kHeadDim;
  // The token's cos / sin row and the norm weights, once per wave.
  const half2_t c2 = as_h2(reinterpret_cast<const uint32_t*>(cos_t + (size_t)t * kHeadDim)[lane]);
  const half2_t s2 = as_h2(reinterpret_cast<const uint32_t*>(sin_t + (size_t)t * kHeadDim)[lane]);
  const half2_t nq = qn_w ? as_h2(reinterpret_cast<const uint32_t*>(qn_w)[lane]) : half2_t{};
  const half2_t nk = kn_w ? as_h2(reinterpret_cast<const uint32_t*>(kn_w)[lane]) : half2_t{};
  // Wave w takes heads w, w + 4, ...; four head rows in flight at a time.
  constexpr int kAhead = 4;
  for (int h0 = wave; h0 < NH; h0 += 4 * kAhead) {
    uint32_t v[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int hh = min(h0 + 4 * u, NH - 1);
      v[u] = reinterpret_cast<const uint32_t*>(src + (size_t)hh * kHeadDim)[lane];
    }
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int hh = h0 + 4 * u;   // wave-uniform
      if (hh >= NH) break;
      if (hh >= H + KV) {
        reinterpret_cast<uint32_t*>(vc + ((size_t)(hh - H - KV) * max_seq + start + t) * kHeadDim)[lane] = v[u];
        continue;
      }
      const bool is_q = hh < H;
      const bool has_w = (is_q ? qn_w : kn_w) != nullptr;
      const half2_t r = norm_rope_pair(as_h2(v[u]), has_w, is_q ? nq : nk, eps, c2, s2, lane);
      half_t* dst = is_q ? q_out + ((size_t)t * H + hh) * kHeadDim
                         : kc + ((size_t)(hh - H) * max_seq + start + t) * kHeadDim;
      reinterpret_cast<uint32_t*>(dst)[lane] = as_u32(r);
    }
  }
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

// ------------------------------------------------------------ embedding row
// out[r] = table[token[r]] for the rows of an fp16 table that may live in
// pinned host memory (read through its device-visible mapping, 16 bytes per
// lane: one row of 5120 is 640 lane loads over the host link).  One
// workgroup per row; a token outside [0, vocab) writes NaN and reads nothing.
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint4_t* __restrict__ table, int64_t vocab,
                                                         int chunks, const int64_t* __restrict__ tokens,
                                                         uint4_t* __restrict__ out, float* __restrict__ sumsq) {
  const int64_t t = tokens[blockIdx.x];
  const bool ok = t >= 0 && t < vocab;
  const uint4_t nan8 = {0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u};
  uint4_t* dst = out + (size_t)blockIdx.x * chunks;
  // Every lane runs every round (the bound is uniform), so the pairs of
  // 8-element chunks that make one 16-element sum of squares meet by a lane
  // swap; lanes past the row only skip their loads and stores.
  for (int c0 = 0; c0 < chunks; c0 += 256) {
    const int c = c0 + (int)threadIdx.x;
    const uint4_t v = c < chunks ? (ok ? table[(size_t)t * chunks + c] : nan8) : uint4_t{0u, 0u, 0u, 0u};
    if (c < chunks) dst[c] = v;
    if (sumsq != nullptr) {
      const half8_t h = __builtin_bit_cast(half8_t, v);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) q += (float)h[e] * (float)h[e];
      q += __shfl_xor(q, 1);
      if (c < chunks && (c & 1) == 0) sumsq[(size_t)blockIdx.x * (chunks / 2) + c / 2] = q;
    }
  }
}

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_host_device_pointer(const void* host_ptr, void** device_ptr) {
  WQ_REQUIRE(host_ptr && device_ptr, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host_ptr), 0);
  WQ_REQUIRE(e == hipSuccess && d, WQ_ERR_INVALID_ARGUMENT,
             "not a device-mapped pinned host allocation (hipHostGetDevicePointer: %s)", hipGetErrorString(e));
  *device_ptr = d;
  return WQ_OK;
}

extern "C" int wq_embed_rows(const uint16_t* table, int64_t vocab, int64_t hidden, const int64_t* tokens,
                             int64_t rows, uint16_t* out, float* sumsq_out, void* stream) {
  if (rows == 0) return WQ_OK;
  WQ_REQUIRE(table && tokens && out, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(vocab > 0 && hidden > 0 && hidden % 8 == 0 && hidden <= (1 << 24) && rows > 0 && rows <= 65535,
             WQ_ERR_INVALID_ARGUMENT, "need vocab > 0, 0 < hidden, hidden %% 8 == 0, 0 < rows <= 65535");
  WQ_REQUIRE(sumsq_out == nullptr || (hidden % 16 == 0 && (uintptr_t)sumsq_out % 4 == 0), WQ_ERR_INVALID_ARGUMENT,
             "sums of squares need hidden %% 16 == 0");
  WQ_REQUIRE(((uintptr_t)table | (uintptr_t)out) % 16 == 0 && (uintptr_t)tokens % 8 == 0, WQ_ERR_INVALID_ARGUMENT,
             "table and out must be 16-byte aligned, tokens 8-byte");
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4_t*>(table), vocab, (int)(hidden / 8), tokens,
                     reinterpret_cast<uint4_t*>(out), sumsq_out);
  return check_launch("embed_rows");
}

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
  const AttnSplit split = attn_split(kv_heads, max_seq);
  const int64_t nc = split.nc;
  const size_t need = attention_workspace_bytes(q_heads, kv_heads, max_seq);
  WQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), WQ_ERR_WORKSPACE,
             "decode attention needs a workspace of %zu bytes (got %zu)", need, workspace_bytes);
  float* ml = need ? reinterpret_cast<float*>(workspace) : nullptr;
  float* po = need ? reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) +
                                              align256((size_t)kv_heads * nc * (q_heads / kv_heads) * 2 * 4))
                   : nullptr;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3((unsigned)(kv_heads * nc)), dim3(64 * split.sw), 0, as_stream(stream),
                       reinterpret_cast<const half_t*>(qkv), (int)q_heads, (int)kv_heads,
                       reinterpret_cast<const half_t*>(q_norm_weight), reinterpret_cast<const half_t*>(k_norm_weight),
                       eps, reinterpret_cast<const half_t*>(cos_table), reinterpret_cast<const half_t*>(sin_table),
                       position, reinterpret_cast<half_t*>(key_cache), reinterpret_cast<half_t*>(value_cache),
                       (int)max_seq, scale * kLog2e, split.nbc, reinterpret_cast<half_t*>(out), po, ml);
  };
  const int g = (int)(q_heads / kv_heads);
#define WQ_ATTN_CASE(GG)                                                                     \
  case GG:                                                                                   \
    if (split.sw == 5) {                                                                     \
      if (split.bpw == 1) launch(decode_attention_kernel<GG, 1, 5>);                        \
      else launch(decode_attention_kernel<GG, 2, 5>);                                        \
    } else {                                                                                 \
      switch (split.bpw) {                                                                   \
        case 1: launch(decode_attention_kernel<GG, 1, 4>); break;                            \
        case 2: launch(decode_attention_kernel<GG, 2, 4>); break;                            \
        case 3: launch(decode_attention_kernel<GG, 3, 4>); break;                            \
        default: launch(decode_attention_kernel<GG, 4, 4>); break;                           \
      }                                                                                      \
    }                                                                                        \
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
    auto merge = nc <= 16   ? decode_attention_merge_kernel<16>
                 : nc <= 32 ? decode_attention_merge_kernel<32>
                 : nc <= 48 ? decode_attention_merge_kernel<48>
                            : decode_attention_merge_kernel<64>;
    const int xcd_group = kv_heads == 8 ? g : 0;   // 11.14 -> 11.03 us per layer with the merge (40 / 8 heads)
    hipLaunchKernelGGL(merge, dim3((unsigned)q_heads), dim3(kHeadDim), 0, as_stream(stream), (int)nc, po,
                       reinterpret_cast<const float2_t*>(ml), reinterpret_cast<half_t*>(out), xcd_group);
    return check_launch("decode_attention_merge");
  }
  return check_launch("decode_attention");
}

extern "C" int wq_prefill_qk_rope(const uint16_t* qkv, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                                  float eps, const uint16_t* cos_rows, const uint16_t* sin_rows, int64_t start,
                                  uint16_t* key_cache, uint16_t* value_cache, int64_t max_seq, uint16_t* q_out,
                                  void* stream) {
  if (tokens == 0) return WQ_OK;
  WQ_REQUIRE(tokens > 0 && tokens <= 0x7fffffff, WQ_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
  WQ_REQUIRE(q_heads > 0 && kv_heads > 0 && max_seq > 0 && q_heads + 2 * kv_heads <= 4 * 65535,
             WQ_ERR_INVALID_ARGUMENT, "bad head counts or max_seq");
  WQ_REQUIRE(head_dim == kHeadDim, WQ_ERR_UNSUPPORTED, "prefill q/k RoPE is built for head_dim 128 (got %lld)",
             (long long)head_dim);
  WQ_REQUIRE(start >= 0 && start + tokens <= max_seq && max_seq <= 0x7fffffff, WQ_ERR_INVALID_ARGUMENT,
             "KV cache capacity exceeded: rows %lld .. %lld of %lld", (long long)start, (long long)(start + tokens),
             (long long)max_seq);
  WQ_REQUIRE(qkv && cos_rows && sin_rows && key_cache && value_cache && q_out, WQ_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  WQ_REQUIRE(((uintptr_t)qkv | (uintptr_t)cos_rows | (uintptr_t)sin_rows | (uintptr_t)key_cache |
              (uintptr_t)value_cache | (uintptr_t)q_out | (uintptr_t)q_norm_weight | (uintptr_t)k_norm_weight) % 4 == 0,
             WQ_ERR_INVALID_ARGUMENT, "operands must be 4-byte aligned");
  hipLaunchKernelGGL(prefill_qk_rope_kernel, dim3((unsigned)tokens), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const half_t*>(qkv), (int)tokens, (int)q_heads, (int)kv_heads,
                     reinterpret_cast<const half_t*>(q_norm_weight), reinterpret_cast<const half_t*>(k_norm_weight),
                     eps, reinterpret_cast<const half_t*>(cos_rows), reinterpret_cast<const half_t*>(sin_rows),
                     (int)start, reinterpret_cast<half_t*>(key_cache), reinterpret_cast<half_t*>(value_cache),
                     (int)max_seq, reinterpret_cast<half_t*>(q_out));
  return check_launch("prefill_qk_rope");
}
