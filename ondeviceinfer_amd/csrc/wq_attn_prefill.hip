// Prefill (multi-token, batch 1) causal grouped-query attention over the
// resident fp16 KV cache, flash-attention style: each workgroup streams its
// query block's keys once through LDS and keeps the softmax online, so the
// [tokens x keys] score matrix never exists in memory.
//
// Layout and arithmetic (head_dim 128, 16x16x32 fp16 MFMA, fp32 accumulate):
//  * workgroup = 4 waves = 128 queries of one query head; wave w owns the 32
//    queries 32w .. 32w + 31 of the block (two 16-query tiles);
//  * per 64-key block the keys go to LDS as K [key][d] (16-byte chunk c of
//    row r at slot c ^ (r & 15)) and the values transposed as V^T [d][key
//    slot] (chunk c of row d at slot c ^ ((d >> 1) & 7)), so the 16 lanes of
//    a fragment read hit distinct banks;
//  * scores are computed transposed, S^T = K . Q^T (A = 16 keys x 32 d from
//    LDS, B = 32 d x 16 queries held in registers), so lane l holds keys
//    4(l/16) .. 4(l/16)+3 of each 16-key tile for query l % 16;
//  * P^T, rounded to fp16, is then directly the B operand of O^T = V^T . P^T
//    once V^T's key slots follow the same order: slot 8s + j holds key 4s + j
//    and slot 8s + 4 + j key 16 + 4s + j of each 32-key step;
//  * the online softmax runs in log2 units (scale * log2 e folded into the
//    scores); a query's max is reduced over its four lanes with lane swaps;
//    the denominator sums the fp32 P per lane and is reduced once at the end;
//    the accumulators are rescaled only in blocks where some query's maximum
//    moved.
// Causality is by absolute position: query t (position start + t) attends
// keys 0 .. start + t.  Keys past the block's last query position read as
// zero values, so a masked score (P = 0) never meets a NaN row.
#include "ondeviceinfer_decode.h"
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

constexpr int kPD = 128;                    // head_dim
constexpr int kPBM = 128;                   // queries per workgroup
constexpr int kPBN = 64;                    // keys per block
constexpr int kPKBytes = kPBN * kPD * 2;    // K block in LDS
constexpr int kPVBytes = kPD * kPBN * 2;    // V^T block in LDS
constexpr int kPStage = kPKBytes + kPVBytes;

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __builtin_bit_cast(float, __shfl_xor(__builtin_bit_cast(int, v), mask, 64));
}

// LDS byte offset of key slot `pos` (0..63, multiple of 4) in V^T row d.
__device__ __forceinline__ int vt_offset(int d, int pos) {
  return kPKBytes + d * (kPBN * 2) + ((((pos >> 3) ^ ((d >> 1) & 7))) << 4) + (pos & 7) * 2;
}

// grid = ceil(T / 128) * H workgroups, 256 threads.  Workgroup b: kv head
// b % KV (with 8 kv heads, one per XCD: workgroups are dealt to the 8 XCDs
// round-robin by flat id, so a kv head's keys stay in one L2), then its query
// heads and query blocks, the longest (last) query blocks first.
__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(const half_t* __restrict__ q, int T, int H, int KV,
                                                                   const half_t* __restrict__ kc,
                                                                   const half_t* __restrict__ vc, int max_seq,
                                                                   int start, float scale_log2,
                                                                   half_t* __restrict__ out, int nqb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15, s4 = lane >> 4;
  const int G = H / KV;
  const int b = blockIdx.x;
  const int kvh = b % KV, j = b / KV;
  const int qh = kvh * G + j % G;
  const int qb = nqb - 1 - j / G;
  const int q0 = qb * kPBM + 32 * wave;                          // this wave's first query
  const int last_q = min(qb * kPBM + kPBM, T) - 1;               // the workgroup's last query
  const int key_end = start + last_q + 1;                        // keys [0, key_end) matter here
  const int nkb = (key_end + kPBN - 1) / kPBN;
  const int wave_lo = start + q0;                                 // this wave's first query position
  const int wave_hi = start + min(q0 + 31, T - 1);                // ... and last (q0 < T or the wave is idle)

  // Q^T fragments (B operand): query q0 + 16qt + i (clamped; rows past T are
  // computed, never stored), d = 32ks + 8 s4 .. +7.
  half8_t qf[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int t = min(q0 + 16 * qt + i, T - 1);
    const half_t* p = q + ((size_t)t * H + qh) * kPD + 8 * s4;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[qt][ks] = ld_h8(p + 32 * ks);
  }

  // The kv head's cache rows as buffers (rows past max_seq read as zero).
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kc + (size_t)kvh * max_seq * kPD, (int64_t)max_seq * kPD * 2);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vc + (size_t)kvh * max_seq * kPD, (int64_t)max_seq * kPD * 2);
  // Block loads: K rows r = (tid + 256 u) / 16, 16-byte chunk (tid % 16);
  // V keys 4 (tid % 16) .. +3, d chunk tid / 16 (so that the 16 lanes of a
  // transposed V^T write cover one whole 128-byte row, not 16 rows).
  uint4_t kr[4], vr[4];
  const uint32_t ko = (uint32_t)((tid >> 4) * 256 + (tid & 15) * 16);        // + 16 rows per u
  const uint32_t vo = (uint32_t)(4 * (tid & 15) * 256 + (tid >> 4) * 16);   // + 1 row per e
  auto load_block = [&](int kb) {
    const uint32_t so = (uint32_t)kb * kPBN * 256;
#pragma unroll
    for (int u = 0; u < 4; ++u) kr[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 4096 * u, so, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) vr[e] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo + 256 * e, so, 0);
  };
  // The stores zero the values of keys past key_end (not in load_block, so
  // that the loads stay in flight during the block's math; only the last
  // block has such keys).
  auto store_block = [&](int st, int kb) {
    if (kb * kPBN + kPBN > key_end) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (kb * kPBN + 4 * (tid & 15) + e >= key_end) vr[e] = uint4_t{0u, 0u, 0u, 0u};
    }
    uint8_t* base = smem + st * kPStage;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u, r = c >> 4, cc = c & 15;
      *reinterpret_cast<uint4_t*>(base + r * 256 + ((cc ^ (r & 15)) << 4)) = kr[u];
    }
    // Keys 4g .. 4g+3 (g = tid % 16) land in slots pos .. pos+3 of each of
    // the chunk's 8 V^T rows.
    const int g = tid & 15, kk = (4 * g) & 31;
    const int pos = 32 * (g >> 3) + 8 * ((kk & 15) >> 2) + (kk >= 16 ? 4 : 0);
    const int d0 = 8 * (tid >> 4);
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const int w = dd >> 1, hi = dd & 1;
      half4_t h4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // Through a scalar: a bit_cast of an ext-vector component reads
        // component 0 in this hipcc.
        const uint32_t word = vr[e][w];
        h4[e] = __builtin_bit_cast(half2_t, word)[hi];
      }
      *reinterpret_cast<half4_t*>(base + vt_offset(d0 + dd, pos)) = h4;
    }
  };

  float4_t acc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) acc[dt][qt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};

  load_block(0);
  // Q and block 0 land here: the Q fragments must not be left in flight
  // into the loop, where every iteration's wait would then also cover the
  // next block's loads (the empty asm pins the Q loads above this point).
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" : "+v"(qf[qt][ks]));
  __builtin_amdgcn_s_waitcnt(0);
  store_block(0, 0);
  __syncthreads();

  float l_run[2] = {0.f, 0.f};   // this lane's part of each query's denominator

  // One 64-key block of this wave's 32 queries; `masked`: some keys of the
  // block lie past some of the wave's query positions (wave-uniform).
  auto step = [&](const uint8_t* base, int k0, bool masked) {
    // S^T = K . Q^T for the block's four 16-key tiles.
    float4_t sc[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      sc[kt][0] = sc[kt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
      const int r = 16 * kt + i;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int cc = 4 * ks + s4;
        const half8_t a = *reinterpret_cast<const half8_t*>(base + r * 256 + ((cc ^ (r & 15)) << 4));
        sc[kt][0] = mfma16(a, qf[0][ks], sc[kt][0]);
        sc[kt][1] = mfma16(a, qf[1][ks], sc[kt][1]);
      }
    }
    if (masked) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (k0 + 16 * kt + 4 * s4 + v > start + q0 + 16 * qt + i) sc[kt][qt][v] = -INFINITY;
    }
    half8_t pb[2][2];
    float alpha[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float mb = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) mb = fmaxf(mb, sc[kt][qt][v]);
      mb = fmaxf(mb, shfl_xor_f(mb, 16));
      mb = fmaxf(mb, shfl_xor_f(mb, 32));
      // scale_log2 > 0, so the scaled maximum is the maximum of the scaled scores.
      const float m_new = fmaxf(m_run[qt], mb * scale_log2);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      alpha[qt] = exp2_hw(m_run[qt] - m_use);   // 0 on the first block with a key
      m_run[qt] = m_new;
      half_t ph[4][4];
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float p = exp2_hw(__builtin_fmaf(sc[kt][qt][v], scale_log2, -m_use));
          ls += p;
          ph[kt][v] = (half_t)p;
        }
      l_run[qt] = l_run[qt] * alpha[qt] + ls;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv)
        pb[qt][kv] = half8_t{ph[2 * kv][0], ph[2 * kv][1], ph[2 * kv][2], ph[2 * kv][3],
                             ph[2 * kv + 1][0], ph[2 * kv + 1][1], ph[2 * kv + 1][2], ph[2 * kv + 1][3]};
    }
    // Rescale only when some query's maximum moved (wave-uniform test).
    if (__builtin_amdgcn_ballot_w64(alpha[0] != 1.f || alpha[1] != 1.f) != 0) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt][qt] *= alpha[qt];
    }
    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = 16 * dt + i;
#pragma unroll
      for (int kv = 0; kv < 2; ++kv) {
        const int ch = 4 * kv + s4;
        const half8_t a =
            *reinterpret_cast<const half8_t*>(base + kPKBytes + d * (kPBN * 2) + ((ch ^ ((d >> 1) & 7)) << 4));
        acc[dt][0] = mfma16(a, pb[0][kv], acc[dt][0]);
        acc[dt][1] = mfma16(a, pb[1][kv], acc[dt][1]);
      }
    }
  };

  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) load_block(kb + 1);
    const int k0 = kb * kPBN;
    if (q0 < T && k0 <= wave_hi) {
      const uint8_t* base = smem + st * kPStage;
      step(base, k0, k0 + kPBN - 1 > wave_lo);
    }
    if (more) store_block(st ^ 1, kb + 1);   // that stage was last read before the previous barrier
    __syncthreads();
  }

  // out[t][qh][d] = O / l; lane (i, s4) holds d = 16 dt + 4 s4 .. +3 of query 16 qt + i.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float l = l_run[qt];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const float inv = 1.0f / l;
    const int t = q0 + 16 * qt + i;
    if (t < T) {
      half_t* o = out + ((size_t)t * H + qh) * kPD + 4 * s4;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        half4_t h;
#pragma unroll
        for (int v = 0; v < 4; ++v) h[v] = (half_t)(acc[dt][qt][v] * inv);
        *reinterpret_cast<half4_t*>(o + 16 * dt) = h;
      }
    }
  }
}

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_prefill_attention(const uint16_t* q, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                    int64_t head_dim, const uint16_t* key_cache, const uint16_t* value_cache,
                                    int64_t max_seq, int64_t start, float scale, uint16_t* out, void* stream) {
  if (tokens == 0) return WQ_OK;
  WQ_REQUIRE(tokens > 0 && tokens <= 0x7fffffff, WQ_ERR_INVALID_ARGUMENT, "tokens must be >= 0");
  WQ_REQUIRE(head_dim == kPD, WQ_ERR_UNSUPPORTED, "prefill attention is built for head_dim 128 (got %lld)",
             (long long)head_dim);
  WQ_REQUIRE(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0, WQ_ERR_INVALID_ARGUMENT,
             "q_heads (%lld) must be a positive multiple of kv_heads (%lld)", (long long)q_heads, (long long)kv_heads);
  WQ_REQUIRE(start >= 0 && start + tokens <= max_seq && max_seq <= 0x7fffffff, WQ_ERR_INVALID_ARGUMENT,
             "KV cache rows %lld .. %lld exceed its %lld rows", (long long)start, (long long)(start + tokens),
             (long long)max_seq);
  const int64_t nqb = (tokens + kPBM - 1) / kPBM;
  WQ_REQUIRE(nqb * q_heads <= 0x7fffffff, WQ_ERR_UNSUPPORTED, "too many query blocks");
  WQ_REQUIRE(q && key_cache && value_cache && out, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(((uintptr_t)q | (uintptr_t)key_cache | (uintptr_t)value_cache | (uintptr_t)out) % 16 == 0,
             WQ_ERR_INVALID_ARGUMENT, "q, the caches and out must be 16-byte aligned");
  hipLaunchKernelGGL(prefill_attention_kernel, dim3((unsigned)(nqb * q_heads)), dim3(256), 2 * kPStage,
                     as_stream(stream), reinterpret_cast<const half_t*>(q), (int)tokens, (int)q_heads,
                     (int)kv_heads, reinterpret_cast<const half_t*>(key_cache),
                     reinterpret_cast<const half_t*>(value_cache), (int)max_seq, (int)start, scale * kLog2e,
                     reinterpret_cast<half_t*>(out), (int)nqb);
  return check_launch("prefill_attention");
}
