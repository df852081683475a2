// Prefill (multi-token, batch 1) causal grouped-query attention over the
// resident fp16 KV cache, flash-attention style: each workgroup streams its
// query block's keys once through LDS and keeps the softmax online, so the
// [tokens x keys] score matrix never exists in memory.
//
// Layout and arithmetic (head_dim 128, 32x32x16 fp16 MFMA, fp32 accumulate):
//  * workgroup = 4 waves = 128 queries of one query head; wave w owns the 32
//    queries 32w .. 32w + 31 of the block (one 32-query tile);
//  * per 64-key block the keys go to LDS as K [key][d] (16-byte chunk c of
//    row r at slot c ^ (r & 15)) and the values transposed as V^T [d][key
//    slot] (chunk c of row d at slot c ^ ((d >> 1) & 7)), so the 16 lanes of
//    a fragment read hit distinct banks;
//  * scores are computed transposed, S^T = K . Q^T (A = 32 keys x 16 d from
//    LDS, B = 16 d x 32 queries held in registers): lane l = (q, h) =
//    (l % 32, l / 32) holds, in register r, key 8(r/4) + 4h + r%4 of each
//    32-key tile for query q;
//  * P^T, rounded to fp16, is then directly the B operand of O^T = V^T . P^T
//    (registers 8s .. 8s+7 for 16-key step s of a tile) once V^T's key slots
//    follow the same order: slot 8h + 4j + e of a 16-key step holds key
//    8j + 4h + e;
//  * the online softmax runs in log2 units (scale * log2 e folded into the
//    scores); a query's max is reduced over its two lanes with one lane swap;
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

typedef float float16_t __attribute__((ext_vector_type(16)));

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
  const int ql = lane & 31, hh = lane >> 5;   // this lane's query within the wave's tile, and lane half
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
  const int qpos = start + q0 + ql;                               // this lane's query position

  // Q^T fragments (B operand): query q0 + ql (clamped; rows past T are
  // computed, never stored), d = 16ks + 8hh .. +7.
  half8_t qf[8];
  {
    const int t = min(q0 + ql, T - 1);
    const half_t* p = q + ((size_t)t * H + qh) * kPD + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = ld_h8(p + 16 * ks);
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
    // the chunk's 8 V^T rows: within 16-key step g / 4, key 8jj + 4h + e
    // sits at slot 8h + 4jj + e.
    const int g = tid & 15, kk = (4 * g) & 15;
    const int pos = 16 * (g >> 2) + 8 * ((kk & 7) >> 2) + 4 * (kk >> 3);
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

  float16_t acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;   // this lane's part of its query's denominator

  load_block(0);
  // Q and block 0 land here: the Q fragments must not be left in flight
  // into the loop, where every iteration's wait would then also cover the
  // next block's loads (the empty asm pins the Q loads above this point).
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) asm volatile("" : "+v"(qf[ks]));
  __builtin_amdgcn_s_waitcnt(0);
  store_block(0, 0);
  __syncthreads();

  // One 64-key block of this wave's 32 queries; `masked`: some keys of the
  // block lie past some of the wave's query positions (wave-uniform).
  auto step = [&](const uint8_t* base, int k0, bool masked) {
    // S^T = K . Q^T for the block's two 32-key tiles.
    float16_t sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[kt][r] = 0.f;
      const int row = 32 * kt + ql;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const int cc = 2 * ks + hh;
        const half8_t a = *reinterpret_cast<const half8_t*>(base + row * 256 + ((cc ^ (row & 15)) << 4));
        sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], sc[kt], 0, 0, 0);
      }
    }
    if (masked) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + 32 * kt + 8 * (r >> 2) + 4 * hh + (r & 3) > qpos) sc[kt][r] = -INFINITY;
    }
    float mb = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mb = fmaxf(mb, sc[kt][r]);
    mb = fmaxf(mb, shfl_xor_f(mb, 32));
    // scale_log2 > 0, so the scaled maximum is the maximum of the scaled scores.
    const float m_new = fmaxf(m_run, mb * scale_log2);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_hw(m_run - m_use);   // 0 on the first block with a key
    m_run = m_new;
    half8_t pb[2][2];
    float ls = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        half8_t h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pv = exp2_hw(__builtin_fmaf(sc[kt][8 * st + e], scale_log2, -m_use));
          ls += pv;
          h[e] = (half_t)pv;
        }
        pb[kt][st] = h;
      }
    l_run = l_run * alpha + ls;
    // Rescale only when some query's maximum moved (wave-uniform test).
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }
    // O^T += V^T . P^T over the block's four 16-key steps.
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = 32 * dt + ql;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int ch = 2 * (2 * kt + st) + hh;
          const half8_t a =
              *reinterpret_cast<const half8_t*>(base + kPKBytes + d * (kPBN * 2) + ((ch ^ ((d >> 1) & 7)) << 4));
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[kt][st], acc[dt], 0, 0, 0);
        }
    }
  };

  for (int kb = 0; kb < nkb; ++kb) {
    const int st = kb & 1;
    const bool more = kb + 1 < nkb;
    if (more) load_block(kb + 1);
    const int k0 = kb * kPBN;
    if (q0 < T && k0 <= wave_hi) step(smem + st * kPStage, k0, k0 + kPBN - 1 > wave_lo);
    if (more) store_block(st ^ 1, kb + 1);   // that stage was last read before the previous barrier
    __syncthreads();
  }

  // out[t][qh][d] = O / l; lane (ql, hh) holds d = 32 dt + 8 (r/4) + 4 hh + r%4 of query ql.
  const float l = l_run + shfl_xor_f(l_run, 32);
  const float inv = 1.0f / l;
  const int t = q0 + ql;
  if (t < T) {
    half_t* o = out + ((size_t)t * H + qh) * kPD + 4 * hh;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        half4_t hv;
#pragma unroll
        for (int e = 0; e < 4; ++e) hv[e] = (half_t)(acc[dt][4 * jj + e] * inv);
        *reinterpret_cast<half4_t*>(o + 32 * dt + 8 * jj) = hv;
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
  // One kv head's cache rows are read through a buffer of at most 2^31 - 1 bytes.
  WQ_REQUIRE(max_seq * kPD * 2 <= 0x7fffffff, WQ_ERR_UNSUPPORTED,
             "prefill attention reads at most %lld cache rows per kv head (max_seq %lld)",
             (long long)(0x7fffffff / (kPD * 2)), (long long)max_seq);
  // The online softmax takes the block maximum of the raw scores as the
  // maximum of the scaled ones, which needs a positive scale.
  WQ_REQUIRE(scale > 0.f && scale < INFINITY, WQ_ERR_INVALID_ARGUMENT, "scale must be positive and finite (got %g)",
             (double)scale);
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
