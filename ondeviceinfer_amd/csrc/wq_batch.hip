// Small-batch W4A16 linear (12 <= M <= 32) for N up to 1152 tiles (18432 rows):
// the activation slice is staged once per workgroup in LDS and shared by its
// eight waves, which own eight different 16-row tiles.
//
// The skinny kernels give every wave its own copy of the activation
// fragments in registers, so at M = 17..32 a wave moves 8 KiB of x (from L2)
// for every 1 KiB block of weights and can keep only two blocks in flight.
// Here workgroup (g, s) owns the tile group g (8 tiles, one per wave) over
// the k range [s*R, (s+1)*R) of 128-k blocks:
//  * the x slice x[0:16*MC, s*R*128 : (s+1)*R*128] is copied buffer -> LDS
//    (buffer_load_dwordx4 ... lds, rows past M read as zero), one stage of
//    16*MC rows x 256 B per block, 16-byte chunk c of row r at slot
//    c ^ (r & 15), so the sixteen rows of a B-fragment read hit sixteen
//    different bank groups;
//  * every wave requests its scale / zero records (one 8-byte load per
//    lane) and all R of its weight blocks at once, behind the x copy: the
//    whole k range is in flight before the first block is used;
//  * per block the wave runs the skinny kernels' arithmetic: the exact fp16
//    (q - z) against x on MFMA 16x16x32, then the group scale times the
//    block sum added into an fp32 accumulator.
// With S > 1 splits the S workgroups of a tile group meet through the
// workspace: each publishes its fp32 partials with device-coherent stores,
// counts in with a device-scope atomic, and the last to arrive adds the S
// partials in split order (independent of arrival order) and stores y.  The
// counters sit in the workspace's fixed counter region (kSplitCounterBytes).
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

constexpr int kBatchWaves = 8;                         // waves (tiles) per workgroup
// Up to the gate / up projections (1088 tiles).  The fused gate_up (2176
// tiles) keeps the skinny ring (M <= 16) and the deep-ring GEMM (M > 16):
// there this kernel's 1088 workgroups at M = 32 took 46 us against 37.
constexpr int kBatchMaxTiles = 1152;
constexpr int kBatchMaxGroups = kBatchMaxTiles / kBatchWaves;
constexpr size_t kBatchCounterBytes = kSplitCounterBytes;
static_assert(kBatchMaxGroups <= kSplitMaxCounters, "one counter per tile group");
// Below 12 rows the skinny kernels stay ahead: the k split's publish, count
// and sum steps cost about 3 us per launch, more than the shared x saves
// there (MI355X, fused QKV 5120->7168: M = 8 9.9 against 9.1 us; M = 16
// 9.8 against 11.6; M = 32 12.4 against 15.0).
constexpr int kBatchMinM = 12;

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS 16-byte read at a byte address, invisible to the compiler's wait
// insertion (see lds_read16_asm); completed by an explicit lgkmcnt wait.
__device__ __forceinline__ uint4_t lds_rd(uint32_t a) {
  uint4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
  return v;
}

// grid = (tile groups, S); block = 512 threads.  nblk == S * R.
template <int MC, int R>
__global__ __launch_bounds__(64 * kBatchWaves) void w4_batch_kernel(const half_t* __restrict__ x, int M, int K,
                                                                    const uint8_t* __restrict__ tiles,
                                                                    const uint8_t* __restrict__ meta, int N, int bpg,
                                                                    half_t* __restrict__ y, float4_t* ws_part,
                                                                    uint32_t* ws_cnt) {
  constexpr int W = kBatchWaves;
  constexpr int ROWS = 16 * MC;
  constexpr int kStageBytes = ROWS * 256;
  constexpr int kRowInstr = ROWS / 4;                 // 1 KiB copies (4 rows each) per stage
  constexpr int kXInstr = R * kRowInstr;
  static_assert(kXInstr % W == 0, "x copies split evenly over the waves");
  constexpr int kXPerWave = kXInstr / W;
  constexpr int kLoads = kXPerWave + 1 + R;           // per wave: x copies, the records, R weight blocks
  static_assert(R * kW4MetaBytes <= 512, "one 8-byte record load per lane covers the wave's groups");
  static_assert(kLoads <= 63, "loads in flight per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t xs[R * kStageBytes];
  __shared__ uint32_t arrival;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, kb = lane >> 4;
  const int ntile = (N + 15) >> 4;
  const int nblk = K / kW4BlockK, ngrp = nblk / bpg;
  const int group = blockIdx.x, split = blockIdx.y, S = gridDim.y;
  const int blk0 = split * R;
  const int tile = group * W + wave;
  const bool live = tile < ntile;

  // 1) x slice -> LDS.  Copy J fills rows 4*(J % kRowInstr) .. +3 of stage
  //    J / kRowInstr; lane L lands in row 4*(J % kRowInstr) + L/16, slot L%16,
  //    so it fetches chunk (L%16) ^ (row & 15) of that row.
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (int64_t)M * K * 2);
#pragma unroll
  for (int j = 0; j < kXPerWave; ++j) {
    const int J = wave * kXPerWave + j;
    const int st = J / kRowInstr, rr = 4 * (J % kRowInstr) + (lane >> 4);
    const uint32_t voff = (uint32_t)(rr * K * 2 + ((lane & 15) ^ (rr & 15)) * 16);
    lds_load16(rx, voff, (uint32_t)((blk0 + st) * kW4BlockK * 2), xs + st * kStageBytes + (J % kRowInstr) * 1024);
  }
  __builtin_amdgcn_sched_barrier(0);   // the copies stay the oldest loads (the wait below counts on it)

  // 2) this wave's records, then its weight blocks, all in flight at once.
  //    A tile past N reads zeros (empty range) and is never stored.
  const __amdgpu_buffer_rsrc_t rw =
      buf_rsrc(tiles + ((size_t)(live ? tile : 0) * nblk + blk0) * 1024, live ? (int64_t)R * 1024 : 0);
  const __amdgpu_buffer_rsrc_t rm =
      buf_rsrc(meta + (size_t)(live ? tile : 0) * ngrp * kW4MetaBytes, live ? (int64_t)ngrp * kW4MetaBytes : 0);
  // The records of the wave's groups are contiguous (40 B each, at most
  // R of them): one 8-byte load per lane covers 512 B, and each block's
  // scale pair and zero word are then fetched from the owning lanes with
  // ds_bpermute (no LDS memory access) instead of two loads per block.
  const int g_lo = blk0 / bpg;
  const uint2_t mrec = __builtin_bit_cast(
      uint2_t, __builtin_amdgcn_raw_buffer_load_b64(rm, (uint32_t)lane * 8, (uint32_t)(g_lo * kW4MetaBytes), 0));
  __builtin_amdgcn_sched_barrier(0);
  uint4_t wv[R];
#pragma unroll
  for (int b = 0; b < R; ++b)
    wv[b] = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)lane * 16, (uint32_t)b * 1024, kNtPolicy);
  __builtin_amdgcn_sched_barrier(0);

  // 3) every wave's x copies have landed (they are its oldest loads), then
  //    the workgroup's: a barrier without a fence, which would wait for the
  //    weight loads as well.
  wait_vm<kLoads - kXPerWave>();
  __builtin_amdgcn_s_barrier();

  // Each block's scale pair and zero word from the lanes holding them.
  // Record gb = group - g_lo: the scales of rows 4kb.. at byte 40gb + 8kb
  // (lane 5gb + kb, both words), zero word (i >> 3) at byte
  // 40gb + 32 + 4(i >> 3) (lane 5gb + 4, word i >> 3).
  uint2_t scb[R];
  uint32_t zwb[R];
#pragma unroll
  for (int b = 0; b < R; ++b) {
    const int gb = (blk0 + b) / bpg - g_lo;
    const int src_s = (5 * gb + kb) * 4, src_z = (5 * gb + 4) * 4;
    scb[b].x = (uint32_t)__builtin_amdgcn_ds_bpermute(src_s, (int)mrec.x);
    scb[b].y = (uint32_t)__builtin_amdgcn_ds_bpermute(src_s, (int)mrec.y);
    const uint32_t z_lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src_z, (int)mrec.x);
    const uint32_t z_hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src_z, (int)mrec.y);
    zwb[b] = (i >> 3) ? z_hi : z_lo;
  }
  __builtin_amdgcn_sched_barrier(0);   // all of them before the block loop's own LDS reads

  float4_t acc[MC];
#pragma unroll
  for (int mc = 0; mc < MC; ++mc) acc[mc] = float4_t{0.f, 0.f, 0.f, 0.f};
  const uint32_t xs_base = (uint32_t)(size_t)((const __attribute__((address_space(3))) uint8_t*)xs);
  // B fragments of block b: row mc*16 + i, chunk 4kb + w at slot (4kb + w) ^ i.
  // Block b + 1's are read while block b computes (LDS reads return in order).
  uint4_t xf[2][MC][4];
  auto read_frags = [&](int b, uint4_t (&f)[MC][4]) {
#pragma unroll
    for (int mc = 0; mc < MC; ++mc)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        f[mc][w] = lds_rd(xs_base + (uint32_t)(b * kStageBytes + (mc * 16 + i) * 256 + (((4 * kb + w) ^ i) * 16)));
  };
  read_frags(0, xf[0]);
#pragma unroll
  for (int b = 0; b < R; ++b) {
    uint4_t (&cur)[MC][4] = xf[b & 1];
    if (b + 1 < R) read_frags(b + 1, xf[(b + 1) & 1]);
    uint32_t c_lo, c_hi;
    w4_zero_consts((zwb[b] >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
    const uint32_t words[4] = {wv[b].x, wv[b].y, wv[b].z, wv[b].w};
    half8_t a[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) a[w] = w4_word_to_h8(words[w], c_lo, c_hi);
    // This block's reads are done once at most the next block's 4*MC remain.
    if constexpr (MC == 1) {
      if (b + 1 < R)
        asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(cur[0][0]), "+v"(cur[0][1]), "+v"(cur[0][2]), "+v"(cur[0][3]));
      else
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0][0]), "+v"(cur[0][1]), "+v"(cur[0][2]), "+v"(cur[0][3]));
    } else {
      if (b + 1 < R)
        asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(cur[0][0]), "+v"(cur[0][1]), "+v"(cur[0][2]), "+v"(cur[0][3]),
                     "+v"(cur[1][0]), "+v"(cur[1][1]), "+v"(cur[1][2]), "+v"(cur[1][3]));
      else
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0][0]), "+v"(cur[0][1]), "+v"(cur[0][2]), "+v"(cur[0][3]),
                     "+v"(cur[1][0]), "+v"(cur[1][1]), "+v"(cur[1][2]), "+v"(cur[1][3]));
    }
    const half4_t s4 = __builtin_bit_cast(half4_t, scb[b]);
#pragma unroll
    for (int mc = 0; mc < MC; ++mc) {
      float4_t cg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; ++w) cg = mfma16(a[w], __builtin_bit_cast(half8_t, cur[mc][w]), cg);
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[mc][v] += (float)s4[v] * cg[v];
    }
    // Keep each block's work in its own step: hoisting a later block's
    // unpack here would wait for that block's weights (vmcnt counts in
    // issue order) and serialize the stream.
    __builtin_amdgcn_sched_barrier(0);
  }

  // 4) Lane (i, kb) holds y[m = mc*16 + i][n = 16*tile + 4kb + v].
  const int n0 = tile * 16 + 4 * kb;
  auto store = [&](int mc, float4_t s) {
    const int m = mc * 16 + i;
    if (live && m < M && n0 < N) {
      half4_t o;
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = (half_t)s[v];
      *reinterpret_cast<half4_t*>(y + (size_t)m * N + n0) = o;
    }
  };
  if (S == 1) {
#pragma unroll
    for (int mc = 0; mc < MC; ++mc) store(mc, acc[mc]);
    return;
  }
  // Partial (group, split, wave, mc) at 1 KiB granules, lane l at +16l.
  auto part_off = [&](int s2, int mc) {
    return (uint32_t)(((((size_t)group * S + s2) * W + wave) * MC + mc) * 1024 + lane * 16);
  };
#pragma unroll
  for (int mc = 0; mc < MC; ++mc) coherent_store16(ws_part, part_off(split, mc), __builtin_bit_cast(uint4_t, acc[mc]));
  __builtin_amdgcn_s_waitcnt(0);   // this wave's partials are acknowledged
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();    // ... and every wave's
  if (threadIdx.x == 0)
    arrival = __hip_atomic_fetch_add(&ws_cnt[group], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrival != (uint32_t)(S - 1)) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // Last to arrive: the S partials in split order (this workgroup's own from
  // its registers), then the counter back to zero for the next call.
#pragma unroll
  for (int mc = 0; mc < MC; ++mc) {
    float4_t s = split == 0 ? acc[mc] : __builtin_bit_cast(float4_t, coherent_load16(ws_part, part_off(0, mc)));
    for (int s2 = 1; s2 < S; ++s2)
      s += s2 == split ? acc[mc] : __builtin_bit_cast(float4_t, coherent_load16(ws_part, part_off(s2, mc)));
    store(mc, s);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&ws_cnt[group], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct BatchPlan {
  int mc, r, s, groups;
};

// The plan for (M, N, K) or r == 0 when this kernel does not take the shape:
// the longest k range R (fewest partials) with at most 16 splits.  The
// narrow shapes then run one eight-wave workgroup per compute unit (fused
// QKV 224 workgroups, q/o 160); the gate and up projections (1088 tiles)
// run 544 workgroups in about two rounds, still ahead of the skinny ring
// (MI355X, 5120->17408: M = 16 25.2 -> 17.9-20.0 us, M = 32 31.8 -> 27.1 us).
BatchPlan batch_plan(int64_t M, int64_t N, int64_t K, int64_t G) {
  BatchPlan p{(int)((M + 15) / 16), 0, 0, 0};
  const int64_t ntile = (N + 15) / 16, nblk = K / kW4BlockK;
  if (M < kBatchMinM || M > 32 || ntile > kBatchMaxTiles || K % kW4BlockK != 0 || G % kW4BlockK != 0 || K % G != 0)
    return p;
  if (K > (1 << 24)) return p;   // the x copy's 32-bit lane offsets (31 rows of 2K bytes)
  p.groups = (int)((ntile + kBatchWaves - 1) / kBatchWaves);
  for (int r : {10, 8, 5, 4}) {
    if (nblk % r != 0) continue;
    const int s = (int)(nblk / r);
    if (s > 16) continue;
    if ((r * p.mc * 4) % kBatchWaves != 0) continue;
    if (s > 1 && kBatchCounterBytes + (size_t)p.groups * s * kBatchWaves * p.mc * 1024 > kSplitWorkspaceMaxBytes)
      continue;
    p.r = r;
    p.s = s;
    return p;
  }
  p.r = 0;
  return p;
}

size_t batch_ws_bytes(const BatchPlan& p) {
  if (p.r == 0 || p.s <= 1) return 0;
  return kBatchCounterBytes + (size_t)p.groups * p.s * kBatchWaves * p.mc * 1024;
}

template <int MC, int R>
int launch_batch(const half_t* x, int M, int K, const uint8_t* tiles, const uint8_t* meta, int N, int bpg, half_t* y,
                 const BatchPlan& p, void* ws, hipStream_t st) {
  float4_t* part = p.s > 1 ? reinterpret_cast<float4_t*>(reinterpret_cast<uint8_t*>(ws) + kBatchCounterBytes) : nullptr;
  hipLaunchKernelGGL((w4_batch_kernel<MC, R>), dim3((unsigned)p.groups, (unsigned)p.s), dim3(64 * kBatchWaves), 0,
                     st, x, M, K, tiles, meta, N, bpg, y, part, reinterpret_cast<uint32_t*>(ws));
  return check_launch("w4_batch");
}

}  // namespace

size_t w4_batch_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t g) {
  return batch_ws_bytes(batch_plan(m, n, k, g));
}

// Returns -1 (not taken) when the shape has no plan or the workspace is
// smaller than the plan needs; the caller then runs the skinny kernels.
int launch_w4_batch(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G, half_t* y,
                    void* ws, size_t ws_bytes, hipStream_t st) {
  const BatchPlan p = batch_plan(M, N, K, G);
  if (p.r == 0) return -1;
  const size_t need = batch_ws_bytes(p);
  if (need > 0 && (ws == nullptr || ws_bytes < need)) return -1;
  const uint8_t* t8 = reinterpret_cast<const uint8_t*>(tiles);
  const int bpg = G / kW4BlockK;
  switch (p.mc * 100 + p.r) {
    case 110: return launch_batch<1, 10>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 108: return launch_batch<1, 8>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 104: return launch_batch<1, 4>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 210: return launch_batch<2, 10>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 208: return launch_batch<2, 8>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 205: return launch_batch<2, 5>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    case 204: return launch_batch<2, 4>(x, M, K, t8, meta, N, bpg, y, p, ws, st);
    default: return -1;
  }
}

}  // namespace wq
