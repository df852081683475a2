// Startup repack, inverse unpack, dequant and explicit QDQ decode kernels.
//
// W4 tile layout (gfx950): one 1 KiB block per (16-row tile t, 128-k block).
// Lane l of the wavefront that streams the block owns row 16t + l%16 and k
// range 128*blk + 32*(l/16) + [0, 32) as four words; word w holds
// k0 = 128*blk + 32*(l/16) + 8w .. k0+7 with nibble p storing element
// {0,2,4,6,1,3,5,7}[p].  A block is therefore one coalesced 16 B-per-lane
// load, and each word converts to four fp16 pairs with one AND-OR apiece.
// meta holds, per (tile, group), the 16 fp16 scales of the tile's rows and
// the two zero-point words of those rows (40 bytes).
//
// INT8 tile layout: one 2 KiB block per (16-row tile, 128-k block), two
// 1 KiB pieces of 16 bytes per lane in the order the INT8 kernels take them
// (W8Layout in wq_common.h); the rows are still scaled per row by the
// caller's fp16 / fp32 scale vector.
#include "wq_common.h"
#include "wq_status.h"

namespace wq {
namespace {

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

__device__ __forceinline__ uint32_t nibble_order_from_natural(uint32_t s) {
  // tile nibble p <- source nibble {0,2,4,6,1,3,5,7}[p]
  uint32_t r = 0;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int e = (p < 4) ? 2 * p : 2 * (p - 4) + 1;
    r |= ((s >> (4 * e)) & 0xFu) << (4 * p);
  }
  return r;
}

__device__ __forceinline__ uint32_t nibble_order_to_natural(uint32_t t) {
  uint32_t r = 0;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int e = (p < 4) ? 2 * p : 2 * (p - 4) + 1;
    r |= ((t >> (4 * p)) & 0xFu) << (4 * e);
  }
  return r;
}

// One thread per (tile, block, lane): gathers 4 source words, writes 16 B.
__global__ void w4_repack_tiles_kernel(const uint32_t* __restrict__ packed, int64_t n, int64_t k,
                                       int64_t nblk, int64_t total, uint4_t* __restrict__ tiles) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  const int64_t tb = idx >> 6;           // tile * nblk + blk
  const int64_t t = tb / nblk, blk = tb - t * nblk;
  const int64_t row = t * 16 + (lane & 15);
  uint4_t out = {0u, 0u, 0u, 0u};
  if (row < n) {
    const uint4_t src = *reinterpret_cast<const uint4_t*>(packed + row * (k / 8) + blk * 16 + (lane >> 4) * 4);
    out.x = nibble_order_from_natural(src.x);
    out.y = nibble_order_from_natural(src.y);
    out.z = nibble_order_from_natural(src.z);
    out.w = nibble_order_from_natural(src.w);
  }
  tiles[idx] = out;
}

// INT8 tiles (W8Layout in wq_common.h): one thread per (tile, block, piece,
// lane) moves the lane's 16 bytes; rows past n are written as zeros.
__global__ void w8_repack_kernel(const int8_t* __restrict__ q, int64_t n, int64_t k, int64_t nblk, int64_t total,
                                 uint4_t* __restrict__ tiles) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63), piece = (int)((idx >> 6) & 1);
  const int64_t tb = idx >> 7;           // tile * nblk + blk
  const int64_t t = tb / nblk, blk = tb - t * nblk;
  const int64_t row = t * 16 + (lane & 15);
  uint4_t v = {0u, 0u, 0u, 0u};
  if (row < n)
    v = *reinterpret_cast<const uint4_t*>(q + row * k + blk * kW8BlockK + 64 * piece + 16 * (lane >> 4));
  tiles[idx] = v;
}

__global__ void w8_unpack_kernel(const uint4_t* __restrict__ tiles, int64_t n, int64_t k, int64_t nblk,
                                 int64_t total, int8_t* __restrict__ q) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63), piece = (int)((idx >> 6) & 1);
  const int64_t tb = idx >> 7;
  const int64_t t = tb / nblk, blk = tb - t * nblk;
  const int64_t row = t * 16 + (lane & 15);
  if (row < n)
    *reinterpret_cast<uint4_t*>(q + row * k + blk * kW8BlockK + 64 * piece + 16 * (lane >> 4)) = tiles[idx];
}

// One thread per (tile, group): 16 scales + 2 zero words.
__global__ void w4_repack_meta_kernel(const uint16_t* __restrict__ scale, const uint32_t* __restrict__ zero,
                                      int64_t n, int64_t ngrp, int64_t total, uint8_t* __restrict__ meta) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t t = idx / ngrp, g = idx - t * ngrp;
  uint16_t* s_out = reinterpret_cast<uint16_t*>(meta + idx * kW4MetaBytes);
  uint32_t* z_out = reinterpret_cast<uint32_t*>(meta + idx * kW4MetaBytes + 32);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = t * 16 + i;
    s_out[i] = row < n ? scale[row * ngrp + g] : (uint16_t)0;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t zrow = t * 2 + j;   // zero-point word row covers rows 8*zrow .. 8*zrow+7
    uint32_t v = 0;
    if (zrow * 8 < n) v = zero ? zero[zrow * ngrp + g] : 0x88888888u;
    z_out[j] = v;
  }
}

__global__ void w4_unpack_tiles_kernel(const uint4_t* __restrict__ tiles, int64_t n, int64_t k, int64_t nblk,
                                       int64_t total, uint32_t* __restrict__ packed) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  const int64_t tb = idx >> 6;
  const int64_t t = tb / nblk, blk = tb - t * nblk;
  const int64_t row = t * 16 + (lane & 15);
  if (row >= n) return;
  const uint4_t v = tiles[idx];
  uint4_t out;
  out.x = nibble_order_to_natural(v.x);
  out.y = nibble_order_to_natural(v.y);
  out.z = nibble_order_to_natural(v.z);
  out.w = nibble_order_to_natural(v.w);
  *reinterpret_cast<uint4_t*>(packed + row * (k / 8) + blk * 16 + (lane >> 4) * 4) = out;
}

__global__ void w4_unpack_meta_kernel(const uint8_t* __restrict__ meta, int64_t n, int64_t ngrp, int64_t total,
                                      uint16_t* __restrict__ scale, uint32_t* __restrict__ zero) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t t = idx / ngrp, g = idx - t * ngrp;
  const uint16_t* s_in = reinterpret_cast<const uint16_t*>(meta + idx * kW4MetaBytes);
  const uint32_t* z_in = reinterpret_cast<const uint32_t*>(meta + idx * kW4MetaBytes + 32);
  for (int i = 0; i < 16; ++i) {
    const int64_t row = t * 16 + i;
    if (row < n) scale[row * ngrp + g] = s_in[i];
  }
  for (int j = 0; j < 2; ++j) {
    const int64_t zrow = t * 2 + j;
    if (zrow * 8 < n) zero[zrow * ngrp + g] = z_in[j];
  }
}

// One thread per (tile, block, lane): 32 fp16 outputs through the same
// unpack helpers the linear kernels use.
__global__ void w4_dequant_tiles_kernel(const uint4_t* __restrict__ tiles, const uint8_t* __restrict__ meta,
                                        int64_t n, int64_t k, int64_t nblk, int64_t ngrp, int64_t group_size,
                                        int64_t total, half_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  const int64_t tb = idx >> 6;
  const int64_t t = tb / nblk, blk = tb - t * nblk;
  const int i = lane & 15;
  const int64_t row = t * 16 + i;
  if (row >= n) return;
  const int64_t g = blk * kW4BlockK / group_size;
  const uint8_t* mp = meta + (t * ngrp + g) * kW4MetaBytes;
  const uint16_t s_bits = reinterpret_cast<const uint16_t*>(mp)[i];
  const uint32_t zw = reinterpret_cast<const uint32_t*>(mp + 32)[i >> 3];
  uint32_t c_lo, c_hi;
  w4_zero_consts((zw >> (4 * (i & 7))) & 0xFu, c_lo, c_hi);
  const half2_t s2 = as_h2((uint32_t)s_bits * 0x00010001u);
  const uint4_t v = tiles[idx];
  half_t* dst = out + row * k + blk * kW4BlockK + (lane >> 4) * 32;
  const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int w = 0; w < 4; ++w)
    *reinterpret_cast<half8_t*>(dst + 8 * w) = w4_word_to_h8_scaled(words[w], c_lo, c_hi, s2);
}

// Explicit QDQ decode from the raw compressed-tensors tensors (any group
// size, optional g_idx): one thread per source word (8 outputs).
__global__ void w4_decode_kernel(const uint32_t* __restrict__ packed, const float* __restrict__ scale,
                                 const uint32_t* __restrict__ zero, const int32_t* __restrict__ g_idx,
                                 int64_t n, int64_t k, int64_t ngrp, int64_t group_size,
                                 uint16_t* __restrict__ out) {
  const int64_t words_per_row = k / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * words_per_row) return;
  const int64_t row = idx / words_per_row, kw = idx - row * words_per_row;
  const uint32_t word = packed[idx];
  uint16_t res[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t col = kw * 8 + e;
    // g_idx is range-checked by the host; the clamp only keeps reads in bounds.
    const int64_t g = g_idx ? min(max((int64_t)g_idx[col], (int64_t)0), ngrp - 1) : col / group_size;
    const float q = (float)((word >> (4 * e)) & 0xFu);
    const float z = zero ? (float)((zero[(row >> 3) * ngrp + g] >> (4 * (row & 7))) & 0xFu) : 8.0f;
    const half_t h = (half_t)((q - z) * scale[row * ngrp + g]);
    res[e] = __builtin_bit_cast(uint16_t, h);
  }
  uint4_t o;
  o.x = res[0] | ((uint32_t)res[1] << 16);
  o.y = res[2] | ((uint32_t)res[3] << 16);
  o.z = res[4] | ((uint32_t)res[5] << 16);
  o.w = res[6] | ((uint32_t)res[7] << 16);
  *reinterpret_cast<uint4_t*>(out + idx * 8) = o;
}

// Row-sampled explicit decode: output row r is weight row rows[r] (one thread
// per source word of a sampled row), groups of `group_size` along k.
__global__ void w4_decode_rows_kernel(const uint32_t* __restrict__ packed, const float* __restrict__ scale,
                                      const uint32_t* __restrict__ zero, const int64_t* __restrict__ rows,
                                      int64_t nrows, int64_t n, int64_t k, int64_t ngrp, int64_t group_size,
                                      uint16_t* __restrict__ out) {
  const int64_t words_per_row = k / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nrows * words_per_row) return;
  const int64_t r = idx / words_per_row, kw = idx - r * words_per_row;
  const int64_t row = min(max(rows[r], (int64_t)0), n - 1);   // range-checked by the host
  const uint32_t word = packed[row * words_per_row + kw];
  uint16_t res[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t g = (kw * 8 + e) / group_size;
    const float q = (float)((word >> (4 * e)) & 0xFu);
    const float z = zero ? (float)((zero[(row >> 3) * ngrp + g] >> (4 * (row & 7))) & 0xFu) : 8.0f;
    res[e] = __builtin_bit_cast(uint16_t, (half_t)((q - z) * scale[row * ngrp + g]));
  }
  uint4_t o;
  o.x = res[0] | ((uint32_t)res[1] << 16);
  o.y = res[2] | ((uint32_t)res[3] << 16);
  o.z = res[4] | ((uint32_t)res[5] << 16);
  o.w = res[6] | ((uint32_t)res[7] << 16);
  *reinterpret_cast<uint4_t*>(out + idx * 8) = o;
}

__global__ void w8_decode_kernel(const int8_t* __restrict__ q, const float* __restrict__ scale, int64_t n,
                                 int64_t k, uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * k) return;
  const int64_t row = idx / k;
  const half_t h = (half_t)((float)q[idx] * scale[row]);
  out[idx] = __builtin_bit_cast(uint16_t, h);
}

// One 256-thread workgroup per row.  The absmax is an exact max, so the
// result does not depend on how rows are grouped (the reference's
// row_block_size only bounds its memory).
__global__ __launch_bounds__(256) void w8_quantize_kernel(const float* __restrict__ w, int64_t k,
                                                          int8_t* __restrict__ q, uint16_t* __restrict__ scale,
                                                          int32_t* __restrict__ flags) {
  const int64_t row = blockIdx.x;
  const float* wr = w + row * k;
  float amax = 0.0f;
  bool finite = true;
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) {
    const float v = wr[c];
    finite &= __builtin_isfinite(v);
    amax = fmaxf(amax, fabsf(v));
  }
  __shared__ float red[256];
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  if (!finite) atomicOr(&bad, 1);
  red[threadIdx.x] = amax;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  __shared__ float s_fp32;
  if (threadIdx.x == 0) {
    const float absmax = red[0];
    float raw = absmax / 127.0f;
    if (absmax == 0.0f) raw = 1.0f;
    half_t stored = (half_t)raw;
    uint16_t bits = __builtin_bit_cast(uint16_t, stored);
    if (absmax != 0.0f && (bits & 0x7FFFu) == 0) bits = 0x0001u;  // smallest positive fp16
    if ((bits & 0x7C00u) == 0x7C00u) atomicOr(flags, 2);        // scale overflowed to inf
    if (bad) atomicOr(flags, 1);
    scale[row] = bits;
    s_fp32 = (float)__builtin_bit_cast(half_t, bits);
  }
  __syncthreads();
  const float s = s_fp32;
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) {
    float v = __builtin_rintf(wr[c] / s);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    q[row * k + c] = (int8_t)v;
  }
}

int launch_1d(int64_t total, int threads, int64_t& blocks) {
  blocks = ceil_div(total, threads);
  if (blocks > 0x7FFFFFFF) return WQ_ERR_UNSUPPORTED;
  return WQ_OK;
}

int w4_shape_check(int64_t n, int64_t k, int64_t g) {
  WQ_REQUIRE(n > 0 && k > 0 && g > 0, WQ_ERR_INVALID_ARGUMENT, "non-positive shape n=%lld k=%lld group=%lld",
             (long long)n, (long long)k, (long long)g);
  WQ_REQUIRE(n % 8 == 0, WQ_ERR_UNSUPPORTED, "W4 tile layout needs n %% 8 == 0 (n=%lld)", (long long)n);
  WQ_REQUIRE(g % kW4BlockK == 0 && k % g == 0, WQ_ERR_UNSUPPORTED,
             "W4 tile layout needs group_size %% 128 == 0 and k %% group_size == 0 (k=%lld group=%lld)",
             (long long)k, (long long)g);
  return WQ_OK;
}

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" int wq_w4_repack_size(int64_t n, int64_t k, int64_t group_size, size_t* tiles_bytes,
                                 size_t* meta_bytes) {
  if (int st = w4_shape_check(n, k, group_size)) return st;
  WQ_REQUIRE(tiles_bytes && meta_bytes, WQ_ERR_INVALID_ARGUMENT, "null size output");
  const int64_t ntile = ceil_div(n, 16);
  *tiles_bytes = (size_t)(ntile * 16) * (size_t)(k / 2);
  *meta_bytes = (size_t)ntile * (size_t)(k / group_size) * kW4MetaBytes;
  return WQ_OK;
}

extern "C" int wq_w4_repack(const int32_t* weight_packed, const uint16_t* weight_scale,
                            const int32_t* weight_zero_point, int64_t n, int64_t k, int64_t group_size,
                            void* tiles, void* meta, void* stream) {
  if (int st = w4_shape_check(n, k, group_size)) return st;
  WQ_REQUIRE(weight_packed && weight_scale && tiles && meta, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t ntile = ceil_div(n, 16), nblk = k / kW4BlockK, ngrp = k / group_size;
  int64_t blocks;
  const int64_t total_t = ntile * nblk * 64;
  if (launch_1d(total_t, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "repack grid too large");
  hipLaunchKernelGGL(w4_repack_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(weight_packed), n, k, nblk, total_t,
                     reinterpret_cast<uint4_t*>(tiles));
  if (int st = check_launch("w4_repack_tiles")) return st;
  const int64_t total_m = ntile * ngrp;
  launch_1d(total_m, 256, blocks);
  hipLaunchKernelGGL(w4_repack_meta_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), weight_scale,
                     reinterpret_cast<const uint32_t*>(weight_zero_point), n, ngrp, total_m,
                     reinterpret_cast<uint8_t*>(meta));
  return check_launch("w4_repack_meta");
}

extern "C" int wq_w4_unpack(const void* tiles, const void* meta, int64_t n, int64_t k, int64_t group_size,
                            int32_t* weight_packed, uint16_t* weight_scale, int32_t* weight_zero_point,
                            void* stream) {
  if (int st = w4_shape_check(n, k, group_size)) return st;
  WQ_REQUIRE(tiles && meta && weight_packed && weight_scale && weight_zero_point, WQ_ERR_INVALID_ARGUMENT,
             "null pointer argument");
  const int64_t ntile = ceil_div(n, 16), nblk = k / kW4BlockK, ngrp = k / group_size;
  int64_t blocks;
  const int64_t total_t = ntile * nblk * 64;
  if (launch_1d(total_t, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "unpack grid too large");
  hipLaunchKernelGGL(w4_unpack_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4_t*>(tiles), n, k, nblk, total_t,
                     reinterpret_cast<uint32_t*>(weight_packed));
  if (int st = check_launch("w4_unpack_tiles")) return st;
  const int64_t total_m = ntile * ngrp;
  launch_1d(total_m, 256, blocks);
  hipLaunchKernelGGL(w4_unpack_meta_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint8_t*>(meta), n, ngrp, total_m, weight_scale,
                     reinterpret_cast<uint32_t*>(weight_zero_point));
  return check_launch("w4_unpack_meta");
}

extern "C" int wq_w4_dequant(const void* tiles, const void* meta, int64_t n, int64_t k, int64_t group_size,
                             uint16_t* weight, void* stream) {
  if (int st = w4_shape_check(n, k, group_size)) return st;
  WQ_REQUIRE(tiles && meta && weight, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t ntile = ceil_div(n, 16), nblk = k / kW4BlockK, ngrp = k / group_size;
  int64_t blocks;
  const int64_t total = ntile * nblk * 64;
  if (launch_1d(total, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "dequant grid too large");
  hipLaunchKernelGGL(w4_dequant_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4_t*>(tiles), reinterpret_cast<const uint8_t*>(meta), n, k, nblk,
                     ngrp, group_size, total, reinterpret_cast<half_t*>(weight));
  return check_launch("w4_dequant_tiles");
}

extern "C" int wq_w4_decode(const int32_t* weight_packed, const float* weight_scale,
                            const int32_t* weight_zero_point, const int32_t* g_idx, int64_t n, int64_t k,
                            int64_t num_groups, int64_t group_size, uint16_t* weight, void* stream) {
  WQ_REQUIRE(n > 0 && k > 0 && num_groups > 0 && group_size > 0, WQ_ERR_INVALID_ARGUMENT,
             "non-positive shape n=%lld k=%lld groups=%lld group_size=%lld", (long long)n, (long long)k,
             (long long)num_groups, (long long)group_size);
  WQ_REQUIRE(k % 8 == 0, WQ_ERR_UNSUPPORTED, "decode needs k %% 8 == 0 (k=%lld)", (long long)k);
  WQ_REQUIRE(g_idx != nullptr || (k - 1) / group_size < num_groups, WQ_ERR_INVALID_ARGUMENT,
             "scale has %lld groups but k=%lld, group_size=%lld needs %lld", (long long)num_groups, (long long)k,
             (long long)group_size, (long long)((k - 1) / group_size + 1));
  WQ_REQUIRE(weight_packed && weight_scale && weight, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  int64_t blocks;
  if (launch_1d(n * (k / 8), 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "decode grid too large");
  hipLaunchKernelGGL(w4_decode_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(weight_packed), weight_scale,
                     reinterpret_cast<const uint32_t*>(weight_zero_point), g_idx, n, k, num_groups, group_size,
                     weight);
  return check_launch("w4_decode");
}

extern "C" int wq_w4_decode_rows(const int32_t* weight_packed, const float* weight_scale,
                                 const int32_t* weight_zero_point, const int64_t* rows, int64_t num_rows, int64_t n,
                                 int64_t k, int64_t num_groups, int64_t group_size, uint16_t* weight, void* stream) {
  WQ_REQUIRE(n > 0 && k > 0 && num_groups > 0 && group_size > 0 && num_rows >= 0, WQ_ERR_INVALID_ARGUMENT,
             "non-positive shape n=%lld k=%lld groups=%lld group_size=%lld rows=%lld", (long long)n, (long long)k,
             (long long)num_groups, (long long)group_size, (long long)num_rows);
  WQ_REQUIRE(k % 8 == 0, WQ_ERR_UNSUPPORTED, "decode needs k %% 8 == 0 (k=%lld)", (long long)k);
  WQ_REQUIRE((k - 1) / group_size < num_groups, WQ_ERR_INVALID_ARGUMENT,
             "scale has %lld groups but k=%lld, group_size=%lld needs %lld", (long long)num_groups, (long long)k,
             (long long)group_size, (long long)((k - 1) / group_size + 1));
  if (num_rows == 0) return WQ_OK;
  WQ_REQUIRE(weight_packed && weight_scale && rows && weight, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  int64_t blocks;
  if (launch_1d(num_rows * (k / 8), 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "decode grid too large");
  hipLaunchKernelGGL(w4_decode_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(weight_packed), weight_scale,
                     reinterpret_cast<const uint32_t*>(weight_zero_point), rows, num_rows, n, k, num_groups,
                     group_size, weight);
  return check_launch("w4_decode_rows");
}

extern "C" int wq_w8_tiles_size(int64_t n, int64_t k, size_t* bytes) {
  WQ_REQUIRE(n > 0 && k > 0, WQ_ERR_INVALID_ARGUMENT, "non-positive shape n=%lld k=%lld", (long long)n,
             (long long)k);
  WQ_REQUIRE(k % kW8BlockK == 0, WQ_ERR_UNSUPPORTED, "INT8 tiles need k %% 128 == 0 (k=%lld)", (long long)k);
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null size output");
  *bytes = (size_t)ceil_div(n, 16) * (size_t)(k / kW8BlockK) * kW8TileBlockBytes;
  return WQ_OK;
}

extern "C" int wq_w8_repack(const int8_t* qweight, int64_t n, int64_t k, void* tiles, void* stream) {
  size_t bytes = 0;
  if (int st = wq_w8_tiles_size(n, k, &bytes)) return st;
  WQ_REQUIRE(qweight && tiles, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(((reinterpret_cast<uintptr_t>(qweight) | reinterpret_cast<uintptr_t>(tiles)) & 15u) == 0,
             WQ_ERR_INVALID_ARGUMENT, "qweight and tiles must be 16-byte aligned");
  const int64_t total = (int64_t)(bytes / 16);
  int64_t blocks;
  if (launch_1d(total, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "repack grid too large");
  hipLaunchKernelGGL(w8_repack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), qweight, n, k,
                     k / kW8BlockK, total, reinterpret_cast<uint4_t*>(tiles));
  return check_launch("w8_repack");
}

extern "C" int wq_w8_unpack(const void* tiles, int64_t n, int64_t k, int8_t* qweight, void* stream) {
  size_t bytes = 0;
  if (int st = wq_w8_tiles_size(n, k, &bytes)) return st;
  WQ_REQUIRE(qweight && tiles, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(((reinterpret_cast<uintptr_t>(qweight) | reinterpret_cast<uintptr_t>(tiles)) & 15u) == 0,
             WQ_ERR_INVALID_ARGUMENT, "qweight and tiles must be 16-byte aligned");
  const int64_t total = (int64_t)(bytes / 16);
  int64_t blocks;
  if (launch_1d(total, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "unpack grid too large");
  hipLaunchKernelGGL(w8_unpack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4_t*>(tiles), n, k, k / kW8BlockK, total, qweight);
  return check_launch("w8_unpack");
}

extern "C" int wq_w8_decode(const int8_t* qweight, const float* scale, int64_t n, int64_t k, uint16_t* weight,
                            void* stream) {
  WQ_REQUIRE(n > 0 && k > 0, WQ_ERR_INVALID_ARGUMENT, "non-positive shape n=%lld k=%lld", (long long)n,
             (long long)k);
  WQ_REQUIRE(qweight && scale && weight, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  int64_t blocks;
  if (launch_1d(n * k, 256, blocks)) return fail(WQ_ERR_UNSUPPORTED, "decode grid too large");
  hipLaunchKernelGGL(w8_decode_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), qweight, scale, n, k,
                     weight);
  return check_launch("w8_decode");
}

extern "C" int wq_w8_quantize(const float* weight, int64_t n, int64_t k, int8_t* qweight, uint16_t* scale,
                              int32_t* status_flags, void* stream) {
  WQ_REQUIRE(n > 0 && k > 0, WQ_ERR_INVALID_ARGUMENT, "linear weight dimensions must be nonzero");
  WQ_REQUIRE(n <= 0x7FFFFFFF, WQ_ERR_UNSUPPORTED, "too many rows");
  WQ_REQUIRE(weight && qweight && scale && status_flags, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  hipLaunchKernelGGL(w8_quantize_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), weight, k, qweight,
                     scale, status_flags);
  return check_launch("w8_quantize");
}
