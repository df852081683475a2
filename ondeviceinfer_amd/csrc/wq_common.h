// Shared device helpers for the gfx950 weight-only quantized Linear.
//
// Conventions used by every kernel in this directory:
//  * fp16 tensors cross the C ABI as uint16_t bit patterns; inside kernels
//    they are _Float16 vectors.
//  * MFMA v_mfma_f32_16x16x32_f16 is used with the *weights* as the A operand
//    (16 output rows n) and the activations as the B operand (16 columns m),
//    so the accumulator lane l holds D[n = 4*(l/16) + v][m = l%16], v = 0..3.
//    Lane l supplies A row l%16 and B column l%16, each with 8 consecutive k
//    taken from k-slot l/16; A and B use the same (lane, register) -> k map,
//    which is all the dot product needs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace wq {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

constexpr int kW4BlockK = 128;     // k extent of one W4 tile block (one 1 KiB wave load)
constexpr int kW4MetaBytes = 40;   // per (16-row tile, group): 16 fp16 scales + 2 zero words
constexpr int kW8BlockK = 128;     // k extent of one INT8 wave block (2 x 16 B per lane)
constexpr int kW8TileBlockBytes = 16 * kW8BlockK;   // one (16-row tile, 128-k block) of INT8 tiles

// INT8 weight addressing, shared by the W8A16 and W8A8 kernels.  For 16-row
// tile t and 128-k block b, lane l = (i, kb) = (l % 16, l / 16) of a wave
// takes piece 0 = bytes k = 128b + 16kb .. +15 and piece 1 = bytes
// k = 128b + 64 + 16kb .. +15 of row 16t + i.
//  * row-major q [N, K]: the lane's base is row * K + 16kb (rows clamped to
//    N - 1, never stored), a block is 128 bytes on, piece 1 64 bytes on;
//  * tiles (wq_w8_repack): 2 KiB per (tile, block), piece p at +1024p and
//    lane l at +16l, so that each piece is one contiguous 1 KiB wave load;
//    the lane's base is t * nblk * 2048 + 16l, a block 2048 bytes on,
//    piece 1 1024 bytes on (rows past N are zero in the tiles).
struct W8Layout {
  int tiled;
  __device__ __forceinline__ int block_bytes() const { return tiled ? kW8TileBlockBytes : kW8BlockK; }
  __device__ __forceinline__ int piece1() const { return tiled ? kW8TileBlockBytes / 2 : 64; }
  __device__ __forceinline__ size_t lane_base(int tile, int lane, int N, int K) const {
    if (tiled) return (size_t)tile * (K / kW8BlockK) * kW8TileBlockBytes + 16 * lane;
    const int row = (tile * 16 + (lane & 15)) < N ? tile * 16 + (lane & 15) : N - 1;
    return (size_t)row * K + 16 * (lane >> 4);
  }
};
// Word 3 of a gfx9 buffer resource: 32-bit data format, so raw dword loads
// are range-checked against num_records and return 0 past it.  On gfx950 the
// check covers the SGPR offset (soffset) as well as the VGPR offset, so a
// tile or row offset passed in soffset past the end also reads zero.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Cache policy of a buffer access that is coherent across the XCDs' L2s
// (sc1): the bits the compiler gives device-scope relaxed atomic loads and
// stores on gfx950, here on 16-byte accesses.
constexpr int kCoherentPolicy = 16;

// 16-byte store / load at base + byte_off that other workgroups on any XCD
// observe once the storing wave has waited for its stores (vmcnt) and
// published that with a device-scope atomic.
__device__ __forceinline__ void coherent_store16(void* base, uint32_t byte_off, uint4_t v) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, kBufferRsrcWord3);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, kCoherentPolicy);
}
__device__ __forceinline__ uint4_t coherent_load16(const void* base, uint32_t byte_off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, kBufferRsrcWord3);
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCoherentPolicy);
}

// Buffer over [base, base + bytes) (bytes clamped to the 31-bit record
// count); accesses at or past the end read as zero.  The range check covers
// the sum of the lane offset (voffset) and the wave-uniform one (soffset):
// on MI355X a load whose soffset alone, or whose voffset + soffset, passes
// the range returned zeros (measured with both inside one allocation), which
// is what the kernels' past-the-end soffsets rely on.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int64_t bytes) {
  const int nrec = (int)(bytes < 0 ? 0 : bytes > 0x7fffffff ? 0x7fffffff : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nrec, kBufferRsrcWord3);
}

constexpr int kNtPolicy = 2;   // non-temporal: data streamed once

// Workspace layout shared by every kernel that splits a tile's k range over
// workgroups (decode GEMV, small-batch kernel, deep-ring GEMM): uint32
// arrival counters in this fixed region at the start, then that kernel's
// fp32 partials.  Every call leaves the counters it used at zero, and no
// kernel's partials reach into the region, so one buffer can serve all the
// kernels and shapes in turn.
constexpr size_t kSplitCounterBytes = 16384;
constexpr int kSplitMaxCounters = (int)(kSplitCounterBytes / 4);
// Largest workspace any split plan asks for (counters + partials): plans
// that would need more take fewer splits, so the allocation-free entry
// point's fixed scratch of this size runs the same plan as a caller
// workspace.
constexpr size_t kSplitWorkspaceMaxBytes = 16u << 20;

// 16 bytes per lane, buffer -> LDS (buffer_load_dwordx4 ... lds): lane L's
// bytes land at lds_base + 16 * L (out-of-range offsets land as zeros).
// Kept out of kernel templates: with the builtin written inside one, the
// host pass drops the kernel's launch stub.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, soff, 0, 0);
}

// 16-byte LDS read issued as inline asm, for kernels that fill LDS with the
// direct copies above: the compiler cannot tell such a copy into the next
// stage from a read of the current one and waits for all of them (vmcnt(0))
// before any LDS read it can see, which serializes the copy with the math.
// These reads are invisible to it; lds_wait_first_half / lds_wait_rest must
// complete them before use.
__device__ __forceinline__ uint4_t lds_read16_asm(const uint8_t* p) {
  const uint32_t a = (uint32_t)(size_t)((const __attribute__((address_space(3))) uint8_t*)p);
  uint4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
  return v;
}

// For MT reads issued in order: wait until the first MT/2 have landed (LDS
// reads return in order), then until all have; each wait is tied to the
// fragments it completes so that no use moves above it.
template <int MT>
__device__ __forceinline__ void lds_wait_first_half(uint4_t (&b)[MT]) {
  static_assert(MT == 1 || MT == 2 || MT == 4 || MT == 8 || MT == 16, "fragment count");
  if constexpr (MT == 1) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b[0]));   // a single read: all of it
  } else if constexpr (MT == 16) {
    asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(b[4]), "+v"(b[5]),
                 "+v"(b[6]), "+v"(b[7]));
  } else if constexpr (MT == 8) {
    asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
  } else if constexpr (MT == 4) {
    asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(b[0]), "+v"(b[1]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(b[0]));
  }
}
template <int MT>
__device__ __forceinline__ void lds_wait_rest(uint4_t (&b)[MT]) {
  static_assert(MT == 1 || MT == 2 || MT == 4 || MT == 8 || MT == 16, "fragment count");
  if constexpr (MT == 1) {
    // completed by lds_wait_first_half
  } else if constexpr (MT == 16) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b[8]), "+v"(b[9]), "+v"(b[10]), "+v"(b[11]), "+v"(b[12]), "+v"(b[13]),
                 "+v"(b[14]), "+v"(b[15]));
  } else if constexpr (MT == 8) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7]));
  } else if constexpr (MT == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b[2]), "+v"(b[3]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b[1]));
  }
}

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Zero-point constants for one row: c_lo = -(1024 + z), c_hi = -(64 + z) as
// fp16 pairs.  -(1024+z) has exponent 25 and mantissa z; -(64+z) has exponent
// 21 and mantissa 16*z.
__device__ __forceinline__ void w4_zero_consts(uint32_t z, uint32_t& c_lo, uint32_t& c_hi) {
  const uint32_t zz = z * 0x00010001u;
  c_lo = zz | 0xE400E400u;
  c_hi = (zz << 4) | 0xD400D400u;
}

// (a & mask) | c in one VALU op.  gfx9 VOP3 cannot take two literal
// operands, so the compiler splits the expression into v_and + v_or; this
// keeps the mask in an SGPR and the OR-constant in a (hoisted) VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(c));
  return r;
}

// One tile word (nibble p holds element {0,2,4,6,1,3,5,7}[p]) -> the eight
// exact fp16 values (q_e - z), e = 0..7 in order.  OR-ing a nibble into the
// mantissa of 1024.0 gives 1024+q exactly; the high nibble of each byte lands
// as 1024+16q and is brought back with an exact fma by 1/16.
__device__ __forceinline__ half8_t w4_word_to_h8(uint32_t w, uint32_t c_lo, uint32_t c_hi) {
  const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
  const uint32_t w8 = w >> 8;
  const half2_t t0 = as_h2(and_or(w, 0x000F000Fu, 0x64006400u));
  const half2_t t1 = as_h2(and_or(w, 0x00F000F0u, 0x64006400u));
  const half2_t t2 = as_h2(and_or(w8, 0x000F000Fu, 0x64006400u));
  const half2_t t3 = as_h2(and_or(w8, 0x00F000F0u, 0x64006400u));
  const half2_t p0 = t0 + as_h2(c_lo);
  const half2_t p1 = __builtin_elementwise_fma(t1, sixteenth, as_h2(c_hi));
  const half2_t p2 = t2 + as_h2(c_lo);
  const half2_t p3 = __builtin_elementwise_fma(t3, sixteenth, as_h2(c_hi));
  half8_t r;
  r.s01 = p0; r.s23 = p1; r.s45 = p2; r.s67 = p3;
  return r;
}

// One tile word -> the eight fp16 values before the zero point is taken off:
// 1024+q_e for e in {0,1,4,5} and 1024+16q_e for e in {2,3,6,7}.  Four VALU
// ops per word; the caller pairs the fragment with x pre-divided by 16 at
// e in {2,3,6,7} and with w4_zero_frag() on the same x, so that
//   raw . x' + zero_frag . x' = sum_e (q_e - z) x_e.
// Every product is exact in fp32 (11 x 11 significant bits).
__device__ __forceinline__ half8_t w4_word_to_h8_raw(uint32_t w) {
  const uint32_t w8 = w >> 8;
  half8_t r;
  r.s01 = as_h2(and_or(w, 0x000F000Fu, 0x64006400u));
  r.s23 = as_h2(and_or(w, 0x00F000F0u, 0x64006400u));
  r.s45 = as_h2(and_or(w8, 0x000F000Fu, 0x64006400u));
  r.s67 = as_h2(and_or(w8, 0x00F000F0u, 0x64006400u));
  return r;
}

// The matching zero-point fragment of one row: -(1024 + z) at e in {0,1,4,5},
// -(1024 + 16z) at e in {2,3,6,7} (exponent 25, mantissa z or 16z: exact).
__device__ __forceinline__ half8_t w4_zero_frag(uint32_t z) {
  const uint32_t zz = z * 0x00010001u;
  const half2_t lo = as_h2(zz | 0xE400E400u);
  const half2_t hi = as_h2((zz << 4) | 0xE400E400u);
  half8_t r;
  r.s01 = lo; r.s23 = hi; r.s45 = lo; r.s67 = hi;
  return r;
}

// x chunk of eight consecutive k (8-aligned) -> the B fragment that pairs
// with w4_word_to_h8_raw: elements 2,3,6,7 divided by 16 (exact for normal
// results).
__device__ __forceinline__ uint4_t w4_prescale_x(uint4_t v) {
  const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
  v.y = as_u32(as_h2(v.y) * sixteenth);
  v.w = as_u32(as_h2(v.w) * sixteenth);
  return v;
}

// Same, multiplied by the group scale: fp16((q - z) * s), which is the
// reference decode bit for bit ((q - z) is exact, the product rounds once).
__device__ __forceinline__ half8_t w4_word_to_h8_scaled(uint32_t w, uint32_t c_lo, uint32_t c_hi, half2_t s2) {
  half8_t v = w4_word_to_h8(w, c_lo, c_hi);
  half8_t s8;
  s8.s01 = s2; s8.s23 = s2; s8.s45 = s2; s8.s67 = s2;
  return v * s8;
}

// Four signed int8 (natural order) -> four exact fp16.  Flipping the sign bit
// gives q+128 as an unsigned byte; placing it under the exponent byte 0x64
// yields 1024+128+q, and subtracting 1152 leaves q.
__device__ __forceinline__ half4_t i8x4_to_h4(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const half2_t bias = as_h2(0xE480E480u);  // -1152
  const half2_t lo = as_h2(__builtin_amdgcn_perm(u, 0x64646464u, 0x00050004u)) + bias;
  const half2_t hi = as_h2(__builtin_amdgcn_perm(u, 0x64646464u, 0x00070006u)) + bias;
  half4_t r;
  r.s01 = lo; r.s23 = hi;
  return r;
}

__device__ __forceinline__ half8_t i8x8_to_h8(uint32_t w0, uint32_t w1) {
  half8_t r;
  r.s0123 = i8x4_to_h4(w0);
  r.s4567 = i8x4_to_h4(w1);
  return r;
}

// Eight signed int8 -> eight fp16 1152+q (the bias is left in; the caller
// takes it off with one MFMA of the constant fragment kI8BiasFrag against
// the same x).  Three VALU ops per word.
__device__ __forceinline__ half8_t i8x8_to_h8_raw(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  half8_t r;
  r.s01 = as_h2(__builtin_amdgcn_perm(u0, 0x64646464u, 0x00050004u));
  r.s23 = as_h2(__builtin_amdgcn_perm(u0, 0x64646464u, 0x00070006u));
  r.s45 = as_h2(__builtin_amdgcn_perm(u1, 0x64646464u, 0x00050004u));
  r.s67 = as_h2(__builtin_amdgcn_perm(u1, 0x64646464u, 0x00070006u));
  return r;
}

// -1152 in every element (fp16 0xE480).
__device__ __forceinline__ half8_t i8_bias_frag() {
  const half2_t b = as_h2(0xE480E480u);
  half8_t r;
  r.s01 = b; r.s23 = b; r.s45 = b; r.s67 = b;
  return r;
}

__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t ld_h8(const half_t* p) {
  return *reinterpret_cast<const half8_t*>(p);
}

// Cross-lane reductions without LDS: DPP moves inside the 16-lane rows, then
// v_readlane for the wave (every lane gets the result; sums in row order).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Over the 16 lanes of a DPP row: quad swaps, then the half-row and row
// mirrors.
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

// Lane c's value, wave-uniform.
__device__ __forceinline__ float lane_f(float v, int c) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), c));
}

__device__ __forceinline__ float wave_max_rl(float v) {
  v = row_max16(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ float wave_sum_rl(float v) {
  v = row_sum16(v);
  return ((lane_f(v, 0) + lane_f(v, 16)) + lane_f(v, 32)) + lane_f(v, 48);
}

// Eight x values -> w * fp16(x * r), the reference's rms_norm order
// (normalize in fp32, cast, scale in fp16).
__device__ __forceinline__ uint4_t rms_scale8(uint4_t xv, uint4_t wv, float r) {
  const half8_t xh = __builtin_bit_cast(half8_t, xv), wh = __builtin_bit_cast(half8_t, wv);
  half8_t o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = wh[e] * (half_t)((float)xh[e] * r);
  return __builtin_bit_cast(uint4_t, o);
}

constexpr float kLog2e = 1.4426950408889634f;

// 2^x on the transcendental unit (v_exp_f32, about 1 ulp; -inf -> 0).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// silu(g) = g / (1 + e^-g) as g * rcp(1 + 2^(-g log2 e)): two transcendental
// ops instead of expf and an IEEE divide.  The fp32 result is within a few
// ulp of the exact quotient, far below the fp16 rounding that follows it;
// g -> -inf gives -0 (rcp(inf) = 0), g -> +inf gives g, silu(-0) = -0.
// The empty asm keeps g and the product as plain fp32 values: otherwise
// hipcc folds the fp16 -> fp32 widening of g, or the fp16 rounding of the
// result, into a mixed-precision FMA with a +0 addend, which returns +0 for
// g = -0 (and then a product with a negative up value differs in sign).
__device__ __forceinline__ float silu_f(float g) {
  asm("" : "+v"(g));
  float r = g * __builtin_amdgcn_rcpf(1.0f + exp2_hw(-g * kLog2e));
  asm("" : "+v"(r));
  return r;
}

}  // namespace wq
