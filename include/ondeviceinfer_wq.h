/*
 * ondeviceinfer_wq.h - C ABI of the MI355X (gfx950) weight-only quantized Linear.
 *
 * These entry points replace the native calls behind OnDeviceInfer's pluggable
 * compressed Linear (ondeviceinfer/weight_quantization/backend.py) and its
 * INT8 explicit-dequant path (ondeviceinfer/quantized_model.py,
 * ondeviceinfer/quantization.py).  Each declaration names the reference call
 * it replaces.
 *
 * Conventions
 *  - Every pointer is a device pointer (hipMalloc'd or torch-owned) unless
 *    noted; fp16 tensors are passed as uint16_t bit patterns; all tensors are
 *    contiguous row-major.
 *  - `stream` is a hipStream_t (NULL = default stream).  Work is only
 *    enqueued; nothing synchronises, nothing allocates.
 *  - Return 0 (WQ_OK) or a WQ_ERR_* code; wq_last_error() then describes the
 *    failure (thread-local, valid until the next failing call on the thread).
 *  - Shapes: N output features, K input features, M activation rows.
 */
#ifndef ONDEVICEINFER_WQ_H
#define ONDEVICEINFER_WQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WQ_OK 0
#define WQ_ERR_INVALID_ARGUMENT 1 /* malformed shape / null pointer (Python: ValueError) */
#define WQ_ERR_UNSUPPORTED 2      /* valid request this build does not implement (ValueError) */
#define WQ_ERR_HIP 3              /* HIP runtime error (RuntimeError) */
#define WQ_ERR_WORKSPACE 4        /* workspace too small (ValueError) */

#define WQ_ABI_VERSION 2

/* Error channel.  The reference raises Python exceptions directly
 * (backend.py:174-175, :212-213, :229-230); the Python host maps codes back. */
const char* wq_last_error(void);
int wq_abi_version(void);

/* ---------------------------------------------------------------- W4 (uint4, G-grouped) */

/* Sizes of the gfx950 tile layout for an [n, k] pack-quantized weight.
 * Requires n % 8 == 0, group_size % 128 == 0, k % group_size == 0.
 * Replaces the allocation inside vllm gptq_marlin_repack (backend.py:214). */
int wq_w4_repack_size(int64_t n, int64_t k, int64_t group_size,
                      size_t* tiles_bytes, size_t* meta_bytes);

/* One-time startup repack of compressed-tensors pack-quantized tensors:
 *   weight_packed int32 [n, k/8] (8 codes per word along k, LSB first),
 *   weight_scale  fp16  [n, k/group_size],
 *   weight_zero_point int32 [n/8, k/group_size] (8 per word along n) or NULL
 *   for the symmetric uint4b8 format (zero point 8)
 * into `tiles` / `meta` (sizes from wq_w4_repack_size).
 * Replaces vllm gptq_marlin_repack + marlin_permute_scales + unpack_unsigned/
 * marlin_zero_points (backend.py:214-221). */
int wq_w4_repack(const int32_t* weight_packed, const uint16_t* weight_scale,
                 const int32_t* weight_zero_point, int64_t n, int64_t k, int64_t group_size,
                 void* tiles, void* meta, void* stream);

/* Exact inverse of wq_w4_repack (zero point words are 0x88888888 when the
 * repack had none).  No reference counterpart: it proves the layout is
 * lossless (the reference's own unpack is unpack_unsigned, backend.py:26-32). */
int wq_w4_unpack(const void* tiles, const void* meta, int64_t n, int64_t k, int64_t group_size,
                 int32_t* weight_packed, uint16_t* weight_scale, int32_t* weight_zero_point,
                 void* stream);

/* fp16 [n, k] = (q - z) * s read from the tile layout, with the same unpack
 * arithmetic the W4A16 kernels use; equals decode_weight bit for bit
 * (backend.py:41-54). */
int wq_w4_dequant(const void* tiles, const void* meta, int64_t n, int64_t k, int64_t group_size,
                  uint16_t* weight, void* stream);

/* Explicit QDQ decode straight from compressed-tensors tensors, any group
 * size and optional act-order g_idx (int32 [k] or NULL):
 * fp16((q - z[g]) * scale[g]) computed in fp32, z = 8 when weight_zero_point is
 * NULL.  weight_scale is fp32 [n, num_groups]; weight_zero_point is int32
 * [ceil(n/8), num_groups]; g_idx entries must lie in [0, num_groups).
 * Replaces decode_weight's W4
 * branch (backend.py:41-54) for the reference_int4 backend. */
int wq_w4_decode(const int32_t* weight_packed, const float* weight_scale,
                 const int32_t* weight_zero_point, const int32_t* g_idx,
                 int64_t n, int64_t k, int64_t num_groups, int64_t group_size,
                 uint16_t* weight, void* stream);

/* Row-sampled form of wq_w4_decode: weight [num_rows, k] row r =
 * fp16((q - z) * s) of source row rows[r] (int64, each in [0, n): the host
 * checks), groups of group_size along k (no g_idx).  Replaces decode_rows
 * (benchmarks/validate_weight_reconstruction.py:20-31), which samples the
 * rows of a large matrix such as the LM head instead of decoding it whole. */
int wq_w4_decode_rows(const int32_t* weight_packed, const float* weight_scale,
                      const int32_t* weight_zero_point, const int64_t* rows, int64_t num_rows,
                      int64_t n, int64_t k, int64_t num_groups, int64_t group_size,
                      uint16_t* weight, void* stream);

/* Workspace bytes wq_w4a16_linear can use for this shape (0 when it needs
 * none).  The workspace holds the arrival counters and fp32 partials of the
 * kernels that split a tile's k range over several workgroups: the decode
 * GEMV (m <= 4), the small-batch kernel (12 <= m <= 32 on n <= 18432) and the
 * deep-ring GEMM on the smallest prefill grids (m > 64 on narrow n).  The
 * counters sit in a fixed 16 KiB region at the start, so one buffer sized for
 * the largest shape serves every shape.  It must be zero-filled once before
 * first use; every call leaves the counters zeroed again, so it can be
 * reused by later calls (and graph replays) on the same stream.  Calls that
 * may run concurrently need separate workspaces.  With a NULL or smaller
 * workspace the linear runs without the split (the decode GEMV keeps each
 * tile in one workgroup: same result; at 12 <= m <= 32 the skinny kernels,
 * and the deep-ring GEMM over the whole k range: the same values up to fp32
 * summation order).  Replaces
 * marlin_make_workspace_new (backend.py:223). */
int wq_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int64_t group_size, size_t* bytes);

/* y fp16 [m, n] = x fp16 [m, k] . dequant(W)^T with fp32 accumulation.
 * Dispatches on m: MFMA GEMV for small m, LDS-staged MFMA GEMM for large m.
 * Replaces vllm gptq_marlin_gemm (backend.py:195-202, called from :233-248). */
int wq_w4a16_linear(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                    int64_t n, int64_t group_size, uint16_t* y,
                    void* workspace, size_t workspace_bytes, void* stream);

/* wq_w4a16_linear without a workspace argument and without any allocation:
 * the k-split counters and partials live in a fixed 16 MiB device array
 * inside the library (one per GPU, held until the process ends), so the call
 * runs the same plan, with the same results, as wq_w4a16_linear with a
 * workspace of wq_w4a16_workspace_size bytes (every split plan fits 16 MiB).
 * Every call on a GPU shares that GPU's array: calls that may overlap on one
 * GPU (different streams, or graphs replayed concurrently) race and must be
 * ordered by the caller.  The first call on a device looks the array up
 * (hipGetSymbolAddress) and queues a clear of it on `stream`; that first call
 * must not be under stream capture (it returns WQ_ERR_UNSUPPORTED there, so
 * no clear is ever recorded into a graph): make one eager call per device
 * before capturing later ones, which then record only the linear.
 * No counterpart in the reference: it exists for callers that cannot
 * allocate (code under HIP graph capture, serving loops and harnesses that
 * forbid hipMalloc). */
int wq_w4a16_linear_noalloc(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                            int64_t n, int64_t group_size, uint16_t* y, void* stream);

/* One decode-token (M = 1) W4A16 linear with the neighbouring elementwise
 * work of the Qwen3 decoder layer folded in (n % 16 == 0):
 *   x_mode 0  x as given ([k]);
 *   x_mode 1  x <- norm_weight * fp16(x * rsqrt(sum(sumsq_in[0..sumsq_count)) / k + eps)),
 *             the RMSNorm of x whose sum of squares the producing linear
 *             left in sumsq_in (one float per 16-row tile, at most 512;
 *             16-byte aligned);
 *   x_mode 2  x is [gate | up] of length 2k and x <- fp16(fp16(silu(gate)) * up);
 *   residual  if not NULL, y = residual + fp16(x . W^T) (fp16 add; may alias y);
 *   sumsq_out if not NULL, receives the sum of squares of y per 16-row tile
 *             (n / 16 floats) for the next linear's x_mode 1.
 * Workspace as for wq_w4a16_linear at m = 1.  Replaces, per decode token,
 * rms_norm before q/k/v and gate/up, `residual + attention_output`,
 * `residual + mlp_output` and `F.silu(gate) * up` around the linears
 * (quantized_model.py:146-227); no counterpart kernel exists in the
 * reference (it runs them as separate torch ops). */
int wq_w4a16_decode_fused(const uint16_t* x, int64_t k, const void* tiles, const void* meta, int64_t n,
                          int64_t group_size, int32_t x_mode, const uint16_t* norm_weight, const float* sumsq_in,
                          int64_t sumsq_count, float eps, const uint16_t* residual, float* sumsq_out, uint16_t* y,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Whether wq_w4a16_linear_epilogue applies to this shape and mode (1) or not
 * (0): m above the decode GEMV's 64 rows, on the prefill GEMM grids that carry
 * a fused epilogue (mode 1 also needs two tiles per wave and n % 32 == 0). */
int wq_w4a16_epilogue_supported(int64_t m, int64_t n, int64_t k, int64_t group_size, int32_t mode);

/* Prefill (m > 64) W4A16 linear with the next elementwise op of the Qwen3 MLP
 * in its epilogue, bit-identical to wq_w4a16_linear followed by that op:
 *   mode 1  W is a fused [gate | up] of n = 2 n_out rows (gate rows first);
 *           y fp16 [m, n_out] = fp16(fp16(silu(g)) * u) with g, u the fp16
 *           outputs of the gate and up rows (wq_silu_mul's arithmetic);
 *   mode 2  y fp16 [m, n] = fp16(residual + fp16(x . W^T)); y may alias
 *           residual.
 * Shapes for which wq_w4a16_epilogue_supported is 0 return WQ_ERR_UNSUPPORTED.
 * Replaces `F.silu(gate) * up` after the gate/up linears and
 * `residual + mlp_output` after the down linear of the prefill forward
 * (quantized_model.py:216-228), which the reference runs as separate torch
 * ops after the linears. */
int wq_w4a16_linear_epilogue(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                             int64_t n, int64_t group_size, int32_t mode, const uint16_t* residual,
                             uint16_t* y, void* stream);

/* Whether wq_w8a16_linear_epilogue applies (1) or not (0): INT8 tiles
 * (k % 128 == 0), m above 64 rows, on the prefill GEMM grids that carry a
 * fused epilogue (mode 1: two tiles per wave and n % 32 == 0). */
int wq_w8a16_epilogue_supported(int64_t m, int64_t n, int64_t k, int32_t mode);

/* wq_w4a16_linear_epilogue for an INT8 weight in the tile layout
 * (wq_w8_repack) with fp16 per-row scale: the linear's output is
 * fp16(sum * scale[n]) as in wq_w8a16_linear_tiled, then mode 1 (fused
 * [gate | up] weight and scale, output [m, n / 2]) or mode 2 (+ residual, y may
 * alias it), bit-identical to wq_w8a16_linear_tiled followed by wq_silu_mul or
 * the fp16 add.  Replaces the same elementwise ops of the INT8 model's
 * prefill (quantized_model.py:216-228). */
int wq_w8a16_linear_epilogue(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const uint16_t* scale,
                             int64_t n, int32_t mode, const uint16_t* residual, uint16_t* y, void* stream);

/* ------------------------------------------------- W8 (int8, per-output-channel scale) */

/* fp16 [n, k] = fp16(q * scale[n]), scale fp32 [n].  Replaces the INT8 branch
 * of decode_weight (backend.py:37-40), dequantize_linear_weight
 * (quantization.py:320-330) and the scratch copy_+mul_ of
 * int8_weight_only_linear (quantized_model.py:101-106). */
int wq_w8_decode(const int8_t* qweight, const float* scale, int64_t n, int64_t k,
                 uint16_t* weight, void* stream);

/* Workspace bytes wq_w8a16_linear can use (same contract as
 * wq_w4a16_workspace_size).  Replaces the fp16 dequant scratch sizing of
 * QuantizedCpuWeightStore.max_dequant_elements (runtime/quantized.py:90-96),
 * with far less memory. */
int wq_w8a16_workspace_size(int64_t m, int64_t n, int64_t k, size_t* bytes);

/* y fp16 [m, n] = x fp16 [m, k] . (q * scale)^T (+ bias fp16 [n] or NULL),
 * consuming the INT8 weight in its stored [n, k] row-major layout with no
 * fp16 scratch (MFMA tiles when k % 128 == 0 and x, qweight are 16-byte
 * aligned; a one-wave-per-output kernel otherwise).  Replaces the dequant + F.linear of
 * int8_weight_only_linear (quantized_model.py:101-121) and quantized_linear
 * (quantization.py:333-353). */
int wq_w8a16_linear(const uint16_t* x, int64_t m, int64_t k, const int8_t* qweight,
                    const uint16_t* scale, int64_t n, const uint16_t* bias, uint16_t* y,
                    void* workspace, size_t workspace_bytes, void* stream);

/* The INT8 counterpart of wq_w4a16_decode_fused: one decode-token (M = 1)
 * INT8 x fp16 linear on the stored [n, k] weight with the fp16 row scale,
 * with the same x_mode / residual / sumsq_out fusions (n % 16 == 0,
 * k % 128 == 0; x, qweight, y, norm_weight and sumsq_in 16-byte aligned,
 * residual 8-byte).  y = residual + fp16(scale[n] * (x . q[n])) when residual
 * is given.  Workspace as for wq_w8a16_linear at m = 1.  Replaces, in the
 * INT8 weight-only decoder layer, the same rms_norm / residual / SiLU*up ops
 * around int8_weight_only_linear (quantized_model.py:146-227, :101-121). */
int wq_w8a16_decode_fused(const uint16_t* x, int64_t k, const int8_t* qweight, const uint16_t* scale, int64_t n,
                          int32_t x_mode, const uint16_t* norm_weight, const float* sumsq_in, int64_t sumsq_count,
                          float eps, const uint16_t* residual, float* sumsq_out, uint16_t* y, void* workspace,
                          size_t workspace_bytes, void* stream);

/* INT8 tile layout (k % 128 == 0): the same int8 values as the row-major
 * [n, k] weight, regrouped into 2 KiB per (16-row tile, 128-k block), rows
 * past n zero, so that each 16-byte-per-lane piece the INT8 kernels take is
 * one contiguous 1 KiB wave load instead of sixteen 64-byte row segments.
 * Within tile t, block b: byte 1024 p + 16 l + j = q[16t + l % 16]
 * [128b + 64p + 16 (l / 16) + j], p in {0, 1}, l in [0, 64), j in [0, 16).
 * Like the W4 tile layout, this one is this library's own (the reference
 * stores INT8 row-major and dequantizes it, quantized_model.py:101-106);
 * wq_w8_repack / wq_w8_unpack are a bit-exact pair and the _tiled linears
 * below return the same bits as their row-major counterparts. */
int wq_w8_tiles_size(int64_t n, int64_t k, size_t* bytes);
int wq_w8_repack(const int8_t* qweight, int64_t n, int64_t k, void* tiles, void* stream);
int wq_w8_unpack(const void* tiles, int64_t n, int64_t k, int8_t* qweight, void* stream);

/* wq_w8a16_linear / wq_w8a16_decode_fused / wq_w8a8_linear over INT8 tiles
 * (16-byte aligned) instead of the row-major weight; k % 128 == 0.  Same
 * arguments, results bit-identical.  Replace the same reference calls as
 * their row-major forms; the decode graph and the prepared INT8 linears of
 * this library use these. */
int wq_w8a16_linear_tiled(const uint16_t* x, int64_t m, int64_t k, const void* tiles,
                          const uint16_t* scale, int64_t n, const uint16_t* bias, uint16_t* y,
                          void* workspace, size_t workspace_bytes, void* stream);
int wq_w8a16_decode_fused_tiled(const uint16_t* x, int64_t k, const void* tiles, const uint16_t* scale,
                                int64_t n, int32_t x_mode, const uint16_t* norm_weight, const float* sumsq_in,
                                int64_t sumsq_count, float eps, const uint16_t* residual, float* sumsq_out,
                                uint16_t* y, void* workspace, size_t workspace_bytes, void* stream);

/* Symmetric per-output-channel INT8 quantizer: weight fp32 [n, k] ->
 * qweight int8 [n, k] + fp16 scale [n] (absmax/127, zero rows scale 1,
 * underflowing scales -> smallest fp16 subnormal, the stored scale divides,
 * round-half-even, clamp +-127).  Non-finite input ORs bit 0 and a scale
 * that overflows fp16 ORs bit 1 into *status_flags (device int32 that the
 * caller zero-fills beforehand).  Replaces quantize_linear_weight
 * (quantization.py:226-285). */
int wq_w8_quantize(const float* weight, int64_t n, int64_t k, int8_t* qweight, uint16_t* scale,
                   int32_t* status_flags, void* stream);

/* W8A8, step 1: dynamic per-token symmetric INT8 quantization of the
 * activations x fp16 [m, k] (k % 8 == 0): x_scale fp32 [m] =
 * max(max_k |x[r, k]|, 1e-12) / 127 and qx int8 [m, k] =
 * clamp(round_half_even(x / x_scale), -127, 127), an IEEE fp32 divide.
 * Replaces vLLM's scaled_int8_quant(x, symmetric=True) in the int8_gemm
 * backend (backend.py:252-253); the formula is the reference's W8A8 oracle
 * (reference_w8a8, backend.py:258-261). */
int wq_w8a8_quantize(const uint16_t* x, int64_t m, int64_t k, int8_t* qx, float* x_scale, void* stream);

/* W8A8, step 2: y fp16 [m, n] = fp16(float(sum_k qx[m, k] * qweight[n, k])
 * * x_scale[m] * w_scale[n] (+ bias[n])): int8 x int8 products summed
 * exactly in int32 on the int8 matrix cores, scaled in fp32 in that order.
 * qweight int8 [n, k] row-major (the compressed-tensors channel-INT8
 * `weight`), w_scale fp32 [n]; k % 64 == 0, qx and qweight 16-byte aligned.
 * Replaces vLLM's cutlass_scaled_mm(qx, qweight^T, x_scale, w_scale, fp16)
 * (backend.py:254). */
int wq_w8a8_linear(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const int8_t* qweight,
                   const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream);
int wq_w8a8_linear_tiled(const int8_t* qx, const float* x_scale, int64_t m, int64_t k, const void* tiles,
                         const float* w_scale, int64_t n, const uint16_t* bias, uint16_t* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ONDEVICEINFER_WQ_H */
