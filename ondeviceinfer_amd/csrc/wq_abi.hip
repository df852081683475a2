// C-ABI entry points for the linear kernels, plus the error channel.
#include "wq_common.h"
#include "wq_status.h"

#include <mutex>

namespace wq {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

size_t gemv_workspace_bytes(bool w4, int64_t m, int64_t n, int64_t k);
size_t w4_batch_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t g);
int launch_w4_skinny(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                     half_t* y, void* ws, size_t ws_bytes, hipStream_t s);
int launch_w8_skinny(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                     half_t* y, void* ws, size_t ws_bytes, hipStream_t s, int tiled);
int launch_w8_generic(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                      half_t* y, hipStream_t s);
int launch_w4_gemm(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G, half_t* y,
                   hipStream_t s, void* ws, size_t ws_bytes);
size_t w4_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);
int launch_w8_gemm(const half_t* x, int M, int K, const int8_t* q, const half_t* scale, const half_t* bias, int N,
                   half_t* y, hipStream_t s, int tiled);
bool w4_gemm_small_fits(int64_t M, int64_t N);
int gemm_epi_plan(int64_t M, int64_t N, int64_t K, int mode, int64_t block_bytes);
int launch_w4_gemm_epi(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                       int mode, const half_t* res, half_t* y, hipStream_t s);
int launch_w8_gemm_epi(const half_t* x, int M, int K, const int8_t* tiles, const half_t* scale, int N, int mode,
                       const half_t* res, half_t* y, hipStream_t s);
int launch_w4_gemm_small(const half_t* x, int M, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         half_t* y, hipStream_t s);

int launch_w4_gemv_fused(const half_t* x, int K, const uint4_t* tiles, const uint8_t* meta, int N, int G,
                         int x_mode, const half_t* norm_w, const float* sumsq_in, int sumsq_count, float eps,
                         const half_t* residual, float* sumsq_out, half_t* y, void* ws, size_t ws_bytes,
                         hipStream_t s);
int launch_w8_gemv_fused(const half_t* x, int K, const int8_t* q, const half_t* scale, int N, int x_mode,
                         const half_t* norm_w, const float* sumsq_in, int sumsq_count, float eps,
                         const half_t* residual, float* sumsq_out, half_t* y, void* ws, size_t ws_bytes,
                         hipStream_t s, int tiled);

// Largest M served by the MFMA GEMV (4 chunks of 16 activation rows).
constexpr int64_t kSkinnyMaxM = 64;
// Largest k of the prefill GEMMs.  A workgroup reads its (up to) 128 x rows
// through one buffer resource whose record count is capped at 2^31 - 1
// bytes: row r of a 128-k block sits at byte r * 2k + [0, 256), so the last
// row (127) must stay below that cap, or its reads would come back as zeros.
// Longer rows run the skinny kernels 64 rows at a time.
constexpr int64_t kGemmMaxRows = 128;
constexpr int64_t kGemmMaxK = 1 << 23;
static_assert((kGemmMaxRows - 1) * 2 * kGemmMaxK + 2 * kW4BlockK <= 0x7fffffff,
              "GEMM x offsets must fit the 31-bit buffer range");

namespace {

int linear_shape_check(int64_t m, int64_t n, int64_t k) {
  WQ_REQUIRE(m >= 0 && n > 0 && k > 0, WQ_ERR_INVALID_ARGUMENT, "bad linear shape m=%lld n=%lld k=%lld",
             (long long)m, (long long)n, (long long)k);
  WQ_REQUIRE(m <= 0x7FFFFFFF && n <= 0x7FFFFFFF && k <= 0x7FFFFFFF && m * k < (1LL << 40), WQ_ERR_UNSUPPORTED,
             "linear shape too large m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  return WQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace wq

using namespace wq;

extern "C" const char* wq_last_error(void) { return g_last_error; }

extern "C" int wq_abi_version(void) { return WQ_ABI_VERSION; }

extern "C" int wq_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int64_t group_size, size_t* bytes) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null size output");
  size_t need = gemv_workspace_bytes(true, m, n, k);
  const size_t batch = w4_batch_workspace_bytes(m, n, k, group_size);
  const size_t gemm = m > kSkinnyMaxM && k <= kGemmMaxK ? w4_gemm_workspace_bytes(m, n, k) : 0;
  if (batch > need) need = batch;
  if (gemm > need) need = gemm;
  *bytes = need;
  return WQ_OK;
}

extern "C" int wq_w8a16_workspace_size(int64_t m, int64_t n, int64_t k, size_t* bytes) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(bytes, WQ_ERR_INVALID_ARGUMENT, "null size output");
  *bytes = k % kW8BlockK == 0 ? gemv_workspace_bytes(false, m, n, k) : 0;
  return WQ_OK;
}

extern "C" int wq_w4a16_linear(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                               int64_t n, int64_t group_size, uint16_t* y, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(n % 8 == 0 && group_size % kW4BlockK == 0 && group_size > 0 && k % group_size == 0,
             WQ_ERR_UNSUPPORTED, "W4A16 needs n %% 8 == 0, group_size %% 128 == 0, k %% group_size == 0 "
             "(n=%lld k=%lld group=%lld)", (long long)n, (long long)k, (long long)group_size);
  WQ_REQUIRE(tiles && meta, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (m == 0) return WQ_OK;   // empty activations: x and y may be null
  WQ_REQUIRE(x && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(aligned16(x) && aligned16(tiles) && aligned16(y) && (reinterpret_cast<uintptr_t>(meta) & 7u) == 0,
             WQ_ERR_INVALID_ARGUMENT, "x, tiles and y must be 16-byte aligned and meta 8-byte aligned");
  const half_t* xh = reinterpret_cast<const half_t*>(x);
  half_t* yh = reinterpret_cast<half_t*>(y);
  if (w4_gemm_small_fits(m, n) && k <= kGemmMaxK)
    return launch_w4_gemm_small(xh, (int)m, (int)k, reinterpret_cast<const uint4_t*>(tiles),
                                reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size, yh, as_stream(stream));
  if (m <= kSkinnyMaxM)
    return launch_w4_skinny(xh, (int)m, (int)k, reinterpret_cast<const uint4_t*>(tiles),
                            reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size, yh, workspace,
                            workspace_bytes, as_stream(stream));
  if (k > kGemmMaxK) {
    for (int64_t r = 0; r < m; r += kSkinnyMaxM) {
      const int64_t mr = m - r < kSkinnyMaxM ? m - r : kSkinnyMaxM;
      const int rc = launch_w4_skinny(xh + r * k, (int)mr, (int)k, reinterpret_cast<const uint4_t*>(tiles),
                                      reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size, yh + r * n,
                                      workspace, workspace_bytes, as_stream(stream));
      if (rc != WQ_OK) return rc;
    }
    return WQ_OK;
  }
  return launch_w4_gemm(xh, (int)m, (int)k, reinterpret_cast<const uint4_t*>(tiles),
                        reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size, yh, as_stream(stream),
                        workspace, workspace_bytes);
}

namespace {
// Whether wq_w4a16_linear takes the prefill GEMM for this shape with a grid
// that carries the fused epilogue `mode`.
bool w4_epilogue_fits(int64_t m, int64_t n, int64_t k, int64_t group_size, int32_t mode) {
  if (mode != 1 && mode != 2) return false;
  if (m <= kSkinnyMaxM || w4_gemm_small_fits(m, n) || k > kGemmMaxK) return false;
  if (n % (mode == 1 ? 32 : 8) != 0 || group_size <= 0 || group_size % kW4BlockK != 0 || k % group_size != 0)
    return false;
  return gemm_epi_plan(m, n, k, mode, 1024) != 0;
}

// The same for INT8 tiles (k % 128 == 0).
bool w8_epilogue_fits(int64_t m, int64_t n, int64_t k, int32_t mode) {
  if (mode != 1 && mode != 2) return false;
  if (m <= kSkinnyMaxM || k > kGemmMaxK || k % kW8BlockK != 0) return false;
  if (n % (mode == 1 ? 32 : 8) != 0) return false;
  return gemm_epi_plan(m, n, k, mode, kW8TileBlockBytes) != 0;
}
}  // namespace

extern "C" int wq_w4a16_epilogue_supported(int64_t m, int64_t n, int64_t k, int64_t group_size, int32_t mode) {
  if (linear_shape_check(m, n, k) != WQ_OK) return 0;
  return w4_epilogue_fits(m, n, k, group_size, mode) ? 1 : 0;
}

extern "C" int wq_w4a16_linear_epilogue(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                                        int64_t n, int64_t group_size, int32_t mode, const uint16_t* residual,
                                        uint16_t* y, void* stream) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(mode == 1 || mode == 2, WQ_ERR_INVALID_ARGUMENT, "mode must be 1 (silu_mul) or 2 (residual)");
  WQ_REQUIRE(w4_epilogue_fits(m, n, k, group_size, mode), WQ_ERR_UNSUPPORTED,
             "W4A16 epilogue mode %d does not apply to m=%lld n=%lld k=%lld group=%lld "
             "(see wq_w4a16_epilogue_supported)", (int)mode, (long long)m, (long long)n, (long long)k,
             (long long)group_size);
  WQ_REQUIRE(x && y && tiles && meta && (mode == 1 || residual), WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(aligned16(x) && aligned16(tiles) && aligned16(y) && (reinterpret_cast<uintptr_t>(meta) & 7u) == 0 &&
                 (mode == 1 || (reinterpret_cast<uintptr_t>(residual) & 7u) == 0),
             WQ_ERR_INVALID_ARGUMENT, "x, tiles and y must be 16-byte aligned, meta and residual 8-byte aligned");
  return launch_w4_gemm_epi(reinterpret_cast<const half_t*>(x), (int)m, (int)k, reinterpret_cast<const uint4_t*>(tiles),
                            reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size,
                            mode, reinterpret_cast<const half_t*>(residual), reinterpret_cast<half_t*>(y),
                            as_stream(stream));
}

extern "C" int wq_w8a16_epilogue_supported(int64_t m, int64_t n, int64_t k, int32_t mode) {
  if (linear_shape_check(m, n, k) != WQ_OK) return 0;
  return w8_epilogue_fits(m, n, k, mode) ? 1 : 0;
}

extern "C" int wq_w8a16_linear_epilogue(const uint16_t* x, int64_t m, int64_t k, const void* tiles,
                                        const uint16_t* scale, int64_t n, int32_t mode, const uint16_t* residual,
                                        uint16_t* y, void* stream) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(mode == 1 || mode == 2, WQ_ERR_INVALID_ARGUMENT, "mode must be 1 (silu_mul) or 2 (residual)");
  WQ_REQUIRE(w8_epilogue_fits(m, n, k, mode), WQ_ERR_UNSUPPORTED,
             "W8A16 epilogue mode %d does not apply to m=%lld n=%lld k=%lld (see wq_w8a16_epilogue_supported)",
             (int)mode, (long long)m, (long long)n, (long long)k);
  WQ_REQUIRE(x && y && tiles && scale && (mode == 1 || residual), WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(aligned16(x) && aligned16(tiles) && aligned16(y) &&
                 (mode == 1 || (reinterpret_cast<uintptr_t>(residual) & 7u) == 0),
             WQ_ERR_INVALID_ARGUMENT, "x, tiles and y must be 16-byte aligned and residual 8-byte aligned");
  return launch_w8_gemm_epi(reinterpret_cast<const half_t*>(x), (int)m, (int)k, reinterpret_cast<const int8_t*>(tiles),
                            reinterpret_cast<const half_t*>(scale), (int)n, mode,
                            reinterpret_cast<const half_t*>(residual), reinterpret_cast<half_t*>(y),
                            as_stream(stream));
}

extern "C" int wq_w4a16_decode_fused(const uint16_t* x, int64_t k, const void* tiles, const void* meta, int64_t n,
                                     int64_t group_size, int32_t x_mode, const uint16_t* norm_weight,
                                     const float* sumsq_in, int64_t sumsq_count, float eps, const uint16_t* residual,
                                     float* sumsq_out, uint16_t* y, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (int st = linear_shape_check(1, n, k)) return st;
  WQ_REQUIRE(n % 16 == 0 && group_size % kW4BlockK == 0 && group_size > 0 && k % group_size == 0,
             WQ_ERR_UNSUPPORTED, "fused decode linear needs n %% 16 == 0, group_size %% 128 == 0, k %% group_size == 0 "
             "(n=%lld k=%lld group=%lld)", (long long)n, (long long)k, (long long)group_size);
  WQ_REQUIRE(x_mode >= 0 && x_mode <= 2, WQ_ERR_INVALID_ARGUMENT, "x_mode must be 0 (plain), 1 (rmsnorm) or 2 (silu_mul)");
  WQ_REQUIRE(x && tiles && meta && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(x_mode != 1 || (norm_weight && sumsq_in && sumsq_count > 0 && sumsq_count <= 512),
             WQ_ERR_INVALID_ARGUMENT, "rmsnorm mode needs norm_weight, sumsq_in and 0 < sumsq_count <= 512");
  WQ_REQUIRE(aligned16(x) && aligned16(tiles) && aligned16(y) && (reinterpret_cast<uintptr_t>(meta) & 7u) == 0 &&
                 aligned16(norm_weight) && aligned16(sumsq_in) && (reinterpret_cast<uintptr_t>(residual) & 7u) == 0,
             WQ_ERR_INVALID_ARGUMENT,
             "x, tiles, y, norm_weight and sumsq_in must be 16-byte aligned, meta and residual 8-byte");
  return launch_w4_gemv_fused(reinterpret_cast<const half_t*>(x), (int)k, reinterpret_cast<const uint4_t*>(tiles),
                              reinterpret_cast<const uint8_t*>(meta), (int)n, (int)group_size, x_mode,
                              reinterpret_cast<const half_t*>(norm_weight), sumsq_in, (int)sumsq_count, eps,
                              reinterpret_cast<const half_t*>(residual), sumsq_out, reinterpret_cast<half_t*>(y),
                              workspace, workspace_bytes, as_stream(stream));
}

namespace {

// INT8 weight-only entry points over either weight layout (W8Layout): the
// caller's row-major [N, K] qweight (tiled = 0) or wq_w8_repack's tiles
// (tiled = 1, which needs k % 128 == 0).
int w8a16_decode_fused_impl(const uint16_t* x, int64_t k, const int8_t* qweight, const uint16_t* scale, int64_t n,
                            int32_t x_mode, const uint16_t* norm_weight, const float* sumsq_in, int64_t sumsq_count,
                            float eps, const uint16_t* residual, float* sumsq_out, uint16_t* y, void* workspace,
                            size_t workspace_bytes, void* stream, int tiled) {
  if (int st = linear_shape_check(1, n, k)) return st;
  WQ_REQUIRE(n % 16 == 0 && k % kW8BlockK == 0, WQ_ERR_UNSUPPORTED,
             "fused decode linear needs n %% 16 == 0 and k %% 128 == 0 (n=%lld k=%lld)", (long long)n, (long long)k);
  WQ_REQUIRE(x_mode >= 0 && x_mode <= 2, WQ_ERR_INVALID_ARGUMENT, "x_mode must be 0 (plain), 1 (rmsnorm) or 2 (silu_mul)");
  WQ_REQUIRE(x && qweight && scale && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(x_mode != 1 || (norm_weight && sumsq_in && sumsq_count > 0 && sumsq_count <= 512),
             WQ_ERR_INVALID_ARGUMENT, "rmsnorm mode needs norm_weight, sumsq_in and 0 < sumsq_count <= 512");
  WQ_REQUIRE(aligned16(x) && aligned16(qweight) && aligned16(y) && aligned16(norm_weight) && aligned16(sumsq_in) &&
                 (reinterpret_cast<uintptr_t>(residual) & 7u) == 0,
             WQ_ERR_INVALID_ARGUMENT, "x, qweight, y, norm_weight and sumsq_in must be 16-byte aligned, residual 8-byte");
  return launch_w8_gemv_fused(reinterpret_cast<const half_t*>(x), (int)k, qweight,
                              reinterpret_cast<const half_t*>(scale), (int)n, x_mode,
                              reinterpret_cast<const half_t*>(norm_weight), sumsq_in, (int)sumsq_count, eps,
                              reinterpret_cast<const half_t*>(residual), sumsq_out, reinterpret_cast<half_t*>(y),
                              workspace, workspace_bytes, as_stream(stream), tiled);
}

int w8a16_linear_impl(const uint16_t* x, int64_t m, int64_t k, const int8_t* qweight, const uint16_t* scale,
                      int64_t n, const uint16_t* bias, uint16_t* y, void* workspace, size_t workspace_bytes,
                      void* stream, int tiled) {
  if (int st = linear_shape_check(m, n, k)) return st;
  WQ_REQUIRE(qweight && scale, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  WQ_REQUIRE(!tiled || (k % kW8BlockK == 0 && aligned16(qweight)), WQ_ERR_UNSUPPORTED,
             "INT8 tiles need k %% 128 == 0 and 16-byte aligned tiles (k=%lld)", (long long)k);
  if (m == 0) return WQ_OK;   // empty activations: x and y may be null
  WQ_REQUIRE(x && y, WQ_ERR_INVALID_ARGUMENT, "null pointer argument");
  const half_t* xh = reinterpret_cast<const half_t*>(x);
  const half_t* sh = reinterpret_cast<const half_t*>(scale);
  const half_t* bh = reinterpret_cast<const half_t*>(bias);
  half_t* yh = reinterpret_cast<half_t*>(y);
  if (tiled) {
    WQ_REQUIRE(aligned16(x), WQ_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
    if (m <= kSkinnyMaxM)
      return launch_w8_skinny(xh, (int)m, (int)k, qweight, sh, bh, (int)n, yh, workspace, workspace_bytes,
                              as_stream(stream), 1);
    if (k <= kGemmMaxK) return launch_w8_gemm(xh, (int)m, (int)k, qweight, sh, bh, (int)n, yh, as_stream(stream), 1);
    for (int64_t r = 0; r < m; r += kSkinnyMaxM) {   // k beyond the GEMM's offsets: 64 rows at a time
      const int64_t mr = m - r < kSkinnyMaxM ? m - r : kSkinnyMaxM;
      const int rc = launch_w8_skinny(xh + r * k, (int)mr, (int)k, qweight, sh, bh, (int)n, yh + r * n, workspace,
                                      workspace_bytes, as_stream(stream), 1);
      if (rc != WQ_OK) return rc;
    }
    return WQ_OK;
  }
  if (k % kW8BlockK != 0 || !aligned16(x) || !aligned16(qweight) || (m > kSkinnyMaxM && k > kGemmMaxK))
    return launch_w8_generic(xh, (int)m, (int)k, qweight, sh, bh, (int)n, yh, as_stream(stream));
  if (m <= kSkinnyMaxM)
    return launch_w8_skinny(xh, (int)m, (int)k, qweight, sh, bh, (int)n, yh, workspace, workspace_bytes,
                            as_stream(stream), 0);
  return launch_w8_gemm(xh, (int)m, (int)k, qweight, sh, bh, (int)n, yh, as_stream(stream), 0);
}

}  // namespace

extern "C" int wq_w8a16_decode_fused(const uint16_t* x, int64_t k, const int8_t* qweight, const uint16_t* scale,
                                     int64_t n, int32_t x_mode, const uint16_t* norm_weight, const float* sumsq_in,
                                     int64_t sumsq_count, float eps, const uint16_t* residual, float* sumsq_out,
                                     uint16_t* y, void* workspace, size_t workspace_bytes, void* stream) {
  return w8a16_decode_fused_impl(x, k, qweight, scale, n, x_mode, norm_weight, sumsq_in, sumsq_count, eps, residual,
                                 sumsq_out, y, workspace, workspace_bytes, stream, 0);
}

extern "C" int wq_w8a16_decode_fused_tiled(const uint16_t* x, int64_t k, const void* tiles, const uint16_t* scale,
                                           int64_t n, int32_t x_mode, const uint16_t* norm_weight,
                                           const float* sumsq_in, int64_t sumsq_count, float eps,
                                           const uint16_t* residual, float* sumsq_out, uint16_t* y, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  return w8a16_decode_fused_impl(x, k, reinterpret_cast<const int8_t*>(tiles), scale, n, x_mode, norm_weight,
                                 sumsq_in, sumsq_count, eps, residual, sumsq_out, y, workspace, workspace_bytes,
                                 stream, 1);
}

extern "C" int wq_w8a16_linear(const uint16_t* x, int64_t m, int64_t k, const int8_t* qweight, const uint16_t* scale,
                               int64_t n, const uint16_t* bias, uint16_t* y, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return w8a16_linear_impl(x, m, k, qweight, scale, n, bias, y, workspace, workspace_bytes, stream, 0);
}

extern "C" int wq_w8a16_linear_tiled(const uint16_t* x, int64_t m, int64_t k, const void* tiles,
                                     const uint16_t* scale, int64_t n, const uint16_t* bias, uint16_t* y,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  return w8a16_linear_impl(x, m, k, reinterpret_cast<const int8_t*>(tiles), scale, n, bias, y, workspace,
                           workspace_bytes, stream, 1);
}

// ---------------------------------------------------------------------------
// Allocation-free W4A16 linear (wq_w4a16_linear_noalloc).
//
// The k-split counters and fp32 partials of the split kernels (decode GEMV,
// small-batch kernel, deep-ring GEMM) live in this file-scope device array
// instead of a caller workspace.  Each GPU holds its own copy for the life of
// the process.  Host code never passes `scratch` itself to a kernel: the name
// is only a host-side handle, so every use goes through the device address
// that hipGetSymbolAddress returns for the current device, kept in
// g_scratch_ptr.  Every split plan fits its 16 MiB (kSplitWorkspaceMaxBytes:
// plans that would need more take fewer splits), e.g. the decode GEMV's
// largest 2.0 MiB, the deep ring's up to 16 MiB.
namespace wq {
constexpr size_t kNoAllocScratchBytes = kSplitWorkspaceMaxBytes;
}  // namespace wq

static __device__ __align__(256) uint8_t scratch[wq::kNoAllocScratchBytes];

namespace wq {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ __launch_bounds__(256) void zero_words_kernel(uint4_t* p, size_t n16) {
  for (size_t j = (size_t)blockIdx.x * blockDim.x + threadIdx.x; j < n16; j += (size_t)gridDim.x * blockDim.x)
    p[j] = uint4_t{0u, 0u, 0u, 0u};
}

// Device address of `scratch` on the current device.  The first call on a
// device looks the address up and queues a clear of the whole array on
// `stream` (the split counters must start at zero; every later call leaves
// them at zero again), ahead of the caller's kernels on that stream.  That
// set-up is refused while `stream` is being captured: the clear would be
// recorded into the caller's graph and rerun on every replay, and eager calls
// before the first replay would find the counters uncleared.  One eager call
// on the device, before capture, does the set-up.
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return WQ_ERR_HIP;
  }
  WQ_REQUIRE(dev >= 0 && dev < kMaxDevices, WQ_ERR_UNSUPPORTED, "device %d is beyond the %d this library tracks",
             dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) {
      set_error("hipStreamIsCapturing failed: %s", hipGetErrorString(e));
      return WQ_ERR_HIP;
    }
    WQ_REQUIRE(capture == hipStreamCaptureStatusNone, WQ_ERR_UNSUPPORTED,
               "wq_w4a16_linear_noalloc: the first call on device %d sets up its scratch and must not be captured; "
               "make one call outside graph capture first", dev);
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return WQ_ERR_HIP;
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, stream, reinterpret_cast<uint4_t*>(ptr),
                       kNoAllocScratchBytes / 16);
    if (int rc = check_launch("noalloc scratch clear")) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return WQ_OK;
}

}  // namespace
}  // namespace wq

extern "C" int wq_w4a16_linear_noalloc(const uint16_t* x, int64_t m, int64_t k, const void* tiles, const void* meta,
                                       int64_t n, int64_t group_size, uint16_t* y, void* stream) {
  if (int st = linear_shape_check(m, n, k)) return st;
  if (m == 0) return wq_w4a16_linear(x, m, k, tiles, meta, n, group_size, y, nullptr, 0, stream);
  // The same sizing as wq_w4a16_workspace_size: every split plan (decode
  // GEMV, small-batch kernel, deep-ring GEMM) fits kSplitWorkspaceMaxBytes,
  // so this runs the plan a caller workspace would.
  size_t need = 0;
  if (int st = wq_w4a16_workspace_size(m, n, k, group_size, &need)) return st;
  WQ_REQUIRE(need <= kNoAllocScratchBytes, WQ_ERR_WORKSPACE,
             "wq_w4a16_linear_noalloc: m=%lld n=%lld k=%lld needs %zu scratch bytes, more than the %zu it holds",
             (long long)m, (long long)n, (long long)k, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = noalloc_scratch(as_stream(stream), &ws)) return rc;
  }
  return wq_w4a16_linear(x, m, k, tiles, meta, n, group_size, y, ws, need, stream);
}
