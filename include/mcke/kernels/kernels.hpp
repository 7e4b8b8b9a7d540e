// mcke/kernels/kernels.hpp -- the kernel launcher API.
//
// Same names, argument order and error behaviour as the reference's
// include/mcke/kernels/kernels.hpp:59-302; each launcher is an inline wrapper
// over the C-ABI in mcke_amd.h (libmcke_amd.so), which owns the gfx950 kernels.
// Launchers never allocate and never synchronise; work goes onto `stream`.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "mcke/core/dtype.hpp"
#include "mcke/core/status.hpp"
#include "mcke/kernels/gemm_tile.hpp"
#include "mcke/runtime/stream.hpp"
#include "mcke_amd.h"

namespace mcke::kernels {

namespace detail {
inline Status status_of(int rc) {
  if (rc == MCKE_STATUS_OK) return OkStatus();
  return Status(static_cast<StatusCode>(rc), mcke_last_error());
}
inline mcke_gemm_tile to_c(const GemmTile& t) { return mcke_gemm_tile{t.bm, t.bn, t.bk, t.tm, t.tn}; }
}  // namespace detail

[[nodiscard]] inline Status launch_vector_add_f32(const float* a, const float* b, float* out,
                                                 std::size_t n, rt::StreamHandle stream) {
  return detail::status_of(mcke_launch_vector_add_f32(a, b, out, n, stream));
}

enum class Activation : std::uint8_t { kNone, kRelu, kGeluErf, kGeluTanh };

[[nodiscard]] inline Status launch_bias_act_f32(const float* x, const float* bias, float* y,
                                               std::int64_t rows, std::int64_t cols,
                                               Activation act, int vector_width,
                                               rt::StreamHandle stream, int max_row_blocks = 0) {
  return detail::status_of(mcke_launch_bias_act_f32(x, bias, y, rows, cols, static_cast<int>(act),
                                                    vector_width, stream, max_row_blocks));
}

[[nodiscard]] inline Status launch_bias_add_f32(const float* x, const float* bias, float* y,
                                               std::int64_t rows, std::int64_t cols,
                                               int vector_width, rt::StreamHandle stream) {
  return detail::status_of(mcke_launch_bias_add_f32(x, bias, y, rows, cols, vector_width, stream));
}

[[nodiscard]] inline Status launch_activation_f32(const float* x, float* y, std::int64_t n,
                                                 Activation act, int vector_width,
                                                 rt::StreamHandle stream) {
  return detail::status_of(
      mcke_launch_activation_f32(x, y, n, static_cast<int>(act), vector_width, stream));
}

// Largest width in {4, 2, 1} legal for this pointer and column count.
[[nodiscard]] inline int max_vector_width_f32(const void* p, std::int64_t cols) noexcept {
  const auto addr = reinterpret_cast<std::uintptr_t>(p);
  for (int w = 4; w > 1; w >>= 1)
    if (cols % w == 0 && addr % (sizeof(float) * static_cast<std::size_t>(w)) == 0) return w;
  return 1;
}

enum class ReduceKind : std::uint8_t { kSum, kMax, kMean };
enum class ReduceVariant : std::uint8_t { kSmemTree, kWarpShuffle, kTwoPass };

[[nodiscard]] inline std::size_t row_reduce_workspace_bytes(std::int64_t rows, std::int64_t cols,
                                                           ReduceVariant variant) noexcept {
  return mcke_row_reduce_workspace_bytes(rows, cols, static_cast<int>(variant));
}

[[nodiscard]] inline Status launch_row_reduce_f32(const float* x, float* out, std::int64_t rows,
                                                 std::int64_t cols, ReduceKind kind,
                                                 ReduceVariant variant, rt::StreamHandle stream) {
  return detail::status_of(mcke_launch_row_reduce_f32(x, out, rows, cols, static_cast<int>(kind),
                                                      static_cast<int>(variant), stream));
}

[[nodiscard]] inline Status launch_row_reduce_f32(const float* x, float* out, std::int64_t rows,
                                                 std::int64_t cols, ReduceKind kind,
                                                 ReduceVariant variant, float* workspace,
                                                 std::size_t workspace_bytes,
                                                 rt::StreamHandle stream) {
  return detail::status_of(mcke_launch_row_reduce_ws_f32(
      x, out, rows, cols, static_cast<int>(kind), static_cast<int>(variant), workspace,
      workspace_bytes, stream));
}

enum class SoftmaxVariant : std::uint8_t { kThreePass, kOnlineOnePass };

[[nodiscard]] inline Status launch_row_softmax_f32(const float* x, float* y, std::int64_t rows,
                                                  std::int64_t cols, SoftmaxVariant variant,
                                                  rt::StreamHandle stream) {
  return detail::status_of(
      mcke_launch_row_softmax_f32(x, y, rows, cols, static_cast<int>(variant), stream));
}

[[nodiscard]] inline Status launch_gemm_f32(const float* a, const float* b, float* c,
                                           std::int64_t m, std::int64_t n, std::int64_t k,
                                           float alpha, float beta, GemmVariant variant,
                                           GemmTile tile, rt::StreamHandle stream) {
  const mcke_gemm_tile t = detail::to_c(tile);
  return detail::status_of(mcke_launch_gemm_f32(a, b, c, m, n, k, alpha, beta,
                                                static_cast<int>(variant), &t, stream));
}

// No reference counterpart: launch_gemm_f32 (kMfmaF32, beta = 0) and
// launch_bias_act_f32 in one launch, y = act(alpha * A B + bias[col]), with the
// bits of the two launches in sequence (mcke_launch_gemm_bias_act_f32).
[[nodiscard]] inline Status launch_gemm_bias_act_f32(const float* a, const float* b,
                                                    const float* bias, float* y, std::int64_t m,
                                                    std::int64_t n, std::int64_t k, float alpha,
                                                    Activation act, GemmTile tile,
                                                    rt::StreamHandle stream) {
  const mcke_gemm_tile t = detail::to_c(tile);
  return detail::status_of(mcke_launch_gemm_bias_act_f32(a, b, bias, y, m, n, k, alpha,
                                                         static_cast<int>(act), &t, stream));
}

struct GemmKernelAttrs {
  int regs_per_thread = 0;
  std::size_t static_smem_bytes = 0;
  std::size_t local_bytes = 0;
  int threads_per_block = 0;
  int max_blocks_per_sm_api = 0;
};

[[nodiscard]] inline StatusOr<GemmKernelAttrs> gemm_kernel_attrs(GemmVariant variant, GemmTile tile) {
  const mcke_gemm_tile t = detail::to_c(tile);
  mcke_kernel_attrs a{};
  MCKE_RETURN_IF_ERROR(detail::status_of(mcke_gemm_kernel_attrs(static_cast<int>(variant), &t, &a)));
  GemmKernelAttrs out;
  out.regs_per_thread = a.regs_per_thread;
  out.static_smem_bytes = a.static_smem_bytes;
  out.local_bytes = a.local_bytes;
  out.threads_per_block = a.threads_per_block;
  out.max_blocks_per_sm_api = a.max_blocks_per_sm_api;
  return out;
}

// No reference counterpart: the MFMA tile this build picks for a shape.
[[nodiscard]] inline GemmTile mfma_default_tile(std::int64_t m, std::int64_t n, std::int64_t k) {
  mcke_gemm_tile t{};
  (void)mcke_gemm_mfma_default_tile(m, n, k, &t);
  return GemmTile{t.bm, t.bn, t.bk, t.tm, t.tn};
}

// ---------------------------------------------------------------------------
// 16-bit-input GEMM.  No reference counterpart: the reference reserves
// DType::kF16 / kBF16 (dtype.hpp:33-41) but launches fp32 only.  A and B hold
// `ab` values (kBF16 or kF16), products accumulate in fp32, C holds `c` values
// (kF32 or `ab`).  Argument order, validation and status codes follow
// launch_gemm_f32.
// ---------------------------------------------------------------------------
[[nodiscard]] inline Status launch_gemm_lp(const void* a, const void* b, void* c, DType ab, DType cd,
                                          std::int64_t m, std::int64_t n, std::int64_t k,
                                          float alpha, float beta, GemmTile tile,
                                          rt::StreamHandle stream) {
  const mcke_gemm_tile t = detail::to_c(tile);
  return detail::status_of(mcke_launch_gemm_lp(a, b, c, static_cast<int>(ab), static_cast<int>(cd),
                                               m, n, k, alpha, beta, &t, stream));
}

// The 16-bit GEMM tile this build picks for a shape.
[[nodiscard]] inline GemmTile lp_default_tile(std::int64_t m, std::int64_t n, std::int64_t k) {
  mcke_gemm_tile t{};
  (void)mcke_gemm_lp_default_tile(m, n, k, &t);
  return GemmTile{t.bm, t.bn, t.bk, t.tm, t.tn};
}

// Whether the 16-bit GEMM is instantiated for a tile: (256,256,64,16,16),
// (128,128,64,8,8) or (64,64,64,4,4).
[[nodiscard]] constexpr bool gemm_lp_tile_is_supported(const GemmTile& t) {
  return t.bk == 64 && t.bm == t.bn && (t.bm == 256 || t.bm == 128 || t.bm == 64) &&
         t.tm == t.bm / 16 && t.tn == t.bn / 16;
}

}  // namespace mcke::kernels
