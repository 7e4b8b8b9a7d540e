// gemm_lp.hip -- the 16-bit-input GEMM entry points (bf16 / fp16 in, fp32
// accumulation, fp32 or 16-bit out) over gemm_lp.hpp.
//
// The reference reserves DType::kF16 and kBF16 (include/mcke/core/dtype.hpp:33-41)
// for tensor-core inputs but ships only the fp32 launcher (kernels.hpp:265-269,
// gemm.cu:829-882).  mcke_launch_gemm_lp keeps that launcher's argument order,
// validation and status codes, with the two dtypes added after the pointers.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "gemm_lp.hpp"

namespace mcke_amd {
namespace {

using LpKernel = const void*;

// LDS stages of the direct-to-LDS kernel per tile (32 KiB per stage at 256 x 256).
template <int BM, int BN> struct LpDmaStages { static constexpr int value = 4; };

template <typename T, typename OutT, int BM, int BN>
struct LpTile {
  // Whole tiles with 16-byte aligned operands take a direct-to-LDS kernel (tiles
  // with BN >= 128), whose per-lane source offsets are 32-bit: BM rows of A and 32
  // rows of B must span less than 4 GiB.  K % 64 == 0 takes the 16x16x32 kernel,
  // the other multiples of 32 the 32x32x16 one.
  static bool use_dma(bool vec, int m, int n, int k) {
    if constexpr (BN < 128) {
      return false;
    } else {
      return vec && m % BM == 0 && n % BN == 0 && k % LpDmaShape<BM, BN, 4>::BK == 0 &&
             static_cast<int64_t>(BM) * k * 2 < (int64_t{1} << 32) &&
             static_cast<int64_t>(32) * n * 2 < (int64_t{1} << 32);
    }
  }
  static bool use_dma16(int k) { return k % 64 == 0; }

  static int launch(const void* a, const void* b, void* c, int m, int n, int k, float alpha,
                    float beta, bool vec, hipStream_t s) {
    const int64_t tiles_m = (static_cast<int64_t>(m) + BM - 1) / BM;
    const int64_t tiles_n = (static_cast<int64_t>(n) + BN - 1) / BN;
    if (tiles_m * tiles_n * kMfmaThreads > int64_t{UINT32_MAX})
      return invalid("launch_gemm_lp: tiles x lanes exceed the grid's 32-bit work size; use a "
                     "larger tile");
    const bool even = vec && m % BM == 0 && n % BN == 0 && k % kLpBK == 0;
    const auto* A = static_cast<const uint16_t*>(a);
    const auto* B = static_cast<const uint16_t*>(b);
    auto* C = static_cast<OutT*>(c);
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n)), block(kMfmaThreads);
    const int tmi = static_cast<int>(tiles_m), tni = static_cast<int>(tiles_n);
    if constexpr (BN >= 128) {
      if (use_dma(vec, m, n, k)) {
        if (use_dma16(k)) {
          gemm_lp_dma16_kernel<T, OutT, BM, BN>
              <<<grid, block, 0, s>>>(A, B, C, m, n, k, alpha, beta, tmi, tni);
          MCKE_LAUNCH_CHECK("gemm_lp_dma16_kernel");
        } else {
          gemm_lp_dma_kernel<T, OutT, BM, BN, LpDmaStages<BM, BN>::value>
              <<<grid, block, 0, s>>>(A, B, C, m, n, k, alpha, beta, tmi, tni);
          MCKE_LAUNCH_CHECK("gemm_lp_dma_kernel");
        }
        return ok();
      }
    }
    if (even)
      gemm_lp_kernel<T, OutT, BM, BN, true, true>
          <<<grid, block, 0, s>>>(A, B, C, m, n, k, alpha, beta, tmi, tni);
    else if (vec)
      gemm_lp_kernel<T, OutT, BM, BN, true, false>
          <<<grid, block, 0, s>>>(A, B, C, m, n, k, alpha, beta, tmi, tni);
    else
      gemm_lp_kernel<T, OutT, BM, BN, false, false>
          <<<grid, block, 0, s>>>(A, B, C, m, n, k, alpha, beta, tmi, tni);
    MCKE_LAUNCH_CHECK("gemm_lp_kernel");
    return ok();
  }
  // The instantiation whole-tile shapes run, for attribute queries.
  static LpKernel kernel() {
    using Fn = void (*)(const uint16_t*, const uint16_t*, OutT*, int, int, int, float, float, int,
                        int);
    Fn fn;
    if constexpr (BN >= 128) fn = &gemm_lp_dma16_kernel<T, OutT, BM, BN>;
    else fn = &gemm_lp_kernel<T, OutT, BM, BN, true, true>;
    return reinterpret_cast<LpKernel>(fn);
  }
};

// Instantiated tiles: (bm, bn) with bk = 64 and 256 lanes, so (tm, tn) = (bm/16, bn/16).
constexpr int kLpTiles[][2] = {{256, 256}, {128, 128}, {64, 64}};

int lp_tile_index(const mcke_gemm_tile* t) {
  if (!t) return -1;
  for (int i = 0; i < 3; ++i) {
    const int bm = kLpTiles[i][0], bn = kLpTiles[i][1];
    if (t->bm == bm && t->bn == bn && t->bk == kLpBK && t->tm == bm / 16 && t->tn == bn / 16)
      return i;
  }
  return -1;
}

template <typename T, typename OutT>
struct LpTable {
  static int launch(int ti, const void* a, const void* b, void* c, int m, int n, int k,
                    float alpha, float beta, bool vec, hipStream_t s) {
    switch (ti) {
      case 0: return LpTile<T, OutT, 256, 256>::launch(a, b, c, m, n, k, alpha, beta, vec, s);
      case 1: return LpTile<T, OutT, 128, 128>::launch(a, b, c, m, n, k, alpha, beta, vec, s);
      default: return LpTile<T, OutT, 64, 64>::launch(a, b, c, m, n, k, alpha, beta, vec, s);
    }
  }
  static LpKernel kernel(int ti) {
    switch (ti) {
      case 0: return LpTile<T, OutT, 256, 256>::kernel();
      case 1: return LpTile<T, OutT, 128, 128>::kernel();
      default: return LpTile<T, OutT, 64, 64>::kernel();
    }
  }
};

// (ab_dtype, c_dtype) -> 0..3, or -1 when the pair is not supported.
int lp_combo(int ab, int cd) {
  if (ab == MCKE_DTYPE_BF16) return cd == MCKE_DTYPE_F32 ? 0 : cd == MCKE_DTYPE_BF16 ? 1 : -1;
  if (ab == MCKE_DTYPE_F16) return cd == MCKE_DTYPE_F32 ? 2 : cd == MCKE_DTYPE_F16 ? 3 : -1;
  return -1;
}

int check_combo(const char* who, int ab, int cd, int* combo) {
  if (ab != MCKE_DTYPE_BF16 && ab != MCKE_DTYPE_F16)
    return invalid(std::string(who) + ": ab_dtype must be MCKE_DTYPE_BF16 or MCKE_DTYPE_F16, got " +
                   std::to_string(ab));
  *combo = lp_combo(ab, cd);
  if (*combo < 0)
    return invalid(std::string(who) + ": c_dtype must be MCKE_DTYPE_F32 or ab_dtype, got " +
                   std::to_string(cd));
  return ok();
}

int check_tile(const char* who, const mcke_gemm_tile* tile, int* ti) {
  *ti = lp_tile_index(tile);
  if (*ti < 0)
    return invalid(std::string(who) +
                   ": instantiated for tiles (bm,bn,bk,tm,tn) = (256,256,64,16,16), "
                   "(128,128,64,8,8) and (64,64,64,4,4); no fallback is applied");
  return ok();
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

int mcke_launch_gemm_lp(const void* a, const void* b, void* c, int ab_dtype, int c_dtype,
                        int64_t m, int64_t n, int64_t k, float alpha, float beta,
                        const mcke_gemm_tile* tile, void* stream) {
  int combo = -1, ti = -1;
  if (int rc = check_combo("launch_gemm_lp", ab_dtype, c_dtype, &combo)) return rc;
  if (int rc = check_tile("launch_gemm_lp", tile, &ti)) return rc;
  if (m == 0 || n == 0) return ok();
  if (m < 0 || n < 0 || k < 0) return invalid("launch_gemm_lp: negative extent");
  if (!a || !b || !c) return invalid("launch_gemm_lp: null pointer");
  if (a == c || b == c)
    return invalid("launch_gemm_lp: output aliases an input, which violates the "
                   "__restrict__ contract");
  if (m > 2147483647LL || n > 2147483647LL || k > 2147483647LL)
    return invalid("launch_gemm_lp: extent exceeds INT32_MAX");
  // 16-byte loads of eight elements need k % 8, n % 8 and 16-byte aligned bases;
  // the C vector stores need C 16-byte aligned as well.
  const bool vec = (k % 8 == 0) && (n % 8 == 0) && aligned(a, 16) && aligned(b, 16) &&
                   aligned(c, 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  switch (combo) {
    case 0: return LpTable<__bf16, float>::launch(ti, a, b, c, mi, ni, ki, alpha, beta, vec, s);
    case 1: return LpTable<__bf16, __bf16>::launch(ti, a, b, c, mi, ni, ki, alpha, beta, vec, s);
    case 2: return LpTable<_Float16, float>::launch(ti, a, b, c, mi, ni, ki, alpha, beta, vec, s);
    default:
      return LpTable<_Float16, _Float16>::launch(ti, a, b, c, mi, ni, ki, alpha, beta, vec, s);
  }
}

int mcke_gemm_lp_kernel_attrs(int ab_dtype, int c_dtype, const mcke_gemm_tile* tile,
                              mcke_kernel_attrs* out) {
  if (!out) return invalid("gemm_lp_kernel_attrs: null out");
  int combo = -1, ti = -1;
  if (int rc = check_combo("gemm_lp_kernel_attrs", ab_dtype, c_dtype, &combo)) return rc;
  if (int rc = check_tile("gemm_lp_kernel_attrs", tile, &ti)) return rc;
  LpKernel kern = nullptr;
  switch (combo) {
    case 0: kern = LpTable<__bf16, float>::kernel(ti); break;
    case 1: kern = LpTable<__bf16, __bf16>::kernel(ti); break;
    case 2: kern = LpTable<_Float16, float>::kernel(ti); break;
    default: kern = LpTable<_Float16, _Float16>::kernel(ti); break;
  }
  hipFuncAttributes fa{};
  MCKE_HIP_TRY(hipFuncGetAttributes(&fa, kern));
  out->regs_per_thread = fa.numRegs;
  out->agprs_per_thread = 0;
  out->static_smem_bytes = fa.sharedSizeBytes;
  out->local_bytes = fa.localSizeBytes;
  out->threads_per_block = kMfmaThreads;
  int blocks = 0;
  MCKE_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kern, kMfmaThreads, 0));
  out->max_blocks_per_sm_api = blocks;
  return ok();
}

int mcke_gemm_lp_default_tile(int64_t m, int64_t n, int64_t k, mcke_gemm_tile* out) {
  if (!out) return invalid("gemm_lp_default_tile: null out");
  (void)k;
  // The largest tile that still gives every CU of a 256-CU part a workgroup:
  // measured on MI355X, 256 x 256 wins at 4096^3 (256 tiles) and 128 x 128 at
  // 2048^3 (256 tiles), each over the next smaller tile with more rounds.
  const int64_t want = 256;
  auto tiles = [&](int64_t t) { return ((m + t - 1) / t) * ((n + t - 1) / t); };
  if (tiles(256) >= want) *out = mcke_gemm_tile{256, 256, kLpBK, 16, 16};
  else if (tiles(128) >= want) *out = mcke_gemm_tile{128, 128, kLpBK, 8, 8};
  else *out = mcke_gemm_tile{64, 64, kLpBK, 4, 4};
  return ok();
}

}  // extern "C"
