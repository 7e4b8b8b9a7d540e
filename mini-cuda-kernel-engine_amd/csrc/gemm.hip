// gemm.hip -- launch_gemm_f32 and gemm_kernel_attrs for every GemmVariant.
//
// Replaces kernels/gemm.cu (launcher gemm.cu:829-882, dispatch table :595-700,
// attribute query :884-904).  The fast path is the appended kMfmaF32 variant
// (gemm_mfma.hpp).  The reference's FMA ladder is kept so that every variant a
// caller may name still runs and stays correct, re-shaped for wave64:
//   kNaive / kNaiveUncoalesced  one lane per output; 64 x 4 workgroups with lane x
//                               on the C column (coalesced) or on the C row;
//   kTiledSmem                  32 x 32 x 32 LDS tiles, one output per lane
//                               (tile (32,32,32,1,1), 1024 lanes);
//   kTiledRegBlock, kWarpTile,  128 x 128 block tile, BK = 8, 8 x 8 outputs per
//   kWarpTileNoDbuf,            lane, A staged transposed in LDS; the variants
//   kWarpTileVec4               differ in lane map (row-major vs 8 x 8 per wave64),
//                               LDS double buffering, and 16-byte global loads;
//   kCublasRef                  the vendor-library ceiling row (rocBLAS).
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"
#include "device_math.hpp"
#include "gemm_mfma.hpp"

namespace mcke_amd {
namespace {

// ---------------------------------------------------------------------------
// Ladder kernels (CUDA-core-style FMA paths)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_c(float* c, float acc, float alpha, float beta) {
  *c = (beta == 0.0f) ? alpha * acc : alpha * acc + beta * *c;
}

template <bool COALESCED>
__global__ __launch_bounds__(256) void gemm_naive_kernel(const float* __restrict__ a,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ c, int m, int n,
                                                         int k, float alpha, float beta) {
  const int col = COALESCED ? blockIdx.x * 64 + threadIdx.x : blockIdx.x * 4 + threadIdx.y;
  const int row = COALESCED ? blockIdx.y * 4 + threadIdx.y : blockIdx.y * 64 + threadIdx.x;
  if (row >= m || col >= n) return;
  float acc = 0.0f;
  for (int p = 0; p < k; ++p)
    acc += a[static_cast<int64_t>(row) * k + p] * b[static_cast<int64_t>(p) * n + col];
  store_c(c + static_cast<int64_t>(row) * n + col, acc, alpha, beta);
}

__global__ __launch_bounds__(1024) void gemm_tiled_smem_kernel(const float* __restrict__ a,
                                                               const float* __restrict__ b,
                                                               float* __restrict__ c, int m,
                                                               int n, int k, float alpha,
                                                               float beta) {
  constexpr int T = 32;
  __shared__ float As[T][T + 1];
  __shared__ float Bs[T][T];
  const int tx = threadIdx.x, ty = threadIdx.y;
  const int row = blockIdx.y * T + ty, col = blockIdx.x * T + tx;
  float acc = 0.0f;
  for (int k0 = 0; k0 < k; k0 += T) {
    As[ty][tx] = (row < m && k0 + tx < k) ? a[static_cast<int64_t>(row) * k + k0 + tx] : 0.0f;
    Bs[ty][tx] = (k0 + ty < k && col < n) ? b[static_cast<int64_t>(k0 + ty) * n + col] : 0.0f;
    __syncthreads();
#pragma unroll
    for (int p = 0; p < T; ++p) acc += As[ty][p] * Bs[p][tx];
    __syncthreads();
  }
  if (row < m && col < n) store_c(c + static_cast<int64_t>(row) * n + col, acc, alpha, beta);
}

// Register-blocked 128x128x8, 8x8 per lane, 256 lanes.
// LANE_MAP 0: lane t -> (ty, tx) = (t / 16, t % 16), row-major over the 16x16 grid.
// LANE_MAP 1: each wave64 owns an 8x8 patch of the lane grid (64 x 64 outputs), so a
//             wave reads 8 distinct A and 8 distinct B fragments from LDS per k.
template <int LANE_MAP, bool DBUF, int VW>
__global__ __launch_bounds__(256) void gemm_regblock_kernel(const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            float* __restrict__ c, int m,
                                                            int n, int k, float alpha,
                                                            float beta) {
  constexpr int BM = 128, BN = 128, BK = 8, TM = 8, TN = 8;
  constexpr int APAD = 4;
  constexpr int NBUF = DBUF ? 2 : 1;
  __shared__ __attribute__((aligned(16))) float As[NBUF][BK][BM + APAD];
  __shared__ __attribute__((aligned(16))) float Bs[NBUF][BK][BN];

  const int t = threadIdx.x;
  int ty, tx;
  if (LANE_MAP == 0) {
    ty = t / 16;
    tx = t % 16;
  } else {
    const int w = t / 64, l = t % 64;
    ty = (w / 2) * 8 + l / 8;
    tx = (w % 2) * 8 + l % 8;
  }
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  // Global -> LDS mapping: A tile 128 x 8 (1024 floats), B tile 8 x 128 (1024 floats);
  // four floats per lane each, as one float4 (VW == 4) or four scalars.
  const int a_row = t / 2, a_col = (t % 2) * 4;      // A: 2 lanes per row of 8
  const int b_row = t / 32, b_col = (t % 32) * 4;    // B: 32 lanes per row of 128

  float ra[4], rb[4];
  auto gload = [&](int k0) {
    const int gm = m0 + a_row;
    if (VW == 4) {
      f32x4 va{0.f, 0.f, 0.f, 0.f}, vb{0.f, 0.f, 0.f, 0.f};
      if (gm < m && k0 + a_col < k)
        va = *reinterpret_cast<const f32x4*>(a + static_cast<int64_t>(gm) * k + k0 + a_col);
      if (k0 + b_row < k && n0 + b_col < n)
        vb = *reinterpret_cast<const f32x4*>(b + static_cast<int64_t>(k0 + b_row) * n + n0 + b_col);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ra[i] = va[i];
        rb[i] = vb[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gk = k0 + a_col + i;
        ra[i] = (gm < m && gk < k) ? a[static_cast<int64_t>(gm) * k + gk] : 0.0f;
        const int gn = n0 + b_col + i;
        rb[i] = (k0 + b_row < k && gn < n) ? b[static_cast<int64_t>(k0 + b_row) * n + gn] : 0.0f;
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) As[buf][a_col + i][a_row] = ra[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) Bs[buf][b_row][b_col + i] = rb[i];
  };

  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int p = 0; p < BK; ++p) {
      float av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = As[buf][p][ty * TM + i];
#pragma unroll
      for (int j = 0; j < TN; ++j) bv[j] = Bs[buf][p][tx * TN + j];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += av[i] * bv[j];
    }
  };

  const int ktiles = (k + BK - 1) / BK;
  if (DBUF) {
    if (ktiles > 0) {
      gload(0);
      sstore(0);
    }
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < ktiles;
      if (more) gload((kt + 1) * BK);
      compute(cur);
      if (more) sstore(cur ^ 1);
      __syncthreads();
    }
  } else {
    for (int kt = 0; kt < ktiles; ++kt) {
      gload(kt * BK);
      sstore(0);
      __syncthreads();
      compute(0);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + ty * TM + i;
    if (row >= m) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + tx * TN + j;
      if (col < n) store_c(c + static_cast<int64_t>(row) * n + col, acc[i][j], alpha, beta);
    }
  }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------
bool tile_eq(const mcke_gemm_tile& t, int bm, int bn, int bk, int tm, int tn) {
  return t.bm == bm && t.bn == bn && t.bk == bk && t.tm == tm && t.tn == tn;
}

// gemm_tile.hpp:112-124 with a 64-lane wavefront.
bool tile_self_consistent(const mcke_gemm_tile& t) {
  if (t.bm <= 0 || t.bn <= 0 || t.bk <= 0 || t.tm <= 0 || t.tn <= 0) return false;
  if (t.bm % t.tm != 0 || t.bn % t.tn != 0) return false;
  const int threads = (t.bm / t.tm) * (t.bn / t.tn);
  if (threads <= 0 || threads > 1024) return false;
  if (threads % kWave != 0) return false;
  if ((t.bm * t.bk) % threads != 0) return false;
  if ((t.bk * t.bn) % threads != 0) return false;
  return true;
}

// CUs of the current device (cached per device); 256, the gfx950 part's count,
// when no device can be queried (a CPU-only host asking for a tile).
int64_t device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cached;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (static_cast<int>(cached.size()) <= dev) cached.resize(dev + 1, 0);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    cached[dev] = cus;
  }
  return cached[dev];
}

using GemmFn = void (*)(const float*, const float*, float*, int, int, int, float, float);
using MfmaFn = void (*)(const float*, const float*, float*, int, int, int, float, float, int,
                        int, EpiArgs);

// MFMA instantiations: (bm, bn, bk) with tm = bm/16, tn = bn/16 (256 lanes).
// `even`: 16-byte path for M, N, K multiples of the tile (no bounds checks);
// `vec`: 16-byte path with bounds checks; `scalar`: any shape and alignment.
struct MfmaCfg {
  int bm, bn, bk;
  MfmaFn even, vec, scalar;
  int even_threads;   // block size of `even` (the staged kernels use 256)
  // `even` is the direct-to-LDS kernel, whose per-lane source offsets are 32-bit
  // byte offsets within a tile's BM rows of A and 32 rows of B.
  bool even_dma = false;
  // The same three kernels with the fused bias + activation epilogue.
  MfmaFn even_f = nullptr, vec_f = nullptr, scalar_f = nullptr;
};

#define MCKE_MFMA_CFG(BM, BN, BK)                                                     \
  {BM, BN, BK, &gemm_mfma_kernel<BM, BN, BK, true, true>,                            \
   &gemm_mfma_kernel<BM, BN, BK, true, false>, &gemm_mfma_kernel<BM, BN, BK, false, false>, \
   kMfmaThreads, false, &gemm_mfma_kernel<BM, BN, BK, true, true, true>,             \
   &gemm_mfma_kernel<BM, BN, BK, true, false, true>,                                  \
   &gemm_mfma_kernel<BM, BN, BK, false, false, true>}
// BK = 32 whole tiles take the direct-to-LDS kernel (ST stages, KS wave groups
// splitting each stage's K range).
#define MCKE_MFMA_CFG_DMA(BM, BN, ST, KS)                                             \
  {BM, BN, 32, &gemm_mfma_dma_kernel<BM, BN, ST, KS>,                                \
   &gemm_mfma_kernel<BM, BN, 32, true, false>, &gemm_mfma_kernel<BM, BN, 32, false, false>, \
   kDmaThreads<BM, BN, KS>, true, &gemm_mfma_dma_kernel<BM, BN, ST, KS, true>,        \
   &gemm_mfma_kernel<BM, BN, 32, true, false, true>,                                  \
   &gemm_mfma_kernel<BM, BN, 32, false, false, true>}

// 64 x 64 tiles serve small problems, whose single round of tiles leaves one
// workgroup per CU.  Their direct-to-LDS kernel meets at its barrier in the
// middle of a K step and keeps the fragment reads one sub-step ahead across it,
// so one wave group of 4 waves and a 4-stage ring measured best (1024^3: 109-110
// TFLOP/s vs 106-107 with two wave groups and 99-106 with the earlier 8-stage
// two-group ring; 2048^3 with 64 x 64 tiles: 134-135 vs 131; 3072^3: 136.5 vs
// 134; 3, 5, 6 and 8 stages all measured slower).  For 128 x 128 a 4-stage ring
// bought nothing over 2 at 2048^3 (137-139 either way).  32 x 32 tiles (one wave
// wide, four groups) give the smallest problems four times the workgroups of
// 64 x 64: 40.0 vs 22.6 TFLOP/s at 512^3, 7.0 vs 4.5 at 256^3.
const MfmaCfg kMfmaCfgs[] = {
    MCKE_MFMA_CFG_DMA(256, 256, 2, 1), MCKE_MFMA_CFG(256, 256, 16),
    MCKE_MFMA_CFG_DMA(128, 128, 2, 1), MCKE_MFMA_CFG(128, 128, 16),
    MCKE_MFMA_CFG_DMA(64, 64, 4, 1), MCKE_MFMA_CFG_DMA(32, 32, 4, 4),
};
#undef MCKE_MFMA_CFG
#undef MCKE_MFMA_CFG_DMA

const MfmaCfg* find_mfma(const mcke_gemm_tile& t) {
  for (const MfmaCfg& c : kMfmaCfgs)
    if (tile_eq(t, c.bm, c.bn, c.bk, c.bm / 16, c.bn / 16)) return &c;
  return nullptr;
}

struct Spec {
  const void* kernel = nullptr;   // for attribute queries
  GemmFn fn = nullptr;
  MfmaFn mfma = nullptr;
  MfmaFn mfma_even = nullptr;     // unchecked 16-byte variant for whole tiles
  MfmaFn mfma_f = nullptr;        // the two with the fused bias + activation epilogue
  MfmaFn mfma_even_f = nullptr;
  int even_threads = 0;           // their block size
  bool even_dma = false;          // they take 32-bit per-lane source offsets
  dim3 block{1, 1, 1};
  int threads = 0;                // block size of `kernel`
  int tile_m = 0, tile_n = 0, tile_k = 0;
};

int gemm_spec(int variant, const mcke_gemm_tile* tile, bool vec4, Spec& s) {
  switch (variant) {
    case MCKE_GEMM_NAIVE:
      s.fn = &gemm_naive_kernel<true>;
      s.block = dim3(64, 4, 1);
      s.threads = 256;
      s.tile_m = 4;
      s.tile_n = 64;
      break;
    case MCKE_GEMM_NAIVE_UNCOALESCED:
      s.fn = &gemm_naive_kernel<false>;
      s.block = dim3(64, 4, 1);
      s.threads = 256;
      s.tile_m = 64;
      s.tile_n = 4;
      break;
    case MCKE_GEMM_TILED_SMEM:
      if (!tile || !tile_self_consistent(*tile))
        return invalid("launch_gemm_f32: tile is not self-consistent");
      if (!tile_eq(*tile, 32, 32, 32, 1, 1))
        return invalid("launch_gemm_f32: kTiledSmem is only instantiated for tile "
                       "(bm,bn,bk,tm,tn) = (32,32,32,1,1); no fallback is applied");
      s.fn = &gemm_tiled_smem_kernel;
      s.block = dim3(32, 32, 1);
      s.threads = 1024;
      s.tile_m = s.tile_n = 32;
      break;
    case MCKE_GEMM_TILED_REGBLOCK:
    case MCKE_GEMM_WARP_TILE:
    case MCKE_GEMM_WARP_TILE_NODBUF:
    case MCKE_GEMM_WARP_TILE_VEC4:
      if (!tile || !tile_self_consistent(*tile))
        return invalid("launch_gemm_f32: tile is not self-consistent");
      if (!tile_eq(*tile, 128, 128, 8, 8, 8))
        return invalid("launch_gemm_f32: the register-blocked variants are only instantiated "
                       "for tile (bm,bn,bk,tm,tn) = (128,128,8,8,8); no fallback is applied");
      if (variant == MCKE_GEMM_TILED_REGBLOCK) s.fn = &gemm_regblock_kernel<0, false, 1>;
      else if (variant == MCKE_GEMM_WARP_TILE_NODBUF) s.fn = &gemm_regblock_kernel<1, false, 1>;
      else if (variant == MCKE_GEMM_WARP_TILE) s.fn = &gemm_regblock_kernel<1, true, 1>;
      else s.fn = vec4 ? &gemm_regblock_kernel<1, true, 4> : &gemm_regblock_kernel<1, true, 1>;
      s.block = dim3(256, 1, 1);
      s.threads = 256;
      s.tile_m = s.tile_n = 128;
      break;
    case MCKE_GEMM_MFMA_F32: {
      if (!tile || !tile_self_consistent(*tile))
        return invalid("launch_gemm_f32: tile is not self-consistent");
      const MfmaCfg* cfg = find_mfma(*tile);
      if (!cfg)
        return invalid("launch_gemm_f32: kMfmaF32 is instantiated for tiles (256,256,32,16,16), "
                       "(256,256,16,16,16), (128,128,32,8,8), (128,128,16,8,8), "
                       "(64,64,32,4,4) and (32,32,32,2,2); no fallback is applied");
      s.mfma = vec4 ? cfg->vec : cfg->scalar;
      s.mfma_even = vec4 ? cfg->even : nullptr;
      s.mfma_f = vec4 ? cfg->vec_f : cfg->scalar_f;
      s.mfma_even_f = vec4 ? cfg->even_f : nullptr;
      s.even_threads = cfg->even_threads;
      s.even_dma = cfg->even_dma;
      s.tile_k = cfg->bk;
      s.block = dim3(kMfmaThreads, 1, 1);
      s.threads = s.mfma_even ? cfg->even_threads : kMfmaThreads;
      s.tile_m = cfg->bm;
      s.tile_n = cfg->bn;
      break;
    }
    case MCKE_GEMM_CUBLAS_REF:
      return invalid("gemm_spec: the library ceiling row has no kernel of this library");
    default:
      return invalid("launch_gemm_f32: unknown GemmVariant " + std::to_string(variant));
  }
  // Attribute queries report the instantiation that whole-tile shapes run.
  s.kernel = s.fn ? reinterpret_cast<const void*>(s.fn)
                  : reinterpret_cast<const void*>(s.mfma_even ? s.mfma_even : s.mfma);
  return ok();
}

// ---------------------------------------------------------------------------
// kCublasRef: rocBLAS sgemm as the ceiling row.  Row-major C = A B is the
// column-major C^T = B^T A^T, i.e. a no-transpose sgemm with the operands swapped.
// One handle per stream, created on first use and kept for the process lifetime.
// ---------------------------------------------------------------------------
int rocblas_for_stream(hipStream_t s, rocblas_handle* out) {
  static std::mutex mu;
  static std::vector<std::pair<hipStream_t, rocblas_handle>> cache;
  std::lock_guard<std::mutex> lk(mu);
  for (const auto& kv : cache)
    if (kv.first == s) {
      *out = kv.second;
      return ok();
    }
  rocblas_handle h = nullptr;
  if (rocblas_create_handle(&h) != rocblas_status_success)
    return fail(MCKE_STATUS_DEVICE_ERROR, "rocblas_create_handle failed");
  if (rocblas_set_stream(h, s) != rocblas_status_success)
    return fail(MCKE_STATUS_DEVICE_ERROR, "rocblas_set_stream failed");
  cache.emplace_back(s, h);
  *out = h;
  return ok();
}

int launch_rocblas(const float* a, const float* b, float* c, int m, int n, int k, float alpha,
                   float beta, hipStream_t s) {
  rocblas_handle h = nullptr;
  if (int rc = rocblas_for_stream(s, &h)) return rc;
  const rocblas_status st = rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none,
                                          n, m, k, &alpha, b, n, a, k, &beta, c, n);
  if (st != rocblas_status_success)
    return fail(MCKE_STATUS_DEVICE_ERROR,
                std::string("rocblas_sgemm failed: ") + rocblas_status_to_string(st));
  return ok();
}

// One kMfmaF32 launch: whole tiles take the direct-to-LDS kernel, other shapes the
// staged one; `fused` picks the instantiations with the bias + activation
// epilogue, which route shapes exactly as the plain ones do (so a fused launch
// accumulates in the plain launch's order).
int launch_mfma(const char* who, const Spec& sp, bool fused, const float* a, const float* b,
                float* c, int64_t m, int64_t n, int64_t k, float alpha, float beta, EpiArgs epi,
                hipStream_t s) {
  const int64_t tiles_m = (m + sp.tile_m - 1) / sp.tile_m;
  const int64_t tiles_n = (n + sp.tile_n - 1) / sp.tile_n;
  if (tiles_m * tiles_n > 2147483647LL)
    return invalid(std::string(who) + ": too many tiles for one launch");
  const bool whole = sp.mfma_even && m % sp.tile_m == 0 && n % sp.tile_n == 0 &&
                     k % sp.tile_k == 0 &&
                     (!sp.even_dma || (static_cast<int64_t>(sp.tile_m) * k < (int64_t{1} << 30) &&
                                       static_cast<int64_t>(32) * n < (int64_t{1} << 30)));
  MfmaFn fn = whole ? (fused ? sp.mfma_even_f : sp.mfma_even) : (fused ? sp.mfma_f : sp.mfma);
  const dim3 block = whole ? dim3(static_cast<unsigned>(sp.even_threads), 1, 1) : sp.block;
  if (tiles_m * tiles_n * static_cast<int64_t>(block.x) > int64_t{UINT32_MAX})
    return invalid(std::string(who) + ": tiles x lanes exceed the grid's 32-bit work size; use a "
                   "larger tile");
  fn<<<static_cast<unsigned>(tiles_m * tiles_n), block, 0, s>>>(
      a, b, c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), alpha, beta,
      static_cast<int>(tiles_m), static_cast<int>(tiles_n), epi);
  MCKE_LAUNCH_CHECK(fused ? "gemm_mfma_kernel (bias + activation)" : "gemm_mfma_kernel");
  return ok();
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

int mcke_launch_gemm_f32(const float* a, const float* b, float* c, int64_t m, int64_t n,
                         int64_t k, float alpha, float beta, int variant,
                         const mcke_gemm_tile* tile, void* stream) {
  if (m == 0 || n == 0) return ok();
  if (m < 0 || n < 0 || k < 0) return invalid("launch_gemm_f32: negative extent");
  if (!a || !b || !c) return invalid("launch_gemm_f32: null pointer");
  if (a == c || b == c)
    return invalid("launch_gemm_f32: output aliases an input, which violates the "
                   "__restrict__ contract");
  if (m > 2147483647LL || n > 2147483647LL || k > 2147483647LL)
    return invalid("launch_gemm_f32: extent exceeds INT32_MAX");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);

  if (variant == MCKE_GEMM_CUBLAS_REF) return launch_rocblas(a, b, c, mi, ni, ki, alpha, beta, s);

  // 16-byte loads need every row start of A and B aligned: k % 4, n % 4 and the
  // base pointers (m is unconstrained).
  const bool vec4 = (k % 4 == 0) && (n % 4 == 0) && aligned(a, 16) && aligned(b, 16) &&
                    aligned(c, 16);
  Spec sp;
  if (int rc = gemm_spec(variant, tile, vec4, sp)) return rc;

  if (sp.mfma)
    return launch_mfma("launch_gemm_f32", sp, false, a, b, c, m, n, k, alpha, beta,
                       EpiArgs{nullptr, 0}, s);

  // grid.x walks C column tiles and grid.y C row tiles for every ladder kernel
  // (kNaiveUncoalesced only changes which lane index runs along a row).
  const int64_t gx = (n + sp.tile_n - 1) / sp.tile_n;
  const int64_t gy = (m + sp.tile_m - 1) / sp.tile_m;
  if (gy > 65535) return invalid("launch_gemm_f32: m too large for the grid's y limit");
  if (gx * static_cast<int64_t>(sp.block.x) > int64_t{UINT32_MAX})
    return invalid("launch_gemm_f32: n too large for the grid's 32-bit work size");
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), 1);
  sp.fn<<<grid, sp.block, 0, s>>>(a, b, c, mi, ni, ki, alpha, beta);
  MCKE_LAUNCH_CHECK("gemm kernel");
  return ok();
}

int mcke_launch_gemm_bias_act_f32(const float* a, const float* b, const float* bias, float* y,
                                  int64_t m, int64_t n, int64_t k, float alpha, int activation,
                                  const mcke_gemm_tile* tile, void* stream) {
  if (m == 0 || n == 0) return ok();
  if (m < 0 || n < 0 || k < 0) return invalid("launch_gemm_bias_act_f32: negative extent");
  if (!a || !b || !bias || !y) return invalid("launch_gemm_bias_act_f32: null pointer");
  if (y == a || y == b || y == bias)
    return invalid("launch_gemm_bias_act_f32: the output aliases an input, which violates the "
                   "__restrict__ contract");
  if (activation < MCKE_ACT_NONE || activation > MCKE_ACT_GELU_TANH)
    return invalid("launch_gemm_bias_act_f32: unknown Activation " + std::to_string(activation));
  if (m > 2147483647LL || n > 2147483647LL || k > 2147483647LL)
    return invalid("launch_gemm_bias_act_f32: extent exceeds INT32_MAX");
  const bool vec4 = (k % 4 == 0) && (n % 4 == 0) && aligned(a, 16) && aligned(b, 16) &&
                    aligned(y, 16);
  Spec sp;
  if (int rc = gemm_spec(MCKE_GEMM_MFMA_F32, tile, vec4, sp)) return rc;
  return launch_mfma("launch_gemm_bias_act_f32", sp, true, a, b, y, m, n, k, alpha, 0.0f,
                     EpiArgs{bias, activation}, static_cast<hipStream_t>(stream));
}

int mcke_gemm_kernel_attrs(int variant, const mcke_gemm_tile* tile, mcke_kernel_attrs* out) {
  if (!out) return invalid("gemm_kernel_attrs: null out");
  if (variant == MCKE_GEMM_CUBLAS_REF)
    return fail(MCKE_STATUS_UNIMPLEMENTED,
                "gemm_kernel_attrs: the library ceiling row's kernels are not ours to introspect");
  Spec sp;
  if (int rc = gemm_spec(variant, tile, true, sp)) return rc;
  hipFuncAttributes fa{};
  MCKE_HIP_TRY(hipFuncGetAttributes(&fa, sp.kernel));
  out->regs_per_thread = fa.numRegs;
  out->agprs_per_thread = 0;   // not reported by the HIP runtime
  out->static_smem_bytes = fa.sharedSizeBytes;
  out->local_bytes = fa.localSizeBytes;
  out->threads_per_block = sp.threads;
  int blocks = 0;
  MCKE_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, sp.kernel, sp.threads, 0));
  out->max_blocks_per_sm_api = blocks;
  return ok();
}

int mcke_launch_gemm_lp_vendor(const void* a, const void* b, void* c, int ab_dtype,
                               int c_dtype, int64_t m, int64_t n, int64_t k, float alpha,
                               float beta, void* stream) {
  if ((ab_dtype != MCKE_DTYPE_BF16 && ab_dtype != MCKE_DTYPE_F16) ||
      (c_dtype != MCKE_DTYPE_F32 && c_dtype != ab_dtype))
    return invalid("launch_gemm_lp_vendor: (ab_dtype, c_dtype) must be (BF16|F16, F32|ab_dtype)");
  if (m == 0 || n == 0) return ok();
  if (m < 0 || n < 0 || k < 0) return invalid("launch_gemm_lp_vendor: negative extent");
  if (!a || !b || !c) return invalid("launch_gemm_lp_vendor: null pointer");
  if (a == c || b == c) return invalid("launch_gemm_lp_vendor: output aliases an input");
  if (m > 2147483647LL || n > 2147483647LL || k > 2147483647LL)
    return invalid("launch_gemm_lp_vendor: extent exceeds INT32_MAX");
  rocblas_handle h = nullptr;
  if (int rc = rocblas_for_stream(static_cast<hipStream_t>(stream), &h)) return rc;
  const rocblas_datatype ab =
      ab_dtype == MCKE_DTYPE_BF16 ? rocblas_datatype_bf16_r : rocblas_datatype_f16_r;
  const rocblas_datatype cd = c_dtype == MCKE_DTYPE_F32 ? rocblas_datatype_f32_r : ab;
  const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
  // Row-major C = A B is the column-major C^T = B^T A^T: operands swapped.
  const rocblas_status st = rocblas_gemm_ex(
      h, rocblas_operation_none, rocblas_operation_none, ni, mi, ki, &alpha, b, ab, ni, a, ab, ki,
      &beta, c, cd, ni, c, cd, ni, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MCKE_STATUS_DEVICE_ERROR,
                std::string("rocblas_gemm_ex failed: ") + rocblas_status_to_string(st));
  return ok();
}

int mcke_gemm_mfma_default_tile(int64_t m, int64_t n, int64_t k, mcke_gemm_tile* out) {
  if (!out) return invalid("gemm_mfma_default_tile: null out");
  (void)k;
  // What decides is how evenly a tile size fills whole rounds of CUs: a launch
  // takes as long as its busiest CU, so a partial last round costs a full one.
  // Each candidate is scored by its sustained rate with every CU busy, times the
  // share of its rounds' tile area that is useful work (m*n over rounds * CUs *
  // tile area: partial rounds and the padding of edge tiles both count against
  // it); the best score wins (ties: larger tile).
  // Rates measured on MI355X (gfx950, 256 CUs), fp32, whole-tile shapes: 256 x 256
  // (one workgroup per CU) ~145, 128 x 128 (two per CU) ~137, 64 x 64 ~135, 32 x 32
  // (four wave groups) ~100 TFLOP/s.  The scores pick the measured winner at every shape timed:
  // 8192^3 and 8192 x 8192 x {512..2048} -> 256; 4096^3 -> 256 (140 vs 131);
  // 6144^3 -> 128 (137 vs 107 for 256, 2.25 rounds); 2048^3 and 2048 x 2048 x
  // 8192 -> 128 (125 vs 120 for 64); 3072^3 -> 64 (125 vs 101); 1024^3 -> 64
  // (103 vs 85 for 32); 512^3 -> 32 (40 vs 23 for 64); 256^3 -> 32.
  // Short K costs every tile alike (measured down to K = 512), so K is not weighed.
  struct Cand { int t; double rate; mcke_gemm_tile tile; };
  static const Cand cands[] = {{256, 145.0, {256, 256, 32, 16, 16}},
                               {128, 137.0, {128, 128, 32, 8, 8}},
                               {64, 135.0, {64, 64, 32, 4, 4}},
                               {32, 100.0, {32, 32, 32, 2, 2}}};
  const int64_t cus = device_cu_count();
  double best = -1.0;
  for (const Cand& c : cands) {
    const int64_t tiles = ((m + c.t - 1) / c.t) * ((n + c.t - 1) / c.t);
    const int64_t rounds = (tiles + cus - 1) / cus;
    const double area = static_cast<double>(rounds * cus) * c.t * c.t;
    const double score = rounds > 0 ? c.rate * static_cast<double>(m) * static_cast<double>(n) / area
                                    : 0.0;
    if (score > best) {
      best = score;
      *out = c.tile;
    }
  }
  return ok();
}

}  // extern "C"
