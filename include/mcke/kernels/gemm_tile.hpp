// mcke/kernels/gemm_tile.hpp -- GEMM tile descriptor, (variant, tile) validity,
// the double-buffer schedule and a CDNA occupancy model.  Pure host arithmetic.
//
// Same API as the reference's include/mcke/kernels/gemm_tile.hpp:47-426, with
// the constants of gfx950 instead of sm_75:
//   * a tile's lane count must be a multiple of the 64-lane wavefront;
//   * GemmVariant is append-only and gains kMfmaF32 (= 8), whose tiles are
//     (256,256,32,16,16), (256,256,16,16,16), (128,128,32,8,8), (128,128,16,8,8),
//     (64,64,32,4,4) and (32,32,32,2,2): 256 lanes in the (bm/tm) x (bn/tn)
//     descriptor (the whole-tile kernels of the two smallest tiles split each
//     K stage over wave groups; the descriptor stays the tile's identity);
//   * occupancy is limited per SIMD by the 512-entry unified VGPR file (arch +
//     accumulation registers, allocated in granules of 8) and 8 waves, per CU by
//     160 KiB of LDS, the 2048-lane cap and the workgroup cap.
#pragma once

#include <cstddef>
#include <cstdint>

#include "mcke/core/config.hpp"
#include "mcke/core/device.hpp"

namespace mcke::kernels {

struct GemmTile {
  int bm = 128, bn = 128, bk = 8;
  int tm = 8, tn = 8;
};

[[nodiscard]] constexpr int threads_per_block(const GemmTile& t) {
  if (t.tm <= 0 || t.tn <= 0) return 0;
  return (t.bm / t.tm) * (t.bn / t.tn);
}

[[nodiscard]] constexpr int smem_floats(const GemmTile& t, bool double_buffered, int a_row_pad = 0) {
  return (t.bk * (t.bm + a_row_pad) + t.bk * t.bn) * (double_buffered ? 2 : 1);
}

[[nodiscard]] constexpr std::size_t smem_bytes(const GemmTile& t, bool double_buffered, int a_row_pad = 0) {
  return static_cast<std::size_t>(smem_floats(t, double_buffered, a_row_pad)) * sizeof(float);
}

// Every lane owns the same whole number of outputs and of staged elements, and
// the workgroup is whole wavefronts (gemm_tile.hpp:112-124 with 64-lane waves).
[[nodiscard]] constexpr bool tile_is_self_consistent(const GemmTile& t) {
  if (t.bm <= 0 || t.bn <= 0 || t.bk <= 0 || t.tm <= 0 || t.tn <= 0) return false;
  if (t.bm % t.tm != 0 || t.bn % t.tn != 0) return false;
  const int threads = threads_per_block(t);
  if (threads <= 0 || threads > 1024) return false;
  if (threads % kWarpSize != 0) return false;
  if ((t.bm * t.bk) % threads != 0) return false;
  if ((t.bk * t.bn) % threads != 0) return false;
  return true;
}

// K loop unrolled by two over a double buffer: pair_iters full pairs, then one
// tail tile from buffer 0 when the tile count is odd (gemm_tile.hpp:151-159).
struct DbufSchedule {
  std::int64_t pair_iters = 0;
  bool has_tail = false;
};

[[nodiscard]] constexpr DbufSchedule dbuf_schedule(std::int64_t k_tiles) {
  if (k_tiles <= 0) return {};
  return DbufSchedule{k_tiles / 2, (k_tiles % 2) != 0};
}

enum class GemmTileConfig : std::uint8_t {
  k32x32x32_1x1,
  k128x128x8_8x8,
  kUnsupported,
  // appended: the MFMA instantiations
  kMfma256x256x32,
  kMfma256x256x16,
  kMfma128x128x32,
  kMfma128x128x16,
  kMfma64x64x32,
  kMfma32x32x32,
};

[[nodiscard]] constexpr GemmTileConfig select_tile_config(const GemmTile& t) {
  if (t.bm == 32 && t.bn == 32 && t.bk == 32 && t.tm == 1 && t.tn == 1) return GemmTileConfig::k32x32x32_1x1;
  if (t.bm == 128 && t.bn == 128 && t.bk == 8 && t.tm == 8 && t.tn == 8) return GemmTileConfig::k128x128x8_8x8;
  if (t.bm == 256 && t.bn == 256 && t.tm == 16 && t.tn == 16) {
    if (t.bk == 32) return GemmTileConfig::kMfma256x256x32;
    if (t.bk == 16) return GemmTileConfig::kMfma256x256x16;
  }
  if (t.bm == 128 && t.bn == 128 && t.tm == 8 && t.tn == 8) {
    if (t.bk == 32) return GemmTileConfig::kMfma128x128x32;
    if (t.bk == 16) return GemmTileConfig::kMfma128x128x16;
  }
  if (t.bm == 64 && t.bn == 64 && t.bk == 32 && t.tm == 4 && t.tn == 4) return GemmTileConfig::kMfma64x64x32;
  if (t.bm == 32 && t.bn == 32 && t.bk == 32 && t.tm == 2 && t.tn == 2) return GemmTileConfig::kMfma32x32x32;
  return GemmTileConfig::kUnsupported;
}

enum class GemmVariant : std::uint8_t {
  kNaive,
  kTiledSmem,
  kTiledRegBlock,
  kWarpTile,
  kCublasRef,          // the vendor-library ceiling row (rocBLAS)
  kWarpTileNoDbuf,
  kWarpTileVec4,
  kNaiveUncoalesced,
  kMfmaF32,            // appended: fp32 MFMA, LDS double-buffered
};

[[nodiscard]] constexpr bool gemm_variant_uses_tile(GemmVariant v) {
  return v != GemmVariant::kNaive && v != GemmVariant::kNaiveUncoalesced &&
         v != GemmVariant::kCublasRef;
}

[[nodiscard]] constexpr bool is_mfma_config(GemmTileConfig c) {
  return c == GemmTileConfig::kMfma256x256x32 || c == GemmTileConfig::kMfma256x256x16 ||
         c == GemmTileConfig::kMfma128x128x32 || c == GemmTileConfig::kMfma128x128x16 ||
         c == GemmTileConfig::kMfma64x64x32 || c == GemmTileConfig::kMfma32x32x32;
}

// The instantiation a tile-using variant requires (for kMfmaF32 any MFMA config).
[[nodiscard]] constexpr GemmTileConfig gemm_required_config(GemmVariant v) {
  return v == GemmVariant::kTiledSmem ? GemmTileConfig::k32x32x32_1x1 : GemmTileConfig::k128x128x8_8x8;
}

[[nodiscard]] constexpr bool gemm_tile_is_supported(GemmVariant v, const GemmTile& t) {
  if (!gemm_variant_uses_tile(v)) return true;
  if (!tile_is_self_consistent(t)) return false;
  if (v == GemmVariant::kMfmaF32) return is_mfma_config(select_tile_config(t));
  return select_tile_config(t) == gemm_required_config(v);
}

// ---------------------------------------------------------------------------
// Occupancy on CDNA: the minimum of four limiters (gemm_tile.hpp:304-426 for the
// structure; the constants are gfx950's).
// ---------------------------------------------------------------------------
enum class OccupancyLimiter : std::uint8_t {
  kRegisters,
  kSharedMemory,
  kThreadsPerSm,
  kBlocksPerSm,
  kInvalid,
};

[[nodiscard]] constexpr const char* limiter_name(OccupancyLimiter l) {
  switch (l) {
    case OccupancyLimiter::kRegisters: return "registers";
    case OccupancyLimiter::kSharedMemory: return "LDS";
    case OccupancyLimiter::kThreadsPerSm: return "lanes/CU cap";
    case OccupancyLimiter::kBlocksPerSm: return "workgroups/CU cap";
    case OccupancyLimiter::kInvalid: return "WILL NOT LAUNCH";
  }
  return "?";
}

struct OccupancyEstimate {
  int blocks_per_sm = 0;
  int warps_per_sm = 0;
  double occupancy = 0.0;   // resident lanes / max lanes per CU
  OccupancyLimiter limiter = OccupancyLimiter::kInvalid;
  bool tied = false;
  int by_registers = 0, by_smem = 0, by_threads = 0, by_blocks = 0;
};

inline constexpr int kNoLimit = 1 << 24;
inline constexpr int kSimdsPerCu = 4;
inline constexpr int kVgprsPerSimdLane = 512;   // unified arch + accumulation VGPRs
inline constexpr int kVgprGranule = 8;
inline constexpr int kMaxWavesPerSimd = 8;
inline constexpr int kMaxRegsPerThread = 512;
inline constexpr std::size_t kSmemAllocUnit = 512;

namespace detail {
[[nodiscard]] constexpr int round_up_div(int a, int b) { return (a + b - 1) / b; }
[[nodiscard]] constexpr int round_up(int a, int unit) { return round_up_div(a, unit) * unit; }
[[nodiscard]] constexpr std::size_t round_up_sz(std::size_t a, std::size_t unit) {
  return ((a + unit - 1) / unit) * unit;
}
[[nodiscard]] constexpr int min4(int a, int b, int c, int d) {
  const int ab = a < b ? a : b;
  const int cd = c < d ? c : d;
  return ab < cd ? ab : cd;
}
}  // namespace detail

// regs_per_thread counts unified VGPRs (architectural + accumulation).  A
// workgroup's waves are spread over the 4 SIMDs, so a workgroup of W waves needs
// ceil(W / 4) wave slots on each SIMD.
[[nodiscard]] constexpr OccupancyEstimate occupancy_blocks_per_sm(
    const DeviceInfo& d, int threads_per_blk, int regs_per_thread, std::size_t smem_bytes_per_block) {
  OccupancyEstimate e;
  if (threads_per_blk <= 0 || d.sm_count <= 0 || d.max_threads_per_sm <= 0 ||
      d.max_blocks_per_sm <= 0 || d.shared_mem_per_sm == 0)
    return e;
  if (d.max_threads_per_block > 0 && threads_per_blk > d.max_threads_per_block) return e;
  if (regs_per_thread > kMaxRegsPerThread) return e;
  if (smem_bytes_per_block > d.shared_mem_per_sm) return e;

  const int waves_per_blk = detail::round_up_div(threads_per_blk, kWarpSize);
  const int waves_per_simd_per_blk = detail::round_up_div(waves_per_blk, kSimdsPerCu);

  if (regs_per_thread <= 0) {
    e.by_registers = kNoLimit;
  } else {
    int waves_per_simd = kVgprsPerSimdLane / detail::round_up(regs_per_thread, kVgprGranule);
    if (waves_per_simd > kMaxWavesPerSimd) waves_per_simd = kMaxWavesPerSimd;
    e.by_registers = waves_per_simd / waves_per_simd_per_blk;
  }
  if (smem_bytes_per_block == 0) {
    e.by_smem = kNoLimit;
  } else {
    e.by_smem = static_cast<int>(d.shared_mem_per_sm /
                                 detail::round_up_sz(smem_bytes_per_block, kSmemAllocUnit));
  }
  e.by_threads = d.max_threads_per_sm / threads_per_blk;
  e.by_blocks = d.max_blocks_per_sm;

  const int best = detail::min4(e.by_registers, e.by_smem, e.by_threads, e.by_blocks);
  if (best <= 0) return e;
  OccupancyLimiter which = OccupancyLimiter::kRegisters;
  if (e.by_threads == best) which = OccupancyLimiter::kThreadsPerSm;
  else if (e.by_blocks == best) which = OccupancyLimiter::kBlocksPerSm;
  else if (e.by_registers == best) which = OccupancyLimiter::kRegisters;
  else which = OccupancyLimiter::kSharedMemory;
  e.tied = ((e.by_registers == best) + (e.by_smem == best) + (e.by_threads == best) +
            (e.by_blocks == best)) > 1;
  e.blocks_per_sm = best;
  e.limiter = which;
  e.warps_per_sm = best * waves_per_blk;
  e.occupancy = static_cast<double>(best * threads_per_blk) / static_cast<double>(d.max_threads_per_sm);
  return e;
}

}  // namespace mcke::kernels
