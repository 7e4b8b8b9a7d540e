// mcke/core/config.hpp -- architectural constants of the host API (gfx950).
//
// Counterpart of the reference's include/mcke/core/config.hpp:26-82.  The
// reference hard-codes NVIDIA's 32-lane warp; CDNA's wavefront is 64 lanes, and
// every tile/occupancy rule in this tree is written against kWarpSize = 64.
#pragma once

#include <cstddef>

#if defined(__HIPCC__)
#define MCKE_HOST_DEVICE __host__ __device__
#define MCKE_DEVICE __device__
#else
#define MCKE_HOST_DEVICE
#define MCKE_DEVICE
#endif

// The host layers always have a device backend here (the C-ABI library); the
// reference's MCKE_WITH_CUDA switch has no counterpart.

namespace mcke {

// Lanes per wavefront on CDNA (gfx9).
inline constexpr int kWarpSize = 64;
// Global memory is fetched in 64-byte requests and cached in 128-byte lines.
inline constexpr std::size_t kSectorBytes = 64;
inline constexpr std::size_t kCacheLineBytes = 128;
// hipMalloc returns 256-byte aligned blocks; every allocator here keeps that.
inline constexpr std::size_t kDeviceAlignment = 256;
// Smallest block the buddy allocator hands out.
inline constexpr std::size_t kMinBlockBytes = 256;

}  // namespace mcke
