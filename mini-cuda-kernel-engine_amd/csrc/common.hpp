// common.hpp -- internal helpers shared by every translation unit of libmcke_amd.
//
// Status plumbing for the C-ABI: a failing entry point records its message in a
// thread-local buffer and returns an mcke_status code (the reference's
// mcke::StatusCode values, include/mcke/core/status.hpp:42-50).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "mcke_amd.h"

namespace mcke_amd {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears nothing; OK is just 0 (the last message is kept until the next failure).
inline int ok() { return MCKE_STATUS_OK; }

inline int invalid(const std::string& msg) { return fail(MCKE_STATUS_INVALID_ARGUMENT, msg); }

// A HIP runtime error -> MCKE_STATUS_DEVICE_ERROR with name, string, file, line
// (the reference's cuda_check.hpp:51-67 convention).  hipErrorOutOfMemory maps to
// MCKE_STATUS_OUT_OF_MEMORY so allocators can recover from it.
int hip_fail(hipError_t e, const char* what, const char* file, int line);

#define MCKE_HIP_TRY(expr)                                                    \
  do {                                                                        \
    const hipError_t _e = (expr);                                             \
    if (_e != hipSuccess) return ::mcke_amd::hip_fail(_e, #expr, __FILE__, __LINE__); \
  } while (0)

// After a <<<>>> launch: surface launch-configuration errors now.
#define MCKE_LAUNCH_CHECK(what) MCKE_HIP_TRY(hipGetLastError())

inline bool aligned(const void* p, std::size_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(p) % bytes) == 0;
}

// Wavefront width on CDNA.  Kernels are written for 64 lanes.
constexpr int kWave = 64;

}  // namespace mcke_amd
