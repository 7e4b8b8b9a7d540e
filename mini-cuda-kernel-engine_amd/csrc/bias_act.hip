// bias_act.hip -- fused y = act(x + bias[col]) and the unfused baseline pair.
//
// Replaces kernels/bias_act.cu (launchers bias_act.cu:269-331, validation :208-229).
// HBM-bound: 4 bytes in + 4 bytes out per element (+ the bias row once per
// column strip).  The design for gfx950:
//   * lane t of column strip blockIdx.x owns VW consecutive columns, so a wave
//     issues 64 x VW x 4 contiguous bytes (1 KiB at VW = 4: a 16-byte
//     global_load_dwordx4 per lane);
//   * the bias vector for those columns is loaded once and kept in registers;
//   * large launches at VW = 4: one one-wave workgroup per 1 KiB strip of a row
//     over a flat 1-D grid, so every lane has one 16-byte load in flight, each
//     wave's life is short (its row and strip come from a multiply-shift
//     division, no loop), and the hardware streams workgroups through the CUs in
//     address order;
//   * narrower widths, launches with a capped grid (max_row_blocks, the
//     reference's starvation lever) and tensors beyond the flat grid's 32-bit
//     limits: a 2-D grid of column strips x row blocks that walks rows with a
//     stride of gridDim.y, four per iteration (4 / VW rows per workgroup at once);
//   * small launches (at most two rounds of resident workgroups at one row each):
//     256-lane workgroups that each own kChunkRows adjacent rows of their column
//     strip and issue all their loads before any store, so the launch is one
//     round of long-latency loads instead of two;
//   * x and y are streamed with non-temporal loads/stores.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "device_math.hpp"
#include "fast_div.hpp"

namespace mcke_amd {
namespace {

constexpr int kThreads = 256;
// Workgroups of the row kernel move kRowBytes of a row: one wave at VW = 4, 128
// lanes at VW = 2, 256 at VW = 1, each workgroup over 4 / VW rows at once.  The flat activation kernel
// runs one-wave workgroups (kRowLanes).  On gfx950 one-wave workgroups each
// moving one 16-byte vector per lane streamed a 2 x 256 MiB copy 3% faster than
// 256-lane workgroups of the same shape (80.0 vs 82.5 us); workgroups moving less
// than 1 KiB a row are slower again (GELU_tanh at 16384 x 4096 with one-wave
// workgroups: 227 us at VW = 1, 124 us at VW = 2, 83 us at VW = 4).
constexpr int kRowLanes = 64;
constexpr int kRowBytes = 1024;
constexpr int kRowUnroll = 4;
constexpr int kChunkRows = 8;
// At or below this many one-row workgroups a launch takes the chunked kernel.
constexpr int64_t kChunkMaxBlocks = 4096;

template <int VW, int ACT, int NT>
__global__ __launch_bounds__(NT) void bias_act_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int64_t rows,
                                                      int64_t cols_v) {
  using V = Vec<VW>;
  const int64_t cv = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (cv >= cols_v) return;
  const V bv = reinterpret_cast<const V*>(bias)[cv];
  const V* __restrict__ xv = reinterpret_cast<const V*>(x) + cv;
  V* __restrict__ yv = reinterpret_cast<V*>(y) + cv;
  const int64_t stride = gridDim.y;
  for (int64_t r = blockIdx.y; r < rows; r += kRowUnroll * stride) {
    V a[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t rr = r + u * stride;
      if (rr < rows) a[u] = ld_stream(xv + rr * cols_v);
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      const int64_t rr = r + u * stride;
      if (rr < rows) {
        V o;
        if constexpr (VW == 1) {
          o = act_xb<ACT>(a[u], bv);
        } else {
#pragma unroll
          for (int i = 0; i < VW; ++i) o[i] = act_xb<ACT>(a[u][i], bv[i]);
        }
        st_stream(yv + rr * cols_v, o);
      }
    }
  }
}

// Large launches at VW = 4: workgroup w of a flat grid owns strip (w mod strips) of
// row (w / strips), NT lanes of VW columns each.  One load per lane, no loop: on gfx950
// this streamed 16384 x 4096 at 80.5 us against 83.0 us for the 2-D grid with its
// row walk, and 16384 x 1024 (4 strips a row) at 21.3 us against 30 us, where the
// 2-D grid dispatches poorly.
template <int VW, int ACT, int NT>
__global__ __launch_bounds__(NT) void bias_act_strip_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ y, uint32_t cols_v,
                                                            uint32_t strips, FastDivU32 by_strips) {
  using V = Vec<VW>;
  const uint32_t w = blockIdx.x;
  const uint32_t row = by_strips.div(w);
  const uint32_t cv = (w - row * strips) * NT + threadIdx.x;
  if (cv >= cols_v) return;
  const std::size_t i = static_cast<std::size_t>(row) * cols_v + cv;
  const V a = ld_stream(reinterpret_cast<const V*>(x) + i);
  const V bv = reinterpret_cast<const V*>(bias)[cv];
  V o;
  if constexpr (VW == 1) {
    o = act_xb<ACT>(a, bv);
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) o[k] = act_xb<ACT>(a[k], bv[k]);
  }
  st_stream(reinterpret_cast<V*>(y) + i, o);
}

// Small launches: workgroup row blockIdx.y owns R adjacent matrix rows at a time
// (chunks strided by gridDim.y), all R loads issued before the first store.
template <int VW, int ACT, int R>
__global__ __launch_bounds__(kThreads) void bias_act_chunk_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ y,
                                                                  int64_t rows, int64_t cols_v) {
  using V = Vec<VW>;
  const int64_t cv = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (cv >= cols_v) return;
  const V bv = reinterpret_cast<const V*>(bias)[cv];
  const V* __restrict__ xv = reinterpret_cast<const V*>(x) + cv;
  V* __restrict__ yv = reinterpret_cast<V*>(y) + cv;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.y) * R; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.y) * R) {
    V a[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (r0 + u < rows) a[u] = ld_stream(xv + (r0 + u) * cols_v);
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      if (r0 + u < rows) {
        V o;
        if constexpr (VW == 1) {
          o = act_xb<ACT>(a[u], bv);
        } else {
#pragma unroll
          for (int i = 0; i < VW; ++i) o[i] = act_xb<ACT>(a[u][i], bv[i]);
        }
        st_stream(yv + (r0 + u) * cols_v, o);
      }
    }
  }
}

// y = act(x) over a flat array (the unfused pair's second kernel): one vector
// per lane and one wave per workgroup over the whole array (the layout of the
// fastest plain copy on gfx950).  ONE_SHOT: the grid covers the array, one
// vector per lane and no loop (below 2^32 vectors); otherwise lanes stride on
// past the grid's limit.
template <int VW, int ACT>
__global__ __launch_bounds__(kRowLanes) void activation_flat_kernel(const float* __restrict__ x,
                                                                    float* __restrict__ y,
                                                                    uint32_t n_v) {
  using V = Vec<VW>;
  const uint32_t i = blockIdx.x * kRowLanes + threadIdx.x;
  if (i >= n_v) return;
  const V a = ld_stream(reinterpret_cast<const V*>(x) + i);
  V o;
  if constexpr (VW == 1) {
    o = act_xb<ACT>(a, 0.0f);
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) o[j] = act_xb<ACT>(a[j], 0.0f);
  }
  st_stream(reinterpret_cast<V*>(y) + i, o);
}

template <int VW, int ACT>
__global__ __launch_bounds__(kRowLanes) void activation_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y,
                                                               int64_t n_v) {
  using V = Vec<VW>;
  const V* __restrict__ xv = reinterpret_cast<const V*>(x);
  V* __restrict__ yv = reinterpret_cast<V*>(y);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowLanes;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kRowLanes + threadIdx.x; i < n_v;
       i += stride) {
    const V a = ld_stream(xv + i);
    V o;
    if constexpr (VW == 1) {
      o = act_xb<ACT>(a, 0.0f);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) o[j] = act_xb<ACT>(a[j], 0.0f);
    }
    st_stream(yv + i, o);
  }
}

__global__ __launch_bounds__(kThreads) void vector_add_kernel(const float* __restrict__ a,
                                                              const float* __restrict__ b,
                                                              float* __restrict__ out,
                                                              size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(kThreads) void fill_u32_kernel(uint32_t* __restrict__ dst,
                                                            uint32_t value, size_t count) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride)
    dst[i] = value;
}

int validate_2d(const char* who, const float* x, const float* y, int64_t rows, int64_t cols,
                int vw) {
  if (!x || !y) return invalid(std::string(who) + ": null pointer");
  if (rows < 0 || cols < 0) return invalid(std::string(who) + ": negative extent");
  if (vw != 1 && vw != 2 && vw != 4)
    return invalid(std::string(who) + ": vector_width must be 1, 2 or 4, got " +
                   std::to_string(vw));
  if (cols % vw != 0)
    return invalid(std::string(who) + ": cols (" + std::to_string(cols) +
                   ") must be a multiple of vector_width (" + std::to_string(vw) +
                   "); use max_vector_width_f32() to pick a legal width");
  const std::size_t align = sizeof(float) * static_cast<std::size_t>(vw);
  if (!aligned(x, align) || !aligned(y, align))
    return invalid(std::string(who) + ": pointer not " + std::to_string(align) +
                   "-byte aligned");
  return ok();
}

// Row dimension of the grid: one workgroup row per matrix row, so each lane moves
// one 16-byte vector in and out and the whole launch is in flight at once (on
// gfx950 this streams at the rate of a plain copy; walking several rows per lane
// with a smaller grid measured 3-10% slower).  Capped at the hardware's 65535,
// beyond which lanes walk the remaining rows kRowUnroll at a time, and at the
// caller's max_row_blocks.
dim3 grid_2d(int64_t rows, int64_t cols_v, int max_row_blocks, int lanes, int rows_per_block = 1) {
  const int64_t gx = (cols_v + lanes - 1) / lanes;
  int64_t gy = (rows + rows_per_block - 1) / rows_per_block;
  if (gy > 65535) gy = 65535;
  if (max_row_blocks > 0 && gy > max_row_blocks) gy = max_row_blocks;
  if (gy < 1) gy = 1;
  return dim3(static_cast<unsigned>(gx > 0 ? gx : 1), static_cast<unsigned>(gy), 1u);
}

template <int VW>
int launch_fused_vw(const float* x, const float* bias, float* y, int64_t rows, int64_t cols,
                    int act, hipStream_t s, int max_row_blocks) {
  const int64_t cols_v = cols / VW;
  const int64_t gx = (cols_v + kThreads - 1) / kThreads;
  if (gx * rows <= kChunkMaxBlocks) {
    const dim3 grid = grid_2d(rows, cols_v, max_row_blocks, kThreads, kChunkRows);
#define MCKE_CHUNK(A) bias_act_chunk_kernel<VW, A, kChunkRows><<<grid, kThreads, 0, s>>>(x, bias, y, rows, cols_v)
    switch (act) {
      case kActNone: MCKE_CHUNK(kActNone); break;
      case kActRelu: MCKE_CHUNK(kActRelu); break;
      case kActGeluErf: MCKE_CHUNK(kActGeluErf); break;
      case kActGeluTanh: MCKE_CHUNK(kActGeluTanh); break;
      default: return invalid("launch_bias_act_f32: unknown activation " + std::to_string(act));
    }
#undef MCKE_CHUNK
    MCKE_LAUNCH_CHECK("bias_act_chunk_kernel");
    return ok();
  }
  constexpr int L = kRowBytes / (4 * VW);
  // The flat grid: rows x strips workgroups of L lanes, within the 32-bit limits
  // of the grid, of the global work size and of FastDivU32's operands.  At VW = 4
  // only: a lane then has a 16-byte load in flight, where at VW = 1 and 2 it would
  // have 4 or 8 bytes (16384 x 4096: 153 us and 102 us, against 87 and 82 us for the
  // 2-D grid, whose workgroups take 4 / VW rows at once).
  if constexpr (VW == 4) {
    const int64_t strips = (cols_v + L - 1) / L;
    const int64_t flat = rows * strips;
    if (max_row_blocks <= 0 && cols_v <= INT32_MAX && flat <= INT32_MAX &&
        flat * L <= int64_t{UINT32_MAX}) {
      const FastDivU32 by = FastDivU32::make(static_cast<uint32_t>(strips));
      const dim3 g(static_cast<unsigned>(flat));
      const uint32_t cv32 = static_cast<uint32_t>(cols_v), st32 = static_cast<uint32_t>(strips);
#define MCKE_STRIP(A) bias_act_strip_kernel<VW, A, L><<<g, L, 0, s>>>(x, bias, y, cv32, st32, by)
      switch (act) {
        case kActNone: MCKE_STRIP(kActNone); break;
        case kActRelu: MCKE_STRIP(kActRelu); break;
        case kActGeluErf: MCKE_STRIP(kActGeluErf); break;
        case kActGeluTanh: MCKE_STRIP(kActGeluTanh); break;
        default: return invalid("launch_bias_act_f32: unknown activation " + std::to_string(act));
      }
#undef MCKE_STRIP
      MCKE_LAUNCH_CHECK("bias_act_strip_kernel");
      return ok();
    }
  }
  // Narrower widths, capped grids and very large tensors: the 2-D grid.  Below
  // VW = 4 each workgroup takes 4 / VW rows at once (the kernel's unrolled row
  // walk), so a lane still has 16 bytes of loads in flight.
  const dim3 grid = grid_2d(rows, cols_v, max_row_blocks, L, 4 / VW);
  switch (act) {
    case kActNone: bias_act_kernel<VW, kActNone, L><<<grid, L, 0, s>>>(x, bias, y, rows, cols_v); break;
    case kActRelu: bias_act_kernel<VW, kActRelu, L><<<grid, L, 0, s>>>(x, bias, y, rows, cols_v); break;
    case kActGeluErf: bias_act_kernel<VW, kActGeluErf, L><<<grid, L, 0, s>>>(x, bias, y, rows, cols_v); break;
    case kActGeluTanh: bias_act_kernel<VW, kActGeluTanh, L><<<grid, L, 0, s>>>(x, bias, y, rows, cols_v); break;
    default: return invalid("launch_bias_act_f32: unknown activation " + std::to_string(act));
  }
  MCKE_LAUNCH_CHECK("bias_act_kernel");
  return ok();
}

template <int VW>
int launch_act_vw(const float* x, float* y, int64_t n, int act, hipStream_t s) {
  const int64_t n_v = n / VW;
  int64_t blocks = (n_v + kRowLanes - 1) / kRowLanes;
  // One vector per lane while the global work size (blocks x kRowLanes) fits 32 bits.
  if (blocks * kRowLanes <= int64_t{UINT32_MAX}) {
    const dim3 g1(static_cast<unsigned>(blocks));
    const uint32_t n32 = static_cast<uint32_t>(n_v);
    switch (act) {
      case kActNone: activation_flat_kernel<VW, kActNone><<<g1, kRowLanes, 0, s>>>(x, y, n32); break;
      case kActRelu: activation_flat_kernel<VW, kActRelu><<<g1, kRowLanes, 0, s>>>(x, y, n32); break;
      case kActGeluErf: activation_flat_kernel<VW, kActGeluErf><<<g1, kRowLanes, 0, s>>>(x, y, n32); break;
      case kActGeluTanh: activation_flat_kernel<VW, kActGeluTanh><<<g1, kRowLanes, 0, s>>>(x, y, n32); break;
      default: return invalid("launch_activation_f32: unknown activation " + std::to_string(act));
    }
    MCKE_LAUNCH_CHECK("activation_flat_kernel");
    return ok();
  }
  // Beyond that, 2^24 one-wave workgroups (2^30 lanes) stay below the limit and
  // still fill the chip many times over; the kernel's grid-stride loop covers the rest.
  constexpr int64_t kMaxBlocks = int64_t{1} << 24;
  static_assert(kMaxBlocks * kRowLanes <= (int64_t{1} << 32) - 1, "global work size fits 32 bits");
  if (blocks > kMaxBlocks) blocks = kMaxBlocks;
  const unsigned g = static_cast<unsigned>(blocks);
  constexpr int L = kRowLanes;
  switch (act) {
    case kActNone: activation_kernel<VW, kActNone><<<g, L, 0, s>>>(x, y, n_v); break;
    case kActRelu: activation_kernel<VW, kActRelu><<<g, L, 0, s>>>(x, y, n_v); break;
    case kActGeluErf: activation_kernel<VW, kActGeluErf><<<g, L, 0, s>>>(x, y, n_v); break;
    case kActGeluTanh: activation_kernel<VW, kActGeluTanh><<<g, L, 0, s>>>(x, y, n_v); break;
    default: return invalid("launch_activation_f32: unknown activation " + std::to_string(act));
  }
  MCKE_LAUNCH_CHECK("activation_kernel");
  return ok();
}

}  // namespace
}  // namespace mcke_amd

using namespace mcke_amd;

extern "C" {

int mcke_max_vector_width_f32(const void* p, int64_t cols) {
  for (int w = 4; w > 1; w >>= 1)
    if (cols % w == 0 && aligned(p, sizeof(float) * static_cast<std::size_t>(w))) return w;
  return 1;
}

int mcke_launch_bias_act_f32(const float* x, const float* bias, float* y, int64_t rows,
                             int64_t cols, int act, int vector_width, void* stream,
                             int max_row_blocks) {
  if (rows == 0 || cols == 0) return ok();   // an empty grid is a launch error
  if (!bias) return invalid("launch_bias_act_f32: null bias");
  if (int rc = validate_2d("launch_bias_act_f32", x, y, rows, cols, vector_width)) return rc;
  if (!aligned(bias, sizeof(float) * static_cast<std::size_t>(vector_width)))
    return invalid("launch_bias_act_f32: bias pointer not aligned");
  if (x == y)
    return invalid("launch_bias_act_f32: in-place (x == y) violates the __restrict__ contract");
  if (act < 0 || act > 3)
    return invalid("launch_bias_act_f32: unknown activation " + std::to_string(act));
  // Column strips x their lanes (at most 1024 a strip) must fit the grid's 32-bit
  // global work size along x.
  if (cols / vector_width > int64_t{UINT32_MAX} - 1023)
    return invalid("launch_bias_act_f32: cols / vector_width exceeds the grid's 32-bit work size");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vector_width) {
    case 1: return launch_fused_vw<1>(x, bias, y, rows, cols, act, s, max_row_blocks);
    case 2: return launch_fused_vw<2>(x, bias, y, rows, cols, act, s, max_row_blocks);
    default: return launch_fused_vw<4>(x, bias, y, rows, cols, act, s, max_row_blocks);
  }
}

int mcke_launch_bias_add_f32(const float* x, const float* bias, float* y, int64_t rows,
                             int64_t cols, int vector_width, void* stream) {
  return mcke_launch_bias_act_f32(x, bias, y, rows, cols, kActNone, vector_width, stream, 0);
}

int mcke_launch_activation_f32(const float* x, float* y, int64_t n, int act, int vector_width,
                               void* stream) {
  if (n == 0) return ok();
  if (!x || !y) return invalid("launch_activation_f32: null pointer");
  if (n < 0) return invalid("launch_activation_f32: negative extent");
  if (vector_width != 1 && vector_width != 2 && vector_width != 4)
    return invalid("launch_activation_f32: vector_width must be 1, 2 or 4");
  if (n % vector_width != 0)
    return invalid("launch_activation_f32: n must be a multiple of vector_width");
  const std::size_t align = sizeof(float) * static_cast<std::size_t>(vector_width);
  if (!aligned(x, align) || !aligned(y, align))
    return invalid("launch_activation_f32: pointer not aligned");
  if (act < 0 || act > 3)
    return invalid("launch_activation_f32: unknown activation " + std::to_string(act));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vector_width) {
    case 1: return launch_act_vw<1>(x, y, n, act, s);
    case 2: return launch_act_vw<2>(x, y, n, act, s);
    default: return launch_act_vw<4>(x, y, n, act, s);
  }
}

int mcke_launch_vector_add_f32(const float* a, const float* b, float* out, size_t n,
                               void* stream) {
  if (n == 0) return ok();
  if (!a || !b || !out) return invalid("launch_vector_add_f32: null pointer");
  size_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 8192) blocks = 8192;
  vector_add_kernel<<<static_cast<unsigned>(blocks), kThreads, 0,
                      static_cast<hipStream_t>(stream)>>>(a, b, out, n);
  MCKE_LAUNCH_CHECK("vector_add_kernel");
  return ok();
}

int mcke_fill_u32_async(void* dst, uint32_t value, size_t count, void* stream) {
  if (count == 0) return ok();
  if (!dst) return invalid("fill_u32_async: null pointer");
  if (!aligned(dst, 4)) return invalid("fill_u32_async: pointer not 4-byte aligned");
  size_t blocks = (count + kThreads - 1) / kThreads;
  if (blocks > 16384) blocks = 16384;
  fill_u32_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<uint32_t*>(dst), value, count);
  MCKE_LAUNCH_CHECK("fill_u32_kernel");
  return ok();
}

}  // extern "C"
