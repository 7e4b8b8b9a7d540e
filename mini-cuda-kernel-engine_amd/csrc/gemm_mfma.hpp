// gemm_mfma.hpp -- fp32 GEMM on the CDNA matrix cores (v_mfma_f32_32x32x2_f32).
//
// C[M,N] = alpha * A[M,K] B[K,N] + beta * C, row-major, fp32 in and out, fp32
// accumulation.  This is the new appended GemmVariant (kMfmaF32); the reference's
// ladder kernels (gemm.cu:125-588) have no counterpart because the reference has
// no matrix-core path.
//
// Workgroup: 256 lanes = 4 wave64s in a 2 x 2 grid; the workgroup owns a BM x BN
// tile of C, each wave a WM x WN sub-tile = (WM/32) x (WN/32) MFMA 32x32 tiles,
// kept in accumulation registers for the whole K loop.
//
// K is staged BK at a time through an LDS double buffer:
//   As[BM][BK + 4]   A row-major (k contiguous); the +4 pad puts the 8 rows read
//                    by an 8-lane 16-byte group on 8 disjoint bank quads;
//   Bs[BK][BN]       B row-major (n contiguous).
// One barrier per K step: the next step's global loads are issued before the
// MFMAs of the current step and written to the other buffer after them.
//
// Operand delivery.  v_mfma_f32_32x32x2_f32 takes one A and one B value per lane:
// lane l supplies A[i = l%32][kslot = l/32] and B[kslot = l/32][j = l%32].  The
// K order inside a step is free (a sum), so lane half h = l/32 walks the k range
// [h*BK/2, (h+1)*BK/2): then a lane's next four A values are contiguous in As and
// arrive in one 16-byte ds_read per m-tile.  For B the N order is permuted
// instead: within a wave's WN columns, MFMA n-tile j at lane column c holds
// actual column NT*c + j, so one 4*NT-byte ds_read per k delivers a lane's
// values for all NT n-tiles -- and in the epilogue the same lane holds NT
// adjacent columns of each output row, which become one 16-byte global store.
//
// Accumulator layout of one 32x32 tile (lane l, register r = 0..15):
//   row = 8*(r/4) + 4*(l/32) + (r%4),   col = l%32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

#include "device_math.hpp"

namespace mcke_amd {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMfmaThreads = 256;
constexpr int kXcds = 8;       // gfx950: workgroups are dealt round-robin to 8 XCDs
constexpr int kGroupM = 8;     // tile-row grouping for L2 reuse within an XCD

// MFMA order within a step.  Block row i of a wave's MT x NT accumulators walks
// its columns left to right when i is even and right to left when i is odd, so
// each MFMA shares one operand register with the one before it: the A fragment
// along a row, the B fragment at a row turn.  With random operands the matrix
// pipe runs at the board's power limit, where fewer operand bits changing from
// one MFMA to the next buy engine clock (measured on MI355X, same process,
// alternating blocks: 16-bit GEMM 8192^3 +0.8%, 4096^3 +0.7%; fp32 8192^3 +0.3%,
// 2048^3 +1.7%).  Every accumulator still takes its K sub-steps in the same
// order, so the results are bit-identical to row order.
__host__ __device__ constexpr int mfma_snake_col(int i, int jj, int nt) {
  return (i % 2) ? nt - 1 - jj : jj;
}

template <int NT> struct BVec;
template <> struct BVec<1> { using type = float; };
template <> struct BVec<2> { using type = f32x2; };
template <> struct BVec<4> { using type = f32x4; };

// Workgroup id -> (tile_m, tile_n).  Consecutive workgroup ids land on different
// XCDs (id % 8), so ids are first regrouped so that each XCD sees a contiguous
// run of logical tiles, and logical tiles are then walked kGroupM tile-rows at a
// time so concurrently running tiles share A row-slabs and B column-slabs in
// that XCD's L2.
__device__ __forceinline__ void mfma_tile_coords(int wg, int tiles_m, int tiles_n, int& tm,
                                                 int& tn) {
  const int total = tiles_m * tiles_n;
  const int full = total - (total % kXcds);
  int t = wg;
  if (wg < full) t = (wg % kXcds) * (full / kXcds) + wg / kXcds;
  const int in_group = kGroupM * tiles_n;
  const int g = t / in_group;
  const int first_m = g * kGroupM;
  const int gsz = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int local = t % in_group;
  tm = first_m + local % gsz;
  tn = local / gsz;
}

template <int BM, int BN, int BK, bool VEC>
struct MfmaStage {
  static constexpr int kLdA = BK + 4;
  static constexpr int kLdB = BN;
  static constexpr int kAFloats = BM * kLdA;
  static constexpr int kBFloats = BK * kLdB;
  static constexpr int kStageFloats = kAFloats + kBFloats;
  // Per-lane global loads per stage.
  static constexpr int kAVec = BM * BK / 4 / kMfmaThreads;   // float4 loads of A
  static constexpr int kBVec = BK * BN / 4 / kMfmaThreads;   // float4 loads of B
  static constexpr int kAScl = BM * BK / kMfmaThreads;       // scalar loads of A
  static constexpr int kBScl = BK * BN / kMfmaThreads;       // scalar loads of B
  static_assert(BM * BK % (4 * kMfmaThreads) == 0 && BK * BN % (4 * kMfmaThreads) == 0,
                "stage must divide evenly over the workgroup");

  // Registers holding one stage between its global load and its LDS store.
  struct Regs {
    f32x4 a[VEC ? kAVec : 1];
    f32x4 b[VEC ? kBVec : 1];
    float as[VEC ? 1 : kAScl];
    float bs[VEC ? 1 : kBScl];
  };

  // Loads K columns [k0, k0 + BK) of the block's A rows and B columns, zero-filling
  // everything outside [0, M) x [0, K) and [0, K) x [0, N).
  static __device__ __forceinline__ void load(Regs& R, const float* __restrict__ A,
                                              const float* __restrict__ B, int M, int N,
                                              int K, int m0, int n0, int k0) {
    const int t = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < kAVec; ++i) {
        const int li = i * kMfmaThreads + t;
        const int row = li / (BK / 4), c4 = li % (BK / 4);
        const int gm = m0 + row, gk = k0 + 4 * c4;
        // K % 4 == 0 on this path, so a float4 is either fully in range or fully out.
        if (gm < M && gk < K)
          R.a[i] = *reinterpret_cast<const f32x4*>(A + static_cast<int64_t>(gm) * K + gk);
        else
          R.a[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < kBVec; ++i) {
        const int li = i * kMfmaThreads + t;
        const int kr = li / (BN / 4), c4 = li % (BN / 4);
        const int gk = k0 + kr, gn = n0 + 4 * c4;
        if (gk < K && gn < N)
          R.b[i] = *reinterpret_cast<const f32x4*>(B + static_cast<int64_t>(gk) * N + gn);
        else
          R.b[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    } else {
#pragma unroll
      for (int i = 0; i < kAScl; ++i) {
        const int li = i * kMfmaThreads + t;
        const int row = li / BK, col = li % BK;
        const int gm = m0 + row, gk = k0 + col;
        R.as[i] = (gm < M && gk < K) ? A[static_cast<int64_t>(gm) * K + gk] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kBScl; ++i) {
        const int li = i * kMfmaThreads + t;
        const int kr = li / BN, col = li % BN;
        const int gk = k0 + kr, gn = n0 + col;
        R.bs[i] = (gk < K && gn < N) ? B[static_cast<int64_t>(gk) * N + gn] : 0.0f;
      }
    }
  }

  static __device__ __forceinline__ void store(const Regs& R, float* __restrict__ stage) {
    float* As = stage;
    float* Bs = stage + kAFloats;
    const int t = threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < kAVec; ++i) {
        const int li = i * kMfmaThreads + t;
        const int row = li / (BK / 4), c4 = li % (BK / 4);
        *reinterpret_cast<f32x4*>(As + row * kLdA + 4 * c4) = R.a[i];
      }
#pragma unroll
      for (int i = 0; i < kBVec; ++i) {
        const int li = i * kMfmaThreads + t;
        const int kr = li / (BN / 4), c4 = li % (BN / 4);
        *reinterpret_cast<f32x4*>(Bs + kr * kLdB + 4 * c4) = R.b[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kAScl; ++i) {
        const int li = i * kMfmaThreads + t;
        As[(li / BK) * kLdA + li % BK] = R.as[i];
      }
#pragma unroll
      for (int i = 0; i < kBScl; ++i) {
        const int li = i * kMfmaThreads + t;
        Bs[(li / BN) * kLdB + li % BN] = R.bs[i];
      }
    }
  }
};

// Epilogue shared by the MFMA kernels: C = alpha * acc + beta * C for one wave's
// MT x NT accumulator tiles, the WM x WN = 32 MT x 32 NT block at wave position
// (wm, wn) of the workgroup's tile at (m0, n0) (C is not read when beta == 0).
// Lane (h, c) holds, for MFMA tile (i, j) and accumulator register r, row
// 8*(r/4) + 4h + r%4 of the tile's 32 rows and column NT*c + j of the wave's WN.
// The epilogue's extra operands.  A plain GEMM ignores them; a fused launch
// (FUSED = true, beta = 0) stores y = act(alpha * acc + bias[col]) instead of
// alpha * acc: the same fp32 value of alpha * acc that a plain launch writes to C,
// then the activation exactly as bias_act computes it from C -- so the fused
// result has the bits of mcke_launch_gemm_f32 followed by mcke_launch_bias_act_f32.
struct EpiArgs {
  const float* bias;   // N values
  int act;             // MCKE activation, 0 .. 3
};

// alpha * acc rounded to fp32 before the bias is added: the empty asm makes the
// product a register value, so the compiler cannot contract it with the add
// into one fused multiply-add (which the unfused pair, storing C in between, never
// does).
__device__ __forceinline__ float epi_round(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int ACT> __device__ __forceinline__ float epi_act(float o, float b) {
  return act_xb<ACT>(epi_round(o), b);
}

// mfma_store_c's fused form (beta = 0): the bias of a lane's NT columns is read
// once, before its rows.
template <int MT, int NT, bool VEC, int ACT>
__device__ __forceinline__ void mfma_store_c_act(const f32x16 (&acc)[MT][NT],
                                                 float* __restrict__ C, int M, int N, int m0,
                                                 int n0, int wm, int wn, int h, int c,
                                                 float alpha, const float* __restrict__ bias) {
  constexpr int WM = 32 * MT, WN = 32 * NT;
  const bool vec_store = VEC && (NT == 4) && ((N & 3) == 0);
  const int col0 = n0 + wn * WN + NT * c;
  float bj[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) bj[j] = col0 + j < N ? bias[col0 + j] : 0.0f;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= M) continue;
      float* crow = C + static_cast<int64_t>(row) * N;
      float v[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) v[j] = epi_act<ACT>(alpha * acc[i][j][r], bj[j]);
      if (vec_store && col0 + 3 < N) {
        *reinterpret_cast<f32x4*>(crow + col0) =
            f32x4{v[0], v[NT > 1 ? 1 : 0], v[NT > 2 ? 2 : 0], v[NT > 3 ? 3 : 0]};
      } else {
#pragma unroll
        for (int j = 0; j < NT; ++j)
          if (col0 + j < N) crow[col0 + j] = v[j];
      }
    }
  }
}

template <int MT, int NT, bool VEC>
__device__ __forceinline__ void mfma_store_c(const f32x16 (&acc)[MT][NT],
                                             float* __restrict__ C, int M, int N, int m0, int n0,
                                             int wm, int wn, int h, int c, float alpha,
                                             float beta) {
  constexpr int WM = 32 * MT, WN = 32 * NT;
  const bool vec_store = VEC && (NT == 4) && ((N & 3) == 0);
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= M) continue;
      const int col0 = n0 + wn * WN + NT * c;
      float* crow = C + static_cast<int64_t>(row) * N;
      float v[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) v[j] = alpha * acc[i][j][r];
      if (vec_store && col0 + 3 < N) {
        f32x4 o{v[0], v[NT > 1 ? 1 : 0], v[NT > 2 ? 2 : 0], v[NT > 3 ? 3 : 0]};
        if (beta != 0.0f) o += beta * *reinterpret_cast<const f32x4*>(crow + col0);
        *reinterpret_cast<f32x4*>(crow + col0) = o;
      } else {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = col0 + j;
          if (col < N) {
            float o = v[j];
            if (beta != 0.0f) o += beta * crow[col];
            crow[col] = o;
          }
        }
      }
    }
  }
}

// One butterfly step of a 4 x 4 transpose inside each quad of lanes: lane t
// exchanges one of the register pair (lo, hi_reg) with lane t ^ BIT, by DPP
// quad_perm and selects (no branches, so the values stay in registers).
template <int BIT>
__device__ __forceinline__ void quad_exchange(float& lo, float& hi_reg, bool upper) {
  constexpr int kCtrl = BIT == 1 ? 0xB1 : 0x4E;   // quad_perm [1,0,3,2] / [2,3,0,1]
  const float send = upper ? lo : hi_reg;
  const float recv = __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), kCtrl, 0xF, 0xF, true));
  lo = upper ? recv : lo;
  hi_reg = upper ? hi_reg : recv;
}

// (lane t of a quad, register s) -> (lane s, register t): the two butterfly
// rounds swap bit 0, then bit 1, of the lane and register indices.
__device__ __forceinline__ void quad_transpose(float& v0, float& v1, float& v2, float& v3,
                                               int t) {
  const bool b0 = (t & 1) != 0, b1 = (t & 2) != 0;
  quad_exchange<1>(v0, v1, b0);
  quad_exchange<1>(v2, v3, b0);
  quad_exchange<2>(v0, v2, b1);
  quad_exchange<2>(v1, v3, b1);
}

// The C store of whole tiles (the direct-to-LDS kernel: M % BM == N % BN == 0,
// N % 4 == 0, C 16-byte aligned), in the widest stores the accumulator layout
// allows.  Same values as mfma_store_c, only fewer and wider instructions:
//   NT == 4: a lane holds 4 adjacent columns of a row already (16-byte stores);
//   NT == 2: it holds 2 (8-byte stores);
//   NT == 1: it holds one column of registers r = 4q .. 4q+3, i.e. rows
//            8q + 4h + 0..3.  A 4 x 4 transpose inside each quad of lanes gives
//            lane 4j + t row 8q + 4h + t at columns 4j .. 4j+3 (16-byte stores:
//            4 per 32 x 32 tile instead of 16 single-float ones; 64 x 64 tile at
//            1024^3: 19.20 vs 19.46 us).
template <int MT, int NT>
__device__ __forceinline__ void mfma_store_c_whole(const f32x16 (&acc)[MT][NT],
                                                   float* __restrict__ C, int N, int m0, int n0,
                                                   int wm, int wn, int h, int c, float alpha,
                                                   float beta) {
  constexpr int WM = 32 * MT, WN = 32 * NT;
  if constexpr (NT == 1) {
    const int t = c & 3;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v0 = acc[i][0][4 * q], v1 = acc[i][0][4 * q + 1], v2 = acc[i][0][4 * q + 2],
              v3 = acc[i][0][4 * q + 3];
        quad_transpose(v0, v1, v2, v3, t);
        const int row = m0 + wm * WM + i * 32 + 8 * q + 4 * h + t;
        float* p = C + static_cast<int64_t>(row) * N + n0 + wn * WN + (c & ~3);
        f32x4 o{alpha * v0, alpha * v1, alpha * v2, alpha * v3};
        if (beta != 0.0f) o += beta * *reinterpret_cast<const f32x4*>(p);
        *reinterpret_cast<f32x4*>(p) = o;
      }
    }
  } else if constexpr (NT == 2) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        float* p = C + static_cast<int64_t>(row) * N + n0 + wn * WN + 2 * c;
        f32x2 o{alpha * acc[i][0][r], alpha * acc[i][1][r]};
        if (beta != 0.0f) o += beta * *reinterpret_cast<const f32x2*>(p);
        *reinterpret_cast<f32x2*>(p) = o;
      }
    }
  } else {
    static_assert(NT == 4, "wave tiles are 1, 2 or 4 MFMA tiles wide");
    mfma_store_c<MT, NT, true>(acc, C, m0 + wm * WM + WM, N, m0, n0, wm, wn, h, c, alpha, beta);
  }
}

// mfma_store_c_whole's fused form (beta = 0), the same stores.
template <int MT, int NT, int ACT>
__device__ __forceinline__ void mfma_store_c_whole_act(const f32x16 (&acc)[MT][NT],
                                                       float* __restrict__ C, int N, int m0,
                                                       int n0, int wm, int wn, int h, int c,
                                                       float alpha,
                                                       const float* __restrict__ bias) {
  constexpr int WM = 32 * MT, WN = 32 * NT;
  if constexpr (NT == 1) {
    const int t = c & 3;
    const int col = n0 + wn * WN + (c & ~3);
    const float b0 = bias[col], b1 = bias[col + 1], b2 = bias[col + 2], b3 = bias[col + 3];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v0 = acc[i][0][4 * q], v1 = acc[i][0][4 * q + 1], v2 = acc[i][0][4 * q + 2],
              v3 = acc[i][0][4 * q + 3];
        quad_transpose(v0, v1, v2, v3, t);
        const int row = m0 + wm * WM + i * 32 + 8 * q + 4 * h + t;
        *reinterpret_cast<f32x4*>(C + static_cast<int64_t>(row) * N + col) =
            f32x4{epi_act<ACT>(alpha * v0, b0), epi_act<ACT>(alpha * v1, b1),
                  epi_act<ACT>(alpha * v2, b2), epi_act<ACT>(alpha * v3, b3)};
      }
    }
  } else if constexpr (NT == 2) {
    const int col = n0 + wn * WN + 2 * c;
    const float b0 = bias[col], b1 = bias[col + 1];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        *reinterpret_cast<f32x2*>(C + static_cast<int64_t>(row) * N + col) =
            f32x2{epi_act<ACT>(alpha * acc[i][0][r], b0), epi_act<ACT>(alpha * acc[i][1][r], b1)};
      }
    }
  } else {
    static_assert(NT == 4, "wave tiles are 1, 2 or 4 MFMA tiles wide");
    const int col = n0 + wn * WN + 4 * c;
    const float b0 = bias[col], b1 = bias[col + 1], b2 = bias[col + 2], b3 = bias[col + 3];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        *reinterpret_cast<f32x4*>(C + static_cast<int64_t>(row) * N + col) =
            f32x4{epi_act<ACT>(alpha * acc[i][0][r], b0), epi_act<ACT>(alpha * acc[i][1][r], b1),
                  epi_act<ACT>(alpha * acc[i][2][r], b2), epi_act<ACT>(alpha * acc[i][3][r], b3)};
      }
    }
  }
}

// The store at a kernel's end: plain, or fused with the activation picked once
// (a uniform branch around four copies of the store loop).
template <int MT, int NT, bool VEC, bool WHOLE, bool FUSED>
__device__ __forceinline__ void mfma_epilogue(const f32x16 (&acc)[MT][NT], float* __restrict__ C,
                                              int M, int N, int m0, int n0, int wm, int wn, int h,
                                              int c, float alpha, float beta, EpiArgs epi) {
  if constexpr (!FUSED) {
    if constexpr (WHOLE)
      mfma_store_c_whole<MT, NT>(acc, C, N, m0, n0, wm, wn, h, c, alpha, beta);
    else
      mfma_store_c<MT, NT, VEC>(acc, C, M, N, m0, n0, wm, wn, h, c, alpha, beta);
  } else {
    auto store = [&]<int ACT>() {
      if constexpr (WHOLE)
        mfma_store_c_whole_act<MT, NT, ACT>(acc, C, N, m0, n0, wm, wn, h, c, alpha, epi.bias);
      else
        mfma_store_c_act<MT, NT, VEC, ACT>(acc, C, M, N, m0, n0, wm, wn, h, c, alpha, epi.bias);
    };
    switch (epi.act) {
      case kActNone: store.template operator()<kActNone>(); break;
      case kActRelu: store.template operator()<kActRelu>(); break;
      case kActGeluErf: store.template operator()<kActGeluErf>(); break;
      default: store.template operator()<kActGeluTanh>(); break;
    }
  }
}

template <int BM, int BN, int BK>
struct MfmaVecIO {
  using S = MfmaStage<BM, BN, BK, true>;
  static constexpr int kLoads = S::kAVec + S::kBVec;

  // One of the stage's float4 loads: i < kAVec is A's i-th, else B's (i - kAVec)-th.
  // EVEN (M, N, K multiples of the tile) drops the bounds checks.
  template <bool EVEN>
  static __device__ __forceinline__ void load_one(typename S::Regs& R, int i,
                                                  const float* __restrict__ A,
                                                  const float* __restrict__ B, int M, int N,
                                                  int K, int m0, int n0, int k0) {
    const int t = threadIdx.x;
    if (i < S::kAVec) {
      const int li = i * kMfmaThreads + t;
      const int row = li / (BK / 4), c4 = li % (BK / 4);
      const int gm = m0 + row, gk = k0 + 4 * c4;
      if (EVEN || (gm < M && gk < K))
        R.a[i] = *reinterpret_cast<const f32x4*>(A + static_cast<int64_t>(gm) * K + gk);
      else
        R.a[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      const int ib = i - S::kAVec;
      const int li = ib * kMfmaThreads + t;
      const int kr = li / (BN / 4), c4 = li % (BN / 4);
      const int gk = k0 + kr, gn = n0 + 4 * c4;
      if (EVEN || (gk < K && gn < N))
        R.b[ib] = *reinterpret_cast<const f32x4*>(B + static_cast<int64_t>(gk) * N + gn);
      else
        R.b[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  static __device__ __forceinline__ void store_one(const typename S::Regs& R, int i,
                                                   float* __restrict__ stage) {
    const int t = threadIdx.x;
    if (i < S::kAVec) {
      const int li = i * kMfmaThreads + t;
      const int row = li / (BK / 4), c4 = li % (BK / 4);
      *reinterpret_cast<f32x4*>(stage + row * S::kLdA + 4 * c4) = R.a[i];
    } else {
      const int ib = i - S::kAVec;
      const int li = ib * kMfmaThreads + t;
      const int kr = li / (BN / 4), c4 = li % (BN / 4);
      *reinterpret_cast<f32x4*>(stage + S::kAFloats + kr * S::kLdB + 4 * c4) = R.b[ib];
    }
  }
};

// Waves of one group: a 2 x 2 grid over the tile for tiles of 64 and more, one
// wave across a dimension of 32.  A kernel with more waves than one group runs
// several groups, which split each stage's K range (see gemm_mfma_dma_kernel).
template <int BM> constexpr int kMfmaWaveRows = BM >= 64 ? 2 : 1;
template <int BN> constexpr int kMfmaWaveCols = BN >= 64 ? 2 : 1;
template <int BM, int BN, int KS>
constexpr int kDmaThreads = kWave * kMfmaWaveRows<BM> * kMfmaWaveCols<BN> * KS;

template <int BM, int BN, int BK, bool VEC, bool EVEN, bool FUSED = false>
__global__ __launch_bounds__(kMfmaThreads, 1) void gemm_mfma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, float alpha, float beta, int tiles_m, int tiles_n, EpiArgs epi) {
  // The 256 lanes form one 2 x 2 wave grid for tiles of 64 and more; a 32 x 32
  // tile is one wave wide and high, and its 4 waves are 4 groups splitting each
  // stage's K range, folded in group order at the end.
  constexpr int WGM = kMfmaWaveRows<BM>, WGN = kMfmaWaveCols<BN>;
  constexpr int WPG = WGM * WGN;
  constexpr int KS = (kMfmaThreads / kWave) / WPG;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MT = WM / 32, NT = WN / 32;
  static_assert(MT >= 1 && WM == 32 * MT && (NT == 1 || NT == 2 || NT == 4),
                "unsupported wave tile");
  static_assert(KS * WPG * kWave == kMfmaThreads, "the waves must form whole groups");
  static_assert(BK % 8 == 0, "BK must be a multiple of 8 (two halves of 4-deep reads)");
  constexpr int Q = BK / 8;             // k-quarters per stage
  static_assert(Q % KS == 0, "the k-quarters must split over the wave groups");
  constexpr int QG = Q / KS;            // k-quarters per wave group
  using S = MfmaStage<BM, BN, BK, VEC>;
  static_assert(KS == 1 || (KS - 1) * WPG * MT * NT * 16 * kWave <= 2 * S::kStageFloats,
                "the groups' accumulators must fit in the stage buffers");
  using BV = typename BVec<NT>::type;

  __shared__ __attribute__((aligned(16))) float smem[2 * S::kStageFloats];

  int tm, tn;
  mfma_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int kg = wave / WPG;            // wave group (K split)
  const int wg = wave % WPG;            // wave within its group
  const int wm = wg / WGN, wn = wg % WGN;
  const int h = lane / 32, c = lane % 32;

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ksteps = (K + BK - 1) / BK;
  typename S::Regs R;
  if (ksteps > 0) {
    S::load(R, A, B, M, N, K, m0, n0, 0);
    S::store(R, smem);
  }
  __syncthreads();

  // Per-lane LDS offsets (floats) inside a stage, at this wave group's first
  // k-quarter.
  const int a_off = (wm * WM + c) * S::kLdA + h * (BK / 2) + 4 * kg * QG;
  const int b_off = S::kAFloats + (h * (BK / 2) + 4 * kg * QG) * S::kLdB + wn * WN + NT * c;

  // The next stage's global loads and LDS stores.  On the 16-byte path they are
  // spread over the MFMA stream of the current stage -- loads over the first half
  // of its P = BK/2 MFMA sub-steps, stores (into the other LDS buffer, free since
  // the previous barrier) over the second half -- so the matrix pipe never waits
  // for their issue.  The last stage re-loads itself (k0 clamped) and stores into
  // the unused buffer: harmless, and it keeps the loop free of branches.
  constexpr int P = 4 * QG;              // MFMA sub-steps per wave per stage
  using IO = MfmaVecIO<BM, BN, BK>;
  constexpr int L = IO::kLoads;

  for (int ks = 0; ks < ksteps; ++ks) {
    const float* stage = smem + (ks & 1) * S::kStageFloats;
    float* next_stage = smem + ((ks + 1) & 1) * S::kStageFloats;
    const bool more = (ks + 1) < ksteps;
    const int k_next = (more ? ks + 1 : ks) * BK;
    if constexpr (!VEC) {
      if (more) S::load(R, A, B, M, N, K, m0, n0, k_next);
    }

    // LDS -> register fragments, software-pipelined one MFMA step ahead: the
    // reads for step (q, s+1) are issued before the MFMAs of step (q, s), so the
    // LDS latency hides under 64 * MT * NT MFMA cycles instead of stalling them.
    f32x4 av[MT], av_next[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
      av[i] = *reinterpret_cast<const f32x4*>(stage + a_off + i * 32 * S::kLdA);
    BV bv = *reinterpret_cast<const BV*>(stage + b_off);
#pragma unroll
    for (int q = 0; q < QG; ++q) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int p = 4 * q + s;
        BV bv_next = bv;
        if (s < 3) {
          bv_next = *reinterpret_cast<const BV*>(stage + b_off + (4 * q + s + 1) * S::kLdB);
        } else if (q + 1 < QG) {
          bv_next = *reinterpret_cast<const BV*>(stage + b_off + (4 * q + 4) * S::kLdB);
#pragma unroll
          for (int i = 0; i < MT; ++i)
            av_next[i] = *reinterpret_cast<const f32x4*>(stage + a_off + i * 32 * S::kLdA +
                                                         4 * (q + 1));
        }
        if constexpr (VEC) {
#pragma unroll
          for (int i = 0; i < L; ++i)
            if ((i * (P / 2)) / L == p)
              IO::template load_one<EVEN>(R, i, A, B, M, N, K, m0, n0, k_next);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
          for (int jj = 0; jj < NT; ++jj) {
            const int j = mfma_snake_col(i, jj, NT);
            float bj;
            if constexpr (NT == 1) bj = bv; else bj = bv[j];
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bj, acc[i][j], 0, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (VEC) {
#pragma unroll
          for (int i = 0; i < L; ++i)
            if (P / 2 + (i * (P / 2)) / L == p) IO::store_one(R, i, next_stage);
        }
        bv = bv_next;
        if (s == 3 && q + 1 < QG) {
#pragma unroll
          for (int i = 0; i < MT; ++i) av[i] = av_next[i];
        }
      }
    }

    if constexpr (!VEC) {
      if (more) S::store(R, next_stage);
    }
    __syncthreads();
  }

  if constexpr (KS > 1) {
    // Groups 1 .. KS-1 park their accumulators in the stage buffers (free after
    // the loop's last barrier), lane-contiguous per register; group 0 adds them in
    // group order.
    auto slot = [&](int g, int i, int j, int r) {
      return ((((g - 1) * WPG + wg) * MT + i) * NT + j) * 16 * kWave + r * kWave + lane;
    };
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) smem[slot(kg, i, j, r)] = acc[i][j][r];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += smem[slot(g, i, j, r)];
  }

  mfma_epilogue<MT, NT, VEC, false, FUSED>(acc, C, M, N, m0, n0, wm, wn, h, c, alpha, beta, epi);
}


// ---------------------------------------------------------------------------
// Whole-tile variant with direct-to-LDS loads (gfx950 global_load_lds_dwordx4).
//
// For M % BM == N % BN == K % 32 == 0 and 16-byte aligned A and B.  The next
// stage is fetched straight from global memory into the other LDS buffer: no
// VGPR staging, no ds_write, and no wait on the loads until the step's closing
// barrier.  One such instruction writes its 64 lanes' 16 bytes to 1 KB of
// contiguous LDS (lane j at byte 16 j of a wave-uniform base), so the layouts are
// chosen per 1 KB chunk:
//   B (BK x BN, row-major, unpadded): chunk c holds elements [256 c, 256 c + 256)
//     of the stage, lane j the float4 at element 256 c + 4 j;
//   A (BM x 32, 128-byte rows, unpadded): chunk c holds rows 8c .. 8c+7; the
//     float4 at position p of row r holds k-slot p ^ f(r), f(r) = (r & 7) ^
//     ((r >> 3) & 1).  The MFMA fragment reads fetch one k-slot from 32
//     consecutive rows; the swizzle puts any 8 (or 16) consecutive rows of a slot
//     on distinct 16-byte bank groups, so they are conflict-free without padding.
// ---------------------------------------------------------------------------
// One global_load_lds_dwordx4 in its SGPR-base form: lane l's 16 bytes at
// base + voff + OFF land at LDS byte m0 + OFF + 16 l (the immediate offset applies
// to both addresses, so up to four consecutive 1 KB chunks share one M0).  The
// 64-bit base is wave-uniform and the per-lane offset 32-bit: the generic form's
// 64-bit per-lane address cost a 64-bit VALU add and a v_readfirstlane for M0
// per instruction, issued between the MFMAs (16-bit GEMM, 8192^3 bf16: 1345 vs
// 1215 cycles per K step).  The s_nop covers an M0 write just before the
// instruction.
template <int OFF>
__device__ __forceinline__ void lds_dma16(uint32_t voff, const void* base, uint32_t m0) {
  static_assert(OFF >= 0 && OFF < 4096, "immediate offsets are 12-bit here");
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:%2"
               :: "v"(voff), "s"(base), "i"(OFF), "{m0}"(m0) : "memory");
}

// Issues direct-to-LDS instruction I of a wave's share of one stage (A chunks
// first, then B chunks) for K columns [k0, k0 + 32): 16 bytes per lane into the
// 1 KB chunk of the stage at LDS address `stage` that the instruction owns.
// offA / offB are the lanes' byte offsets from a_base / b_base for k0 = 0, less
// the instruction's immediate offset ((I % 4) KB within its operand); `wave` is
// the wave index as a uniform value.
template <int I, int NA, int NB>
__device__ __forceinline__ void mfma_dma_issue(int a_floats, const uint32_t (&offA)[NA],
                                               const uint32_t (&offB)[NB], const char* a_base,
                                               const char* b_base, int64_t stepB_bytes,
                                               uint32_t stage, int k0, uint32_t wave) {
  if constexpr (I < NA) {
    lds_dma16<(I % 4) * 1024>(offA[I], a_base + static_cast<int64_t>(k0) * 4,
                              stage + (wave * NA + (I & ~3)) * 1024);
  } else {
    constexpr int IB = I - NA;
    lds_dma16<(IB % 4) * 1024>(offB[IB], b_base + static_cast<int64_t>(k0 / 32) * stepB_bytes,
                               stage + a_floats * 4 + (wave * NB + (IB & ~3)) * 1024);
  }
}

// KS > 1 splits each stage's K range over KS groups of waves (each group a 2 x 2
// grid, or 1 x 1 for a 32 x 32 tile): group g runs the MFMA sub-steps of k-quarters [g Q/KS, (g+1) Q/KS)
// of every stage into accumulators of its own, all groups read the same LDS
// stages, and at the end groups 1 .. KS-1 hand their accumulators to group 0
// through LDS, which adds them in group order and writes C.  The 32 x 32 tile,
// one wave wide and high, uses it to give its workgroup four waves.  The sum
// order over K differs from KS = 1 (the groups' partials are added last), and is
// fixed for a given KS.
template <int BM, int BN, int STAGES, int KS = 1, bool FUSED = false>
__global__ __launch_bounds__((kDmaThreads<BM, BN, KS>), 1) void gemm_mfma_dma_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, float alpha, float beta, int tiles_m, int tiles_n, EpiArgs epi) {
  constexpr int BK = 32;
  constexpr int WGM = kMfmaWaveRows<BM>, WGN = kMfmaWaveCols<BN>;
  constexpr int WPG = WGM * WGN;        // waves per group
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int MT = WM / 32, NT = WN / 32;
  static_assert(MT >= 1 && WM == 32 * MT && (NT == 1 || NT == 2 || NT == 4),
                "unsupported wave tile");
  constexpr int kWaves = WPG * KS;
  constexpr int kAFloats = BM * BK;
  constexpr int kStageFloats = kAFloats + BK * BN;
  constexpr int kAChunks = kAFloats / 256, kBChunks = BK * BN / 256;   // 1 KB chunks
  constexpr int NA = kAChunks / kWaves, NB = kBChunks / kWaves;         // per wave
  static_assert(kAChunks % kWaves == 0 && kBChunks % kWaves == 0,
                "chunks must split over the workgroup's waves");
  constexpr int L = NA + NB;            // DMA instructions per wave per stage
  constexpr int Q = BK / 8;             // k-quarters per stage (4 MFMA sub-steps each)
  static_assert(Q % KS == 0, "the k-quarters must split over the wave groups");
  constexpr int QG = Q / KS;            // k-quarters per wave group
  constexpr int P = 4 * QG;             // MFMA sub-steps per wave per stage
  using BV = typename BVec<NT>::type;
  static_assert(STAGES >= 2 && (STAGES - 2) * L <= 63, "vmcnt counts at most 63 loads");
  static_assert(KS == 1 || (KS - 1) * WPG * MT * NT * 16 * kWave <= STAGES * kStageFloats,
                "the groups' accumulators must fit in the stage buffers");

  __shared__ __attribute__((aligned(16))) float smem[STAGES * kStageFloats];

  int tm, tn;
  mfma_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int kg = wave / WPG;            // wave group (K split)
  const int wg = wave % WPG;            // wave within its group
  const int wm = wg / WGN, wn = wg % WGN;
  const int h = lane / 32, c = lane % 32;

  // This lane's source byte offsets for its wave's chunks of stage 0, from the
  // uniform bases A + m0 K and B + n0 (advanced by BK columns of A and BK rows of
  // B per stage), less each instruction's immediate offset.  The launcher keeps
  // BM K and 32 N below 2^30 floats, so they fit 32 bits; row >= 8 ii (A) and
  // (e / BN) N + e % BN >= e >= 256 ii (B, N >= BN) keep them non-negative.
  const int jr = lane / 8, jp = lane % 8;
  uint32_t offA[NA], offB[NB];
#pragma unroll
  for (int ii = 0; ii < NA; ++ii) {
    const int ch = wave * NA + ii;
    const int row = 8 * ch + jr;
    const int slot = jp ^ jr ^ (ch & 1);          // f(row) = jr ^ (ch & 1)
    offA[ii] = (static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + 4u * slot) * 4u -
               1024u * (ii % 4);
  }
#pragma unroll
  for (int ii = 0; ii < NB; ++ii) {
    const int e = (wave * NB + ii) * 256 + 4 * lane;
    offB[ii] = (static_cast<uint32_t>(e / BN) * static_cast<uint32_t>(N) + e % BN) * 4u -
               1024u * (ii % 4);
  }
  const char* a_base = reinterpret_cast<const char*>(A + static_cast<int64_t>(m0) * K);
  const char* b_base = reinterpret_cast<const char*>(B + n0);
  const int64_t stepB_bytes = static_cast<int64_t>(BK) * N * 4;
  const uint32_t wave_u = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wave));
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char*)(smem)));

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ksteps = K / BK;
  // Prologue: stages 0 .. STAGES-2 in flight.  Past the last K step a stage
  // re-fetches the last one into a buffer nobody reads, which keeps the number of
  // loads per stage -- and so the vmcnt arithmetic below -- uniform.
  if (ksteps > 0) {
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) {
      const int kk = (st < ksteps ? st : ksteps - 1) * BK;
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (mfma_dma_issue<I, NA, NB>(kAFloats, offA, offB, a_base, b_base, stepB_bytes,
                                   lds0 + st * kStageFloats * 4, kk, wave_u),
         ...);
      }(std::make_integer_sequence<int, L>{});
    }
  }

  // Fragment addressing: rows wm*WM + i*32 + c all share f = f(c) (the row base
  // is a multiple of 16); k-slot 4h + q sits at position (4h + q) ^ f.  This
  // wave's group walks k-quarters q = kg*QG + qq, qq < QG.
  const int f = (c & 7) ^ ((c >> 3) & 1);
  const int a_row = (wm * WM + c) * BK;
  int a_q[QG];
#pragma unroll
  for (int qq = 0; qq < QG; ++qq) a_q[qq] = 4 * ((4 * h + kg * QG + qq) ^ f);
  const int b_off = kAFloats + (h * (BK / 2) + 4 * kg * QG) * BN + wn * WN + NT * c;

  if constexpr (STAGES >= 3 && KS > 1) {
    // The ring with its barrier in the middle of a step (as below), for wave
    // groups that split K: a group's share of a stage is only P = 4 QG sub-steps,
    // too short for reads one sub-step ahead to hide LDS latency.  Instead all of
    // stage ks + 1's fragments are read right after the barrier that publishes it,
    // into the other of two register sets, while the second half of stage ks's
    // MFMAs runs; the next step's MFMAs then never wait on a read (32 x 32 tile at
    // 512^3: 5.27 vs 5.88 us, the same bits; for the 64 x 64 tile, one group of 16
    // sub-steps, it measured slower than the reads one ahead: 20.0 vs 19.2 us at
    // 1024^3).  Steps come in pairs so that the register sets alternate by name.
    if (ksteps > 0) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 2) * L) : "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    static_assert(P % 2 == 0 && QG <= P / 2, "reads of the next stage fit the second half");
    f32x4 af[2][QG][MT];
    BV bf[2][P];
#pragma unroll
    for (int qq = 0; qq < QG; ++qq)
#pragma unroll
      for (int i = 0; i < MT; ++i)
        af[0][qq][i] = *reinterpret_cast<const f32x4*>(smem + a_row + i * 32 * BK + a_q[qq]);
#pragma unroll
    for (int p = 0; p < P; ++p) bf[0][p] = *reinterpret_cast<const BV*>(smem + b_off + p * BN);
    auto step = [&]<int PP>(int ks) {
      // Past the last step the reads below fetch a buffer whose values go unused.
      const float* stage_n = smem + ((ks + 1) % STAGES) * kStageFloats;
      const uint32_t next_stage = lds0 + ((ks + STAGES - 1) % STAGES) * kStageFloats * 4;
      const int kf = ks + STAGES - 1;
      const int k_next = (kf < ksteps ? kf : ksteps - 1) * BK;
#pragma unroll
      for (int qq = 0; qq < QG; ++qq) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int p = 4 * qq + s;
          if (p == P / 2) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 3) * L) : "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
          }
          if (p >= P / 2) {
            // Sub-step P/2 + x reads B rows 2x, 2x + 1 and, for x < QG, A quarter x.
            const int x = p - P / 2;
            bf[1 - PP][2 * x] = *reinterpret_cast<const BV*>(stage_n + b_off + (2 * x) * BN);
            bf[1 - PP][2 * x + 1] =
                *reinterpret_cast<const BV*>(stage_n + b_off + (2 * x + 1) * BN);
            if (x < QG) {
              const int xq = x < QG ? x : 0;   // (keeps the unrolled indices in range)
#pragma unroll
              for (int i = 0; i < MT; ++i)
                af[1 - PP][xq][i] =
                    *reinterpret_cast<const f32x4*>(stage_n + a_row + i * 32 * BK + a_q[xq]);
            }
          }
          // The fetch of stage ks + STAGES - 1, spread over the second half.
          [&]<int... I>(std::integer_sequence<int, I...>) {
            ((P / 2 + (I * (P / 2)) / L == p
                  ? mfma_dma_issue<I, NA, NB>(kAFloats, offA, offB, a_base, b_base, stepB_bytes,
                                              next_stage, k_next, wave_u)
                  : void()),
             ...);
          }(std::make_integer_sequence<int, L>{});
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              const int j = mfma_snake_col(i, jj, NT);
              float bj;
              if constexpr (NT == 1) bj = bf[PP][p]; else bj = bf[PP][p][j];
              acc[i][j] =
                  __builtin_amdgcn_mfma_f32_32x32x2f32(af[PP][qq][i][s], bj, acc[i][j], 0, 0, 0);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    for (int ks = 0; ks < ksteps; ks += 2) {
      step.template operator()<0>(ks);
      if (ks + 1 < ksteps) step.template operator()<1>(ks + 1);
    }
  } else if constexpr (STAGES >= 3) {
    // With three or more stages the barrier sits in the middle of a step: after
    // half of stage ks's sub-steps it publishes stage ks + 1 and retires the
    // buffer of stage ks - 1, whose fetch (stage ks + STAGES - 1) then issues over
    // the second half.  The fragment reads run one sub-step ahead of the MFMAs,
    // across the barrier and across steps, so the matrix pipe does not drain at
    // the barrier or wait on a fresh fragment read at the top of a step (1024^3,
    // 64 x 64 tile, the two-group 8-stage ring of the time: 103.6-104.3 vs 100.5
    // TFLOP/s; reading B two sub-steps ahead measured the same).
    if (ksteps > 0) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 2) * L) : "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    f32x4 av[MT], av_next[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
      av[i] = *reinterpret_cast<const f32x4*>(smem + a_row + i * 32 * BK + a_q[0]);
    BV bv = *reinterpret_cast<const BV*>(smem + b_off);
    auto mfmas = [&](int s) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int jj = 0; jj < NT; ++jj) {
          const int j = mfma_snake_col(i, jj, NT);
          float bj;
          if constexpr (NT == 1) bj = bv; else bj = bv[j];
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bj, acc[i][j], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int ks = 0; ks < ksteps; ++ks) {
#pragma unroll
      for (int qq = 0; qq < QG; ++qq) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int p = 4 * qq + s;
          if (p == P / 2) {
            // Stage ks + 1 has landed once at most the (STAGES - 3) younger stages'
            // loads are outstanding.  A bare s_barrier, as below.
            asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 3) * L) : "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
          }
          // Sub-step 0 issues its MFMAs before its reads: a read issued at the top of
          // a step would be waited for by the step's first MFMA, since the wait at the
          // loop's head cannot tell it from the fragments read in the step before
          // (64 x 64 tile, in-process A/B on MI355X: 1-1.5% faster at 1024^3,
          // 1024 x 1024 x 4096 and 1536^3, the same bits).  The other sub-steps read
          // one ahead before their MFMAs.
          if (p == 0) mfmas(0);
          const float* stage = smem + (ks % STAGES) * kStageFloats;
          const float* stage_n = smem + ((ks + 1) % STAGES) * kStageFloats;
          BV bv_next;
          if (s < 3) {
            bv_next = *reinterpret_cast<const BV*>(stage + b_off + (p + 1) * BN);
          } else if (qq + 1 < QG) {
            bv_next = *reinterpret_cast<const BV*>(stage + b_off + (p + 1) * BN);
#pragma unroll
            for (int i = 0; i < MT; ++i)
              av_next[i] =
                  *reinterpret_cast<const f32x4*>(stage + a_row + i * 32 * BK + a_q[qq + 1]);
          } else {
            // First sub-step of stage ks + 1 (published by this step's barrier).
            bv_next = *reinterpret_cast<const BV*>(stage_n + b_off);
#pragma unroll
            for (int i = 0; i < MT; ++i)
              av_next[i] = *reinterpret_cast<const f32x4*>(stage_n + a_row + i * 32 * BK + a_q[0]);
          }
          if (p >= P / 2) {
            // The fetch of stage ks + STAGES - 1, spread over the second half.
            const uint32_t next_stage = lds0 + ((ks + STAGES - 1) % STAGES) * kStageFloats * 4;
            const int kf = ks + STAGES - 1;
            const int k_next = (kf < ksteps ? kf : ksteps - 1) * BK;
            [&]<int... I>(std::integer_sequence<int, I...>) {
              ((P / 2 + (I * (P / 2)) / L == p
                    ? mfma_dma_issue<I, NA, NB>(kAFloats, offA, offB, a_base, b_base, stepB_bytes,
                                                next_stage, k_next, wave_u)
                    : void()),
               ...);
            }(std::make_integer_sequence<int, L>{});
          }
          if (p != 0) mfmas(s);
          bv = bv_next;
          if (s == 3) {
#pragma unroll
            for (int i = 0; i < MT; ++i) av[i] = av_next[i];
          }
        }
      }
    }
  } else {
    for (int ks = 0; ks < ksteps; ++ks) {
      // Stage ks has landed once at most the (STAGES - 2) younger stages' loads are
      // still outstanding; the barrier then publishes every wave's share of it and
      // retires every wave's reads of the buffer that the next fetch overwrites
      // (the one read in step ks - 1).
      // A bare s_barrier: __syncthreads() would also drain every outstanding load
      // (vmcnt(0)), which serialises the pipeline.  Each wave's ds_reads of the
      // buffer being refilled were already waited on by the MFMAs that used them,
      // and the asm statements keep the compiler from moving memory accesses
      // across the barrier.
      asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 2) * L) : "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const float* stage = smem + (ks % STAGES) * kStageFloats;
      const uint32_t next_stage = lds0 + ((ks + STAGES - 1) % STAGES) * kStageFloats * 4;
      const int kf = ks + STAGES - 1;
      const int k_next = (kf < ksteps ? kf : ksteps - 1) * BK;

      f32x4 av[MT], av_next[MT];
  #pragma unroll
      for (int i = 0; i < MT; ++i)
        av[i] = *reinterpret_cast<const f32x4*>(stage + a_row + i * 32 * BK + a_q[0]);
      BV bv = *reinterpret_cast<const BV*>(stage + b_off);
  #pragma unroll
      for (int qq = 0; qq < QG; ++qq) {
  #pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int p = 4 * qq + s;
          BV bv_next = bv;
          if (s < 3) {
            bv_next = *reinterpret_cast<const BV*>(stage + b_off + (4 * qq + s + 1) * BN);
          } else if (qq + 1 < QG) {
            bv_next = *reinterpret_cast<const BV*>(stage + b_off + (4 * qq + 4) * BN);
  #pragma unroll
            for (int i = 0; i < MT; ++i)
              av_next[i] =
                  *reinterpret_cast<const f32x4*>(stage + a_row + i * 32 * BK + a_q[qq + 1]);
          }
          // The fetch of stage ks + STAGES - 1, spread over the first half of the
          // sub-steps so that its issue hides under the MFMAs.
          [&]<int... I>(std::integer_sequence<int, I...>) {
            (((I * (P / 2)) / L == p
                  ? mfma_dma_issue<I, NA, NB>(kAFloats, offA, offB, a_base, b_base, stepB_bytes,
                                              next_stage, k_next, wave_u)
                  : void()),
             ...);
          }(std::make_integer_sequence<int, L>{});
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int i = 0; i < MT; ++i) {
  #pragma unroll
            for (int jj = 0; jj < NT; ++jj) {
              const int j = mfma_snake_col(i, jj, NT);
              float bj;
              if constexpr (NT == 1) bj = bv; else bj = bv[j];
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bj, acc[i][j], 0, 0, 0);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          bv = bv_next;
          if (s == 3 && qq + 1 < QG) {
  #pragma unroll
            for (int i = 0; i < MT; ++i) av[i] = av_next[i];
          }
        }
      }
    }
  }
  // No LDS DMA may still be landing when the workgroup retires (or, with KS > 1,
  // when the stage buffers are reused below).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (KS > 1) {
    // Groups 1 .. KS-1 park their accumulators in the (now idle) stage buffers,
    // lane-contiguous per register; group 0 adds them in group order.
    __syncthreads();
    auto slot = [&](int g, int i, int j, int r) {
      return ((((g - 1) * WPG + wg) * MT + i) * NT + j) * 16 * kWave + r * kWave + lane;
    };
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) smem[slot(kg, i, j, r)] = acc[i][j][r];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += smem[slot(g, i, j, r)];
  }

  mfma_epilogue<MT, NT, true, true, FUSED>(acc, C, M, N, m0, n0, wm, wn, h, c, alpha, beta, epi);
}

}  // namespace mcke_amd
