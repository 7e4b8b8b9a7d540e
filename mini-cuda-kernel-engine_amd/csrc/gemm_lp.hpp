// gemm_lp.hpp -- 16-bit-input GEMM on the CDNA4 matrix cores
// (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x16_f16), fp32 accumulation.
//
// C[M,N] = alpha * A[M,K] B[K,N] + beta * C, row-major; A and B in bf16 or fp16,
// C in fp32 or in the input type (rounded to nearest even on the store).
//
// Workgroup: 256 lanes = 4 wave64s in a 2 x 2 grid; the workgroup owns a BM x BN
// tile of C, each wave a WM x WN sub-tile of (WM/32) x (WN/32) MFMA 32x32 tiles
// held in accumulation registers for the whole K loop.  K is staged 64 deep.
//
// Operand delivery.  One v_mfma_f32_32x32x16 takes, per lane l, eight 16-bit A
// values of row l%32 and eight B values of column l%32, the two lane halves
// (h = l/32) covering disjoint k ranges.  Which eight k's a lane half takes is
// free (the sum over k does not care) as long as A and B agree, so both operands
// are kept k-contiguous in LDS and each fragment is one 16-byte ds_read:
//   As[BM][64]   row m of A, k contiguous (the global layout, copied as is);
//   Bs[BN][64]   column n of B, k contiguous: B arrives row-major (n contiguous),
//                so each lane loads an 8(or 4, 2)-row x 8-column block of B and
//                transposes it in registers (16-bit lane shuffles within dwords)
//                before its LDS store.
// MFMA sub-step s (of 4) reads 16-byte chunk q = 2s + h of each row.
//
// LDS rows are 128 bytes (8 chunks); chunk q of row r is stored at position
// q ^ g(r), g(r) = (r & 7) ^ ((r >> 3) & 7).  A fragment read touches 32
// consecutive rows at one chunk: any 8 of them land on 8 distinct positions, and
// rows 8 apart differ in (r >> 3) & 1, which XOR-flips the position's low bit
// against the row's own parity, so 16 consecutive rows also cover every bank.
//
// Columns are permuted per wave, as in the fp32 MFMA kernel: n-tile j at lane
// column c computes block column WN*wn + NT*c + j, so in the epilogue a lane
// holds NT adjacent columns of an output row (one vector store).  Bs row
// WN*wn + 32*j + c holds that column, so the fragment reads stay on 32
// consecutive rows.
//
// Accumulator layout of one 32x32 tile (lane l, register r = 0..15):
//   row = 8*(r/4) + 4*(l/32) + (r%4),   col = l%32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gemm_mfma.hpp"

namespace mcke_amd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kLpBK = 64;            // K depth of one LDS stage (elements)
constexpr int kLpRowBytes = 128;     // one LDS row: 64 16-bit values

// Input element type -> its MFMA.
template <typename T> struct LpMfma;
template <> struct LpMfma<__bf16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct LpMfma<_Float16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Output element conversions (round to nearest even for the 16-bit types).
template <typename O> struct LpOut;
template <> struct LpOut<float> {
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};
template <> struct LpOut<__bf16> {
  static __device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }
  static __device__ __forceinline__ __bf16 from_f32(float v) { return static_cast<__bf16>(v); }
};
template <> struct LpOut<_Float16> {
  static __device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
  static __device__ __forceinline__ _Float16 from_f32(float v) {
    return static_cast<_Float16>(v);
  }
};

__device__ __forceinline__ int lp_swz(int r) { return (r & 7) ^ ((r >> 3) & 7); }

// Loads eight consecutive 16-bit values p[0..7] whose first index is `k` along a
// row of length `len`; VEC: one 16-byte load (len % 8 == 0, p 16-byte aligned,
// so the chunk is wholly in or out of range); else per-element loads.  Elements
// outside [0, len) -- and the whole chunk when !in_row -- read as +0.
template <bool VEC, bool EVEN>
__device__ __forceinline__ u32x4 lp_load8(const uint16_t* __restrict__ p, int k, int len,
                                          bool in_row) {
  if constexpr (VEC) {
    if (EVEN || (in_row && k < len)) return *reinterpret_cast<const u32x4*>(p);
    return u32x4{0u, 0u, 0u, 0u};
  } else {
    unsigned v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (in_row && k + e < len) ? p[e] : 0u;
    return u32x4{v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                 v[6] | (v[7] << 16)};
  }
}

template <int BM, int BN>
struct LpStage {
  static constexpr int kThreads = kMfmaThreads;
  static constexpr int WN = BN / 2;
  static constexpr int NT = WN / 32;
  static constexpr int kABytes = BM * kLpRowBytes;
  static constexpr int kBytes = (BM + BN) * kLpRowBytes;
  // A: BM rows x 8 chunks, spread over the workgroup.
  static constexpr int kAChunks = BM * 8 / kThreads;
  // B: the K x BN slab cut into KR x 8 blocks, one per lane.
  static constexpr int KR = BN / 32;
  static constexpr int kBGroups = BN / 8;       // 8-column groups across the slab
  static_assert(BM * 8 % kThreads == 0, "A stage must split over the workgroup");
  static_assert(KR == 2 || KR == 4 || KR == 8, "BN must be 64, 128 or 256");
  static_assert((kLpBK / KR) * kBGroups == kThreads, "one B block per lane");

  struct Regs {
    u32x4 a[kAChunks];
    u32x4 b[KR];
  };

  // LDS row of block column n (the per-wave column permutation).
  static __device__ __forceinline__ int brow(int n) {
    const int w = n / WN, nl = n % WN;
    return w * WN + (nl % NT) * 32 + nl / NT;
  }

  template <bool VEC, bool EVEN>
  static __device__ __forceinline__ void load_a(Regs& R, int i, const uint16_t* __restrict__ A,
                                                int M, int K, int m0, int k0) {
    const int li = i * kThreads + static_cast<int>(threadIdx.x);
    const int row = li / 8, kc = li % 8;
    const int gm = m0 + row, gk = k0 + 8 * kc;
    const uint16_t* p = A + static_cast<int64_t>(EVEN || gm < M ? gm : 0) * K + gk;
    R.a[i] = lp_load8<VEC, EVEN>(p, gk, K, EVEN || gm < M);
  }

  template <bool VEC, bool EVEN>
  static __device__ __forceinline__ void load_b(Regs& R, int i, const uint16_t* __restrict__ B,
                                                int N, int K, int n0, int k0) {
    const int t = static_cast<int>(threadIdx.x);
    const int nb = t % kBGroups, kb = t / kBGroups;
    const int gk = k0 + kb * KR + i, gn = n0 + 8 * nb;
    const bool in_k = EVEN || gk < K;
    const uint16_t* p = B + static_cast<int64_t>(in_k ? gk : 0) * N + gn;
    R.b[i] = lp_load8<VEC, EVEN>(p, gn, N, in_k);
  }

  static __device__ __forceinline__ void store_a(const Regs& R, int i, char* stage) {
    const int li = i * kThreads + static_cast<int>(threadIdx.x);
    const int row = li / 8, kc = li % 8;
    *reinterpret_cast<u32x4*>(stage + row * kLpRowBytes + 16 * (kc ^ lp_swz(row))) = R.a[i];
  }

  // Transposes the lane's KR x 8 block of B (KR k-rows of 8 columns) into 8
  // column vectors of KR k-values and stores them to their LDS rows.
  static __device__ __forceinline__ void store_b(const Regs& R, char* stage) {
    const int t = static_cast<int>(threadIdx.x);
    const int nb = t % kBGroups, kb = t / kBGroups;
    const int kofs = kb * KR;                      // first k of the block in the stage
    const int kc = kofs / 8, kin = kofs % 8;       // chunk, element offset in it
    char* bs = stage + kABytes;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      unsigned d[KR / 2];
#pragma unroll
      for (int e = 0; e < KR / 2; ++e) {
        const unsigned x = R.b[2 * e][j / 2], y = R.b[2 * e + 1][j / 2];
        d[e] = (j % 2 == 0) ? ((x & 0xffffu) | (y << 16)) : ((x >> 16) | (y & 0xffff0000u));
      }
      const int row = brow(8 * nb + j);
      char* dst = bs + row * kLpRowBytes + 16 * (kc ^ lp_swz(row)) + 2 * kin;
      if constexpr (KR == 8) *reinterpret_cast<u32x4*>(dst) = u32x4{d[0], d[1], d[2], d[3]};
      else if constexpr (KR == 4) *reinterpret_cast<u32x2*>(dst) = u32x2{d[0], d[1]};
      else *reinterpret_cast<unsigned*>(dst) = d[0];
    }
  }
};

// Epilogue: C = alpha * acc + beta * C (C not read when beta == 0).  VEC: C rows
// are 16-byte aligned when N % NT == 0, so a lane's NT adjacent outputs go out as
// one store.
template <typename OutT, int BM, int BN, bool VEC>
__device__ __forceinline__ void lp_store_c(const f32x16 (&acc)[BM / 64][BN / 64],
                                           OutT* __restrict__ C, int M, int N, int m0, int n0,
                                           int wm, int wn, int h, int c, float alpha,
                                           float beta) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MT = WM / 32, NT = WN / 32;
  using O = LpOut<OutT>;
  const int col0 = n0 + wn * WN + NT * c;
  const bool vec_store = VEC && (N % NT == 0) && col0 + NT - 1 < N;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
      if (row >= M) continue;
      OutT* crow = C + static_cast<int64_t>(row) * N;
      if (vec_store) {
        struct alignas(NT * sizeof(OutT)) Pack { OutT v[NT]; };
        Pack o;
        if (beta != 0.0f) {
          const Pack old = *reinterpret_cast<const Pack*>(crow + col0);
#pragma unroll
          for (int j = 0; j < NT; ++j)
            o.v[j] = O::from_f32(alpha * acc[i][j][r] + beta * O::to_f32(old.v[j]));
        } else {
#pragma unroll
          for (int j = 0; j < NT; ++j) o.v[j] = O::from_f32(alpha * acc[i][j][r]);
        }
        *reinterpret_cast<Pack*>(crow + col0) = o;
      } else {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = col0 + j;
          if (col < N) {
            float v = alpha * acc[i][j][r];
            if (beta != 0.0f) v += beta * O::to_f32(crow[col]);
            crow[col] = O::from_f32(v);
          }
        }
      }
    }
  }
}

// VEC: K % 8 == 0, N % 8 == 0, A/B/C 16-byte aligned.  EVEN: additionally M, N, K
// multiples of the tile (no bounds checks at all).
template <typename T, typename OutT, int BM, int BN, bool VEC, bool EVEN>
__global__ __launch_bounds__(kMfmaThreads, 1) void gemm_lp_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, OutT* __restrict__ C,
    int M, int N, int K, float alpha, float beta, int tiles_m, int tiles_n) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MT = WM / 32, NT = WN / 32;
  static_assert(MT >= 1 && (NT == 1 || NT == 2 || NT == 4), "unsupported wave tile");
  static_assert(!EVEN || VEC, "whole tiles take the 16-byte path");
  using S = LpStage<BM, BN>;
  using MF = LpMfma<T>;

  __shared__ __attribute__((aligned(16))) char smem[2 * S::kBytes];

  int tm, tn;
  mfma_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int h = lane / 32, c = lane % 32;

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ksteps = (K + kLpBK - 1) / kLpBK;
  typename S::Regs R;
  if (ksteps > 0) {
#pragma unroll
    for (int i = 0; i < S::kAChunks; ++i)
      S::template load_a<VEC, EVEN>(R, i, A, M, K, m0, 0);
#pragma unroll
    for (int i = 0; i < S::KR; ++i) S::template load_b<VEC, EVEN>(R, i, B, N, K, n0, 0);
#pragma unroll
    for (int i = 0; i < S::kAChunks; ++i) S::store_a(R, i, smem);
    S::store_b(R, smem);
  }
  __syncthreads();

  // Per-lane fragment rows (byte offsets in a stage) and their swizzle: row
  // base + c with base a multiple of 32, so g(row) = g(c) ^ ((base >> 3) & 4).
  int a_row[MT], a_x[MT], b_row[NT], b_x[NT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int r = wm * WM + 32 * i + c;
    a_row[i] = r * kLpRowBytes;
    a_x[i] = lp_swz(r);
  }
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int r = wn * WN + 32 * j + c;
    b_row[j] = S::kABytes + r * kLpRowBytes;
    b_x[j] = lp_swz(r);
  }

  constexpr int kLoads = S::kAChunks + S::KR;
  for (int ks = 0; ks < ksteps; ++ks) {
    const char* stage = smem + (ks & 1) * S::kBytes;
    char* next_stage = smem + ((ks + 1) & 1) * S::kBytes;
    const bool more = (ks + 1) < ksteps;
    // The last step re-loads itself (k clamped) into the unused buffer: harmless,
    // and it keeps the loop free of branches around the loads.
    const int k_next = (more ? ks + 1 : ks) * kLpBK;

    u32x4 av[MT], bv[NT], av_n[MT], bv_n[NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
      av[i] = *reinterpret_cast<const u32x4*>(stage + a_row[i] + 16 * (h ^ a_x[i]));
#pragma unroll
    for (int j = 0; j < NT; ++j)
      bv[j] = *reinterpret_cast<const u32x4*>(stage + b_row[j] + 16 * (h ^ b_x[j]));

#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
        const int q = 2 * (s + 1) + h;
#pragma unroll
        for (int i = 0; i < MT; ++i)
          av_n[i] = *reinterpret_cast<const u32x4*>(stage + a_row[i] + 16 * (q ^ a_x[i]));
#pragma unroll
        for (int j = 0; j < NT; ++j)
          bv_n[j] = *reinterpret_cast<const u32x4*>(stage + b_row[j] + 16 * (q ^ b_x[j]));
      }
      // Next stage's global loads over sub-steps 0-1.
#pragma unroll
      for (int l = 0; l < kLoads; ++l) {
        if ((2 * l) / kLoads == s) {
          if (l < S::kAChunks) S::template load_a<VEC, EVEN>(R, l, A, M, K, m0, k_next);
          else S::template load_b<VEC, EVEN>(R, l - S::kAChunks, B, N, K, n0, k_next);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = MF::run(av[i], bv[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
      // ...and their LDS stores (into the buffer nobody reads this step) over 2-3.
      if (s == 2) {
#pragma unroll
        for (int i = 0; i < S::kAChunks; ++i) S::store_a(R, i, next_stage);
      } else if (s == 3) {
        S::store_b(R, next_stage);
      }
      if (s < 3) {
#pragma unroll
        for (int i = 0; i < MT; ++i) av[i] = av_n[i];
#pragma unroll
        for (int j = 0; j < NT; ++j) bv[j] = bv_n[j];
      }
    }
    __syncthreads();
  }

  lp_store_c<OutT, BM, BN, VEC>(acc, C, M, N, m0, n0, wm, wn, h, c, alpha, beta);
}

}  // namespace mcke_amd
