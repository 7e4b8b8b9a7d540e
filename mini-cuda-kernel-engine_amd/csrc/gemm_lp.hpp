// gemm_lp.hpp -- 16-bit-input GEMM on the CDNA4 matrix cores, fp32 accumulation.
// Three kernels: gemm_lp_kernel (any shape, register-staged, 32x32x16 MFMAs, the
// layout described first below), gemm_lp_dma_kernel (whole tiles, direct-to-LDS,
// 32x32x16, K % 64 == 32) and gemm_lp_dma16_kernel (whole tiles, direct-to-LDS,
// 16x16x32, K % 64 == 0), each described where it is defined.
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
#include <utility>

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
        for (int jj = 0; jj < NT; ++jj) {
          const int j = mfma_snake_col(i, jj, NT);
          acc[i][j] = MF::run(av[i], bv[j], acc[i][j]);
        }
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

// ---------------------------------------------------------------------------
// Whole-tile kernel (M % BM == N % BN == K % 32 == 0, 16-byte aligned operands):
// both operands go straight from global memory into LDS (global_load_lds_dwordx4:
// one instruction writes its 64 lanes' 16 bytes to 1 KB of contiguous LDS, lane j
// at byte 16 j), STAGES deep, and B is read back transposed by the LDS
// (ds_read_b64_tr_b16), so no operand passes through VGPRs or ds_writes.
//
// ds_read_b64_tr_b16, per 16-lane group: lane r supplies the address of four
// consecutive 16-bit values R[r][0..3]; lane 4a + b receives
// { R[a][b], R[4+a][b], R[8+a][b], R[12+a][b] }.  With lane 4j + a pointing at
// B[k0 + j][n0 + 4a .. n0 + 4a + 3], lane 4a + b receives column n0 + 4a + b at
// rows k0 .. k0 + 3: a k-contiguous MFMA B fragment, four values per read, two
// reads per MFMA.  The 16 lanes of a group are the 16 consecutive columns
// n0 .. n0 + 15, so here B fragments use the plain column order (lane c of an
// n-tile is column c).
//
// Epilogue layout.  For fp32 C, A is the MFMA's first operand: lane c of a tile
// holds one column, and the 32 lanes of a half-wave store 128 contiguous bytes of
// a row per instruction (whole cache lines).  For 16-bit C the operands are
// swapped, so each MFMA accumulates a transposed 32 x 32 tile in which a lane
// holds runs of four adjacent columns (one 8-byte store each) -- fewer, wider
// stores than 2-byte ones, which measure faster there.
//
// K is staged 32 deep: sub-step s (0, 1) of a stage covers k = 16 s .. 16 s + 15,
// lane half h the eight k = 16 s + 8 h + e (e = 0..7) -- one 16-byte chunk of an
// A row, two transposed reads (e = 4 t + j, t = 0, 1) of B.
//
// LDS layouts (per stage; XOR swizzles keep every access conflict-free):
//   A: BM rows of 64 bytes (4 chunks); chunk q of row r sits at position
//      q ^ ((r / 4) % 4).  A fragment read covers 32 consecutive rows at one
//      chunk; any 16 of them hit 16 distinct 16-byte bank groups.
//   B: 32 rows (k) of BN * 2 bytes, n contiguous; 16-byte chunk c of row k sits
//      at position c ^ (4 (k % 4)).  A transposed read touches rows
//      k0 .. k0 + 3 (k0 % 4 == 0) and, per lane half, 32 consecutive columns
//      (4 chunks): the swizzle puts the four rows' chunk quads on distinct
//      64-byte bank groups.
// The DMA source of each lane is chosen so that it lands on these positions.
//
// Pipeline: the barrier that publishes stage ks + 1 sits between the two
// sub-steps of stage ks, so the first fragment reads of stage ks + 1 and the
// DMA of stage ks + STAGES - 1 are issued under the MFMAs of stage ks's second
// sub-step, and no fragment read is exposed at a barrier.
// ---------------------------------------------------------------------------
// Fragment reads are issued as inline asm and waited on explicitly: the
// compiler cannot tell that a read of stage ks is disjoint from the DMA still
// landing in other stages, and would otherwise drain every outstanding load
// (vmcnt(0)) in front of it.  Nothing else in the kernel reads LDS, so the
// compiler tracks no LDS read of its own, and lds_wait() is the only wait the
// fragments need: it waits for every read issued so far and re-defines the
// fragment registers after the wait, so no MFMA that uses them can be scheduled
// above it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  // A C-style cast is the address-space cast from the generic pointer.
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (const __attribute__((address_space(3))) char*)(p)));
}

template <int OFF>
__device__ __forceinline__ u32x4 lds_read128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

template <int MT, int NT>
__device__ __forceinline__ void lds_wait(u32x4 (&av)[MT], u32x2 (&bv)[NT][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < MT; ++i) asm volatile("" : "+v"(av[i]));
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    asm volatile("" : "+v"(bv[j][0]));
    asm volatile("" : "+v"(bv[j][1]));
  }
}

template <int BM, int BN, int STAGES>
struct LpDmaShape {
  static constexpr int BK = 32;
  static constexpr int kARow = BK * 2;                    // 64 bytes
  static constexpr int kBRow = BN * 2;                    // 256 or 512 bytes
  static constexpr int kABytes = BM * kARow;
  static constexpr int kBBytes = BK * kBRow;
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int NA = kABytes / 1024 / 4;          // DMA instructions per wave per stage
  static constexpr int NB = kBBytes / 1024 / 4;
  static constexpr int L = NA + NB;
  static constexpr int kBChunksPerRow = BN / 8;
  static constexpr int kBRowsPerChunk = 1024 / kBRow;
  static constexpr int MT = BM / 64, NT = BN / 64;       // MFMA tiles per wave
  static constexpr int kMfmas = MT * NT;                 // per sub-step
  static constexpr int kReads = MT + 2 * NT;             // fragment reads per sub-step
  static constexpr int kReadSpan = kMfmas;               // reads go after the first kReadSpan MFMAs
  static_assert(BN == 128 || BN == 256, "B rows of 16 or 32 chunks");
  static_assert(kABytes % 4096 == 0 && kBBytes % 4096 == 0, "stage must split over 4 waves");
  static_assert(STAGES >= 3 && (STAGES - 2) * L <= 63, "vmcnt counts at most 63 loads");
  static_assert(STAGES * kStageBytes <= 160 * 1024, "LDS holds 160 KiB");
  static_assert((16 + 4) * kBRow + 4 * 32 * kARow < 65536, "ds offsets are 16-bit");
  static_assert(NA <= 4 && NB <= 4, "DMA immediate offsets stay below 4 KiB");

  // Issues DMA instruction II (A chunks first, then B) of this wave's share of
  // K step `kstep` into the stage at LDS address `stage`.  a_src / b_src are the
  // per-lane source offsets less the instruction's immediate offset (II * 1024
  // within its operand), `wave` the wave index as a uniform value.
  template <int II>
  static __device__ __forceinline__ void issue_dma(const char* a_base, const char* b_base,
                                                   int64_t b_step, const uint32_t (&a_src)[NA],
                                                   const uint32_t (&b_src)[NB], int kstep,
                                                   uint32_t stage, uint32_t wave) {
    if constexpr (II < NA) {
      lds_dma16<II * 1024>(a_src[II], a_base + static_cast<int64_t>(kstep) * (BK * 2),
                           stage + wave * (NA * 1024));
    } else {
      constexpr int IB = II - NA;
      lds_dma16<IB * 1024>(b_src[IB], b_base + kstep * b_step,
                           stage + kABytes + wave * (NB * 1024));
    }
  }

  // Fragment read rr of sub-step S of the stage at LDS address `st`: rr < MT
  // reads A for m-tile rr, then B for n-tile (rr - MT) / 2, transposed read t =
  // (rr - MT) % 2.
  template <int SUB, int RR>
  static __device__ __forceinline__ void read_one(uint32_t st, const uint32_t (&a_off)[2],
                                                  const uint32_t (&b_off)[NT], u32x4 (&av)[MT],
                                                  u32x2 (&bv)[NT][2]) {
    if constexpr (RR < MT) {
      av[RR] = lds_read128<RR * 32 * kARow>(st + a_off[SUB]);
    } else {
      constexpr int jn = (RR - MT) / 2, t = (RR - MT) % 2;
      bv[jn][t] = lds_read_tr16<(16 * SUB + 4 * t) * kBRow>(st + b_off[jn]);
    }
  }
};

// Sub-step helper: MFMA idx of the MT x NT grid, then whichever fragment reads
// (of sub-step SUB of the stage at `st`) and DMA instructions fall in its slot,
// so that they issue while the matrix pipe is busy.
template <typename T, bool TRANS, int BM, int BN, int STAGES, int SUB, int IDX>
__device__ __forceinline__ void lp_dma_slot(f32x16 (&acc)[BM / 64][BN / 64],
                                            const u32x4 (&cav)[BM / 64],
                                            const u32x2 (&cbv)[BN / 64][2], uint32_t st,
                                            const uint32_t (&a_off)[2],
                                            const uint32_t (&b_off)[BN / 64],
                                            u32x4 (&nav)[BM / 64], u32x2 (&nbv)[BN / 64][2],
                                            bool dma, const char* a_base, const char* b_base,
                                            int64_t b_step, const uint32_t (&a_src)[LpDmaShape<BM, BN, STAGES>::NA],
                                            const uint32_t (&b_src)[LpDmaShape<BM, BN, STAGES>::NB],
                                            int kstep, uint32_t dstage, uint32_t wave) {
  using S = LpDmaShape<BM, BN, STAGES>;
  constexpr int i = IDX / S::NT, j = mfma_snake_col(i, IDX % S::NT, S::NT);
  const u32x4 b = u32x4{cbv[j][0][0], cbv[j][0][1], cbv[j][1][0], cbv[j][1][1]};
  // TRANS: operands swapped, the MFMA computes the transposed tile (n rows, m columns).
  if constexpr (TRANS) acc[i][j] = LpMfma<T>::run(b, cav[i], acc[i][j]);
  else acc[i][j] = LpMfma<T>::run(cav[i], b, acc[i][j]);
  __builtin_amdgcn_sched_barrier(0);
  // Reads RR with RR * kReadSpan / kReads == IDX go after this MFMA.
  [&]<int... RR>(std::integer_sequence<int, RR...>) {
    ((RR * S::kReadSpan / S::kReads == IDX
          ? S::template read_one<SUB, RR>(st, a_off, b_off, nav, nbv)
          : void()),
     ...);
  }(std::make_integer_sequence<int, S::kReads>{});
  if (dma) {
    [&]<int... II>(std::integer_sequence<int, II...>) {
      ((II * S::kMfmas / S::L == IDX
            ? S::template issue_dma<II>(a_base, b_base, b_step, a_src, b_src, kstep, dstage, wave)
            : void()),
       ...);
    }(std::make_integer_sequence<int, S::L>{});
  }
  __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------
// Whole-tile kernel (M % BM == N % BN == K % 32 == 0, 16-byte aligned operands):
// both operands go straight from global memory into LDS (global_load_lds_dwordx4:
// one instruction writes its 64 lanes' 16 bytes to 1 KB of contiguous LDS, lane j
// at byte 16 j), STAGES deep, and B is read back transposed by the LDS
// (ds_read_b64_tr_b16), so no operand passes through VGPRs or ds_writes.
//
// ds_read_b64_tr_b16, per 16-lane group: lane r supplies the address of four
// consecutive 16-bit values R[r][0..3]; lane 4a + b receives
// { R[a][b], R[4+a][b], R[8+a][b], R[12+a][b] }.  With lane 4j + a pointing at
// B[k0 + j][n0 + 4a .. n0 + 4a + 3], lane 4a + b receives column n0 + 4a + b at
// rows k0 .. k0 + 3: a k-contiguous MFMA B fragment, four values per read, two
// reads per MFMA.  The 16 lanes of a group are the 16 consecutive columns
// n0 .. n0 + 15, so here B fragments use the plain column order (lane c of an
// n-tile is column c).
//
// K is staged 32 deep: sub-step s (0, 1) of a stage covers k = 16 s .. 16 s + 15,
// lane half h the eight k = 16 s + 8 h + e (e = 0..7) -- one 16-byte chunk of an
// A row, two transposed reads (e = 4 t + j, t = 0, 1) of B.
//
// LDS layouts (per stage; XOR swizzles keep every access conflict-free):
//   A: BM rows of 64 bytes (4 chunks); chunk q of row r sits at position
//      q ^ ((r / 4) % 4).  A fragment read covers 32 consecutive rows at one
//      chunk; any 16 of them hit 16 distinct 16-byte bank groups.
//   B: 32 rows (k) of BN * 2 bytes, n contiguous; 16-byte chunk c of row k sits
//      at position c ^ (4 (k % 4)).  A transposed read touches rows
//      k0 .. k0 + 3 (k0 % 4 == 0) and, per lane half, 32 consecutive columns
//      (4 chunks): the swizzle puts the four rows' chunk quads on distinct
//      64-byte bank groups.
// The DMA source of each lane is chosen so that it lands on these positions.
//
// Pipeline, per stage ks:
//   sub-step 0: MFMAs on fragments read earlier, interleaved with the reads of
//               sub-step 1;
//   barrier:    publishes stage ks + 1 (its DMA was issued STAGES - 2 stages
//               earlier) and retires every read of stage ks - 1's buffer;
//   sub-step 1: MFMAs interleaved with the DMA of stage ks + STAGES - 1 (into
//               stage ks - 1's buffer) and the sub-step 0 reads of stage ks + 1.
// ---------------------------------------------------------------------------
template <typename T, typename OutT, int BM, int BN, int STAGES>
__global__ __launch_bounds__(kMfmaThreads, 1) void gemm_lp_dma_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, OutT* __restrict__ C,
    int M, int N, int K, float alpha, float beta, int tiles_m, int tiles_n) {
  using S = LpDmaShape<BM, BN, STAGES>;
  constexpr int BK = S::BK;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MT = S::MT, NT = S::NT;
  constexpr int L = S::L;
  constexpr bool TRANS = sizeof(OutT) == 2;

  __shared__ __attribute__((aligned(1024))) char smem[STAGES * S::kStageBytes];

  int tm, tn;
  mfma_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int h = lane / 32, c = lane % 32;

  // DMA sources: a wave-uniform base per stage plus a per-lane byte offset.
  const char* a_base = reinterpret_cast<const char*>(A + static_cast<int64_t>(m0) * K);
  const char* b_base = reinterpret_cast<const char*>(B + n0);
  const int64_t b_step = static_cast<int64_t>(BK) * N * 2;        // bytes per stage
  // Less the immediate offset of instruction ii (ii * 1024), which the DMA adds to
  // both addresses; row >= 16 ii (A) and >= kBRowsPerChunk ii with N >= BN (B) keep
  // the difference non-negative.
  uint32_t a_src[S::NA], b_src[S::NB];
#pragma unroll
  for (int ii = 0; ii < S::NA; ++ii) {
    const int row = 16 * (wave * S::NA + ii) + lane / 4;       // (row / 4) % 4 == lane / 16
    const int q = (lane % 4) ^ (lane / 16);
    a_src[ii] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) * 2u + 16u * q -
                1024u * ii;
  }
#pragma unroll
  for (int ii = 0; ii < S::NB; ++ii) {
    const int row = S::kBRowsPerChunk * (wave * S::NB + ii) + lane / S::kBChunksPerRow;
    const int cg = (lane % S::kBChunksPerRow) ^ (4 * (row % 4));
    b_src[ii] = static_cast<uint32_t>(row) * static_cast<uint32_t>(N) * 2u + 16u * cg -
                1024u * ii;
  }
  const uint32_t wave_u = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wave));

  // Fragment addressing (bytes within a stage).
  //   A, m-tile i, sub-step s: row wm*WM + 32 i + c, chunk 2 s + h at position
  //   (2 s + h) ^ ((c / 4) % 4)   (the row base is a multiple of 32).
  uint32_t a_off[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
    a_off[s] = (wm * WM + c) * S::kARow + 16 * ((2 * s + h) ^ ((c / 4) % 4));
  //   B, n-tile jn, sub-step s, read t: lane r = 4 jq + a of its 16-lane group g
  //   reads row k = 16 s + 8 h + 4 t + jq at columns wn*WN + 32 jn + 16 (g % 2) + 4 a.
  const int r16 = lane % 16, jq = r16 / 4, qa = r16 % 4, g2 = (lane / 16) % 2;
  uint32_t b_off[NT];
#pragma unroll
  for (int jn = 0; jn < NT; ++jn) {
    const int cc = (wn * WN + 32 * jn + 16 * g2 + 4 * qa) / 8;
    b_off[jn] = S::kABytes + (8 * h + jq) * S::kBRow + 16 * (cc ^ (4 * jq)) + (qa % 2) * 8;
  }

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t lds0 = lds_addr(smem);
  const int ksteps = K / BK;
  u32x4 av0[MT], av1[MT];
  u32x2 bv0[NT][2], bv1[NT][2];
  if (ksteps > 0) {
    // Prologue: stages 0 .. STAGES-2 in flight (past the last K step a stage
    // re-fetches the last one into a buffer nobody reads, which keeps the number
    // of loads per stage -- and so the vmcnt arithmetic -- uniform).
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) {
      const int kst = st < ksteps ? st : ksteps - 1;
      [&]<int... II>(std::integer_sequence<int, II...>) {
        (S::template issue_dma<II>(a_base, b_base, b_step, a_src, b_src, kst,
                                   lds0 + st * S::kStageBytes, wave_u),
         ...);
      }(std::make_integer_sequence<int, L>{});
    }
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 2) * L) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    [&]<int... RR>(std::integer_sequence<int, RR...>) {
      (S::template read_one<0, RR>(lds0, a_off, b_off, av0, bv0), ...);
    }(std::make_integer_sequence<int, S::kReads>{});
  }

  for (int ks = 0; ks < ksteps; ++ks) {
    const uint32_t st = lds0 + (ks % STAGES) * S::kStageBytes;
    const uint32_t st_next = lds0 + ((ks + 1) % STAGES) * S::kStageBytes;
    const int kf = ks + STAGES - 1;
    const int kdma = kf < ksteps ? kf : ksteps - 1;
    const uint32_t dstage = lds0 + (kf % STAGES) * S::kStageBytes;

    // Sub-step 0 (fragments read in the previous step or the prologue).
    lds_wait<MT, NT>(av0, bv0);
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (lp_dma_slot<T, TRANS, BM, BN, STAGES, 1, I>(acc, av0, bv0, st, a_off, b_off, av1, bv1, false,
                                            a_base, b_base, b_step, a_src, b_src, kdma, dstage,
                                            wave_u),
       ...);
    }(std::make_integer_sequence<int, S::kMfmas>{});

    // Stage ks + 1 has landed once at most the (STAGES - 3) younger stages' loads
    // are outstanding; the barrier publishes every wave's share of it, and it also
    // retires every wave's reads of the buffer refilled next (stage ks - 1's,
    // waited for by lds_wait before its last MFMAs).  A bare s_barrier:
    // __syncthreads() would drain every outstanding load (vmcnt(0)).
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((STAGES - 3) * L) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // Sub-step 1, with the DMA of stage ks + STAGES - 1 and the sub-step 0 reads of
    // stage ks + 1 (in the last step they read a buffer nobody uses: harmless).
    lds_wait<MT, NT>(av1, bv1);
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (lp_dma_slot<T, TRANS, BM, BN, STAGES, 0, I>(acc, av1, bv1, st_next, a_off, b_off, av0, bv0,
                                            true, a_base, b_base, b_step, a_src, b_src, kdma,
                                            dstage, wave_u),
       ...);
    }(std::make_integer_sequence<int, S::kMfmas>{});
  }
  // No LDS DMA may still be landing, and no LDS read outstanding, when the
  // workgroup retires.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

  using O = LpOut<OutT>;
  if constexpr (!TRANS) {
    // Lane (h, c) of n-tile j holds column wn*WN + 32 j + c, register r row
    // 8 (r / 4) + 4 h + r % 4 of m-tile i.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        OutT* crow = C + static_cast<int64_t>(row) * N + n0 + wn * WN + c;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          float v = alpha * acc[i][j][r];
          if (beta != 0.0f) v += beta * O::to_f32(crow[32 * j]);
          crow[32 * j] = O::from_f32(v);
        }
      }
    }
    return;
  }
  // Transposed tiles: lane (h, c), register r = 4 g + e holds C row
  // wm*WM + 32 i + c, column wn*WN + 32 j + 8 g + 4 h + e -- e = 0..3 are four
  // adjacent columns, one 8-byte quad.
  struct alignas(4 * sizeof(OutT)) Quad { OutT v[4]; };
  if (beta == 0.0f) {
    // Staged through the (now idle) stage buffers, so the global stores are whole
    // rows: written straight from the registers, the quads reach each 64-byte row
    // segment in pieces, and the launch ended with a write burst of partial lines
    // (measured at 4096^3: 13 us of a 118 us launch, 1.4x the output bytes).
    // The tile is row-major in LDS, 16-byte chunk q of row r at q ^ (r % kChunks),
    // so the 32 lanes of a quad column write 32 distinct chunks and the 32 lanes
    // reading one row back read 32 distinct chunks.  The values are rounded once,
    // as on the direct path, so both give the same bits.
    constexpr int kRowBytes = BN * 2;
    constexpr int kChunks = kRowBytes / 16;
    static_assert(BM * kRowBytes <= STAGES * S::kStageBytes, "the C tile must fit the stages");
    static_assert(kChunks <= 32 && (BM * kChunks) % kMfmaThreads == 0, "tile rows per pass");
    __syncthreads();   // every wave has finished reading the stage buffers
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int rt = wm * WM + 32 * i + c;            // tile row; rt % 32 == c
#pragma unroll
      for (int j = 0; j < NT; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int q = (wn * WN + 32 * j + 8 * g) / 8;     // 16-byte chunk of the row
          Quad o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o.v[e] = O::from_f32(alpha * acc[i][j][4 * g + e]);
          *reinterpret_cast<Quad*>(smem + rt * kRowBytes + ((q ^ (rt % kChunks)) * 16) + 8 * h) = o;
        }
      }
    }
    __syncthreads();
    constexpr int kRowsPerPass = kMfmaThreads / kChunks;
    const int q = threadIdx.x % kChunks;
#pragma unroll 4
    for (int r0 = 0; r0 < BM; r0 += kRowsPerPass) {
      const int rt = r0 + threadIdx.x / kChunks;
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + rt * kRowBytes + ((q ^ (rt % kChunks)) * 16));
      *reinterpret_cast<u32x4*>(C + static_cast<int64_t>(m0 + rt) * N + n0 + 8 * q) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    OutT* crow = C + static_cast<int64_t>(m0 + wm * WM + 32 * i + c) * N + n0 + wn * WN + 4 * h;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        Quad* dst = reinterpret_cast<Quad*>(crow + 32 * j + 8 * g);
        Quad o;
        if (beta != 0.0f) {
          const Quad old = *dst;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o.v[e] = O::from_f32(alpha * acc[i][j][4 * g + e] + beta * O::to_f32(old.v[e]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) o.v[e] = O::from_f32(alpha * acc[i][j][4 * g + e]);
        }
        *dst = o;
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Whole-tile kernel on v_mfma_f32_16x16x32_{bf16,f16} (K % 64 == 0).
//
// Why this MFMA: with random operands the 16-bit matrix pipe is power-limited,
// and per unit of work the 16x16x32 form draws less than the 32x32x16 one.  Long
// chains of either at the same issue rate, on MI355X, settle at 1.82 GHz
// (32x32x16) against 2.02 GHz (16x16x32); in the GEMM the engine clock is the
// limit at 4096^3 and above.
//
// One v_mfma_f32_16x16x32 takes, per lane l, eight 16-bit A values of row l%16
// and eight B values of column l%16; lane group g = l/16 covers k = 8 g .. 8 g + 7
// of the 32 (A and B must agree on which k each group takes; the sum over k
// does not care).  The result: lane l, register r = C row 4 g + r, column l%16.
// A wave's WM x WN sub-tile is MT x NT blocks of 16 x 16 (MT = WM/16).
//
// Fragments per K step (32 deep): A block i is one ds_read_b128 (lane l reads
// row 16 i + l%16, one 16-byte chunk); B block j is two ds_read_b64_tr_b16
// (t = 0, 1): lane r = 4 jq + qa of group g points at B row k = 8 g + 4 t + jq,
// columns 16 j + 4 qa .. + 3, and receives column 16 j + r at rows 8 g + 4 t .. + 3.
//
// LDS (BM = BN = 256: 160 KiB, all of it):
//   A: three buffers, each 64 k deep (two K steps): BM rows of 128 bytes, chunk
//      c of row r at position c ^ (r % 8).  Step ks reads chunks 4 (ks % 2) + g.
//      Measured on MI355X, this read of 16 rows x 4 chunks has no bank conflicts
//      over 128-byte rows, while over 64-byte rows (A 32 deep) every XOR
//      swizzle tried conflicts 2-way; and 128-byte rows make the DMA fetch whole
//      cache lines (8 lanes per row, one line each).
//   B: four buffers, one K step (32 rows of BN * 2 bytes) each; 16-byte chunk c
//      of row k sits at c ^ (4 (k % 4) + 2 ((k / 8) % 2)).  One half-wave of a
//      transposed read touches two chunks of rows k0 .. k0 + 3 and
//      k0 + 8 .. k0 + 11: the last term separates the two row quads.
//
// Pipeline, per K step ks (fragments double-buffered in registers):
//   barrier: publishes B step ks + 1 (and, for even ks + 1, its A buffer); every
//            wave has by then waited for all its reads of step ks - 1's buffers;
//   MFMAs of step ks (block-row order) from one register set, interleaved with
//            the 24 fragment reads of step ks + 1 into the other set, spread over
//            the whole step, and the DMA of B step ks + 3 and of half an A buffer
//            (A pair (ks + 4) / 2), which refill buffers of step ks - 1 and
//            earlier.  Block row i waits only for A block i of its own set.
// Every step issues the same DMA (half an A buffer, one B step), so one vmcnt
// count covers both rings.
// ---------------------------------------------------------------------------
template <typename T> struct LpMfma16;
template <> struct LpMfma16<__bf16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct LpMfma16<_Float16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <int BM, int BN>
struct Lp16Shape {
  static constexpr int BK = 32;                          // K per step
  // Ring depth: step ks issues the DMA of B step ks + kDepth and of half of A pair
  // (ks + kDepth + 1) / 2, so a step's operands have kDepth - 1 steps to land
  // before the step before it reads them.  B keeps kDepth + 1 buffers, A
  // kDepth / 2 + 2 pairs: a buffer is refilled only after the barrier that
  // follows its last reads.
  static constexpr int kDepth = 3;
  static constexpr int kBStages = kDepth + 1;
  static constexpr int kAStages = kDepth / 2 + 2;
  static constexpr int kARow = 128;                      // A buffer row: 64 k
  static constexpr int kABuf = BM * kARow;               // one A buffer (two steps)
  static constexpr int kBRow = BN * 2;                   // 256 or 512 bytes
  static constexpr int kBBytes = BK * kBRow;             // one B step
  static constexpr int kBBase = kAStages * kABuf;        // B ring after the A ring
  static constexpr int kLdsBytes = kBBase + kBStages * kBBytes;
  static constexpr int NA = kABuf / 1024 / 4 / 2;        // A DMA instructions per wave per step
  static constexpr int NB = kBBytes / 1024 / 4;          // B DMA instructions per wave per step
  static constexpr int L = NA + NB;
  static constexpr int kBChunksPerRow = BN / 8;
  static constexpr int kBRowsPerChunk = 1024 / kBRow;
  static constexpr int MT = BM / 32, NT = BN / 32;       // 16 x 16 blocks per wave
  static constexpr int kMfmas = MT * NT;                 // per step
  static_assert(BN == 128 || BN == 256, "B rows of 16 or 32 chunks");
  static_assert(kABuf % 8192 == 0 && kBBytes % 4096 == 0, "buffers must split over 4 waves");
  static_assert((kBStages - 2) * L <= 63, "vmcnt counts at most 63 loads");
  static_assert(2 * kAStages >= kDepth + 2 && kBStages >= kDepth, "buffers retire in time");
  static_assert(kLdsBytes <= 160 * 1024, "LDS holds 160 KiB");
  static_assert(NA <= 4 && NB <= 4, "DMA immediate offsets stay below 4 KiB");

  static __host__ __device__ constexpr int bswz(int k) { return 4 * (k % 4) + 2 * ((k / 8) % 2); }

  // A half h (0, 1) of the A buffer at LDS `abuf`, fetched from pair `pair` (64 k).
  // Wave w's share of a buffer is 2 NA KiB at 2 NA w KiB; half h is NA KiB of it.
  template <int II>
  static __device__ __forceinline__ void dma_a(const char* a_base, const uint32_t (&a_src)[2 * NA],
                                               int pair, int h, uint32_t abuf, uint32_t wave) {
    const char* src = a_base + static_cast<int64_t>(pair) * kARow;
    const uint32_t m0 = abuf + (wave * (2 * NA) + h * NA) * 1024;
    lds_dma16<II * 1024>(h ? a_src[NA + II] : a_src[II], src, m0);
  }
  template <int II>
  static __device__ __forceinline__ void dma_b(const char* b_base, int64_t b_step,
                                               const uint32_t (&b_src)[NB], int kstep,
                                               uint32_t bbuf, uint32_t wave) {
    lds_dma16<II * 1024>(b_src[II], b_base + kstep * b_step, bbuf + wave * (NB * 1024));
  }

  // B block j (RR / 2), transposed read t = RR % 2, of the B buffer at `bst`.
  template <int RR>
  static __device__ __forceinline__ void read_b(uint32_t bst, const uint32_t (&b_off)[NT],
                                                u32x2 (&bv)[NT][2]) {
    constexpr int j = RR / 2, t = RR % 2;
    bv[j][t] = lds_read_tr16<4 * t * kBRow>(bst + b_off[j]);
  }
  // A block I of a step whose chunk-adjusted base is `ast`.
  template <int I>
  static __device__ __forceinline__ void read_a(uint32_t ast, u32x4 (&av)[MT]) {
    av[I] = lds_read128<I * 16 * kARow>(ast);
  }
  // Reads of the next step: B blocks first (2 NT transposed reads), then A
  // blocks 0 .. MT-1, read rr after MFMA rr * kMfmas / kReads.
  static constexpr int kReads = 2 * NT + MT;
  static constexpr int read_slot(int rr) { return rr * kMfmas / kReads; }
  // DMA instruction ii after MFMA dma_slot(ii).  Measured (in-process A/B on
  // MI355X): 256 x 256 tiles run 1.5-2% faster with the DMA in the middle of a block
  // row than at its first MFMA, next to the row's LDS wait; 128 x 128 tiles 2% faster
  // with it on odd slots of the step's first half.
  static constexpr int dma_slot(int ii) {
    return BM >= 256 ? ii * (kMfmas / L) + (kMfmas / L) / 2 : ii * (kMfmas / 2) / L + 1;
  }
  static_assert(dma_slot(L - 1) < kMfmas, "every DMA instruction has a slot");
  // Block row i waits for A block i of its set: at most the A reads issued after
  // it (MT - 1 - i, in the previous step) and the reads of the next step issued so
  // far may be pending.  lgkmcnt counts to 15; a smaller count only waits for
  // older reads as well.
  static constexpr int wait_before_row(int i) {
    int n = MT - 1 - i;
    for (int rr = 0; rr < kReads; ++rr) n += read_slot(rr) < i * NT ? 1 : 0;
    return n < 15 ? n : 15;
  }
};

// Waits until at most N LDS reads are outstanding, then re-defines the listed
// fragment registers so that no MFMA using them is scheduled above the wait.
template <int N>
__device__ __forceinline__ void lds_wait_n() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}
template <int FIRST, int LAST, int MT>
__device__ __forceinline__ void touch_a(u32x4 (&av)[MT]) {
#pragma unroll
  for (int i = FIRST; i < LAST; ++i) asm volatile("" : "+v"(av[i]));
}
template <int FIRST, int LAST, int NT>
__device__ __forceinline__ void touch_b(u32x2 (&bv)[NT][2]) {
#pragma unroll
  for (int j = FIRST; j < LAST; ++j) {
    asm volatile("" : "+v"(bv[j][0]));
    asm volatile("" : "+v"(bv[j][1]));
  }
}

// Per-step addresses of gemm_lp_dma16_kernel (LDS byte addresses and DMA sources).
struct Lp16Step {
  uint32_t bst_next;   // B buffer of the next step
  uint32_t ast_next;   // A fragment base of the next step (its buffer and chunk half)
  uint32_t abuf_dma;   // A buffer that this step's DMA fills
  uint32_t bbuf_dma;   // B buffer that this step's DMA fills
  int a_pair;          // A pair (64 k) fetched into abuf_dma
  int a_half;          // which half of it
  int b_kstep;         // B step fetched into bbuf_dma
};

// MFMA IDX of a step (block i = IDX / NT, j = IDX % NT) from register set P, then
// the reads of the next step (into set 1 - P) and the DMA instructions that fall
// in its slot.
template <typename T, bool TRANS, int BM, int BN, int P, int IDX>
__device__ __forceinline__ void lp16_slot(f32x4 (&acc)[BM / 32][BN / 32],
                                          u32x4 (&av)[2][BM / 32], u32x2 (&bv)[2][BN / 32][2],
                                          const Lp16Step& sp, const uint32_t (&b_off)[BN / 32],
                                          const char* a_base, const char* b_base, int64_t b_step,
                                          const uint32_t (&a_src)[2 * Lp16Shape<BM, BN>::NA],
                                          const uint32_t (&b_src)[Lp16Shape<BM, BN>::NB],
                                          uint32_t wave) {
  using S = Lp16Shape<BM, BN>;
  constexpr int NT = S::NT;
  // jj: position within block row i; j: the column it computes (mfma_snake_col).
  constexpr int i = IDX / NT, jj = IDX % NT, j = mfma_snake_col(i, jj, NT);
  if constexpr (jj == 0) {
    lds_wait_n<S::wait_before_row(i)>();
    touch_a<i, i + 1>(av[P]);
    if constexpr (i == 0) touch_b<0, NT>(bv[P]);
  }
  const u32x4 b = u32x4{bv[P][j][0][0], bv[P][j][0][1], bv[P][j][1][0], bv[P][j][1][1]};
  // TRANS: operands swapped, the MFMA computes the transposed block (n rows, m columns).
  if constexpr (TRANS) acc[i][j] = LpMfma16<T>::run(b, av[P][i], acc[i][j]);
  else acc[i][j] = LpMfma16<T>::run(av[P][i], b, acc[i][j]);
  __builtin_amdgcn_sched_barrier(0);
  [&]<int... RR>(std::integer_sequence<int, RR...>) {
    ((S::read_slot(RR) == IDX
          ? (RR < 2 * NT ? S::template read_b<(RR < 2 * NT ? RR : 0)>(sp.bst_next, b_off, bv[1 - P])
                         : S::template read_a<(RR < 2 * NT ? 0 : RR - 2 * NT)>(sp.ast_next,
                                                                              av[1 - P]))
          : void()),
     ...);
  }(std::make_integer_sequence<int, S::kReads>{});
  [&]<int... II>(std::integer_sequence<int, II...>) {
    ((S::dma_slot(II) == IDX
          ? (II < S::NA ? S::template dma_a<(II < S::NA ? II : 0)>(a_base, a_src, sp.a_pair,
                                                                   sp.a_half, sp.abuf_dma, wave)
                        : S::template dma_b<(II < S::NA ? 0 : II - S::NA)>(
                              b_base, b_step, b_src, sp.b_kstep, sp.bbuf_dma, wave))
          : void()),
     ...);
  }(std::make_integer_sequence<int, S::L>{});
  __builtin_amdgcn_sched_barrier(0);
}

// One accumulator, copied out of the accumulation registers where it is used.
// The TRANS epilogue reads every accumulator through this: the copies the
// compiler would make are shared by its two branches and get hoisted above them,
// all 256 at once.
__device__ __forceinline__ float acc_get(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

template <typename T, typename OutT, int BM, int BN>
__global__ __launch_bounds__(kMfmaThreads, 1) void gemm_lp_dma16_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, OutT* __restrict__ C,
    int M, int N, int K, float alpha, float beta, int tiles_m, int tiles_n) {
  using S = Lp16Shape<BM, BN>;
  constexpr int BK = S::BK;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MT = S::MT, NT = S::NT, NA = S::NA;
  constexpr int L = S::L;
  constexpr bool TRANS = sizeof(OutT) == 2;

  __shared__ __attribute__((aligned(1024))) char smem[S::kLdsBytes];

  int tm, tn;
  mfma_tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int g = lane / 16, r16 = lane % 16;

  // DMA sources: a wave-uniform base per step plus a per-lane byte offset, less
  // the immediate offset of the instruction (its index within the step, times
  // 1024), which the DMA adds to both addresses.
  //   A: instruction q (0 .. 2 NA - 1) of wave w fills rows 8 (2 NA w + q) ..
  //   + 7 of an A buffer; lane l the chunk at position l % 8 of row l / 8 there,
  //   which holds chunk (l % 8) ^ (row % 8).  row >= 8 q and K >= 64 keep the
  //   difference non-negative.
  //   B: as gemm_lp_dma_kernel with this kernel's B swizzle; row >=
  //   kBRowsPerChunk ii with N >= BN keeps it non-negative.
  const char* a_base = reinterpret_cast<const char*>(A + static_cast<int64_t>(m0) * K);
  const char* b_base = reinterpret_cast<const char*>(B + n0);
  const int64_t b_step = static_cast<int64_t>(BK) * N * 2;        // bytes per step
  uint32_t a_src[2 * NA], b_src[S::NB];
#pragma unroll
  for (int q = 0; q < 2 * NA; ++q) {
    const int row = 8 * (wave * 2 * NA + q) + lane / 8;
    const int cg = (lane % 8) ^ (row % 8);
    a_src[q] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) * 2u + 16u * cg -
               1024u * (q % NA);
  }
#pragma unroll
  for (int ii = 0; ii < S::NB; ++ii) {
    const int row = S::kBRowsPerChunk * (wave * S::NB + ii) + lane / S::kBChunksPerRow;
    const int cg = (lane % S::kBChunksPerRow) ^ S::bswz(row);
    b_src[ii] = static_cast<uint32_t>(row) * static_cast<uint32_t>(N) * 2u + 16u * cg -
                1024u * ii;
  }
  const uint32_t wave_u = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wave));

  // Fragment addressing (bytes within a buffer).
  //   A block i of a step with chunk half s: row wm*WM + 16 i + r16, chunk
  //   4 s + g at position (4 s + g) ^ (r16 % 8) (the row base is a multiple of
  //   16); block i adds 16 rows as an immediate.
  uint32_t a_off[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
    a_off[s] = (wm * WM + r16) * S::kARow + 16 * ((4 * s + g) ^ (r16 % 8));
  //   B block j, read t: lane r16 = 4 jq + qa reads row k = 8 g + 4 t + jq at
  //   columns wn*WN + 16 j + 4 qa .. + 3 (read t adds 4 rows as an immediate).
  const int jq = r16 / 4, qa = r16 % 4;
  uint32_t b_off[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int col = wn * WN + 16 * j + 4 * qa;
    const int k = 8 * g + jq;
    b_off[j] = k * S::kBRow + 16 * ((col / 8) ^ S::bswz(k)) + (col % 8) * 2;
  }

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsb = lds0 + S::kBBase;
  const int ksteps = K / BK;                    // even
  const int last_pair = ksteps / 2 - 1;
  u32x4 av[2][MT];
  u32x2 bv[2][NT][2];

  // The DMA that step ks (or, for ks < 0, the prologue in its place) issues: half
  // ks % 2 of A pair (ks + D + 1) / 2 into that pair's buffer, and B step ks + D
  // (D = kDepth).  Past the end the sources repeat the last pair / step into
  // buffers nobody reads, which keeps the number of loads per step -- and so the
  // vmcnt arithmetic -- uniform.
  auto dma_plan = [&](int ks, Lp16Step& sp) {
    const int pair = (ks + S::kDepth + 1) / 2;      // ks >= -D - 1
    sp.a_pair = pair < last_pair ? pair : last_pair;
    sp.a_half = ks & 1;
    sp.abuf_dma = lds0 + (pair % S::kAStages) * S::kABuf;
    const int kb = ks + S::kDepth;
    sp.b_kstep = kb < ksteps ? kb : ksteps - 1;
    sp.bbuf_dma = ldsb + (kb % S::kBStages) * S::kBBytes;
  };

  if (ksteps > 0) {
    // Prologue: the DMA of steps -D - 1 .. -1 (A pairs 0 .. D / 2, B steps 0 ..
    // D - 1; step -D - 1 has no B), in the order the loop keeps.
#pragma unroll
    for (int ks = -S::kDepth - 1; ks < 0; ++ks) {
      Lp16Step sp;
      dma_plan(ks, sp);
      [&]<int... II>(std::integer_sequence<int, II...>) {
        (S::template dma_a<II>(a_base, a_src, sp.a_pair, sp.a_half, sp.abuf_dma, wave_u), ...);
      }(std::make_integer_sequence<int, NA>{});
      if (ks >= -S::kDepth) {
        [&]<int... II>(std::integer_sequence<int, II...>) {
          (S::template dma_b<II>(b_base, b_step, b_src, sp.b_kstep, sp.bbuf_dma, wave_u), ...);
        }(std::make_integer_sequence<int, S::NB>{});
      }
    }
    // A pair 0 and B step 0 have landed once the D - 1 younger steps' loads at
    // most are outstanding.
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((S::kBStages - 2) * L) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // Step 0's fragments into set 0, in the order the loop reads them.
    [&]<int... RR>(std::integer_sequence<int, RR...>) {
      (S::template read_b<RR>(ldsb, b_off, bv[0]), ...);
    }(std::make_integer_sequence<int, 2 * NT>{});
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (S::template read_a<I>(lds0 + a_off[0], av[0]), ...);
    }(std::make_integer_sequence<int, MT>{});
  }

  // Step ks from register set P.
  auto step = [&]<int P>(int ks) {
    Lp16Step sp;
    dma_plan(ks, sp);
    const int kn = ks + 1;
    sp.bst_next = ldsb + (kn % S::kBStages) * S::kBBytes;
    sp.ast_next = lds0 + ((kn / 2) % S::kAStages) * S::kABuf + (kn & 1 ? a_off[1] : a_off[0]);

    // B step ks + 1 (and A's buffer for it) has landed once at most the D - 2
    // younger steps' loads are outstanding; the barrier publishes every wave's share and
    // retires the buffers refilled in this step (each wave waited for its reads of
    // them in the step before).  A bare s_barrier: __syncthreads() would drain
    // every outstanding load (vmcnt(0)).
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((S::kBStages - 3) * L) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (lp16_slot<T, TRANS, BM, BN, P, I>(acc, av, bv, sp, b_off, a_base, b_base, b_step, a_src,
                                         b_src, wave_u),
       ...);
    }(std::make_integer_sequence<int, S::kMfmas>{});
  };
  // K % 64 == 0: whole pairs of steps, set 0 then set 1.
  for (int ks = 0; ks < ksteps; ks += 2) {
    step.template operator()<0>(ks);
    step.template operator()<1>(ks + 1);
  }
  // The accumulators stay in the accumulation registers past the loop: left to
  // itself the compiler copies all of them out at once where the loop and the
  // K == 0 path meet, more than the other register file holds.
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) asm volatile("" : "+a"(acc[i][j]));
  // acc_get is inline asm, which the hazard checks do not see into: the last
  // MFMA's results are ready well before these 16 cycles are over.
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  // No LDS DMA may still be landing, and no LDS read outstanding, when the
  // workgroup retires.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

  using O = LpOut<OutT>;
  if constexpr (!TRANS) {
    // Lane (g, r16) of block (i, j), register r: row wm*WM + 16 i + 4 g + r,
    // column wn*WN + 16 j + r16.  A 16-lane group stores 64 contiguous bytes of a
    // row; blocks j and j + 1 (j even) complete one 128-byte line.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * WM + 16 * i + 4 * g + r;
        OutT* crow = C + static_cast<int64_t>(row) * N + n0 + wn * WN + r16;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          float v = alpha * acc[i][j][r];
          if (beta != 0.0f) v += beta * O::to_f32(crow[16 * j]);
          crow[16 * j] = O::from_f32(v);
        }
      }
    }
    return;
  }
  // Transposed blocks: lane (g, r16), register r of block (i, j) holds C row
  // wm*WM + 16 i + r16, column wn*WN + 16 j + 4 g + r -- one quad of four
  // adjacent columns.
  struct alignas(4 * sizeof(OutT)) Quad { OutT v[4]; };
  if (beta == 0.0f) {
    // Staged through the (now idle) stage buffers so that the global stores are
    // whole rows, as in gemm_lp_dma_kernel.  Chunk q of tile row r sits at
    // q ^ (r % kChunks): the 16 rows of a half-wave's quads land on 16 distinct
    // chunk positions.
    constexpr int kRowBytes = BN * 2;
    constexpr int kChunks = kRowBytes / 16;
    static_assert(BM * kRowBytes <= S::kLdsBytes, "the C tile must fit the buffers");
    static_assert(kChunks <= 32 && (BM * kChunks) % kMfmaThreads == 0, "tile rows per pass");
    __syncthreads();   // every wave has finished reading the stage buffers
    // Block row by block row: left to itself the scheduler converts every
    // accumulator ahead of the barrier and runs out of registers.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int rt = wm * WM + 16 * i + r16;            // tile row
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int col = wn * WN + 16 * j + 4 * g;
        Quad o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o.v[e] = O::from_f32(alpha * acc_get(acc[i][j][e]));
        *reinterpret_cast<Quad*>(smem + rt * kRowBytes + (((col / 8) ^ (rt % kChunks)) * 16) +
                                 (col % 8) * 2) = o;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    constexpr int kRowsPerPass = kMfmaThreads / kChunks;
    const int q = threadIdx.x % kChunks;
#pragma unroll 4
    for (int r0 = 0; r0 < BM; r0 += kRowsPerPass) {
      const int rt = r0 + threadIdx.x / kChunks;
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + rt * kRowBytes + ((q ^ (rt % kChunks)) * 16));
      *reinterpret_cast<u32x4*>(C + static_cast<int64_t>(m0 + rt) * N + n0 + 8 * q) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    OutT* crow = C + static_cast<int64_t>(m0 + wm * WM + 16 * i + r16) * N + n0 + wn * WN + 4 * g;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      Quad* dst = reinterpret_cast<Quad*>(crow + 16 * j);
      const Quad old = *dst;
      Quad o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o.v[e] = O::from_f32(alpha * acc_get(acc[i][j][e]) + beta * O::to_f32(old.v[e]));
      *dst = o;
    }
  }
}

}  // namespace mcke_amd
