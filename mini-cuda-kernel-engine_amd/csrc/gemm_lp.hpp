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
  constexpr int i = IDX / S::NT, j = IDX % S::NT;
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

}  // namespace mcke_amd
