// Tile engine shared by the dense, batched and MoE grouped GEMM kernels (gfx950).
//
// One workgroup = 256 threads = 4 waves in a WM x WN grid computes a BM x BN tile
// of D[n][m] = sum_k B[n][k] * A[m][k] with v_mfma_f32_32x32x16_{bf16,f16}.
// Operand rows are described by per-thread row pointers chosen by the caller, so a
// caller can gather A rows (MoE token dispatch) or remap B rows (interleaved
// gate/up weights) at no cost in the K loop.
//
// LDS layout: each operand tile is [rows][64] 16-bit values = 128-byte rows; the
// 16-byte chunk c of row r lives at chunk c ^ swz8(r).  Tiles are double buffered:
// the global loads of K step k+1 are in flight while step k is multiplied, with one
// barrier per K step.  B may also be N-contiguous ([K][N] in memory); such a tile
// is transposed in registers (8x8 blocks) before it is written to LDS.
// With AP == 2 the A operand has two planes (A = A0 + A1, e.g. the bf16 high and low
// parts of an fp32 activation): both planes share every B fragment, so the product
// keeps ~16 significand bits of A at the cost of a second MFMA per B fragment.
#pragma once

#include "kore_common.hpp"

namespace kore {

constexpr int kEngineThreads = 256;
constexpr int kBK = 64;  // K elements per step (128 bytes per row)

__device__ __forceinline__ u32x4_t ld16(const void* p) { return *(const u32x4_t*)p; }
__device__ __forceinline__ u32x4_t zero4() { return u32x4_t{0u, 0u, 0u, 0u}; }

// 8x8 transpose of 16-bit values: in[r] holds row r (8 values); out[c] holds column c.
__device__ __forceinline__ void transpose8x8(const u32x4_t in[8], u32x4_t out[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[j][e] = __builtin_amdgcn_perm(in[2 * e + 1][j >> 1], in[2 * e][j >> 1], sel);
  }
}

enum { B_KC = 0, B_NC = 1 };

template <typename T, int BM, int BN, int WM, int WN, int BL, int AP = 1>
struct TileEngine {
  static_assert(AP == 1 || AP == 2, "one or two A planes");
  static_assert(WM * WN == 4, "4 waves per workgroup");
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(MI >= 1 && NI >= 1 && WROWS % 32 == 0 && WCOLS % 32 == 0, "wave tile is a multiple of 32x32");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int STAGE = AP * A_ELEMS + B_ELEMS;
  static constexpr int B_OFF = AP * A_ELEMS;  // B tile offset inside a stage
  static constexpr int LDS_ELEMS = 2 * STAGE;
  static constexpr int LA = BM * 8 / kEngineThreads;
  static_assert(LA >= 1 && BM % 32 == 0, "BM >= 32");
  static constexpr int LB_KC = BN * 8 / kEngineThreads;
  static constexpr int NBLK_NC = (kBK / 8) * (BN / 8);
  static constexpr int LB_NC = (NBLK_NC + kEngineThreads - 1) / kEngineThreads;
  static constexpr int LB = (BL == B_KC) ? LB_KC : LB_NC;
  static constexpr int RB = (BL == B_KC) ? LB_KC : 8 * LB_NC;

  // Row r (0..BM) of the A tile handled by load slot j of this thread.
  static __device__ __forceinline__ int a_row_of(int tid, int j) { return (tid >> 3) + 32 * j; }
  static __device__ __forceinline__ int b_row_of(int tid, int j) { return (tid >> 3) + 32 * j; }
  // N-contiguous B: block q = (kb, nb) of 8 K-rows x 8 columns.
  static __device__ __forceinline__ int nc_kb(int tid, int j) { return (tid + kEngineThreads * j) / (BN / 8); }
  static __device__ __forceinline__ int nc_nb(int tid, int j) { return (tid + kEngineThreads * j) % (BN / 8); }
  static __device__ __forceinline__ bool nc_active(int tid, int j) {
    return (NBLK_NC % kEngineThreads == 0) || (tid + kEngineThreads * j < NBLK_NC);
  }

  // a_src[j]: start of A row a_row_of(tid, j) (any row inside the tensor for rows
  // that fall outside the problem; their results are discarded), offset by the
  // thread's chunk (tid & 7) * 8 elements.
  // B_KC: b_src[j] likewise for B^T rows.  B_NC: b_src[j] points at element
  // (kb*8, column of block nb) and ldb is the K-row stride.
  const uint16_t* a_src[LA];
  const uint16_t* a2_src[AP == 2 ? LA : 1];  // second A plane (AP == 2)
  const uint16_t* b_src[LB];
  int64_t ldb;
  u32x4_t ra[LA];
  u32x4_t ra2[AP == 2 ? LA : 1];
  u32x4_t rb[RB];

  __device__ __forceinline__ void load(int k0, int K, int tid) {
    const int ch = tid & 7;
    const bool kin = (k0 + ch * 8) < K;
#pragma unroll
    for (int j = 0; j < LA; ++j) ra[j] = kin ? ld16(a_src[j] + k0) : zero4();
    if constexpr (AP == 2) {
#pragma unroll
      for (int j = 0; j < LA; ++j) ra2[j] = kin ? ld16(a2_src[j] + k0) : zero4();
    }
    if constexpr (BL == B_KC) {
#pragma unroll
      for (int j = 0; j < LB; ++j) rb[j] = kin ? ld16(b_src[j] + k0) : zero4();
    } else {
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        const int kb = nc_kb(tid, j);
        const bool act = nc_active(tid, j);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const bool ok = act && (k0 + kb * 8 + kk) < K;
          rb[8 * j + kk] = ok ? ld16(b_src[j] + (int64_t)(k0 + kk) * ldb) : zero4();
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, int stage, int tid) const {
    uint16_t* sA = lds + stage * STAGE;
    uint16_t* sB = sA + B_OFF;
    const int ch = tid & 7;
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int r = a_row_of(tid, j);
      *(u32x4_t*)(sA + r * kBK + ((ch ^ swz8(r)) << 3)) = ra[j];
      if constexpr (AP == 2) *(u32x4_t*)(sA + A_ELEMS + r * kBK + ((ch ^ swz8(r)) << 3)) = ra2[j];
    }
    if constexpr (BL == B_KC) {
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        const int r = b_row_of(tid, j);
        *(u32x4_t*)(sB + r * kBK + ((ch ^ swz8(r)) << 3)) = rb[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < LB; ++j) {
        if (nc_active(tid, j)) {
          const int kb = nc_kb(tid, j), nb = nc_nb(tid, j);
          u32x4_t tr[8];
          transpose8x8(&rb[8 * j], tr);
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const int n = nb * 8 + jj;
            *(u32x4_t*)(sB + n * kBK + ((kb ^ swz8(n)) << 3)) = tr[jj];
          }
        }
      }
    }
  }

  // Full K loop; acc must be zeroed by the caller.  Leaves LDS free (barrier) on exit.
  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
    // fragment row R + lr, chunk 2*ks + hh; for R % 32 == 0:
    // swz8(R + lr) = (lr & 7) ^ (lr >> 3) ^ (4 * ((R / 32) & 1))
    int offA[2][4], offB[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int qa = (wm * MI + par) & 1, qb = (wn * NI + par) & 1;
      const int swa = ((lr & 7) ^ (lr >> 3) ^ (4 * qa)) & 7;
      const int swb = ((lr & 7) ^ (lr >> 3) ^ (4 * qb)) & 7;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        offA[par][ks] = lr * kBK + (((2 * ks + hh) ^ swa) << 3);
        offB[par][ks] = lr * kBK + (((2 * ks + hh) ^ swb) << 3);
      }
    }
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    const int nk = (K + kBK - 1) / kBK;
    load(0, K, tid);
    store(lds, 0, tid);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load((kt + 1) * kBK, K, tid);
      const uint16_t* sA = lds + cur * STAGE + rowA0 * kBK;
      const uint16_t* sB = lds + cur * STAGE + B_OFF + rowB0 * kBK;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4_t af[MI], bfr[NI];
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][ks]);
#pragma unroll
        for (int j = 0; j < NI; ++j) bfr[j] = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][ks]);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = Op::mma32(bfr[j], af[i], acc[i][j]);
        if constexpr (AP == 2) {
#pragma unroll
          for (int i = 0; i < MI; ++i) af[i] = *(const u32x4_t*)(sA + A_ELEMS + i * 32 * kBK + offA[i & 1][ks]);
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[i][j] = Op::mma32(bfr[j], af[i], acc[i][j]);
        }
      }
      if (kt + 1 < nk) store(lds, cur ^ 1, tid);
      __syncthreads();
    }
  }

  static __device__ __forceinline__ void zero(f32x16_t (&acc)[MI][NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }
};

// Output coordinates held by a lane: block (i, j) of its wave tile, register group
// g (0..3) holds the 4 consecutive columns  col = j*32 + 8*g + 4*(lane/32) + e
// (e = 0..3) of row  i*32 + lane%32  (wave-tile coordinates).
__device__ __forceinline__ int out_row(int i, int lane) { return i * 32 + (lane & 31); }
__device__ __forceinline__ int out_col(int j, int g, int lane) { return j * 32 + 8 * g + 4 * (lane >> 5); }

// Stage a wave's packed 16-bit output tile [WROWS][WCOLS] in LDS (16-byte chunks,
// XOR swizzled by row) so it can be written with row-contiguous 16-byte stores.
template <int WROWS, int WCOLS>
struct Stager {
  static constexpr int CH = WCOLS / 8;
  static __device__ __forceinline__ void put(uint16_t* stg, int row, int col, u32x2_t w) {
    const int pc = (col >> 3) ^ (row & (CH - 1));
    *(u32x2_t*)(stg + row * WCOLS + pc * 8 + (col & 7)) = w;
  }
  // Iterate the staged tile: fn(row, col, u32x4 value of 8 columns).
  template <typename F>
  static __device__ __forceinline__ void drain(const uint16_t* stg, int lane, F&& fn) {
#pragma unroll 4
    for (int it = 0; it < WROWS * CH / 64; ++it) {
      const int idx = it * 64 + lane;
      const int row = idx / CH, c8 = idx % CH;
      const u32x4_t v = *(const u32x4_t*)(stg + row * WCOLS + ((c8 ^ (row & (CH - 1))) << 3));
      fn(row, c8 * 8, v);
    }
  }
};

// Store 8 packed 16-bit values at dst (columns gn..gn+7 of a row of width N).
__device__ __forceinline__ void store_row8(uint16_t* dst, int gn, int N, bool vec, u32x4_t v) {
  if (vec && gn + 8 <= N) {
    *(u32x4_t*)dst = v;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (gn + e < N) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
  }
}

}  // namespace kore
