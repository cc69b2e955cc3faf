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

namespace kore {

// ---------------------------------------------------------------------------------
// Direct-to-LDS engine (K-contiguous operands).
//
// NW = WM*WN waves (8 -> two waves per SIMD, so one wave's LDS/global waits are
// covered by the other's MFMAs).  Operand tiles are filled with
// global_load_lds_dwordx4: one wave instruction writes 64 x 16 bytes = 8 consecutive
// 128-byte LDS rows, lane l landing at row l/8, chunk l%8.  The XOR swizzle is
// applied on the source side: lane l fetches logical chunk (l%8) ^ swz8(row), so the
// LDS image is identical to the register-staged engine's and no staging VGPRs are
// needed.  Lanes whose chunk lies past K read a zero page instead (no branches).
// Fragments are double buffered in registers across the four 16-wide K sub-steps.
// ---------------------------------------------------------------------------------
__device__ const u32x4_t kZeroPage[4] = {};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void gl_lds16(const void* src, uint16_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)lds_dst, 16, 0, 0);
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename T, int BM, int BN, int WM, int WN>
struct DLEngine {
  static constexpr int NW = WM * WN;
  static constexpr int NT = 64 * NW;
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(MI >= 1 && NI >= 1 && WROWS % 32 == 0 && WCOLS % 32 == 0, "wave tile is a multiple of 32x32");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int STAGE = A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = 2 * STAGE;
  static constexpr int AJ = BM / 8 / NW, BJ = BN / 8 / NW;  // wave-loads per wave per stage
  static_assert(AJ * 8 * NW == BM && BJ * 8 * NW == BN, "8-row wave loads must cover the tile");

  // Row (0..BM) of the tile that lane `lane` of wave `wave` fills in wave-load j, and
  // the logical 16-byte chunk it fetches for that row.
  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ swz8(row); }

  // Per-lane source of each wave-load: row pointer + 8 * chunk(row, lane) elements.
  const uint16_t* a_src[AJ];
  const uint16_t* b_src[BJ];
  int a_k[AJ], b_k[BJ];  // element offset of the lane's chunk inside a K step (8*chunk)

  __device__ __forceinline__ void issue(uint16_t* lds, int stage, int k0, int K, int wave) {
    uint16_t* sA = lds + stage * STAGE;
    uint16_t* sB = sA + A_ELEMS;
    const bool full = k0 + kBK <= K;
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const void* src = full || (k0 + a_k[j] < K) ? (const void*)(a_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sA + (wave + NW * j) * 8 * kBK);
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const void* src = full || (k0 + b_k[j] < K) ? (const void*)(b_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sB + (wave + NW * j) * 8 * kBK);
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

  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
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
    issue(lds, 0, 0, K, wave);
    wait_vmem_all();
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) issue(lds, cur ^ 1, (kt + 1) * kBK, K, wave);
      const uint16_t* sA = lds + cur * STAGE + rowA0 * kBK;
      const uint16_t* sB = lds + cur * STAGE + A_ELEMS + rowB0 * kBK;
      u32x4_t af[2][MI], bfr[2][NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[0][i] = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][0]);
#pragma unroll
      for (int j = 0; j < NI; ++j) bfr[0][j] = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][0]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = ks & 1, n = c ^ 1;
        if (ks < 3) {
#pragma unroll
          for (int i = 0; i < MI; ++i) af[n][i] = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][ks + 1]);
#pragma unroll
          for (int j = 0; j < NI; ++j) bfr[n][j] = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][ks + 1]);
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = Op::mma32(bfr[c][j], af[c][i], acc[i][j]);
      }
      wait_vmem_all();
      __syncthreads();
    }
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Ring engine: direct-to-LDS loads into an NSTAGE-deep ring of 32-wide K stages.
//
// Global latency on MI355X under GEMM load is ~1 us, longer than one K step of MFMA
// work, so stages are issued NSTAGE-1 steps ahead (3 x 32 KiB in flight per CU for a
// 256x256 tile) and a stage is consumed after `s_waitcnt vmcnt(n)` for the loads
// issued later plus one barrier.  LDS rows are 64 bytes (32 x 16-bit); chunk c of
// row r lives at chunk c ^ swz4(r), swz4(r) = ((r >> 1) ^ (r >> 3)) & 3, which keeps
// the 32 fragment rows read by a half-wave on distinct banks for 32- and 64-bank
// LDS.  For rows R + lr with R % 32 == 0, swz4(R + lr) == swz4(lr).
// ---------------------------------------------------------------------------------
constexpr int kRK = 32;  // K elements per ring stage (64-byte rows)

__device__ __forceinline__ int swz4(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Execution barrier without the workgroup release fence of __syncthreads(): that
// fence waits for *all* outstanding vector-memory operations (vmcnt(0)), which would
// drain the prefetched ring stages at every K step.  Callers order their own memory:
// direct-to-LDS loads via wait_vmcnt<N>() before the barrier.  The empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void exec_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename T, int BM, int BN, int WM, int WN, int NSTAGE>
struct RingEngine {
  static constexpr int NW = WM * WN;
  static constexpr int NT = 64 * NW;
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(MI >= 1 && NI >= 1 && WROWS % 32 == 0 && WCOLS % 32 == 0, "wave tile is a multiple of 32x32");
  static constexpr int A_ELEMS = BM * kRK, B_ELEMS = BN * kRK;
  static constexpr int STAGE = A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = NSTAGE * STAGE;
  static constexpr int AJ = BM / 16 / NW, BJ = BN / 16 / NW;  // 16-row wave loads per wave per stage
  static_assert(AJ * 16 * NW == BM && BJ * 16 * NW == BN, "16-row wave loads must cover the tile");
  static constexpr int LPS = AJ + BJ;  // load instructions per wave per stage
  static_assert(NSTAGE >= 2 && NSTAGE <= 4, "2..4 stages");

  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 16 + (lane >> 2); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 16 + (lane >> 2); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 3) ^ swz4(row); }

  const uint16_t* a_src[AJ];
  const uint16_t* b_src[BJ];
  int a_k[AJ], b_k[BJ];

  __device__ __forceinline__ void issue(uint16_t* lds, int slot, int k0, int K, int wave) {
    uint16_t* sA = lds + slot * STAGE;
    uint16_t* sB = sA + A_ELEMS;
    const bool full = k0 + kRK <= K;
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const void* src = full || (k0 + a_k[j] < K) ? (const void*)(a_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sA + (wave + NW * j) * 16 * kRK);
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const void* src = full || (k0 + b_k[j] < K) ? (const void*)(b_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sB + (wave + NW * j) * 16 * kRK);
    }
  }

  // Issue load q (0 .. LPS-1) of a stage: A wave-loads first, then B.
  __device__ __forceinline__ void issue_one(uint16_t* lds, int slot, int k0, int K, int wave, int q) {
    uint16_t* sA = lds + slot * STAGE;
    uint16_t* sB = sA + A_ELEMS;
    const bool full = k0 + kRK <= K;
    if (q < AJ) {
      const void* src = full || (k0 + a_k[q] < K) ? (const void*)(a_src[q] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sA + (wave + NW * q) * 16 * kRK);
    } else {
      const int j = q - AJ;
      const void* src = full || (k0 + b_k[j] < K) ? (const void*)(b_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sB + (wave + NW * j) * 16 * kRK);
    }
  }

  // Wait until the loads of the stage about to be consumed are done, given that
  // `later` more stages have been issued after it.
  static __device__ __forceinline__ void wait_stage(int later) {
    if (later >= 2) wait_vmcnt<2 * LPS>();
    else if (later == 1) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
  }

  static __device__ __forceinline__ void zero(f32x16_t (&acc)[MI][NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
    const int sw = swz4(lr);
    const int off0 = lr * kRK + (((0 + hh) ^ sw) << 3);
    const int off1 = lr * kRK + (((2 + hh) ^ sw) << 3);
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    const int nk = (K + kRK - 1) / kRK;
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s)
      if (s < nk) issue(lds, s, s * kRK, K, wave);
    for (int kt = 0; kt < nk; ++kt) {
      wait_stage(min(NSTAGE - 2, nk - 1 - kt));
      exec_barrier();
      const int slot = kt % NSTAGE;
      const uint16_t* sA = lds + slot * STAGE + rowA0 * kRK;
      const uint16_t* sB = lds + slot * STAGE + A_ELEMS + rowB0 * kRK;
      u32x4_t af[2][MI], bfr[2][NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[0][i] = *(const u32x4_t*)(sA + i * 32 * kRK + off0);
#pragma unroll
      for (int j = 0; j < NI; ++j) bfr[0][j] = *(const u32x4_t*)(sB + j * 32 * kRK + off0);
#pragma unroll
      for (int i = 0; i < MI; ++i) af[1][i] = *(const u32x4_t*)(sA + i * 32 * kRK + off1);
#pragma unroll
      for (int j = 0; j < NI; ++j) bfr[1][j] = *(const u32x4_t*)(sB + j * 32 * kRK + off1);
      // The next stage's direct loads are spread through the MFMA stream (one load per
      // MFMA group) so the per-CU request queue never fills: a full queue stalls the
      // issuing wave and would serialise memory and compute.
      const bool more = kt + NSTAGE - 1 < nk;
      const int nslot = (kt + NSTAGE - 1) % NSTAGE, nk0 = (kt + NSTAGE - 1) * kRK;
      constexpr int NMMA = 2 * MI * NI;
      constexpr int GROUP = (NMMA + LPS - 1) / LPS;
#pragma unroll
      for (int m = 0; m < NMMA; ++m) {
        if (m % GROUP == 0 && m / GROUP < LPS) {
          __builtin_amdgcn_sched_barrier(0);
          if (more) issue_one(lds, nslot, nk0, K, wave, m / GROUP);
          __builtin_amdgcn_sched_barrier(0);
        }
        const int ks = m / (MI * NI), i = (m / NI) % MI, j = m % NI;
        acc[i][j] = Op::mma32(bfr[ks][j], af[ks][i], acc[i][j]);
      }
    }
    __syncthreads();  // every wave is done with the ring before the caller reuses LDS
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Pipelined ring engine: 4 waves (one per SIMD, 128x128 wave tiles, accumulators
// in AGPRs), NSTAGE-deep ring of 32-wide K stages filled by direct-to-LDS loads.
//
// A stage is two 16-wide K sub-steps.  Fragments of sub-step t+1 are read from LDS
// while the MFMAs of sub-step t run, including across the stage boundary: the ring
// barrier sits between the two halves of a stage (after the wave's own LDS reads
// have returned), so the first fragments of stage s+1 are read under the second
// half of stage s's MFMAs.  The next-but-two stage's direct loads are spread through
// both halves (one per four MFMAs).  Slot reuse: stage s+NSTAGE-1 overwrites the
// slot of stage s-1, whose last reads completed before the mid barrier of s-1.
// ---------------------------------------------------------------------------------
template <typename T, int BM, int BN, int NSTAGE>
struct PipeEngine {
  static constexpr int WM = 2, WN = 2, NW = 4;
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(WROWS % 32 == 0 && WCOLS % 32 == 0 && MI >= 1 && NI >= 1, "wave tile");
  static constexpr int A_ELEMS = BM * kRK, B_ELEMS = BN * kRK;
  static constexpr int STAGE = A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = NSTAGE * STAGE;
  static constexpr int AJ = BM / 16 / NW, BJ = BN / 16 / NW;
  static_assert(AJ * 16 * NW == BM && BJ * 16 * NW == BN, "16-row wave loads must cover the tile");
  static constexpr int LPS = AJ + BJ;
  static constexpr int HALF = LPS / 2;  // loads issued in the first half of a stage
  static_assert(NSTAGE == 4, "ring of 4 stages");

  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 16 + (lane >> 2); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 16 + (lane >> 2); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 3) ^ swz4(row); }

  const uint16_t* a_src[AJ];
  const uint16_t* b_src[BJ];
  int a_k[AJ], b_k[BJ];

  __device__ __forceinline__ void issue_one(uint16_t* lds, int slot, int k0, int K, int wave, int q) {
    uint16_t* sA = lds + slot * STAGE;
    uint16_t* sB = sA + A_ELEMS;
    const bool full = k0 + kRK <= K;
    if (q < AJ) {
      const void* src = full || (k0 + a_k[q] < K) ? (const void*)(a_src[q] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sA + (wave + NW * q) * 16 * kRK);
    } else {
      const int j = q - AJ;
      const void* src = full || (k0 + b_k[j] < K) ? (const void*)(b_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sB + (wave + NW * j) * 16 * kRK);
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

  // Wait for the loads of a stage given how many load instructions were issued after it.
  static __device__ __forceinline__ void wait_after(int n) {
    if (n >= LPS + HALF) wait_vmcnt<LPS + HALF>();
    else if (n >= LPS) wait_vmcnt<LPS>();
    else if (n >= HALF) wait_vmcnt<HALF>();
    else wait_vmcnt<0>();
  }

  __device__ __forceinline__ void read_frags(const uint16_t* lds, int slot, int off, int rowA0, int rowB0,
                                             u32x4_t (&af)[MI], u32x4_t (&bf)[NI]) const {
    const uint16_t* sA = lds + slot * STAGE + rowA0 * kRK;
    const uint16_t* sB = lds + slot * STAGE + A_ELEMS + rowB0 * kRK;
#pragma unroll
    for (int i = 0; i < MI; ++i) af[i] = *(const u32x4_t*)(sA + i * 32 * kRK + off);
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[j] = *(const u32x4_t*)(sB + j * 32 * kRK + off);
  }

  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
    const int sw = swz4(lr);
    const int off0 = lr * kRK + (((0 + hh) ^ sw) << 3);
    const int off1 = lr * kRK + (((2 + hh) ^ sw) << 3);
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    const int nk = (K + kRK - 1) / kRK;
    if (nk == 0) return;
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s)
      if (s < nk)
#pragma unroll
        for (int q = 0; q < LPS; ++q) issue_one(lds, s, s * kRK, K, wave, q);
    wait_after((nk > 1 ? LPS : 0) + (nk > 2 ? LPS : 0));
    exec_barrier();
    u32x4_t f0a[MI], f0b[NI], f1a[MI], f1b[NI];
    read_frags(lds, 0, off0, rowA0, rowB0, f0a, f0b);
    constexpr int NMMA = MI * NI;                  // MFMAs per sub-step
    constexpr int GRP_LD = (NMMA + HALF - 1) / HALF;  // MFMAs per direct load
    for (int s = 0; s < nk; ++s) {
      const int slot = s % NSTAGE;
      const bool more = s + NSTAGE - 1 < nk;
      const int nslot = (s + NSTAGE - 1) % NSTAGE, nk0 = (s + NSTAGE - 1) * kRK;
      // ---- first half: MFMAs of sub-step 0, reads of sub-step 1, HALF direct loads
      read_frags(lds, slot, off1, rowA0, rowB0, f1a, f1b);
#pragma unroll
      for (int m = 0; m < NMMA; ++m) {
        if (m % GRP_LD == 0 && m / GRP_LD < HALF) {
          __builtin_amdgcn_sched_barrier(0);
          if (more) issue_one(lds, nslot, nk0, K, wave, m / GRP_LD);
          __builtin_amdgcn_sched_barrier(0);
        }
        const int i = m / NI, j = m % NI;
        acc[i][j] = Op::mma32(f0b[j], f0a[i], acc[i][j]);
      }
      // ---- ring barrier: stage s+1 landed (own loads + everyone past the barrier)
      const bool next = s + 1 < nk;
      if (next) {
        const int after = (s + 2 < nk ? LPS : 0) + (more ? HALF : 0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_after(after);
        exec_barrier();
      }
      // ---- second half: MFMAs of sub-step 1, reads of stage s+1 sub-step 0, rest of the loads
      if (next) read_frags(lds, (s + 1) % NSTAGE, off0, rowA0, rowB0, f0a, f0b);
#pragma unroll
      for (int m = 0; m < NMMA; ++m) {
        if (m % GRP_LD == 0 && m / GRP_LD < LPS - HALF) {
          __builtin_amdgcn_sched_barrier(0);
          if (more) issue_one(lds, nslot, nk0, K, wave, HALF + m / GRP_LD);
          __builtin_amdgcn_sched_barrier(0);
        }
        const int i = m / NI, j = m % NI;
        acc[i][j] = Op::mma32(f1b[j], f1a[i], acc[i][j]);
      }
    }
    __syncthreads();  // every wave is done with the ring before the caller reuses LDS
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Pipe64 engine: 4 waves (one per SIMD, 128x128 wave tiles, AGPR accumulators), two
// LDS stages of 64-wide K (128-byte rows, chunk c of row r at c ^ swz8(r)), filled
// by direct-to-LDS loads whose 8 lanes per row cover one whole 128-byte line (one
// L2 request per line; 64-byte rows would double the request count).
//
// Iteration s (stage s in slot s%2, its sub-step-0 fragments already in registers):
//   issue stage s+1 into slot (s+1)%2, spread over the first two sub-steps' MFMAs;
//   sub-steps 0..2: MFMAs of sub-step t while the fragments of t+1 are read;
//   own LDS reads done + own loads landed, then one barrier;
//   sub-step 3: MFMAs while the first fragments of stage s+1 are read.
// Slot (s+1)%2 last held stage s-1, whose final reads completed before the barrier
// of iteration s-1, so one barrier per 64-wide K step suffices.
// ---------------------------------------------------------------------------------
template <typename T, int BM, int BN>
struct Pipe64Engine {
  static constexpr int WM = 2, WN = 2, NW = 4;
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(WROWS % 32 == 0 && WCOLS % 32 == 0 && MI >= 1 && NI >= 1, "wave tile");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int STAGE = A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = 2 * STAGE;
  static constexpr int AJ = BM / 8 / NW, BJ = BN / 8 / NW;  // 8-row wave loads per wave per stage
  static_assert(AJ * 8 * NW == BM && BJ * 8 * NW == BN, "8-row wave loads must cover the tile");
  static constexpr int LPS = AJ + BJ;

  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ swz8(row); }

  const uint16_t* a_src[AJ];
  const uint16_t* b_src[BJ];
  int a_k[AJ], b_k[BJ];

  __device__ __forceinline__ void issue_one(uint16_t* lds, int slot, int k0, int K, int wave, int q) {
    uint16_t* sA = lds + slot * STAGE;
    uint16_t* sB = sA + A_ELEMS;
    const bool full = k0 + kBK <= K;
    if (q < AJ) {
      const void* src = full || (k0 + a_k[q] < K) ? (const void*)(a_src[q] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sA + (wave + NW * q) * 8 * kBK);
    } else {
      const int j = q - AJ;
      const void* src = full || (k0 + b_k[j] < K) ? (const void*)(b_src[j] + k0) : (const void*)kZeroPage;
      gl_lds16(src, sB + (wave + NW * j) * 8 * kBK);
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

  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
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
    auto read = [&](int slot, int ks, u32x4_t (&af)[MI], u32x4_t (&bf)[NI]) {
      const uint16_t* sA = lds + slot * STAGE + rowA0 * kBK;
      const uint16_t* sB = lds + slot * STAGE + A_ELEMS + rowB0 * kBK;
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][ks]);
#pragma unroll
      for (int j = 0; j < NI; ++j) bf[j] = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][ks]);
    };
    const int nk = (K + kBK - 1) / kBK;
    if (nk == 0) return;
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 0, 0, K, wave, q);
    wait_vmcnt<0>();
    exec_barrier();
    u32x4_t fa[2][MI], fb[2][NI];
    read(0, 0, fa[0], fb[0]);
    constexpr int NMMA = MI * NI;
    constexpr int LD_STEPS = 2;  // sub-steps that carry the next stage's loads
    constexpr int PER = (LPS + LD_STEPS * NMMA - 1) / (LD_STEPS * NMMA);  // loads per MFMA slot
    constexpr int EVERY = (LD_STEPS * NMMA) / ((LPS + PER - 1) / PER);     // MFMAs between load slots
    for (int s = 0; s < nk; ++s) {
      const int slot = s & 1;
      const bool more = s + 1 < nk;
      const int k1 = (s + 1) * kBK;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = ks & 1;
        if (ks < 3) {
          read(slot, ks + 1, fa[c ^ 1], fb[c ^ 1]);
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          wait_vmcnt<0>();
          exec_barrier();
          if (more) read(slot ^ 1, 0, fa[c ^ 1], fb[c ^ 1]);
        }
#pragma unroll
        for (int m = 0; m < NMMA; ++m) {
          if (ks < LD_STEPS) {
            const int g = ks * NMMA + m;
            if (g % EVERY == 0) {
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int u = 0; u < PER; ++u) {
                const int q = (g / EVERY) * PER + u;
                if (q < LPS && more) issue_one(lds, slot ^ 1, k1, K, wave, q);
              }
              __builtin_amdgcn_sched_barrier(0);
            }
          }
          const int i = m / NI, j = m % NI;
          acc[i][j] = Op::mma32(fb[c][j], fa[c][i], acc[i][j]);
        }
      }
    }
    __syncthreads();  // every wave is done with both stages before the caller reuses LDS
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Buffer-load pipelined engine (the production dense/grouped GEMM main loop).
//
// Same schedule as Pipe64Engine (4 waves, 128x128 wave tiles, two 64-wide K stages,
// one barrier per K step, next stage's loads spread over the first half of the
// MFMAs, fragments read one sub-step ahead), but the direct-to-LDS loads are
// buffer_load_dwordx4 ... lds with a buffer resource per operand, a per-lane byte
// offset fixed at setup (row and swizzled chunk) and the K advance in the scalar
// offset -- no per-load vector address arithmetic, which otherwise costs more issue
// slots than the MFMAs leave free.  Rows are gathered for free (any per-lane
// offset).  Requires K % 64 == 0; out-of-range offsets read 0 via the resource size.
// ---------------------------------------------------------------------------------
constexpr int kBufWord3 = 0x00020000;  // gfx9-family raw buffer resource flags

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufWord3);
}

__device__ __forceinline__ void buf_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint16_t* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, (int)voff, (int)soff, 0, 0);
}

template <typename T, int BM, int BN, int WM_ = 2, int WN_ = 2, int AP = 1>
struct BufPipeEngine {
  static constexpr int WM = WM_, WN = WN_, NW = WM * WN;
  static_assert(NW == 4, "4 waves");
  static_assert(AP == 1 || AP == 2, "one or two A planes");
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(WROWS % 32 == 0 && WCOLS % 32 == 0 && MI >= 1 && NI >= 1, "wave tile");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int B_OFF = AP * A_ELEMS;
  static constexpr int STAGE = AP * A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = 2 * STAGE;
  static constexpr int AJ = BM / 8 / NW, BJ = BN / 8 / NW;
  static_assert(AJ * 8 * NW == BM && BJ * 8 * NW == BN, "8-row wave loads must cover the tile");
  static constexpr int LPS = AP * AJ + BJ;
  static_assert(LPS % 2 == 0, "loads of a stage are issued in two equal halves");

  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  // Logical 16-byte chunk lane `lane` fetches for `row` (element offset 8 * chunk).
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ swz8(row); }

  __amdgpu_buffer_rsrc_t ra, ra2, rb;  // ra2: second A plane (same offsets), AP == 2
  uint32_t a_voff[AJ], b_voff[BJ];      // bytes: row * row_stride + 16 * chunk

  __device__ __forceinline__ void issue_one(uint16_t* lds, int slot, uint32_t soff, int wave, int q) {
    uint16_t* sA = lds + slot * STAGE;
    if (q < AJ) {
      buf_lds16(ra, a_voff[q], soff, sA + (wave + NW * q) * 8 * kBK);
    } else if (AP == 2 && q < 2 * AJ) {
      const int j = q - AJ;
      buf_lds16(ra2, a_voff[j], soff, sA + A_ELEMS + (wave + NW * j) * 8 * kBK);
    } else {
      const int j = q - AP * AJ;
      buf_lds16(rb, b_voff[j], soff, sA + B_OFF + (wave + NW * j) * 8 * kBK);
    }
  }

  static __device__ __forceinline__ void zero(f32x16_t (&acc)[MI][NI]) {
    static_assert(MI >= 1, "");
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  // K must be a multiple of 64.
  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    // wave index as a scalar so LDS destinations (M0) are pure scalar arithmetic
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
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
    // Fragment f of a sub-step: f < AP*MI -> A plane f/MI block f%MI, else B block.
    auto read_one = [&](int slot, int ks, int f, u32x4_t (&af)[AP * MI], u32x4_t (&bf)[NI]) {
      if (f < AP * MI) {
        const int pl = f / MI, i = f % MI;
        af[f] = *(const u32x4_t*)(lds + slot * STAGE + pl * A_ELEMS + rowA0 * kBK + i * 32 * kBK + offA[i & 1][ks]);
      } else {
        const int j = f - AP * MI;
        bf[j] = *(const u32x4_t*)(lds + slot * STAGE + B_OFF + rowB0 * kBK + j * 32 * kBK + offB[j & 1][ks]);
      }
    };
    auto read = [&](int slot, int ks, u32x4_t (&af)[AP * MI], u32x4_t (&bf)[NI]) {
#pragma unroll
      for (int f = 0; f < AP * MI + NI; ++f) read_one(slot, ks, f, af, bf);
    };
    const int nk = K / kBK;
    if (nk == 0) return;
    constexpr int HALF = LPS / 2;
    constexpr int NMMA = AP * MI * NI;  // MFMAs per sub-step
    constexpr int EVERY = NMMA / HALF > 0 ? NMMA / HALF : 1;  // MFMAs per load inside a sub-step
    static_assert(HALF * EVERY <= NMMA, "a half stage of loads must fit in one sub-step");
    // Loads of a stage go out in two halves: the first right after the barrier that
    // frees its slot (under the last sub-step of the previous stage), the second
    // under the first sub-step of the next iteration.  Past the last stage the
    // K offset is clamped, re-loading the last stage into the idle slot (no branch).
    const uint32_t kmax = (uint32_t)(nk - 1) * (kBK * 2);
    auto soff_of = [&](int stage) { return min((uint32_t)stage * (kBK * 2), kmax); };
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 0, 0u, wave, q);
#pragma unroll
    for (int q = 0; q < HALF; ++q) issue_one(lds, 1, soff_of(1), wave, q);
    wait_vmcnt<HALF>();
    exec_barrier();
    u32x4_t fa[2][AP * MI], fb[2][NI];
    read(0, 0, fa[0], fb[0]);
    // Per sub-step the instruction order is pinned: the next sub-step's fragment
    // reads (and, in sub-steps 0 and 3, half a stage of direct loads) are interleaved
    // one per MFMA over the first half of the MFMAs, so LDS latency is covered by
    // the second half.
    constexpr int NRD = AP * MI + NI;  // fragment reads per sub-step
    static_assert(NRD <= NMMA && HALF <= NMMA, "interleave needs enough MFMAs");
    for (int s = 0; s < nk; ++s) {
      const int slot = s & 1;
      const uint32_t soff1 = soff_of(s + 1), soff2 = soff_of(s + 2);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int c = ks & 1;
        if (ks == 3) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          wait_vmcnt<0>();
          exec_barrier();
        }
        // MFMA m, then (m < NRD) one fragment read of the next sub-step, then
        // (sub-steps 0 and 3, m < HALF) one direct load; hard scheduling fences keep
        // this order.
        const int rslot = ks < 3 ? slot : (slot ^ 1);
        const int rks = ks < 3 ? ks + 1 : 0;
#pragma unroll
        for (int m = 0; m < NMMA; ++m) {
          __builtin_amdgcn_sched_barrier(0);
          const int pl = m / (MI * NI), i = (m / NI) % MI, j = m % NI;
          acc[i][j] = Op::mma32(fb[c][j], fa[c][pl * MI + i], acc[i][j]);
          if (m < NRD) read_one(rslot, rks, m, fa[c ^ 1], fb[c ^ 1]);
          if (m < HALF) {
            if (ks == 0) issue_one(lds, slot ^ 1, soff1, wave, HALF + m);  // 2nd half of s+1
            else if (ks == 3) issue_one(lds, slot, soff2, wave, m);       // 1st half of s+2
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vmcnt<0>();  // drain the clamped trailing loads before LDS is reused
    __syncthreads();
  }
};

}  // namespace kore
