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
// A layouts of the direct-to-LDS engines: K-contiguous rows, or M-contiguous (a transposed
// view, element (m, k) at a[k * lda + m]) staged as K-rows and read back transposed.
enum { A_KC = 0, A_MC = 1 };

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
// Row / first column of elements 4g .. 4g + 3 of a lane's 32x32-tile accumulator, for
// tiles computed by one 32x32x16 MFMA chain (M16 false: one row per lane, the layout
// above) or by 2 x 2 16x16x32 chains (M16 true: sub-tile g = 2 * sm + sn, lane l holds
// row 16 sm + l % 16, columns 16 sn + 4 (l / 16) .. + 3).
template <bool M16>
__device__ __forceinline__ int acc_row(int i, int g, int lane) {
  return M16 ? i * 32 + 16 * (g >> 1) + (lane & 15) : out_row(i, lane);
}
template <bool M16>
__device__ __forceinline__ int acc_col(int j, int g, int lane) {
  return M16 ? j * 32 + 16 * (g & 1) + 4 * (lane >> 4) : out_col(j, g, lane);
}

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
// Direct-to-LDS helpers.  `buffer_load_dwordx4 ... lds` writes one wave instruction's
// 64 x 16 bytes to 1 KiB of consecutive LDS (lane l at byte 16*l), so a 128-byte LDS
// row gets 8 lanes; the XOR swizzle is applied on the source side (lane l fetches
// logical chunk (l % 8) ^ swz8(row)), which gives the same LDS image as the
// register-staged engine.  vmcnt counts these loads like any other vector load.
// ---------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Execution barrier without the workgroup release fence of __syncthreads(): that
// fence waits for *all* outstanding vector-memory operations (vmcnt(0)), which would
// drain prefetched stages at every K step.  Callers order their own memory:
// direct-to-LDS loads via wait_vmcnt<N>() before the barrier.  The empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void exec_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Buffer-load pipelined engine (the production dense/grouped GEMM main loop).
//
// 4 waves (one per SIMD, wave tiles up to 128x128, accumulators in AGPRs) or 8 waves
// (two per SIMD), two 64-wide K stages, one barrier per K step; the next stage's loads
// are spread over the MFMAs and fragments are read one sub-step (32 K for the 16x16x32
// MFMAs, 16 K for 32x32x16) ahead.  The direct-to-LDS loads are
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

// Cache-policy field of a buffer load: bit 1 is nt, the non-temporal hint.  Operands
// read exactly once (MoE expert weights) use it.  Measured on MI355X, a 100 MB stream of
// 16-byte buffer loads right after a 256 MiB zero fill (which leaves the memory-side
// cache full of dirty lines) runs at 2.8 TB/s with the default policy and 5.4 TB/s
// with nt (5.2 and 5.4 TB/s after a read-only fill), consistent with nt reads not
// allocating in that cache and so not forcing write-backs of its dirty lines.
constexpr int kCpolDefault = 0, kCpolNT = 2;

template <int CPOL>
__device__ __forceinline__ void buf_lds16_cp(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                             uint16_t* lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, (int)voff, (int)soff, 0, CPOL);
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16).  Within each group of 16 lanes, lane
// c supplies the address of 4 consecutive 16-bit values S[c][0..3]; lane i receives
// S[4e + i/4][i % 4] for e = 0..3.  So when lane c points at K-row k0 + c/4, columns
// n0 + 4 (c % 4) .. + 3 of an N-contiguous tile, lane i gets column n0 + i at K-rows
// k0 .. k0 + 3: four K-consecutive values of one column, an MFMA operand fragment.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;

__device__ __forceinline__ u32x2_t lds_read_tr16(const uint16_t* p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)p));
}

// Direct-to-LDS load issued as inline asm (M0 = LDS destination).  With the builtin the
// compiler records an LDS DMA write and, unable to prove that a following transpose
// read does not alias it, puts a vmcnt(0) wait in front of every such read, draining
// the load pipeline.  Loads issued this way are invisible to the compiler: the callers
// order them with explicit vmcnt waits and barriers, and no compiler-generated M0 use
// may sit between them (M0 is not preserved).
template <int CPOL = kCpolDefault>
__device__ __forceinline__ void buf_lds16_asm(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                              const uint16_t* lds_dst) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds_dst);
  // one wait state between the SALU write of M0 and the LDS DMA that reads it
  if constexpr (CPOL == kCpolNT)
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
                 :: "v"(voff), "s"(r), "s"(soff), "s"(m0) : "memory");
  else
    asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(r), "s"(soff), "s"(m0) : "memory");
}

// N-contiguous B stage layout shared by the direct-to-LDS engines: 64 K-rows of BN
// elements (BN = 128 or 256), one direct load instruction (512 elements) fills
// 512 / BN whole K-rows, and 16-byte chunk c of K-row k lives at chunk c ^ nc_x(k & 3)
// with nc_x = {0, 4, 10, 14}: the four K-rows one transpose read touches (32 bytes
// each) then sit in four distinct 32-byte bank slots of a 128-byte window, and with
// the next 16 lanes' chunk pair (same K-rows) in eight distinct slots of 256 bytes.
__device__ __forceinline__ int nc_x(int r) { return ((r & 1) * 4) ^ ((r >> 1) * 10); }
// The 16x16x32 fragments (BufPipeEngine with M16) read K-rows k0 .. k0 + 3 in lanes 0-15
// and k0 + 8 .. k0 + 11 in lanes 16-31 at the same columns, so K-rows with bit 3 set
// move by two more chunks: the 32 lanes of one half-wave then cover 16 distinct
// 16-byte slots of a 256-byte bank window ({0,1,4,5,10,11,14,15} and {2,3,6,7,8,9,12,13}
// for an even first chunk).
__device__ __forceinline__ int nc_x16(int r) { return nc_x(r & 3) ^ (((r >> 3) & 1) * 2); }

// Element offsets (within a stage's B region, sub-step 0, low half) of the transpose
// reads for the NI 32-column fragments of a wave whose columns start at col0: lane
// (16-lane group g, index c) reads K-rows 8 (lane / 32) + c / 4 (+ 4 for the high
// half, + 16 per sub-step), columns col0 + 32 j + 16 (g & 1) + 4 (c % 4) .. + 3.
template <int BN, int NI>
__device__ __forceinline__ void nc_frag_offsets(int lane, int col0, int (&off)[NI]) {
  const int c = lane & 15, x = nc_x(c >> 2), hh = lane >> 5;
  const int low = 2 * ((lane >> 4) & 1) + ((c & 3) >> 1);
#pragma unroll
  for (int j = 0; j < NI; ++j)
    off[j] = (8 * hh + (c >> 2)) * BN + (((col0 / 8 + 4 * j + low) ^ x) << 3) + 4 * (c & 1);
}

// BCPOL: cache policy of the B (weight) loads -- non-temporal where each weight tile
// is read by the row blocks of one expert only.
// M16: each 32x32 output tile is computed as 2 x 2 tiles of v_mfma_f32_16x16x32 (two
// K = 32 sub-steps per stage) instead of v_mfma_f32_32x32x16 (four K = 16 sub-steps).
// Same LDS layout, fragment bytes and load schedule; on MI355X the 16x16x32 shape
// sustains 20-30% more bf16 throughput than 32x32x16 under load (register-only probe,
// all CUs: 1.63-1.87 against 1.36-1.43 PF on random operands).  The accumulator of a
// 32x32 tile then holds sub-tile g = 2 * sm + sn in elements 4g .. 4g + 3
// (acc_row / acc_col<true>).
// AL == A_MC: A staged like an N-contiguous B (64 K-rows of BM elements, nc_x16 chunk
// swizzle) and read through transpose reads; 16x16 engine, one A plane.
template <typename T, int BM, int BN, int WM_ = 2, int WN_ = 2, int AP = 1, int BL = B_KC, int BCPOL = kCpolDefault,
          bool M16_ = false, int AL = A_KC>
struct BufPipeEngine {
  static constexpr bool M16 = M16_;
  static constexpr bool AMC = AL == A_MC;
  static_assert(!AMC || (M16_ && AP == 1 && (BM == 128 || BM == 256)), "M-contiguous A: 16x16 engine, one plane");
  static constexpr int NCRA = 512 / BM, NCHA = BM / 8;  // A_MC: K-rows per load, chunks per K-row
  static __device__ __forceinline__ int amc_krow(int wave, int lane, int j) {
    return (wave + WM_ * WN_ * j) * NCRA + lane / NCHA;
  }
  static __device__ __forceinline__ int amc_chunk(int krow, int lane) { return (lane % NCHA) ^ nc_x16(krow); }
  static constexpr int WM = WM_, WN = WN_, NW = WM * WN;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
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
  // Swizzle key of a K-contiguous row: the 16x16 engine reads 16-row fragments (swz16),
  // the 32x32 engine 32-row ones (swz8).
  static __device__ __forceinline__ int row_key(int row) { return M16 ? swz16(row) : swz8(row); }
  // Logical 16-byte chunk lane `lane` fetches for `row` (element offset 8 * chunk).
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ row_key(row); }

  // N-contiguous B (BL == B_NC): K-rows of BN elements, NCR per direct load
  // instruction, chunk swizzle nc_x.
  static constexpr bool NC = BL == B_NC;
  static constexpr int NCR = 512 / BN, NCH = BN / 8;
  static_assert(!NC || BN == 128 || BN == 256, "N-contiguous B tile width");
  static __device__ __forceinline__ int nc_krow(int wave, int lane, int j) { return (wave + NW * j) * NCR + lane / NCH; }
  static __device__ __forceinline__ int nc_chunk(int krow, int lane) {
    return (lane % NCH) ^ (M16 ? nc_x16(krow) : nc_x(krow & 3));
  }

  __amdgpu_buffer_rsrc_t ra, ra2, rb;  // ra2: second A plane (same offsets), AP == 2
  uint32_t a_voff[AJ], b_voff[BJ];      // bytes: row * row_stride + 16 * chunk
  uint32_t b_kstep;                     // NC: bytes of B between consecutive 64-row K stages
  uint32_t a_kstep;                     // A_MC: bytes of A between consecutive 64-row K stages
  // K tail (mainloop16<true>, K % 64 != 0): the last stage is read from K - 64 (a_klast,
  // b_klast: scalar byte offsets of A / K-contiguous B and of an N-contiguous B) instead
  // of 64 (nk - 1), so no load passes K; its first kdup = 64 nk - K columns, which the
  // stage before already covered, are zeroed in LDS in both operands before any read.
  uint32_t a_klast, b_klast;
  int kdup;

  // Zero K columns [0, kdup) of both operands of the stage at st (every thread takes part).
  __device__ __forceinline__ void zero_dup(uint16_t* st) const {
    static_assert(AP == 1 && !AMC, "K tails: one K-contiguous A plane");
    const int tid = threadIdx.x;
    for (int idx = tid; idx < BM * kdup; idx += NW * 64) {
      const int r = idx / kdup, k = idx - r * kdup;
      st[r * kBK + (((k >> 3) ^ row_key(r)) << 3) + (k & 7)] = 0;
    }
    if constexpr (NC) {
      for (int idx = tid; idx < kdup * BN; idx += NW * 64) st[B_OFF + idx] = 0;  // whole K-rows
    } else {
      for (int idx = tid; idx < BN * kdup; idx += NW * 64) {
        const int r = idx / kdup, k = idx - r * kdup;
        st[B_OFF + r * kBK + (((k >> 3) ^ row_key(r)) << 3) + (k & 7)] = 0;
      }
    }
  }

  __device__ __forceinline__ void issue_one(uint16_t* lds, int slot, uint32_t soff, uint32_t soffb, int wave,
                                            int q) {
    uint16_t* sA = lds + slot * STAGE;
    auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t so, uint16_t* dst) {
      if constexpr (NC) buf_lds16_asm(r, voff, so, dst);
      else buf_lds16(r, voff, so, dst);
    };
    if (q < AJ) {
      if constexpr (AMC) buf_lds16_asm(ra, a_voff[q], soff, sA + (wave + NW * q) * 8 * kBK);
      else ld(ra, a_voff[q], soff, sA + (wave + NW * q) * 8 * kBK);
    } else if (AP == 2 && q < 2 * AJ) {
      const int j = q - AJ;
      ld(ra2, a_voff[j], soff, sA + A_ELEMS + (wave + NW * j) * 8 * kBK);
    } else {
      const int j = q - AP * AJ;
      if constexpr (NC) buf_lds16_asm<BCPOL>(rb, b_voff[j], soffb, sA + B_OFF + (wave + NW * j) * 8 * kBK);
      else buf_lds16_cp<BCPOL>(rb, b_voff[j], soffb, sA + B_OFF + (wave + NW * j) * 8 * kBK);
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
    static_assert(!M16, "the 16x16 engine accumulates in f32x4_t[MI][NI][4] (mainloop16)");
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
    int offNC[NI];
    if constexpr (NC) nc_frag_offsets<BN, NI>(lane, rowB0, offNC);
    // Fragment f of a sub-step: f < AP*MI -> A plane f/MI block f%MI, else B block.
    auto read_one = [&](int slot, int ks, int f, u32x4_t (&af)[AP * MI], u32x4_t (&bf)[NI]) {
      if (f < AP * MI) {
        const int pl = f / MI, i = f % MI;
        af[f] = *(const u32x4_t*)(lds + slot * STAGE + pl * A_ELEMS + rowA0 * kBK + i * 32 * kBK + offA[i & 1][ks]);
      } else {
        const int j = f - AP * MI;
        if constexpr (NC) {
          const uint16_t* q = lds + slot * STAGE + B_OFF + offNC[j] + 16 * ks * BN;
          const u32x2_t lo = lds_read_tr16(q), hi = lds_read_tr16(q + 4 * BN);
          bf[j] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        } else {
          bf[j] = *(const u32x4_t*)(lds + slot * STAGE + B_OFF + rowB0 * kBK + j * 32 * kBK + offB[j & 1][ks]);
        }
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
    auto soffb_of = [&](int stage) { return NC ? (uint32_t)min(stage, nk - 1) * b_kstep : soff_of(stage); };
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 0, 0u, 0u, wave, q);
#pragma unroll
    for (int q = 0; q < HALF; ++q) issue_one(lds, 1, soff_of(1), soffb_of(1), wave, q);
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
      const uint32_t soffb1 = soffb_of(s + 1), soffb2 = soffb_of(s + 2);
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
            if (ks == 0) issue_one(lds, slot ^ 1, soff1, soffb1, wave, HALF + m);  // 2nd half of s+1
            else if (ks == 3) issue_one(lds, slot, soff2, soffb2, wave, m);       // 1st half of s+2
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vmcnt<0>();  // drain the clamped trailing loads before LDS is reused
    __syncthreads();
  }

  // The same pipeline on 16x16x32 MFMAs: per 64-wide stage two sub-steps of K = 32.
  // Lane l reads row 16 * s + (l % 16) of a 32-row block, 16-byte chunk 4 * ks + l / 16.
  // The accumulators stay 4-register tuples from the caller to the epilogue (c4[i][j][g]:
  // sub-tile g of 32x32 tile (i, j)); converting them to and from 16-register tiles made
  // the register allocator copy every chain between AGPRs and VGPRs once per stage.
  static __device__ __forceinline__ void zero16(f32x4_t (&c4)[MI][NI][4]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) c4[i][j][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // KT: K tail mode (K here is the padded length 64 nk; see a_klast / kdup).
  template <bool KT = false>
  __device__ __forceinline__ void mainloop16(uint16_t* lds, int K, f32x4_t (&c4)[MI][NI][4]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    // element offsets within a 32-row block, by block parity (swizzle), 16-row half and sub-step
    int offA[2][2][2], offB[2][2][2];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int ra = rowA0 + 32 * par + 16 * h + r16, rb = rowB0 + 32 * par + 16 * h + r16;
          offA[par][h][ks] = (16 * h + r16) * kBK + (((4 * ks + g4) ^ row_key(ra)) << 3);
          offB[par][h][ks] = (16 * h + r16) * kBK + (((4 * ks + g4) ^ row_key(rb)) << 3);
        }
    constexpr int NFA = AP * MI * 2, NFB = NI * 2;
    // N-contiguous B: fragment q = 2 j + h (columns rowB0 + 32 j + 16 h .. + 15) of lane
    // 16 g + c comes from two transpose reads; lane c points at K-row 8 g + c / 4 (+ 4 for
    // the second read, + 32 per sub-step), columns + 4 (c % 4) .. + 3, and lane c then
    // holds column + c at those four K-rows.  Element offsets of sub-step 0, first read.
    // M-contiguous A: the same transpose reads over A's K-rows, fragment f = 2 i + h at
    // rows rowA0 + 32 i + 16 h .. + 15
    int offMC[AMC ? NFA : 1];
    if constexpr (AMC) {
      const int c = lane & 15, g = lane >> 4;
      const int x = nc_x16(8 * g + (c >> 2));
#pragma unroll
      for (int f = 0; f < NFA; ++f) {
        const int ch = (rowA0 + 32 * (f / 2) + 16 * (f & 1)) / 8 + ((c & 3) >> 1);
        offMC[f] = (8 * g + (c >> 2)) * BM + ((ch ^ x) << 3) + 4 * (c & 1);
      }
    }
    int offNC[NC ? NFB : 1];
    if constexpr (NC) {
      const int c = lane & 15, g = lane >> 4;
      const int x = nc_x16(8 * g + (c >> 2));
#pragma unroll
      for (int q = 0; q < NFB; ++q) {
        const int ch = (rowB0 + 32 * (q / 2) + 16 * (q & 1)) / 8 + ((c & 3) >> 1);
        offNC[q] = (8 * g + (c >> 2)) * BN + ((ch ^ x) << 3) + 4 * (c & 1);
      }
    }
    // fragment f of a sub-step: f < NFA -> A plane, block, half; else B block, half
    auto read_one = [&](int slot, int ks, int f, u32x4_t (&af)[NFA], u32x4_t (&bf)[NFB]) {
      if (f < NFA) {
        const int pl = f / (MI * 2), i = (f / 2) % MI, h = f & 1;
        if constexpr (AMC) {
          const uint16_t* src = lds + slot * STAGE + offMC[f] + 32 * ks * BM;
          const u32x2_t lo = lds_read_tr16(src), hi = lds_read_tr16(src + 4 * BM);
          af[f] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        } else {
          af[f] = *(const u32x4_t*)(lds + slot * STAGE + pl * A_ELEMS + (rowA0 + 32 * i) * kBK + offA[i & 1][h][ks]);
        }
      } else {
        const int q = f - NFA, j = q / 2, h = q & 1;
        if constexpr (NC) {
          const uint16_t* src = lds + slot * STAGE + B_OFF + offNC[q] + 32 * ks * BN;
          const u32x2_t lo = lds_read_tr16(src), hi = lds_read_tr16(src + 4 * BN);
          bf[q] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        } else {
          bf[q] = *(const u32x4_t*)(lds + slot * STAGE + B_OFF + (rowB0 + 32 * j) * kBK + offB[j & 1][h][ks]);
        }
      }
    };
    const int nk = K / kBK;
    if (nk == 0) return;
    constexpr int NMMA = AP * MI * NI * 4;  // MFMAs per sub-step
    constexpr int NRD = NFA + NFB;          // fragment reads per sub-step
    static_assert(NRD <= NMMA && LPS <= NMMA && LPS <= 32, "interleave needs enough MFMAs; vmcnt range");
    const uint32_t kmax = (uint32_t)(nk - 1) * (kBK * 2);
    auto soff_of = [&](int stage) -> uint32_t {
      if constexpr (KT) return stage >= nk - 1 ? a_klast : (uint32_t)stage * (kBK * 2);
      else return min((uint32_t)stage * (kBK * 2), kmax);
    };
    auto soffb_of = [&](int stage) -> uint32_t {
      if constexpr (KT && NC) return stage >= nk - 1 ? b_klast : (uint32_t)stage * b_kstep;
      else return NC ? (uint32_t)min(stage, nk - 1) * b_kstep : soff_of(stage);
    };
    auto soffa_of = [&](int stage) { return AMC ? (uint32_t)min(stage, nk - 1) * a_kstep : soff_of(stage); };
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 0, soffa_of(0), soffb_of(0), wave, q);
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 1, soffa_of(1), soffb_of(1), wave, q);
    wait_vmcnt<LPS>();
    exec_barrier();
    if constexpr (KT) {
      if (nk == 1) {  // the only stage is the last one
        zero_dup(lds);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        exec_barrier();
      }
    }
    // 8 waves: A fragments are single-buffered: A block (pl, i, half sm) of the next
    // sub-step is read right after its last MFMA in this one (tile j = NI - 1, sub-tile
    // g = 2 sm + 1), at least (MI - 1) * NI * 4 MFMAs before its first use; B fragments
    // are double-buffered and read over the first MFMAs.  This keeps 32 VGPRs free, which
    // the register allocator otherwise finds by moving accumulators through AGPR copies.
    // 4 waves (FA2, one wave per SIMD, K-contiguous operands): the accumulators (up to the
    // 256 AGPRs of a 128 x 128 wave tile) stay in place (mma16_acc), so A is double-
    // buffered too and every read of the next sub-step goes out over its first MFMAs.
    constexpr bool FA2 = NW == 4 && !NC && !AMC;
    u32x4_t fa[FA2 ? 2 : 1][NFA], fb[2][NFB], fa_unused[NFA];
#pragma unroll
    for (int f = 0; f < NRD; ++f) read_one(0, 0, f, fa[0], fb[0]);
    // sub-step ks of stage s: its MFMAs, the next sub-step's fragment reads and (ks == 1)
    // the direct loads of stage s + 2
    // (first: the very first sub-step, whose MFMAs start the accumulators)
    auto substep = [&](int s, auto ksc, auto firstc) {
      constexpr int ks = decltype(ksc)::value, c = ks;
      constexpr bool first = decltype(firstc)::value;
      const int slot = s & 1;
      const uint32_t soff2 = soffa_of(s + 2), soffb2 = soffb_of(s + 2);
      const int rslot = ks == 0 ? slot : (slot ^ 1);
      const int rks = ks == 0 ? 1 : 0;
#pragma unroll
      for (int m = 0; m < NMMA; ++m) {
        __builtin_amdgcn_sched_barrier(0);
        const int pl = m / (MI * NI * 4), i = (m / (NI * 4)) % MI, j = (m / 4) % NI, g = m & 3;
        const int sm = g >> 1, sn = g & 1;
        if constexpr (FA2) {
          if (first && pl == 0) mma16_acc0<T>(c4[i][j][g], fb[c][j * 2 + sn], fa[c][(pl * MI + i) * 2 + sm]);
          else mma16_acc<T>(c4[i][j][g], fb[c][j * 2 + sn], fa[c][(pl * MI + i) * 2 + sm]);
          if (m < NRD) read_one(rslot, rks, m, fa[c ^ 1], fb[c ^ 1]);
        } else {
          c4[i][j][g] = Op::mma16(fb[c][j * 2 + sn], fa[0][(pl * MI + i) * 2 + sm], c4[i][j][g]);
          if (j == NI - 1 && (g & 1)) read_one(rslot, rks, (pl * MI + i) * 2 + sm, fa[0], fb[c ^ 1]);
          if (m < NFB) read_one(rslot, rks, NFA + m, fa_unused, fb[c ^ 1]);
        }
        // every load of stage s+2 goes out in sub-step 1, right after the barrier that frees
        // its slot, spread over the MFMAs: a full stage of lead before the vmcnt(0) wait of
        // stage s+1.  Issuing half of them in the next stage's sub-step 0 instead (half a
        // stage of lead) measured slower in the same process, bit-equal outputs: 4096^3 bf16
        // 100.3 against 103.2 us, 8192x4096x4096 195.6 against 204.0 us.
        constexpr int EV = NMMA / LPS > 0 ? NMMA / LPS : 1;
        if (ks == 1 && m % EV == 0 && m / EV < LPS) issue_one(lds, slot, soff2, soffb2, wave, m / EV);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // every wave has read stage s's slot (through sub-step 0) and landed stage s + 1
    auto sync = [&](int s) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      wait_vmcnt<0>();
      exec_barrier();
      if constexpr (KT) {
        if (s == nk - 2) {  // stage s + 1 is the last: zero its repeated columns first
          zero_dup(lds + ((s & 1) ^ 1) * STAGE);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          exec_barrier();
        }
      }
    };
    // The loop runs from barrier to barrier (sub-step 1 of stage s, then sub-step 0 of
    // stage s + 1), so its head follows an lgkmcnt(0) wait.  With the head at sub-step 0
    // the compiler's wait-count analysis merged the loop's two entries into an
    // lgkmcnt(1) wait before the first MFMA of every stage, a full LDS latency with
    // one wave per SIMD (same process, bit-equal, 4096^3 bf16 on 4 waves: 93.6 -> 92.7 us).
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    using F0 = std::integral_constant<bool, false>;
    substep(0, K0(), std::integral_constant<bool, FA2>());
    for (int s = 0; s < nk - 1; ++s) {
      sync(s);
      substep(s, K1(), F0());
      substep(s + 1, K0(), F0());
    }
    sync(nk - 1);
    substep(nk - 1, K1(), F0());
    if constexpr (FA2) mma16_acc_fence();
    wait_vmcnt<0>();  // drain the clamped trailing loads before LDS is reused
    __syncthreads();
  }
  // fp8 (e4m3) operands on the same byte layout (4 waves, K-contiguous A and B): one
  // 16x16x128 MFMA per 16x16 sub-tile and 128-byte stage.  Lane l of a fragment holds the
  // two 16-byte chunks the 16x16x32 engine reads in its two sub-steps (K bytes 16 (l / 16)
  // + [0, 16) and 64 + 16 (l / 16) + [0, 16)); A and B take the same K permutation, so each
  // MFMA still sums all 128 products of a stage.  One barrier per stage, early in it (stage
  // s + 1 landed, every wave done reading stage s), then the direct loads of stage s + 2 into
  // the slot stage s leaves; each fragment of the next stage is read right after its last
  // use in this one (A blocks after their row of tiles, B blocks in the last row; 32-byte
  // fragments of two stages do not fit the registers).  K in 16-bit units (64 per stage).
  __device__ __forceinline__ void mainloop_f8(uint16_t* lds, int K, f32x4_t (&c4)[MI][NI][4]) {
    static_assert(NW == 4 && !NC && !AMC && AP == 1 && M16, "fp8 main loop: 4 waves, K-contiguous operands");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    int offA[2][2][2], offB[2][2][2];
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int ra = rowA0 + 32 * par + 16 * h + r16, rb = rowB0 + 32 * par + 16 * h + r16;
          offA[par][h][ks] = (16 * h + r16) * kBK + (((4 * ks + g4) ^ row_key(ra)) << 3);
          offB[par][h][ks] = (16 * h + r16) * kBK + (((4 * ks + g4) ^ row_key(rb)) << 3);
        }
    constexpr int NFA = MI * 2, NFB = NI * 2;
    auto read_f = [&](int slot, int f, i32x8_t& dst) {
      const uint16_t* base;
      const int* o;
      if (f < NFA) {
        const int i = f / 2, h = f & 1;
        base = lds + slot * STAGE + (rowA0 + 32 * i) * kBK;
        o = offA[i & 1][h];
      } else {
        const int j = (f - NFA) / 2, h = (f - NFA) & 1;
        base = lds + slot * STAGE + B_OFF + (rowB0 + 32 * j) * kBK;
        o = offB[j & 1][h];
      }
      const u32x4_t lo = *(const u32x4_t*)(base + o[0]), hi = *(const u32x4_t*)(base + o[1]);
      dst = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    };
    const int nk = K / kBK;
    if (nk == 0) return;
    constexpr int NMMA = MI * NI * 4;
    static_assert(NFB <= NMMA && LPS <= NMMA && LPS <= 32, "interleave needs enough MFMAs; vmcnt range");
    const uint32_t kmax = (uint32_t)(nk - 1) * (kBK * 2);
    auto soff_of = [&](int stage) { return min((uint32_t)stage * (kBK * 2), kmax); };
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 0, 0u, 0u, wave, q);
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue_one(lds, 1, soff_of(1), soff_of(1), wave, q);
    wait_vmcnt<LPS>();
    exec_barrier();
    i32x8_t fa[NFA], fb[NFB];
#pragma unroll
    for (int f = 0; f < NFA; ++f) read_f(0, f, fa[f]);
#pragma unroll
    for (int f = 0; f < NFB; ++f) read_f(0, NFA + f, fb[f]);
    // stage s: its MFMAs, the reads of stage s + 1 and the direct loads of stage s + 2 (into
    // the slot stage s leaves).  The barrier comes after BARM MFMAs, which hide the
    // lgkmcnt(0) wait for the last fragment reads of the stage before, and before the first
    // read of stage s + 1 (MFMA NI * 4 - 3).  The loads follow every EV MFMAs, so the last
    // leaves NMMA - BARM - (LPS - 1) EV MFMAs of lead before the next barrier.  A barrier at
    // the stage's start with the loads spread over all of it measured slower (same process,
    // bit-equal: 4096^3 58.7 against 54.9 us); EV = 1 too (57.5 us).
    constexpr int BARM = 4, EV = 2;
    static_assert(BARM < NI * 4 - 3 && BARM + (LPS - 1) * EV < NMMA, "barrier before the first read");
    auto phase = [&](int s, auto firstc) {
      constexpr bool first = decltype(firstc)::value;
      const int slot = s & 1, nslot = slot ^ 1;
      const uint32_t soff2 = soff_of(s + 2);
#pragma unroll
      for (int m = 0; m < NMMA; ++m) {
        __builtin_amdgcn_sched_barrier(0);
        if (m == BARM) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          wait_vmcnt<0>();
          exec_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
        const int i = m / (NI * 4), j = (m / 4) % NI, g = m & 3;
        const int sm = g >> 1, sn = g & 1;
        if constexpr (first) mma16_f8_acc0(c4[i][j][g], fb[j * 2 + sn], fa[i * 2 + sm]);
        else mma16_f8_acc(c4[i][j][g], fb[j * 2 + sn], fa[i * 2 + sm]);
        if (j == NI - 1 && (g & 1)) read_f(nslot, i * 2 + sm, fa[i * 2 + sm]);
        if (i == MI - 1 && g >= 2) read_f(nslot, NFA + j * 2 + sn, fb[j * 2 + sn]);
        if (m >= BARM && (m - BARM) % EV == 0 && (m - BARM) / EV < LPS)
          issue_one(lds, slot, soff2, soff2, wave, (m - BARM) / EV);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    phase(0, std::integral_constant<bool, true>());
    for (int s = 1; s < nk; ++s) phase(s, std::integral_constant<bool, false>());
    mma16_acc_fence();
    wait_vmcnt<0>();  // drain the clamped trailing loads before LDS is reused
    __syncthreads();
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Skinny ring engine (weight streaming, M = 32, 64 or 128 rows).
//
// For grouped GEMMs with few rows per expert (MoE decode) the time is the weight
// stream, so what matters is how many bytes each CU keeps in flight.  Four waves sit
// side by side over N (wave tile BM x BN/4); an NSLOT-deep ring of 64-wide K stages
// is filled by direct-to-LDS buffer loads (one wave instruction = 8 whole 128-byte
// rows), NSLOT-1 stages ahead of the MFMAs.  Per K step: wait for the own loads of
// the stage, one barrier (every wave's loads landed and every wave finished the
// previous stage, whose slot is refilled next), issue the stage NSLOT-1 ahead, then
// 4 sub-steps of MFMAs.  Past the last stage the K offset is clamped (the last
// stage is re-loaded into a free slot), so every wave issues the same loads and the
// vmcnt arithmetic is uniform.  AP == 2 multiplies two A planes by the same B
// fragments (the bf16 high/low split of an fp32 activation).  BCPOL is the cache
// policy of the B loads (kCpolNT for weights that no other workgroup reads).
// ---------------------------------------------------------------------------------
template <typename T, int BN, int AP, int NSLOT, int BM_ = 32, int BCPOL = kCpolDefault>
struct SkinnyRingEngine {
  static constexpr int NW = 4, BM = BM_, MI = BM / 32;
  static_assert(BM == 32 || BM == 64 || BM == 128, "32, 64 or 128 rows");
  static constexpr int WCOLS = BN / NW, NI = WCOLS / 32;
  static_assert(WCOLS % 32 == 0 && NI >= 1, "wave tile is BM x (multiple of 32)");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int B_OFF = AP * A_ELEMS;
  static constexpr int STAGE = AP * A_ELEMS + B_ELEMS;
  static constexpr int LDS_ELEMS = NSLOT * STAGE;
  static constexpr int AJ = BM / 32;      // 8-row A loads per wave per plane
  static constexpr int BJ = BN / 8 / NW;  // 8-row B loads per wave per stage
  static_assert(BJ * 8 * NW == BN, "8-row wave loads must cover the B tile");
  static constexpr int LPS = AP * AJ + BJ;
  static_assert(NSLOT >= 2 && (NSLOT - 2) * LPS <= 63, "vmcnt range");

  static __device__ __forceinline__ int a_row(int wave, int lane, int j = 0) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ swz8(row); }

  __amdgpu_buffer_rsrc_t ra, ra2, rb;
  uint32_t a_voff[AJ], b_voff[BJ];

  __device__ __forceinline__ void issue(uint16_t* lds, int slot, uint32_t soff, int wave) const {
    uint16_t* st = lds + slot * STAGE;
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      buf_lds16(ra, a_voff[j], soff, st + (wave + NW * j) * 8 * kBK);
      if constexpr (AP == 2) buf_lds16(ra2, a_voff[j], soff, st + A_ELEMS + (wave + NW * j) * 8 * kBK);
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) buf_lds16_cp<BCPOL>(rb, b_voff[j], soff, st + B_OFF + (wave + NW * j) * 8 * kBK);
  }

  static __device__ __forceinline__ void zero(f32x16_t (&acc)[MI][NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  // Multiply K elements [k_begin, k_end) (multiples of 64; k_end > k_begin).
  __device__ __forceinline__ void mainloop(uint16_t* lds, int k_begin, int k_end, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31, hh = lane >> 5;
    // fragment row R + lr (R % 32 == 0): swz8(R + lr) = (lr & 7) ^ (lr >> 3) ^ (4 * ((R / 32) & 1))
    int offA[2][4], offB[2][4];
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int swa = ((lr & 7) ^ (lr >> 3) ^ (4 * par)) & 7;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        offA[par][ks] = lr * kBK + (((2 * ks + hh) ^ swa) << 3);
        const int qb = (wave * NI + par) & 1;
        offB[par][ks] = lr * kBK + (((2 * ks + hh) ^ ((((lr & 7) ^ (lr >> 3)) & 7) ^ (4 * qb))) << 3);
      }
    }
    const int nk = (k_end - k_begin) / kBK;
    const uint32_t s0 = (uint32_t)k_begin * 2u, smax = (uint32_t)(k_end - kBK) * 2u;
    auto soff_of = [&](int stage) { return min(s0 + (uint32_t)stage * (kBK * 2), smax); };
#pragma unroll
    for (int s = 0; s < NSLOT - 1; ++s) issue(lds, s, soff_of(s), wave);
    int slot = 0;
    for (int s = 0; s < nk; ++s) {
      wait_vmcnt<(NSLOT - 2) * LPS>();
      exec_barrier();
      const int nslot = slot == 0 ? NSLOT - 1 : slot - 1;  // slot of stage s - 1
      issue(lds, nslot, soff_of(s + NSLOT - 1), wave);
      const uint16_t* sA = lds + slot * STAGE;
      const uint16_t* sB = sA + B_OFF + wave * WCOLS * kBK;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4_t af[AP][MI], bf[NI];
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
          for (int i = 0; i < MI; ++i) af[pl][i] = *(const u32x4_t*)(sA + pl * A_ELEMS + i * 32 * kBK + offA[i & 1][ks]);
#pragma unroll
        for (int j = 0; j < NI; ++j) bf[j] = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][ks]);
#pragma unroll
        for (int pl = 0; pl < AP; ++pl)
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[i][j] = Op::mma32(bf[j], af[pl][i], acc[i][j]);
      }
      slot = slot + 1 == NSLOT ? 0 : slot + 1;
    }
    wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
    __syncthreads();
  }
};

}  // namespace kore

namespace kore {

// ---------------------------------------------------------------------------------
// Deep ring engine (mid-size GEMMs: a few hundred tiles and a long K).
//
// A mid-size tile streams 1-2 MiB of operands through its CU; with two 64-wide K
// stages in flight the CU waits most of a memory round trip per stage.  Here an
// NSLOT-deep ring of stages is filled by direct-to-LDS buffer loads NSLOT - 1 stages
// ahead of the MFMAs (~100 KiB in flight per CU).  Four waves in a WM x WN grid.
// Per K step: wait for the own loads of the stage, one barrier (all loads of the
// stage landed, every wave finished the previous stage, whose slot is refilled
// next), issue the stage NSLOT - 1 ahead, then 4 sub-steps of MFMAs.  Past the last
// stage the K offset is clamped (the last stage is re-loaded into a slot nobody
// reads), so every wave issues the same loads and the vmcnt arithmetic is uniform.
// A and K-contiguous B use 128-byte rows with the swz8 chunk swizzle; N-contiguous B
// uses the nc_x layout and LDS transpose reads (loads then go out as inline asm).
// BCPOL is the cache policy of the B loads: non-temporal where every B element is read
// by one workgroup only (the split-K decode GEMM streams its weights once).
// ---------------------------------------------------------------------------------
template <typename T, int BM, int BN, int WM, int WN, int NSLOT, int BL, int BCPOL = kCpolDefault>
struct RingEngine {
  static constexpr bool AMC = false;  // A is K-contiguous
  static constexpr int NW = 4;
  static_assert(WM * WN == NW, "4 waves");
  static constexpr int WROWS = BM / WM, WCOLS = BN / WN;
  static constexpr int MI = WROWS / 32, NI = WCOLS / 32;
  static_assert(WROWS % 32 == 0 && WCOLS % 32 == 0 && MI >= 1 && NI >= 1, "wave tile");
  static constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;
  static constexpr int B_OFF = A_ELEMS, STAGE = A_ELEMS + B_ELEMS, LDS_ELEMS = NSLOT * STAGE;
  static constexpr int AJ = BM / 32, BJ = BN / 32;  // 512-element loads per wave per stage
  static_assert(AJ * 32 == BM && BJ * 32 == BN, "wave loads must cover the tile");
  static constexpr int LPS = AJ + BJ;
  static_assert(NSLOT >= 2 && (NSLOT - 2) * LPS <= 63, "vmcnt range");
  static constexpr bool NC = BL == B_NC;
  static constexpr int NCR = 512 / BN, NCH = BN / 8;
  static_assert(!NC || BN == 128 || BN == 256, "N-contiguous B tile width");

  static __device__ __forceinline__ int a_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int b_row(int wave, int lane, int j) { return (wave + NW * j) * 8 + (lane >> 3); }
  static __device__ __forceinline__ int chunk(int row, int lane) { return (lane & 7) ^ swz8(row); }
  static __device__ __forceinline__ int nc_krow(int wave, int lane, int j) { return (wave + NW * j) * NCR + lane / NCH; }
  static __device__ __forceinline__ int nc_chunk(int krow, int lane) { return (lane % NCH) ^ nc_x(krow & 3); }

  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t a_voff[AJ], b_voff[BJ];
  uint32_t b_kstep;  // NC: bytes of B between consecutive 64-row K stages
  // K tail (mainloop<true>, K % 64 != 0): the last stage is read from K - 64 (scalar byte
  // offsets a_klast, b_klast) and its first kdup columns, which the stage before already
  // covered, are zeroed in LDS in both operands once it has landed.
  uint32_t a_klast, b_klast;
  int kdup;

  // Zero K columns [0, kdup) of both operands of the stage at st (every thread takes part).
  __device__ __forceinline__ void zero_dup(uint16_t* st) const {
    const int tid = threadIdx.x;
    for (int idx = tid; idx < BM * kdup; idx += NW * 64) {
      const int r = idx / kdup, k = idx - r * kdup;
      st[r * kBK + (((k >> 3) ^ swz8(r)) << 3) + (k & 7)] = 0;
    }
    if constexpr (NC) {
      for (int idx = tid; idx < kdup * BN; idx += NW * 64) st[B_OFF + idx] = 0;  // whole K-rows
    } else {
      for (int idx = tid; idx < BN * kdup; idx += NW * 64) {
        const int r = idx / kdup, k = idx - r * kdup;
        st[B_OFF + r * kBK + (((k >> 3) ^ swz8(r)) << 3) + (k & 7)] = 0;
      }
    }
  }

  __device__ __forceinline__ void issue(uint16_t* lds, int slot, uint32_t soff, uint32_t soffb, int wave) const {
    uint16_t* st = lds + slot * STAGE;
    auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t so, uint16_t* dst, auto cpol_tag) {
      constexpr int CP = decltype(cpol_tag)::value;
      if constexpr (NC) buf_lds16_asm<CP>(r, voff, so, dst);
      else buf_lds16_cp<CP>(r, voff, so, dst);
    };
#pragma unroll
    for (int j = 0; j < AJ; ++j)
      ld(ra, a_voff[j], soff, st + (wave + NW * j) * 8 * kBK, std::integral_constant<int, kCpolDefault>{});
#pragma unroll
    for (int j = 0; j < BJ; ++j)
      ld(rb, b_voff[j], soffb, st + B_OFF + (wave + NW * j) * 8 * kBK, std::integral_constant<int, BCPOL>{});
  }

  static __device__ __forceinline__ void zero(f32x16_t (&acc)[MI][NI]) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  }

  // K must be a positive multiple of 64 (KT: the padded length, see a_klast / kdup).
  template <bool KT = false>
  __device__ __forceinline__ void mainloop(uint16_t* lds, int K, f32x16_t (&acc)[MI][NI]) {
    mainloop_range<KT>(lds, 0, K, acc);
  }

  // Multiply K elements [k_begin, k_end) (multiples of 64, k_end > k_begin; KT: the whole K,
  // k_begin == 0).
  template <bool KT = false>
  __device__ __forceinline__ void mainloop_range(uint16_t* lds, int k_begin, int k_end, f32x16_t (&acc)[MI][NI]) {
    using Op = MfmaOp<T>;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, hh = lane >> 5;
    const int rowA0 = wm * WROWS, rowB0 = wn * WCOLS;
    // fragment row R + lr (R % 32 == 0): swz8(R + lr) = (lr & 7) ^ (lr >> 3) ^ (4 * ((R / 32) & 1))
    int offA[2][4], offB[2][4], offNC[NI];
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
    if constexpr (NC) nc_frag_offsets<BN, NI>(lane, rowB0, offNC);
    const int nk = (k_end - k_begin) / kBK, kb0 = k_begin / kBK;
    auto soff_of = [&](int stage) -> uint32_t {
      if (KT && stage >= nk - 1) return a_klast;
      return (uint32_t)(kb0 + min(stage, nk - 1)) * (kBK * 2);
    };
    auto soffb_of = [&](int stage) -> uint32_t {
      if (KT && NC && stage >= nk - 1) return b_klast;
      return NC ? (uint32_t)(kb0 + min(stage, nk - 1)) * b_kstep : soff_of(stage);
    };
#pragma unroll
    for (int s = 0; s < NSLOT - 1; ++s) issue(lds, s, soff_of(s), soffb_of(s), wave);
    int slot = 0;
    for (int s = 0; s < nk; ++s) {
      wait_vmcnt<(NSLOT - 2) * LPS>();
      exec_barrier();
      if constexpr (KT) {
        if (s == nk - 1) {  // the last stage has landed: zero its repeated columns before any read
          zero_dup(lds + slot * STAGE);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          exec_barrier();
        }
      }
      const int nslot = slot == 0 ? NSLOT - 1 : slot - 1;  // slot of stage s - 1
      issue(lds, nslot, soff_of(s + NSLOT - 1), soffb_of(s + NSLOT - 1), wave);
      const uint16_t* sA = lds + slot * STAGE + rowA0 * kBK;
      const uint16_t* sB = lds + slot * STAGE + B_OFF;
      auto read = [&](int ks, u32x4_t (&af)[MI], u32x4_t (&bf)[NI]) {
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][ks]);
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          if constexpr (NC) {
            const uint16_t* q = sB + offNC[j] + 16 * ks * BN;
            const u32x2_t lo = lds_read_tr16(q), hi = lds_read_tr16(q + 4 * BN);
            bf[j] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
          } else {
            bf[j] = *(const u32x4_t*)(sB + rowB0 * kBK + j * 32 * kBK + offB[j & 1][ks]);
          }
        }
      };
      // sub-step ks + 1's fragments are read before sub-step ks's MFMAs go out, so LDS
      // latency hides under them (one wave per SIMD has nothing else to switch to)
      u32x4_t fa[2][MI], fb[2][NI];
      read(0, fa[0], fb[0]);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) read(ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = Op::mma32(fb[ks & 1][j], fa[ks & 1][i], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
      }
      slot = slot + 1 == NSLOT ? 0 : slot + 1;
    }
    wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
    __syncthreads();
  }
};

}  // namespace kore
