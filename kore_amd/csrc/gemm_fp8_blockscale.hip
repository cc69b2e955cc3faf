// fp8 (OCP e4m3) a8w8 block-scaled GEMM for gfx950.
//
// Y[M,N] (bf16) = sum_kb  xs[m,kb] * ws[n/128,kb] * sum_{k in block kb} xq[m,k]*wq[n,k]
// with 1x128 activation scales and 128x128 weight scales (DeepSeek-V3 layout).
//
// A workgroup (4 waves, 2x2) computes a 256x128 tile with v_mfma_f32_32x32x64_f8f6f4.
// One K step is exactly one 128-wide scale block: the two MFMAs of a block accumulate
// into a zeroed partial, which is then promoted into the fp32 accumulator with one
// FMA by the combined scale xs[m,kb]*ws[nb,kb] -- every scale applied exactly once,
// as in the reference oracle.  Operands are staged through LDS with the same
// 128-byte-row XOR swizzle and double buffering as the 16-bit kernels (a 128-byte
// row is 128 fp8 values here).  The B fragment is the first MFMA operand, so each
// lane owns one output row m: its activation scale is a per-lane value and the
// weight scale is uniform per 32-column block.
#include "../../include/kore_amd.h"
#include "kore_common.hpp"
#include "tile_engine.hpp"

#include <type_traits>

namespace kore {
namespace {

struct Fp8Params {
  const uint8_t* xq;
  const uint8_t* wq;
  const float* xs;
  const float* ws;
  uint16_t* y;
  int M, N, K;
  int64_t ldx, ldw, ldy;
  int64_t xs_m, xs_k, ws_n, ws_k;
  int tiles_m, tiles_n;
  int vec_store;
  // grouped (top-1 expert) mode: tile m-block b holds the rows sorted[b*BM ..] of
  // expert block_expert[b] (-1: unused block); a sorted entry >= M is a padding row
  const int32_t* sorted;
  const int32_t* block_expert;
  int64_t w_estride, ws_estride;
};

constexpr int kFp8GroupM = 4;

template <int BM, int BN>
__global__ void __launch_bounds__(kEngineThreads)
    gemm_fp8_bs_kernel(const Fp8Params p) {
  // Byte rows are staged as 64 x 16-bit units: the engine's loader/stager is reused.
  using E = TileEngine<BF16, BM, BN, 2, 2, B_KC>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, hh = lane >> 5;

  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int width = kFp8GroupM * p.tiles_n;
  const int grp = bid / width;
  const int first_m = grp * kFp8GroupM;
  const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
  const int tl = bid - grp * width;
  const int m0 = (first_m + tl % gsz) * BM;
  const int n0 = (tl / gsz) * BN;
  const int M = p.M, N = p.N, K = p.K;

  E eng;
  const int ch16 = (tid & 7) * 16;  // byte offset of this thread's chunk
#pragma unroll
  for (int j = 0; j < E::LA; ++j)
    eng.a_src[j] = (const uint16_t*)(p.xq + (int64_t)min(m0 + E::a_row_of(tid, j), M - 1) * p.ldx + ch16);
#pragma unroll
  for (int j = 0; j < E::LB; ++j)
    eng.b_src[j] = (const uint16_t*)(p.wq + (int64_t)min(n0 + E::b_row_of(tid, j), N - 1) * p.ldw + ch16);
  eng.ldb = 0;

  // Fragment offsets (16-bit units): row R + lr, chunks c and c+1 with c = 4*kk + 2*hh.
  int offA[2][2][2], offB[2][2][2];  // [parity][kk][half]
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int qa = (wm * MI + par) & 1, qb = (wn * NI + par) & 1;
    const int swa = ((lr & 7) ^ (lr >> 3) ^ (4 * qa)) & 7;
    const int swb = ((lr & 7) ^ (lr >> 3) ^ (4 * qb)) & 7;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = 4 * kk + 2 * hh + h;
        offA[par][kk][h] = lr * kBK + ((c ^ swa) << 3);
        offB[par][kk][h] = lr * kBK + ((c ^ swb) << 3);
      }
  }
  const int rowA0 = wm * E::WROWS, rowB0 = wn * E::WCOLS;

  // Per-lane activation-scale rows and per-block weight-scale rows.
  const float* xs_row[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) xs_row[i] = p.xs + (int64_t)min(m0 + rowA0 + i * 32 + lr, M - 1) * p.xs_m;
  const float* ws_row[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) ws_row[j] = p.ws + (int64_t)((n0 + rowB0 + j * 32) / 128) * p.ws_n;

  f32x16_t acc[MI][NI];
  E::zero(acc);

  const int K16 = K / 2;  // K in 16-bit units (128 fp8 = 64 units per step)
  const int nk = K / 128;
  eng.load(0, K16, tid);
  eng.store(lds, 0, tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) eng.load((kt + 1) * kBK, K16, tid);
    float xsv[MI], wsv[NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) xsv[i] = xs_row[i][(int64_t)kt * p.xs_k];
#pragma unroll
    for (int j = 0; j < NI; ++j) wsv[j] = ws_row[j][(int64_t)kt * p.ws_k];

    const uint16_t* sA = lds + cur * E::STAGE + rowA0 * kBK;
    const uint16_t* sB = lds + cur * E::STAGE + E::B_OFF + rowB0 * kBK;
    i32x8_t af[2][MI], bfr[2][NI];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const u32x4_t lo = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][kk][0]);
        const u32x4_t hi = *(const u32x4_t*)(sA + i * 32 * kBK + offA[i & 1][kk][1]);
        af[kk][i] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const u32x4_t lo = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][kk][0]);
        const u32x4_t hi = *(const u32x4_t*)(sB + j * 32 * kBK + offB[j & 1][kk][1]);
        bfr[kk][j] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      }
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        f32x16_t t = {};
        t = mma32_fp8(bfr[0][j], af[0][i], t);
        t = mma32_fp8(bfr[1][j], af[1][i], t);
        const float s = xsv[i] * wsv[j];
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(t[r], s, acc[i][j][r]);
      }
    }
    if (kt + 1 < nk) eng.store(lds, cur ^ 1, tid);
    __syncthreads();
  }

  // ---- epilogue: bf16 pack, stage per wave, 16-byte row stores ----
  using St = Stager<E::WROWS, E::WCOLS>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = lds + wave * (E::WROWS * E::WCOLS);
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        St::put(stg, out_row(i, lane), out_col(j, g, lane),
                u32x2_t{Op::pack2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                        Op::pack2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3])});
  __syncthreads();
  const int mw0 = m0 + rowA0, nw0 = n0 + rowB0;
  const bool vec = p.vec_store != 0;
  St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
    const int gm = mw0 + row, gn = nw0 + col;
    if (gm < M) store_row8(p.y + (int64_t)gm * p.ldy + gn, gn, N, vec, v);
  });
}


// ------------------------------------------------------------------------------
// Pipelined kernel: direct-to-LDS buffer loads into a ring of LDS slots.
//
// Per slot (one K step = one 128-wide scale block): A 256 rows x 128 B, B BN rows x
// 128 B, and the scales of the step -- scales travel through the same DMA pipeline
// as the operands, so their waits are the operands' waits.  Activation scales: 256
// fp32 per step, or, when the scale rows are contiguous in K (XS4), one 16-byte load
// per row bringing four K steps into a two-deep ring (the per-step column of xs is
// 256 strided 4-byte reads, each its own L2 request).  Weight scales: 64 copies per
// 128-column block (16-byte copies of an aligned group of four steps for XS4).  Every
// wave issues the same number of loads per stage; which scale a wave loads is chosen
// with scalar selects, not branches: a branch would split the tile loop into blocks
// and let the compiler sink the promotion FMAs away from the MFMAs they overlap.
//
// The 16-byte chunks of a 128-byte row are XOR-swizzled with key(r) = (r ^ (r >> 3)) & 7,
// r = row % 32: a fragment read (lane l: row l % 32) then hits 8 distinct 16-byte bank
// groups in every 8-lane pass over 32 banks and 16 distinct ones in every 16-lane pass
// over 64 banks, and the key does not depend on which 32-row block a fragment is in.
// (The earlier key ((r >> 1) & 7) ^ ((r >> 4) & 1) gave rows 2j and 2j+1 the same chunk,
// a 2-way conflict per 8-lane pass that SQ_LDS_BANK_CONFLICT measured at 30% of the
// LDS-active cycles.)  Weight scales are read from one address (an LDS broadcast).
//
// NW waves in a WGM x WGN grid, each owning (256/WGM) x 64 outputs as MI x 2 tiles of
// 32x32.  A tile's two MFMAs (K 0..63, 64..127) accumulate into one of two rotating
// partials; the promotion acc += partial * (xs * ws) of tile t-1 is issued between
// the two MFMAs of tile t.  With 8 waves two share a SIMD, so one wave's promotion
// FMAs run while the other's MFMAs occupy the matrix core (a wave's own VALU work
// does not overlap its own MFMAs).
//
// Slot lifecycle (stage s in slot s % NSLOT): the barrier at tile TB (first tile of
// the last block row) guarantees every wave has finished reading slot s % NSLOT and
// stage s+1 has landed.  The loads of stage s + NSLOT then go into that slot, spread
// over the next W tiles (W = NT with three slots: one to two stages of latency; the
// remaining tiles of the stage with two slots: one stage).
// ------------------------------------------------------------------------------
// Scale modes of the 8-bit kernels: DeepSeek block scales promoted once per 128-wide
// K block (fp8), or one activation scale per row and one weight scale per column,
// applied once to the finished accumulator in the epilogue (fp8 or int8 operands).
enum { Q_BLOCK_FP8 = 0, Q_ROW_FP8 = 1, Q_ROW_I8 = 2 };

template <int BM_, int BN_, int NW_, int NSLOT_, bool XS4_, int MODE_ = Q_BLOCK_FP8>
struct F8Cfg {
  static constexpr int BM = BM_, BN = BN_, NW = NW_, NSLOT = NSLOT_, MODE = MODE_;
  static constexpr bool ROW = MODE != Q_BLOCK_FP8;
  static constexpr bool XS4 = XS4_ && !ROW;
  static constexpr int NB = BN / 128;         // weight-scale blocks per tile
  static constexpr int WGN = BN / 64, WGM = NW / WGN;
  static_assert(WGM * WGN == NW && WGM >= 1, "wave grid");
  static constexpr int WROWS = BM / WGM;
  static constexpr int MI = WROWS / 32, NI = 2;
  static constexpr int NT = MI * NI;
  static constexpr int TB = (MI - 1) * NI;
  static_assert(MI >= 2, "the barrier tile follows the last read of the current slot");
  static constexpr int AQ = (BM / 8) / NW, BQ = (BN / 8) / NW;  // 8-row loads per wave
  static_assert(AQ * NW * 8 == BM && BQ * NW * 8 == BN, "row loads cover the tile");
  // scale loads per wave: 4 waves each load 64 xs rows (rows past the tile are
  // clamped and never read) and the ws copies; 8 waves: waves 0-3 xs, waves 4-7 ws
  // (block (w-4) % NB)
  static constexpr int SQ = ROW ? 0 : (NW == 4 ? 2 : 1);
  static_assert(ROW || NW == 8 || NB == 1, "4-wave tiles have one weight-scale block");
  static constexpr int LPS = AQ + BQ + SQ;
  static constexpr int W = NSLOT >= 3 ? NT : NT - TB;  // load window in tiles
  static constexpr int PER = (LPS + W - 1) / W;
  static constexpr int WAITN = (NSLOT - 2) * LPS;    // loads allowed in flight at the barrier
  // LDS layout of a slot
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int XOFF = A_BYTES + B_BYTES;          // xs (per-step mode only)
  static constexpr int WOFF = XOFF + (XS4 || ROW ? 0 : 1024);
  static constexpr int WCOPY = ROW ? 0 : (XS4 ? 1024 : 256);  // bytes of one ws block's copies
  static constexpr int SLOT = WOFF + NB * WCOPY;
  static constexpr int RING = NSLOT * SLOT;                // XS4 activation-scale ring
  static constexpr int LDS = RING + (XS4 ? 2 * 4096 : 0);
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NW * WROWS * 64 * 2 <= LDS, "epilogue staging fits");
};

template <int CPOL = kCpolDefault>
__device__ __forceinline__ void buf_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t* lds_dst,
                                        int size) {
  if (size == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, (int)voff, (int)soff, 0, CPOL);
  else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 4, (int)voff, (int)soff, 0, CPOL);
}

__device__ __forceinline__ int f8_key(int r) { return (r ^ (r >> 3)) & 7; }

// 32 K-consecutive bytes of one row: two 16-byte chunks at their swizzled positions.
__device__ __forceinline__ i32x8_t lds_frag32(const uint8_t* row, const int (&off)[2]) {
  const u32x4_t lo = *(const u32x4_t*)(row + off[0]);
  const u32x4_t hi = *(const u32x4_t*)(row + off[1]);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// FULL_M: every row of the M tile exists, so the A loads of a wave share one per-lane
// offset and differ by a scalar row offset; otherwise rows are clamped per load.
// GROUPED (row-scale modes): the tile's A rows are gathered through p.sorted (padding
// rows read row 0 and are never stored), B and the weight scales are those of the
// block's expert, and output rows are scattered back to token order.
// BNT: the weight loads are non-temporal -- every weight tile is read by one group of
// at most kFp8GroupM row tiles (launched side by side, sharing it through L2), or, in
// the grouped mode, by one expert's row blocks.  The policy is an instruction immediate,
// hence a template flag (a branch would split the tile loop).
template <typename C, bool FULL_M, bool GROUPED = false, bool BNT = false>
__global__ void __launch_bounds__(C::NW * 64)
    gemm_fp8_pipe_kernel(const Fp8Params p) {
  constexpr int NW = C::NW, MI = C::MI, NI = C::NI, NT = C::NT, TB = C::TB;
  constexpr int AQ = C::AQ, BQ = C::BQ, LPS = C::LPS, PER = C::PER, NSLOT = C::NSLOT;
  constexpr bool XS4 = C::XS4, ROW = C::ROW, I8 = C::MODE == Q_ROW_I8;
  static_assert(!GROUPED || (ROW && !FULL_M), "grouped tiles use row scales and gathered rows");
  using AccT = std::conditional_t<I8, i32x16_t, f32x16_t>;

  __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int lr = lane & 31, hh = lane >> 5;

  int m0, n0;
  if constexpr (GROUPED) {
    // m-block major: the live blocks are a prefix of the grid, which the round-robin
    // dispatch spreads evenly over the XCDs (a remap would pack them onto a few)
    m0 = ((int)blockIdx.x / p.tiles_n) * C::BM;
    n0 = ((int)blockIdx.x % p.tiles_n) * C::BN;
  } else {
    const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int width = kFp8GroupM * p.tiles_n;
    const int grp = bid / width;
    const int first_m = grp * kFp8GroupM;
    const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
    const int tl = bid - grp * width;
    m0 = (first_m + tl % gsz) * C::BM;
    n0 = (tl / gsz) * C::BN;
  }
  const int rows_a = GROUPED ? C::BM : min(p.M - m0, C::BM);
  const int nk = p.K / 128;
  int expert = 0;
  if constexpr (GROUPED) {
    expert = p.block_expert[m0 / C::BM];  // uniform: an unused block leaves before any barrier
    if (expert < 0) return;
  }
  // token row of tile row r (grouped: padding rows read token 0)
  auto grow = [&](int r) -> int {
    if constexpr (GROUPED) {
      const int t = p.sorted[m0 + r];
      return t < p.M ? t : 0;
    } else {
      return min(r, rows_a - 1);
    }
  };

  // ---- buffer resources (tile-based) and per-lane load offsets ----
  const __amdgpu_buffer_rsrc_t ra = GROUPED ? make_rsrc(p.xq, (uint32_t)((int64_t)p.M * p.ldx))
                                            : make_rsrc(p.xq + (int64_t)m0 * p.ldx, (uint32_t)(rows_a * p.ldx));
  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(p.wq + (int64_t)expert * p.w_estride + (int64_t)n0 * p.ldw, (uint32_t)(C::BN * p.ldw));
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(p.xs + (int64_t)m0 * p.xs_m, (uint32_t)(((rows_a - 1) * p.xs_m + (nk - 1) * p.xs_k + 1) * 4));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(
      p.ws + (int64_t)(n0 / 128) * p.ws_n, (uint32_t)(((C::NB - 1) * p.ws_n + (nk - 1) * p.ws_k + 1) * 4));
  // 16-byte chunk this lane fetches: row (lane >> 3) of an 8-row group, position
  // lane & 7.  Load q of a wave covers rows 8 * (wave + NW * q) + lane / 8, whose
  // row % 32 is 8 * (wave % 4) + lane / 8 for every q.
  const int lrow = lane >> 3;
  const int dchunk = (lane & 7) ^ f8_key(8 * (wave & 3) + lrow);
  uint32_t a_voff[FULL_M ? 1 : AQ];
  if constexpr (FULL_M) {
    a_voff[0] = (uint32_t)((lrow + 8 * wave) * p.ldx + 16 * dchunk);
  } else {
#pragma unroll
    for (int q = 0; q < AQ; ++q) a_voff[q] = (uint32_t)(grow(lrow + 8 * (wave + NW * q)) * p.ldx + 16 * dchunk);
  }
  const uint32_t b_voff = (uint32_t)((lrow + 8 * wave) * p.ldw + 16 * dchunk);
  const uint32_t x_voff = (uint32_t)(min(64 * (wave & 3) + lane, rows_a - 1) * p.xs_m * 4);
  const uint32_t a_rstep = (uint32_t)(8 * NW * p.ldx), b_rstep = (uint32_t)(8 * NW * p.ldw);
  const uint32_t xs_kstep = (uint32_t)(p.xs_k * 4), ws_kstep = (uint32_t)(p.ws_k * 4);
  // weight-scale block this wave loads (8 waves) and the one its columns use
  const int wblk_ld = (NW == 8) ? ((wave - 4) & 3) % C::NB : 0;
  const uint32_t w_soff_blk = (uint32_t)(wblk_ld * p.ws_n * 4);
  const int wblk_rd = (wn * 64) / 128;

  // load q of stage kb (already clamped to nk - 1) into slot
  auto issue = [&](int slot, int kb, int q) {
    uint8_t* base = lds + slot * C::SLOT;
    if (q < AQ) {
      const uint32_t v = a_voff[FULL_M ? 0 : q];
      const uint32_t so = (uint32_t)kb * 128u + (FULL_M ? (uint32_t)q * a_rstep : 0u);
      buf_lds(ra, v, so, base + (wave + NW * q) * 1024, 16);
    } else if (q < AQ + BQ) {
      buf_lds<(GROUPED || BNT) ? kCpolNT : kCpolDefault>(rb, b_voff, (uint32_t)kb * 128u + (uint32_t)(q - AQ) * b_rstep,
                                                base + C::A_BYTES + (wave + NW * (q - AQ)) * 1024, 16);
    } else if constexpr (!ROW) {
      // scale load (wave-uniform selects): activation scales, or weight-scale copies
      const bool xload = (NW == 4 ? q == AQ + BQ : wave < 4) && (!XS4 || (kb & 3) == 0);
      if constexpr (XS4) {
        uint8_t* dst = xload ? lds + C::RING + ((kb >> 2) & 1) * 4096 + (wave & 3) * 1024
                             : base + C::WOFF + wblk_ld * C::WCOPY;
        buf_lds(xload ? rx : rw, xload ? x_voff : 0u,
                xload ? (uint32_t)kb * 4u : w_soff_blk + (uint32_t)(kb & ~3) * 4u, dst, 16);
      } else {
        uint8_t* dst = xload ? base + C::XOFF + (wave & 3) * 256 : base + C::WOFF + wblk_ld * C::WCOPY;
        buf_lds(xload ? rx : rw, xload ? x_voff : 0u,
                xload ? (uint32_t)kb * xs_kstep : w_soff_blk + (uint32_t)kb * ws_kstep, dst, 4);
      }
    }
  };

  // ---- fragment read offsets: row lr of a 32-row block, K sub-step h, 16-byte half e:
  // chunk 4h + 2hh + e ----
  const int key = f8_key(lr);
  int off[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) off[h][e] = lr * 128 + (((4 * h + 2 * hh + e) ^ key) << 4);
  const int rowA0 = wm * C::WROWS, rowB0 = wn * 64;

  AccT acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  // row-scale modes: one K half of a 32x32 tile straight into its accumulator
  auto row_mma = [&](AccT& c, const i32x8_t& b, const i32x8_t& a) {
    if constexpr (I8) {
      c = mma32_i8(u32x4_t{(uint32_t)b[0], (uint32_t)b[1], (uint32_t)b[2], (uint32_t)b[3]},
                   u32x4_t{(uint32_t)a[0], (uint32_t)a[1], (uint32_t)a[2], (uint32_t)a[3]}, c);
      c = mma32_i8(u32x4_t{(uint32_t)b[4], (uint32_t)b[5], (uint32_t)b[6], (uint32_t)b[7]},
                   u32x4_t{(uint32_t)a[4], (uint32_t)a[5], (uint32_t)a[6], (uint32_t)a[7]}, c);
    } else if constexpr (ROW) {
      c = mma32_fp8(b, a, c);
    }
  };
  f32x16_t part[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) part[1][r] = 0.0f;
  const f32x16_t zero = {};
  float sc[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) sc[i] = 0.0f;
  float xsv[MI], wsv;
  i32x8_t af[2][2], bf[2][2];  // af[buffer][h], bf[j][h]

  // ---- prologue: stages 0 .. NSLOT-2 in flight, wait for stage 0, first fragments,
  // then the post-barrier share of stage NSLOT-1 ----
#pragma unroll
  for (int st = 0; st + 1 < NSLOT; ++st)
#pragma unroll
    for (int q = 0; q < LPS; ++q) issue(st, min(st, nk - 1), q);
  wait_vmcnt<C::WAITN>();
  exec_barrier();
  af[0][0] = lds_frag32(lds + rowA0 * 128, off[0]);
  af[0][1] = lds_frag32(lds + rowA0 * 128, off[1]);
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    bf[j][0] = lds_frag32(lds + C::A_BYTES + (rowB0 + 32 * j) * 128, off[0]);
    bf[j][1] = lds_frag32(lds + C::A_BYTES + (rowB0 + 32 * j) * 128, off[1]);
  }
#pragma unroll
  for (int q = 0; q < PER * (NT - TB) && q < LPS; ++q) issue(NSLOT - 1, min(NSLOT - 1, nk - 1), q);

  int slot = 0;
  for (int s = 0; s < nk; ++s) {
    const int slot1 = slot + 1 == NSLOT ? 0 : slot + 1;
    const int slotp = slot == 0 ? NSLOT - 1 : slot - 1;  // slot of stage s + NSLOT - 1
    const uint8_t* cur = lds + slot * C::SLOT;
    const uint8_t* nxt = lds + slot1 * C::SLOT;
    const int kbn = min(s + NSLOT, nk - 1), kbp = min(s + NSLOT - 1, nk - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int i = t / NI, j = t % NI;
      if (t == TB) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<C::WAITN>();
        exec_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (ROW) {
        row_mma(acc[i][j], bf[j][0], af[i & 1][0]);
      } else {
        part[j] = mma32_fp8(bf[j][0], af[i & 1][0], zero);
        __builtin_amdgcn_sched_barrier(0);
        if (t == 1) {
#pragma unroll
          for (int q = 0; q < MI; ++q) sc[q] = xsv[q] * wsv;
        }
        {
          // promote the previous tile (t == 0: the last tile of the previous stage,
          // whose scale sc[MI-1] is still live; zeros before the first stage)
          const int pt = (t + NT - 1) % NT;
          const float f = sc[pt / NI];
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[pt / NI][pt % NI][r] = fmaf(part[j ^ 1][r], f, acc[pt / NI][pt % NI][r]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (ROW) row_mma(acc[i][j], bf[j][1], af[i & 1][1]);
      else part[j] = mma32_fp8(bf[j][1], af[i & 1][1], part[j]);
      __builtin_amdgcn_sched_barrier(0);
      // LDS reads: scales of this stage; A block i+1 (both K halves) at the first
      // tile of block i, two MFMA pairs before its first use; after the barrier A
      // block 0 of the next stage; B of the next stage right after its last use.
      if (!ROW && t == 0) {
        if constexpr (XS4) {
          const uint8_t* ring = lds + C::RING + ((s >> 2) & 1) * 4096 + (s & 3) * 4;
#pragma unroll
          for (int q = 0; q < MI; ++q) xsv[q] = *(const float*)(ring + (rowA0 + 32 * q + lr) * 16);
          wsv = *(const float*)(cur + C::WOFF + wblk_rd * C::WCOPY + (s & 3) * 4);
        } else {
#pragma unroll
          for (int q = 0; q < MI; ++q) xsv[q] = *(const float*)(cur + C::XOFF + (rowA0 + 32 * q + lr) * 4);
          wsv = *(const float*)(cur + C::WOFF + wblk_rd * C::WCOPY);
        }
      }
      if (j == 0 && i + 1 < MI) {
        af[(i + 1) & 1][0] = lds_frag32(cur + (rowA0 + 32 * (i + 1)) * 128, off[0]);
        af[(i + 1) & 1][1] = lds_frag32(cur + (rowA0 + 32 * (i + 1)) * 128, off[1]);
      } else if (t == TB) {
        af[0][0] = lds_frag32(nxt + rowA0 * 128, off[0]);
        af[0][1] = lds_frag32(nxt + rowA0 * 128, off[1]);
      }
      if (t >= TB) {
        bf[j][0] = lds_frag32(nxt + C::A_BYTES + (rowB0 + 32 * j) * 128, off[0]);
        bf[j][1] = lds_frag32(nxt + C::A_BYTES + (rowB0 + 32 * j) * 128, off[1]);
      }
      // direct loads, PER per tile over the window: tiles TB.. of stage s start stage
      // s + NSLOT (into the slot just released); with three slots tiles ..TB-1 finish
      // stage s + NSLOT - 1
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        if (t >= TB) {
          const int q = PER * (t - TB) + e;
          if (q < LPS) issue(slot, kbn, q);
        } else if (NSLOT >= 3) {
          const int q = PER * (t + NT - TB) + e;
          if (q < LPS) issue(slotp, kbp, q);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    slot = slot1;
  }
  if constexpr (!ROW) {
    // promote the last tile of the last stage
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[MI - 1][NI - 1][r] = fmaf(part[1][r], sc[MI - 1], acc[MI - 1][NI - 1][r]);
  }
  wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
  __syncthreads();

  // ---- epilogue: (row modes: x scale of the row times w scale of the column), bf16
  // pack, stage per wave, 16-byte row stores ----
  using St = Stager<C::WROWS, 64>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = (uint16_t*)lds + wave * (C::WROWS * 64);
  float xrow[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    if constexpr (GROUPED) xrow[i] = p.xs[(int64_t)grow(rowA0 + 32 * i + lr) * p.xs_m];
    else xrow[i] = ROW ? p.xs[(int64_t)min(m0 + rowA0 + 32 * i + lr, p.M - 1) * p.xs_m] : 1.0f;
  }
  const float* wsx = p.ws + (int64_t)expert * p.ws_estride;
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float wcol[4] = {1.0f, 1.0f, 1.0f, 1.0f};
      if constexpr (ROW) {
        const int64_t n = n0 + rowB0 + out_col(j, g, lane);  // n + 3 < N: N % BN == 0
#pragma unroll
        for (int e = 0; e < 4; ++e) wcol[e] = wsx[(n + e) * p.ws_n];
      }
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = (float)acc[i][j][4 * g + e];
          if constexpr (ROW) v[e] = v[e] * xrow[i] * wcol[e];
        }
        St::put(stg, out_row(i, lane), out_col(j, g, lane), u32x2_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3])});
      }
    }
  __syncthreads();
  const int mw0 = m0 + rowA0, nw0 = n0 + rowB0;
  const bool vec = p.vec_store != 0;
  St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
    const int gn = nw0 + col;
    const int gm = GROUPED ? p.sorted[mw0 + row] : mw0 + row;
    if (gm < p.M) store_row8(p.y + (int64_t)gm * p.ldy + gn, gn, p.N, vec, v);
  });
}

template <typename C>
int launch_fp8_pipe(Fp8Params p, hipStream_t st) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = p.N / C::BN;
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n)), block(C::NW * 64);
  // Block scales with one group of row tiles (kFp8GroupM of them sweep the column tiles
  // together): each weight tile is read once from memory.  Same process, cold cache:
  // M=256 / 512 33.5 / 33.3 -> 27.7 / 28.3 us, warm 21.1 / 24.0 -> 23.1 / 25.0 us.
  bool bnt = false;
  if constexpr (C::MODE == Q_BLOCK_FP8) bnt = p.tiles_m <= kFp8GroupM;
  if (bnt) {
    if constexpr (C::MODE == Q_BLOCK_FP8) {
      if (p.M % C::BM == 0) hipLaunchKernelGGL((gemm_fp8_pipe_kernel<C, true, false, true>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((gemm_fp8_pipe_kernel<C, false, false, true>), grid, block, 0, st, p);
    }
  } else if (p.M % C::BM == 0) {
    hipLaunchKernelGGL((gemm_fp8_pipe_kernel<C, true>), grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((gemm_fp8_pipe_kernel<C, false>), grid, block, 0, st, p);
  }
  return check_launch("gemm_fp8_pipe_kernel");
}

// ------------------------------------------------------------------------------
// Wide block-scale kernel: 256 x 224 tiles, 8 waves.  2048 x 7168 (the BASELINE
// shape) has exactly 8 x 32 = 256 such tiles, one per CU, where 256 x 256 tiles leave
// 32 of the 256 CUs idle.  Waves form a 4 (M) x 2 (N) grid: every wave owns 64 rows
// (two 32-row tiles); waves 0-3 own columns 0..127 of the tile (four 32-column tiles)
// and waves 4-7 columns 128..223 (three).  Wave w runs on SIMD w % 4 next to wave
// w + 4, so every SIMD multiplies 2 x (4 + 3) = 14 tiles of 32 x 32 per K block.
//
// Per 128-wide K block (= one scale block) a wave walks its tiles column by column:
// tile (j, i) is two 32x32x64 MFMAs into a zeroed partial, and the partial of the
// previous tile is promoted acc += partial * xs[m, kb] * ws[n/128, kb] between them
// (each scale applied once, as in the oracle).  The A fragments of both row tiles stay
// in registers for the whole block; B fragments are read one column ahead into a
// double buffer.  The LDS ring (two slots; XOR-swizzled 128-byte rows, filled by
// direct-to-LDS loads; scales travel in the same DMA stream) and the one barrier per
// block follow the pipelined kernel above: the barrier sits at the first tile of
// the last column, after the block's last B read and before the next block's first.
// Requires M % 256 == 0, N % 224 == 0, K % 512 == 0 and K-contiguous scale rows.
// ------------------------------------------------------------------------------
// LDS: the A tiles of both slots, then the B tiles of both slots, then the ws copies
// of both slots and the xs ring, so that every fragment read is one base register per
// operand plus an immediate offset below 64 KiB.
// LDS reads through a 32-bit LDS byte offset held in a VGPR plus a compile-time
// immediate.  The offset is made opaque to the compiler (an empty asm), so it keeps
// one register per base and folds the constant into the ds_read offset field instead
// of materialising a new address register per read.
// Calls f(std::integral_constant<int, t>) for t = 0 .. N-1 (a compile-time loop).
template <int T, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (T < N) {
    f(std::integral_constant<int, T>{});
    static_for<T + 1, N>(f);
  }
}

typedef __attribute__((address_space(3))) const u32x4_t* lds_cv4;
typedef __attribute__((address_space(3))) const float* lds_cf;
typedef __attribute__((address_space(3))) uint8_t* lds_u8;
__device__ __forceinline__ uint32_t lds_offset_of(const void* p) {
  uint32_t v = (uint32_t)(uintptr_t)(lds_u8)(p);
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ u32x4_t lds_ld16(uint32_t off) { return *(lds_cv4)(uintptr_t)off; }
__device__ __forceinline__ float lds_ldf(uint32_t off) { return *(lds_cf)(uintptr_t)off; }
template <int IMM>
__device__ __forceinline__ i32x8_t lds_frag32_imm(const uint32_t (&base)[2]) {
  const u32x4_t lo = lds_ld16(base[0] + IMM);
  const u32x4_t hi = lds_ld16(base[1] + IMM);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

struct WideCfg {
  static constexpr int BM = 256, BN = 224, NW = 8, MI = 2;
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int B_BASE = 2 * A_BYTES;            // B tile of slot s at B_BASE + s * B_BYTES
  static constexpr int NWB = 3;                         // weight-scale blocks a tile can touch
  static constexpr int W_BASE = B_BASE + 2 * B_BYTES;   // ws copies of slot s (1 KiB per block)
  static constexpr int RING = W_BASE + 2 * NWB * 1024;  // xs ring (2 x 4 K blocks)
  static constexpr int LDS = RING + 2 * 4096;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(NW * 64 * 128 * 2 <= LDS, "epilogue staging fits");
};

// Main loop and epilogue of one wave with NI column tiles (4: waves 0-3, 3: waves
// 4-7).  A wave issues 4 A loads, NI B loads and 1 scale load per stage.
template <int NI>
__device__ __forceinline__ void fp8_wide_wave(const Fp8Params& p, uint8_t* lds, int wave, int lane, int m0, int n0) {
  using C = WideCfg;
  constexpr int MI = C::MI, AQ = 4, BQ = NI, LPS = AQ + BQ + 1;
  constexpr int NT = MI * NI, TB = 2 * (NI - 1);  // barrier tile: (j = NI-1, i = 0)
  // The loads of block s+2 (into the slot released at block s's barrier) are spread
  // over NU = NT - 2 issue tiles: tiles TB .. NT-1 of block s, then tiles 0 .. TB-3 of
  // block s+1 (they must land by its barrier).  Issue tile u takes loads
  // [u * LPS / NU, (u + 1) * LPS / NU): bunching them into two tiles filled the TA
  // queue and stalled the waves at issue.
  constexpr int NU = NT - 2, U0 = NT - TB;  // U0: issue tiles in the releasing block
  const int lr = lane & 31, hh = lane >> 5;
  const int wm = wave & 3;
  const int rowA0 = 64 * wm, colB0 = wave < 4 ? 0 : 128;
  const int nk = p.K / 128;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.xq + (int64_t)m0 * p.ldx, (uint32_t)(C::BM * p.ldx));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.wq + (int64_t)n0 * p.ldw, (uint32_t)(C::BN * p.ldw));
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(p.xs + (int64_t)m0 * p.xs_m, (uint32_t)(((C::BM - 1) * p.xs_m + (nk - 1) + 1) * 4));
  const int wblk0 = n0 / 128;  // first weight-scale block of the tile
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(p.ws + (int64_t)wblk0 * p.ws_n,
                (uint32_t)((((int64_t)p.N / 128 - 1 - wblk0) * p.ws_n + (nk - 1) + 1) * 4));
  // DMA: load q of a wave covers tile rows 8 * (wave + 8q) + lane / 8, whose row % 32 is
  // 8 * (wave % 4) + lane / 8 for every q; lane l fetches chunk (l % 8) ^ key(row % 32)
  const int lrow = lane >> 3;
  const int dchunk = (lane & 7) ^ f8_key(8 * (wave & 3) + lrow);
  const uint32_t a_voff = (uint32_t)((lrow + 8 * wave) * p.ldx + 16 * dchunk);
  const uint32_t b_voff = (uint32_t)((lrow + 8 * wave) * p.ldw + 16 * dchunk);
  const uint32_t a_rstep = (uint32_t)(64 * p.ldx), b_rstep = (uint32_t)(64 * p.ldw);
  const uint32_t x_voff = (uint32_t)((64 * (wave & 3) + lane) * p.xs_m * 4);
  // scale load of this wave: waves 0-3 load the xs of 64 rows (4 K blocks per 16 bytes)
  // at every fourth block and otherwise a copy of ws block wave % 3; waves 4-7 load
  // ws block (wave - 4) % 3 (64 copies of 4 K blocks each)
  const int wblk_ld = wave < 4 ? wave % 3 : (wave - 4) % 3;
  const uint32_t w_soff = (uint32_t)(wblk_ld * p.ws_n * 4);

  auto issue = [&](int slot, int kb, int q) {
    if (q < AQ) {
      buf_lds(ra, a_voff, (uint32_t)kb * 128u + (uint32_t)q * a_rstep,
              lds + slot * C::A_BYTES + (wave + 8 * q) * 1024, 16);
    } else if (q < AQ + BQ) {
      buf_lds(rb, b_voff, (uint32_t)kb * 128u + (uint32_t)(q - AQ) * b_rstep,
              lds + C::B_BASE + slot * C::B_BYTES + (wave + 8 * (q - AQ)) * 1024, 16);
    } else {
      const bool xload = wave < 4 && (kb & 3) == 0;
      uint8_t* dst = xload ? lds + C::RING + ((kb >> 2) & 1) * 4096 + (wave & 3) * 1024
                           : lds + C::W_BASE + (slot * C::NWB + wblk_ld) * 1024;
      buf_lds(xload ? rx : rw, xload ? x_voff : 0u, xload ? (uint32_t)kb * 4u : w_soff + (uint32_t)(kb & ~3) * 4u,
              dst, 16);
    }
  };

  // fragment read offsets: row lr of a 32-row block, K half h, 16-byte half e
  const int key = f8_key(lr);
  int off[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) off[h][e] = lr * 128 + (((4 * h + 2 * hh + e) ^ key) << 4);
  // weight-scale block of each column tile, relative to the tile's first block
  int wsb[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) wsb[j] = (n0 + colB0 + 32 * j) / 128 - wblk0;

  f32x16_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  f32x16_t part[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) part[1][r] = 0.0f;
  const f32x16_t zero = {};
  float sc_last = 0.0f, xsv_[MI] = {}, wsv_[NI] = {};
  i32x8_t af[MI][2], bf[2][2];  // af[i][h]; bf[buffer][h]

  // prologue: block 0, and the share of block 1 normally issued at the end of the
  // block before it; wait for block 0
  constexpr int P1 = U0 * LPS / NU;
#pragma unroll
  for (int q = 0; q < LPS; ++q) issue(0, 0, q);
#pragma unroll
  for (int q = 0; q < P1; ++q) issue(1, min(1, nk - 1), q);
  wait_vmcnt<P1>();
  exec_barrier();
  // fragment bases (LDS byte offsets): A row block 0 and B column block 0 of slot 0,
  // per K half h and 16-byte half e; slot, row and column offsets are immediates
  uint32_t ab[2][2], bbv[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      ab[h][e] = lds_offset_of(lds + rowA0 * 128 + off[h][e]);
      bbv[h][e] = lds_offset_of(lds + C::B_BASE + colB0 * 128 + off[h][e]);
    }
  // xs of row block 0 (16 bytes per row: 4 K blocks) and the ws copies of slot 0
  const uint32_t xbase = lds_offset_of(lds + C::RING + (rowA0 + lr) * 16);
  const uint32_t wbase = lds_offset_of(lds + C::W_BASE);
  af[0][0] = lds_frag32_imm<0>(ab[0]);
  af[0][1] = lds_frag32_imm<0>(ab[1]);
  af[1][0] = lds_frag32_imm<32 * 128>(ab[0]);
  af[1][1] = lds_frag32_imm<32 * 128>(ab[1]);
  bf[0][0] = lds_frag32_imm<0>(bbv[0]);
  bf[0][1] = lds_frag32_imm<0>(bbv[1]);

  // one K block; SL: its slot, PB: the bf buffer of its column 0 (both compile-time)
  auto stage = [&](int s, auto sl_tag, auto pb_tag) {
    constexpr int SL = decltype(sl_tag)::value, PB = decltype(pb_tag)::value;
    constexpr int A_NXT = (SL ^ 1) * C::A_BYTES, B_CUR = SL * C::B_BYTES, B_NXT = (SL ^ 1) * C::B_BYTES;
    constexpr int W_CUR = SL * C::NWB * 1024;
    const int kb1 = min(s + 1, nk - 1), kb2 = min(s + 2, nk - 1);
    static_for<0, NT>([&](auto tt) {
      constexpr int t = decltype(tt)::value;
      constexpr int j = t / MI, i = t % MI;
      constexpr int bb = (PB + j) & 1;
      if constexpr (t == TB) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<0>();
        exec_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      part[t & 1] = mma32_fp8(bf[bb][0], af[i][0], zero);
      __builtin_amdgcn_sched_barrier(0);
      // promote the previous tile (t == 0: the last tile of the previous block), half
      // on each side of the second MFMA: the FMAs fill the MFMA's dependency shadow
      // instead of one run of 16 that waits out the first MFMA's result (0.5% on
      // 2048 x 7168 x 4096, measured)
      constexpr int pi = t == 0 ? MI - 1 : (t - 1) % MI, pj = t == 0 ? NI - 1 : (t - 1) / MI;
      const float f = t == 0 ? sc_last : xsv_[pi] * wsv_[pj];
      f32x16_t& a = acc[pi][pj];
#pragma unroll
      for (int r = 0; r < 8; ++r) a[r] = fmaf(part[(t + 1) & 1][r], f, a[r]);
      __builtin_amdgcn_sched_barrier(0);
      part[t & 1] = mma32_fp8(bf[bb][1], af[i][1], part[t & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 8; r < 16; ++r) a[r] = fmaf(part[(t + 1) & 1][r], f, a[r]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (t == NT - 1) sc_last = xsv_[MI - 1] * wsv_[NI - 1];
      // LDS reads: this block's scales at t == 0; B column j + 1 at tile (j, 0); after
      // the barrier B column 0 and the A fragments of the next block
      if constexpr (t == 0) {
        const uint32_t xo = xbase + (uint32_t)(((s >> 2) & 1) * 4096 + (s & 3) * 4);
        const uint32_t wo = wbase + (uint32_t)((s & 3) * 4);
        xsv_[0] = lds_ldf(xo);
        xsv_[1] = lds_ldf(xo + 32 * 16);
        const float w0 = lds_ldf(wo + W_CUR), w1 = lds_ldf(wo + W_CUR + 1024), w2 = lds_ldf(wo + W_CUR + 2048);
#pragma unroll
        for (int jj = 0; jj < NI; ++jj) wsv_[jj] = wsb[jj] == 0 ? w0 : (wsb[jj] == 1 ? w1 : w2);
      }
      if constexpr (i == 0 && j + 1 < NI) {
        bf[bb ^ 1][0] = lds_frag32_imm<B_CUR + 32 * 128 * (j + 1)>(bbv[0]);
        bf[bb ^ 1][1] = lds_frag32_imm<B_CUR + 32 * 128 * (j + 1)>(bbv[1]);
      }
      if constexpr (t == TB) {
        bf[bb ^ 1][0] = lds_frag32_imm<B_NXT>(bbv[0]);
        bf[bb ^ 1][1] = lds_frag32_imm<B_NXT>(bbv[1]);
        af[0][0] = lds_frag32_imm<A_NXT>(ab[0]);
        af[0][1] = lds_frag32_imm<A_NXT>(ab[1]);
      }
      if constexpr (t == NT - 1) {
        af[1][0] = lds_frag32_imm<A_NXT + 32 * 128>(ab[0]);
        af[1][1] = lds_frag32_imm<A_NXT + 32 * 128>(ab[1]);
      }
      // loads: the rest of block s+1 (slot SL^1) early in the block, the first share of
      // block s+2 (slot SL, released at this block's barrier) after the barrier
      if constexpr (t < TB - 2 || t >= TB) {
        constexpr int u = t >= TB ? t - TB : U0 + t;
        constexpr int q0 = u * LPS / NU, q1 = (u + 1) * LPS / NU;
#pragma unroll
        for (int q = q0; q < q1; ++q) {
          if constexpr (t >= TB) issue(SL, kb2, q);
          else issue(SL ^ 1, kb1, q);
        }
      }
    });
  };
  // blocks in pairs so that the slot and the bf buffer parity are compile-time
  for (int s = 0; s < nk; s += 2) {
    stage(s, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    stage(s + 1, std::integral_constant<int, 1>{}, std::integral_constant<int, NI & 1>{});
  }
  // promote the last tile of the last block
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[MI - 1][NI - 1][r] = fmaf(part[(NT - 1) & 1][r], sc_last, acc[MI - 1][NI - 1][r]);
  wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
  __syncthreads();

  // epilogue: bf16 pack, stage the wave's 64 x 128 tile in LDS, 16-byte row stores
  using St = Stager<64, 128>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = (uint16_t*)lds + wave * (64 * 128);
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        St::put(stg, out_row(i, lane), out_col(j, g, lane),
                u32x2_t{Op::pack2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                        Op::pack2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3])});
  __syncthreads();
  const int mw0 = m0 + rowA0, nw0 = n0 + colB0;
  const bool vec = p.vec_store != 0;
  St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
    if (col < 32 * NI) store_row8(p.y + (int64_t)(mw0 + row) * p.ldy + nw0 + col, nw0 + col, p.N, vec, v);
  });
}

__global__ void __launch_bounds__(512) gemm_fp8_wide_kernel(const Fp8Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[WideCfg::LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // XCD-aware order: each XCD's 32 consecutive tiles form 4 M-tiles x 8 N-tiles
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int width = kFp8GroupM * p.tiles_n;
  const int grp = bid / width;
  const int first_m = grp * kFp8GroupM;
  const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
  const int tl = bid - grp * width;
  const int m0 = (first_m + tl % gsz) * WideCfg::BM;
  const int n0 = (tl / gsz) * WideCfg::BN;
  if (wave < 4) fp8_wide_wave<4>(p, lds, wave, lane, m0, n0);
  else fp8_wide_wave<3>(p, lds, wave, lane, m0, n0);
}

int launch_fp8_wide(Fp8Params p, hipStream_t st) {
  p.tiles_m = p.M / WideCfg::BM;
  p.tiles_n = p.N / WideCfg::BN;
  hipLaunchKernelGGL(gemm_fp8_wide_kernel, dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(512), 0, st, p);
  return check_launch("gemm_fp8_wide_kernel");
}

// ------------------------------------------------------------------------------
// K-split block-scale kernel: 128 x 128 tiles, 8 waves, for problems whose 128 x 128
// grid covers at least three quarters of the CUs (M = 512 at N = 7168: 224 tiles).  The 4-wave
// 128 x 128 tile puts one wave on each SIMD, whose promotion FMAs then serialise with
// its own MFMAs; here the two waves of a SIMD own the same 64 x 64 outputs and split
// the K blocks: waves 0-3 (group 0) take the even blocks, waves 4-7 (group 1) the odd
// ones, so one wave's promotion runs under the other's MFMAs at the 4-wave tile's
// fragment traffic per MFMA.  A stage is two consecutive K blocks (one per group) in
// one LDS slot: A 2 x 128 rows, B 2 x 128 rows, one copy of the weight scales; two
// slots, one barrier per stage, the xs of four blocks per 16-byte row load in a
// two-entry ring.  LDS holds the A blocks of both slots, then their B blocks, so every
// fragment read is a base register plus an immediate offset below 64 KiB.  Each block is promoted once, with its own xs[m, kb] * ws[nb, kb],
// by the wave that multiplies it; the two partial sums of an output are added once
// after the K loop (group 0's registers + group 1's, through LDS), so every output
// is reproducible run to run.  Requires M % 128 == 0, N % 128 == 0, K % 512 == 0 and
// K-contiguous scale rows.
// ------------------------------------------------------------------------------
struct KsCfg {
  static constexpr int BM = 128, BN = 128, NW = 8, MI = 2, NI = 2, NT = MI * NI;
  static constexpr int A_BLK = BM * 128, B_BLK = BN * 128;  // one K block
  static constexpr int A_SLOT = 2 * A_BLK, B_SLOT = 2 * B_BLK;
  // A block b of slot s at s * A_SLOT + b * A_BLK; B at B_BASE + s * B_SLOT + b * B_BLK;
  // the ws copy (four blocks) of slot s at W_BASE + s * 1024; the xs ring after them
  static constexpr int B_BASE = 2 * A_SLOT, W_BASE = B_BASE + 2 * B_SLOT;
  static constexpr int RING = W_BASE + 2 * 1024;  // xs ring: 2 x (128 rows x 16 B)
  static constexpr int LDS = RING + 2 * 2048;
  static constexpr int XCH = 4 * 64 * 64 * 4;                     // epilogue: group 1's partials
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(XCH + 4 * 64 * 64 * 2 <= LDS, "epilogue exchange + staging fit");
  static_assert(A_SLOT == B_SLOT && A_SLOT + 4 * 1024 < 65536, "fragment immediates below 64 KiB");
};

__global__ void __launch_bounds__(512) gemm_fp8_ksplit_kernel(const Fp8Params p) {
  using C = KsCfg;
  constexpr int MI = C::MI, NI = C::NI, NT = C::NT;
  constexpr int TB = 2 * (NI - 1);  // barrier tile: the first tile of the last column
  constexpr int LPS = 4 + 4 + 1;    // per wave and stage: 4 A and 4 B row loads, one scale load
  constexpr int NU = NT - TB;       // the next-but-one stage's loads go out in tiles TB .. NT-1
  __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wq = wave & 3;  // K-block parity, position in the 2 x 2 wave grid
  const int wm = wq >> 1, wn = wq & 1;
  const int lr = lane & 31, hh = lane >> 5;

  // XCD-aware raster, groups of kFp8GroupM row tiles sweeping the column tiles
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int width = kFp8GroupM * p.tiles_n;
  const int gi = bid / width;
  const int first_m = gi * kFp8GroupM;
  const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
  const int tl = bid - gi * width;
  const int m0 = (first_m + tl % gsz) * C::BM;
  const int n0 = (tl / gsz) * C::BN;
  const int nk = p.K / 128, ns = nk / 2;  // K blocks, stages

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.xq + (int64_t)m0 * p.ldx, (uint32_t)(C::BM * p.ldx));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.wq + (int64_t)n0 * p.ldw, (uint32_t)(C::BN * p.ldw));
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(p.xs + (int64_t)m0 * p.xs_m, (uint32_t)(((C::BM - 1) * p.xs_m + (nk - 1) + 1) * 4));
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(p.ws + (int64_t)(n0 / 128) * p.ws_n, (uint32_t)(((int64_t)nk - 1 + 1) * 4));
  // DMA: load q of a wave covers 8 rows of the stage's stacked A (or B) region: rows
  // 8 * (wave + 8 q) + lane / 8 of 256 (block 2s for rows < 128, block 2s+1 above);
  // row % 32 = 8 * (wave % 4) + lane / 8 for every q, so one chunk key per lane
  const int lrow = lane >> 3;
  const int dchunk = (lane & 7) ^ f8_key(8 * (wave & 3) + lrow);
  const int drow = lrow + 8 * wave;  // tile row of loads 0 and 2 (loads 1 and 3: + 64)
  const uint32_t a_voff = (uint32_t)(drow * p.ldx + 16 * dchunk);
  const uint32_t b_voff = (uint32_t)(drow * p.ldw + 16 * dchunk);
  const uint32_t a_r64 = (uint32_t)(64 * p.ldx), b_r64 = (uint32_t)(64 * p.ldw);
  const uint32_t x_voff = (uint32_t)(min(64 * wave + lane, C::BM - 1) * p.xs_m * 4);

  // load q of stage st (K blocks 2 st and 2 st + 1) into slot sl; the scale load is the
  // xs of rows 64 w .. 64 w + 63 for blocks 4 k .. 4 k + 3 (waves 0-1, even stages)
  // and otherwise the one copy of ws[nb, 4 k .. 4 k + 3] (identical bytes from every
  // wave that writes it)
  auto issue = [&](int sl, int st, int q) {
    const uint32_t kb0 = (uint32_t)(2 * st);
    if (q < 4) {  // A: q / 2 selects the K block, q % 2 the 64-row half
      buf_lds(ra, a_voff, (kb0 + (uint32_t)(q >> 1)) * 128u + (uint32_t)(q & 1) * a_r64,
              lds + sl * C::A_SLOT + (q >> 1) * C::A_BLK + (wave + 8 * (q & 1)) * 1024, 16);
    } else if (q < 8) {
      const int r = q - 4;
      buf_lds(rb, b_voff, (kb0 + (uint32_t)(r >> 1)) * 128u + (uint32_t)(r & 1) * b_r64,
              lds + C::B_BASE + sl * C::B_SLOT + (r >> 1) * C::B_BLK + (wave + 8 * (r & 1)) * 1024, 16);
    } else {
      const bool xload = wave < 2 && (st & 1) == 0;
      uint8_t* dst = xload ? lds + C::RING + ((st >> 1) & 1) * 2048 + wave * 1024 : lds + C::W_BASE + sl * 1024;
      buf_lds(xload ? rx : rw, xload ? x_voff : 0u, xload ? kb0 * 4u : (kb0 & ~3u) * 4u, dst, 16);
    }
  };

  // fragment reads: row lr of a 32-row block, K half h, 16-byte half e
  const int key = f8_key(lr);
  uint32_t ab[2][2], bbv[2][2];
  f32x16_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  f32x16_t part[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) part[1][r] = 0.0f;
  const f32x16_t zero = {};
  float sc_last = 0.0f, xsv_[MI] = {}, wsv_ = 0.0f;
  i32x8_t af[MI][2], bf[2][2];

  // prologue: stages 0 and 1 in flight, wait for stage 0
#pragma unroll
  for (int q = 0; q < LPS; ++q) issue(0, 0, q);
#pragma unroll
  for (int q = 0; q < LPS; ++q) issue(1, min(1, ns - 1), q);
  wait_vmcnt<LPS>();
  exec_barrier();
  const int rowA0 = 64 * wm, colB0 = 64 * wn;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int o = lr * 128 + (((4 * h + 2 * hh + e) ^ key) << 4);
      ab[h][e] = lds_offset_of(lds + grp * C::A_BLK + rowA0 * 128 + o);
      bbv[h][e] = lds_offset_of(lds + C::B_BASE + grp * C::B_BLK + colB0 * 128 + o);
    }
  const uint32_t xbase = lds_offset_of(lds + C::RING + (rowA0 + lr) * 16);
  const uint32_t wbase = lds_offset_of(lds + C::W_BASE);
  af[0][0] = lds_frag32_imm<0>(ab[0]);
  af[0][1] = lds_frag32_imm<0>(ab[1]);
  af[1][0] = lds_frag32_imm<32 * 128>(ab[0]);
  af[1][1] = lds_frag32_imm<32 * 128>(ab[1]);
  bf[0][0] = lds_frag32_imm<0>(bbv[0]);
  bf[0][1] = lds_frag32_imm<0>(bbv[1]);

  // one stage; SL: its slot (compile-time)
  auto stage = [&](int s, auto sl_tag) {
    constexpr int SL = decltype(sl_tag)::value;
    constexpr int CUR = SL * C::A_SLOT, NXT = (SL ^ 1) * C::A_SLOT;  // A_SLOT == B_SLOT
    const int s2 = min(s + 2, ns - 1);
    const int kb = 2 * s + grp;  // this wave's K block
    static_for<0, NT>([&](auto tt) {
      constexpr int t = decltype(tt)::value;
      constexpr int j = t / MI, i = t % MI;
      constexpr int bb = j & 1;
      if constexpr (t == TB) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<0>();
        exec_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      part[t & 1] = mma32_fp8(bf[bb][0], af[i][0], zero);
      __builtin_amdgcn_sched_barrier(0);
      {
        // promote the previous tile (t == 0: the last tile of the previous stage)
        constexpr int pi = t == 0 ? MI - 1 : (t - 1) % MI, pj = t == 0 ? NI - 1 : (t - 1) / MI;
        const float f = t == 0 ? sc_last : xsv_[pi] * wsv_;
        f32x16_t& a = acc[pi][pj];
#pragma unroll
        for (int r = 0; r < 16; ++r) a[r] = fmaf(part[(t + 1) & 1][r], f, a[r]);
      }
      __builtin_amdgcn_sched_barrier(0);
      part[t & 1] = mma32_fp8(bf[bb][1], af[i][1], part[t & 1]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (t == NT - 1) sc_last = xsv_[MI - 1] * wsv_;
      if constexpr (t == 0) {
        // this block's scales: xs[m, kb] from the ring, ws[nb, kb] from the slot's copy
        const uint32_t xo = xbase + (uint32_t)(((s >> 1) & 1) * 2048 + (kb & 3) * 4);
        xsv_[0] = lds_ldf(xo);
        xsv_[1] = lds_ldf(xo + 32 * 16);
        wsv_ = lds_ldf(wbase + (uint32_t)(SL * 1024 + (kb & 3) * 4));
      }
      if constexpr (i == 0 && j + 1 < NI) {  // B column j + 1 of this block
        bf[bb ^ 1][0] = lds_frag32_imm<CUR + 32 * 128 * (j + 1)>(bbv[0]);
        bf[bb ^ 1][1] = lds_frag32_imm<CUR + 32 * 128 * (j + 1)>(bbv[1]);
      }
      if constexpr (t == TB) {  // after the barrier: column 0 and A row tile 0 of the next stage
        bf[bb ^ 1][0] = lds_frag32_imm<NXT>(bbv[0]);
        bf[bb ^ 1][1] = lds_frag32_imm<NXT>(bbv[1]);
        af[0][0] = lds_frag32_imm<NXT>(ab[0]);
        af[0][1] = lds_frag32_imm<NXT>(ab[1]);
      }
      if constexpr (t == NT - 1) {
        af[1][0] = lds_frag32_imm<NXT + 32 * 128>(ab[0]);
        af[1][1] = lds_frag32_imm<NXT + 32 * 128>(ab[1]);
      }
      // loads of stage s + 2 into this slot, released at this stage's barrier
      if constexpr (t >= TB) {
        constexpr int u = t - TB;
        constexpr int q0 = u * LPS / NU, q1 = (u + 1) * LPS / NU;
#pragma unroll
        for (int q = q0; q < q1; ++q) issue(SL, s2, q);
      }
    });
  };
  for (int s = 0; s < ns; s += 2) {
    stage(s, std::integral_constant<int, 0>{});
    stage(s + 1, std::integral_constant<int, 1>{});
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[MI - 1][NI - 1][r] = fmaf(part[(NT - 1) & 1][r], sc_last, acc[MI - 1][NI - 1][r]);
  wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
  __syncthreads();

  // group 1 hands its partial sums to group 0 (same outputs, the other K blocks)
  float* xch = (float*)lds + wq * (64 * 64);
  if (grp == 1) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) xch[((i * NI + j) * 16 + r) * 64 + lane] = acc[i][j][r];
  }
  __syncthreads();
  using St = Stager<64, 64>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = (uint16_t*)(lds + C::XCH) + wq * (64 * 64);
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] + xch[((i * NI + j) * 16 + 4 * g + e) * 64 + lane];
          St::put(stg, out_row(i, lane), out_col(j, g, lane), u32x2_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3])});
        }
  }
  __syncthreads();
  if (grp == 0) {
    const int mw0 = m0 + rowA0, nw0 = n0 + colB0;
    const bool vec = p.vec_store != 0;
    St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
      store_row8(p.y + (int64_t)(mw0 + row) * p.ldy + nw0 + col, nw0 + col, p.N, vec, v);
    });
  }
}

int launch_fp8_ksplit(Fp8Params p, hipStream_t st) {
  p.tiles_m = p.M / KsCfg::BM;
  p.tiles_n = p.N / KsCfg::BN;
  hipLaunchKernelGGL(gemm_fp8_ksplit_kernel, dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(512), 0, st, p);
  return check_launch("gemm_fp8_ksplit_kernel");
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ------------------------------------------------------------------------------
// Skinny-M kernel (M <= 128): the product is bound by streaming W once from HBM, and
// a 256-row tile would leave most CUs idle (N / 128 workgroups).  A workgroup owns
// BN = 16*NB columns (32, or 16 when N / 32 workgroups would not cover the CUs) and
// every row of M (padded to MT); its NW waves split the K blocks (wave w takes blocks
// w, w+NW, ...), so the grid is N / BN workgroups that each stream their BN rows of W
// exactly once.
//
// Each wave has a private ring of S LDS stages (one K block each: MT rows of X, then
// BN rows of W, 128 bytes per row) filled by direct-to-LDS buffer loads in which one
// wave instruction covers 8 whole 128-byte rows (full cache lines: an MFMA-layout
// register load would split every line over two instructions, which measured 1.5x
// slower for the weight stream).  Waves share nothing, so a stage is consumed after
// the wave's own `s_waitcnt vmcnt` and no barrier is needed.  The block's scales
// travel in the same DMA stream (4-byte loads, one activation scale per lane and the
// weight scale), so the only memory waits in the loop are those vmcnt waits.  16-byte
// chunks are XOR swizzled by key(r) = (r ^ (r >> 3)) & 7 (see sk_key below for why this
// kernel keeps that key although its 16-row fragment reads take a 2-way bank conflict
// with it: rocprof's SQ_LDS_BANK_CONFLICT reads 0.76 conflict cycles per access cycle).
//
// v_mfma_f32_16x16x128_f8f6f4 with the W fragment first: D[n][m], lane l owns column
// m = l % 16 (one activation scale) and rows n = 4*(l/16) + i of a 16-column block
// (one weight-scale block, as 16 divides 128).  Each lane's 32 fragment bytes are the
// K chunks g and 4 + g (g = l / 16) of the block; only the pairing of the two
// operands' K slots matters for the product.  A block's MFMA starts from zero and is
// promoted with one FMA by xs[m,kb] * ws[nb,kb], every scale applied exactly once as
// in the reference oracle.  The per-wave partials are summed through LDS in wave
// order (fixed order: bit-reproducible) and written as bf16.
// ------------------------------------------------------------------------------
template <int MT, int NW, int S, int MODE = Q_BLOCK_FP8, int NB_ = 2>
struct SkinnyCfg {
  static constexpr int MT_ = MT, NW_ = NW, S_ = S, MODE_ = MODE;
  static constexpr bool ROW = MODE != Q_BLOCK_FP8;          // scales in the epilogue only
  static constexpr int NB = NB_, BN = 16 * NB, MB = MT / 16;  // 16-column blocks per workgroup
  static constexpr int XQ = MT / 8, WQ = BN / 8;          // 8-row DMA loads per block
  static constexpr int SQ = ROW ? 0 : (MT + 63) / 64;      // 64-row activation-scale loads
  static constexpr int LPB = XQ + WQ + (ROW ? 0 : SQ + 1); // DMA instructions per block
  static constexpr int XS_OFF = (MT + BN) * 128;           // xs[m] of the block (fp32)
  static constexpr int WS_OFF = XS_OFF + SQ * 256;         // ws of the block (64 copies)
  static constexpr int STAGE = WS_OFF + (ROW ? 0 : 256);   // bytes
  static constexpr int RING = NW * S * STAGE;
  static constexpr int BNP = BN + 4;                       // padded fp32 row of the reduction
  static constexpr int RED = NW * MT * BNP * 4;
  static constexpr int LDS = RING > RED ? RING : RED;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(S >= 1 && S <= 3 && LPB * (S - 1) <= 63, "vmcnt range");
};

// Fragment reads are the 16-row shape (lane (r, g) reads row r of a 16-row group), which
// this 32-row key serves with a 2-way bank conflict.  The conflict-free 16-row key swz16
// was measured in the same process and is kept out: M=128 7% slower, M=96 4% faster,
// M=16..64 within 3% -- the kernel's time is its L2-to-LDS operand stream, not LDS reads.
__device__ __forceinline__ int sk_key(int r) { return (r ^ (r >> 3)) & 7; }

template <typename C>
__global__ void __launch_bounds__(C::NW_ * 64)
    gemm_fp8_skinny_kernel(const Fp8Params p) {
  constexpr int MT = C::MT_, NW = C::NW_, S = C::S_, MB = C::MB, NB = C::NB, BN = C::BN;
  constexpr int XQ = C::XQ, WQ = C::WQ, SQ = C::SQ, LPB = C::LPB, STAGE = C::STAGE, BNP = C::BNP;
  constexpr bool ROW = C::ROW, I8 = C::MODE_ == Q_ROW_I8;
  using AccT = std::conditional_t<I8, i32x4_t, f32x4_t>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int n0 = (int)blockIdx.x * BN;
  const int nk = p.K / 128;
  const int cnt = nk > wave ? (nk - wave + NW - 1) / NW : 0;  // K blocks of this wave

  // buffer resources: X rows [0, M), this workgroup's BN rows of W
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.xq, (uint32_t)((int64_t)(p.M - 1) * p.ldx + p.K));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.wq + (int64_t)n0 * p.ldw, (uint32_t)((BN - 1) * p.ldw + p.K));
  // DMA load q covers LDS rows 8q .. 8q+7; lane l fetches row 8q + l/8, logical chunk
  // (l % 8) ^ key(row) into position l % 8
  uint32_t xoff[XQ], woff[WQ];
#pragma unroll
  for (int q = 0; q < XQ; ++q) {
    const int row = 8 * q + (lane >> 3);
    xoff[q] = (uint32_t)((int64_t)min(row, p.M - 1) * p.ldx + 16 * ((lane & 7) ^ sk_key(row)));
  }
#pragma unroll
  for (int q = 0; q < WQ; ++q) {
    const int row = 8 * q + (lane >> 3);
    woff[q] = (uint32_t)((int64_t)row * p.ldw + 16 * ((lane & 7) ^ sk_key(row)));
  }
  const __amdgpu_buffer_rsrc_t rxs =
      make_rsrc(p.xs, (uint32_t)(((int64_t)(p.M - 1) * p.xs_m + (int64_t)(nk - 1) * p.xs_k + 1) * 4));
  const __amdgpu_buffer_rsrc_t rws = make_rsrc(
      p.ws, (uint32_t)(((int64_t)(p.N / 128 - 1) * p.ws_n + (int64_t)(nk - 1) * p.ws_k + 1) * 4));
  uint32_t xsoff[SQ > 0 ? SQ : 1];
#pragma unroll
  for (int q = 0; q < SQ; ++q) xsoff[q] = (uint32_t)((int64_t)min(64 * q + lane, p.M - 1) * p.xs_m * 4);
  const uint32_t ws_base = (uint32_t)((int64_t)(n0 / 128) * p.ws_n * 4);
  uint8_t* ring = lds + wave * (S * STAGE);

  // fragment read offsets inside a stage: row R + r, chunks g and 4 + g
  const int k0 = sk_key(r);  // key(R + r) = (key(r) ^ (R / 8)) & 7 for R % 16 == 0

  // issue the loads of block j into stage slot s (DMA operands, then scales)
  auto issue = [&](int s, int j) {
    const uint32_t ko = (uint32_t)(wave + NW * j) * 128u;
    uint8_t* st = ring + s * STAGE;
#pragma unroll
    for (int q = 0; q < XQ; ++q) buf_lds(rx, xoff[q], ko, st + q * 1024, 16);
#pragma unroll
    for (int q = 0; q < WQ; ++q) buf_lds<kCpolNT>(rw, woff[q], ko, st + MT * 128 + q * 1024, 16);  // W: read once
    if constexpr (!ROW) {
      const uint32_t kb = (uint32_t)(wave + NW * j);
#pragma unroll
      for (int q = 0; q < SQ; ++q) buf_lds(rxs, xsoff[q], kb * (uint32_t)(p.xs_k * 4), st + C::XS_OFF + q * 256, 4);
      buf_lds(rws, 0u, ws_base + kb * (uint32_t)(p.ws_k * 4), st + C::WS_OFF, 4);
    }
  };

  AccT acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = AccT{0, 0, 0, 0};

#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < cnt) issue(s, s);
  for (int j0 = 0; j0 < cnt; j0 += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int j = j0 + s;
      if (j < cnt) {
        // blocks issued after j: min(S - 1, cnt - 1 - j)
        const int later = min(S - 1, cnt - 1 - j);
        if (S >= 3 && later >= 2) wait_vmcnt<(S >= 3 ? 2 * LPB : 0)>();
        else if (S >= 2 && later >= 1) wait_vmcnt<(S >= 2 ? LPB : 0)>();
        else wait_vmcnt<0>();
        const uint8_t* st = ring + s * STAGE;
        i32x8_t xf[MB], wf[NB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const uint8_t* row = st + (mb * 16 + r) * 128;
          const int key = (k0 ^ (2 * mb)) & 7;
          const u32x4_t lo = *(const u32x4_t*)(row + ((g ^ key) << 4));
          const u32x4_t hi = *(const u32x4_t*)(row + (((4 + g) ^ key) << 4));
          xf[mb] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint8_t* row = st + (MT + nb * 16 + r) * 128;
          const int key = (k0 ^ (2 * nb)) & 7;
          const u32x4_t lo = *(const u32x4_t*)(row + ((g ^ key) << 4));
          const u32x4_t hi = *(const u32x4_t*)(row + (((4 + g) ^ key) << 4));
          wf[nb] = i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        }
        float sc[MB];
        if constexpr (!ROW) {
          const float wsv = *(const float*)(st + C::WS_OFF);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) sc[mb] = *(const float*)(st + C::XS_OFF + (mb * 16 + r) * 4) * wsv;
        }
        // the slot is free once its fragments are in registers
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (j + S < cnt) issue(s, j + S);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            if constexpr (I8) {
              // int8 16x16x64: the 16-byte chunks g and 4 + g are two K slices
              const i32x8_t w = wf[nb], x = xf[mb];
              acc[mb][nb] = mma16_i8(u32x4_t{(uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]},
                                     u32x4_t{(uint32_t)x[0], (uint32_t)x[1], (uint32_t)x[2], (uint32_t)x[3]},
                                     acc[mb][nb]);
              acc[mb][nb] = mma16_i8(u32x4_t{(uint32_t)w[4], (uint32_t)w[5], (uint32_t)w[6], (uint32_t)w[7]},
                                     u32x4_t{(uint32_t)x[4], (uint32_t)x[5], (uint32_t)x[6], (uint32_t)x[7]},
                                     acc[mb][nb]);
            } else if constexpr (ROW) {
              acc[mb][nb] = mma16_fp8(wf[nb], xf[mb], acc[mb][nb]);
            } else {
              const f32x4_t part = mma16_fp8(wf[nb], xf[mb], f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[mb][nb][i] = fmaf(part[i], sc[mb], acc[mb][nb][i]);
            }
          }
      }
    }
  }

  // ---- cross-wave reduction: red[wave][m][n] over the (now idle) ring, fixed-order sum ----
  wait_vmcnt<0>();
  __syncthreads();
  float* red = (float*)lds;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      *(f32x4_t*)(red + (wave * MT + mb * 16 + r) * BNP + nb * 16 + 4 * g) =
          f32x4_t{(float)acc[mb][nb][0], (float)acc[mb][nb][1], (float)acc[mb][nb][2], (float)acc[mb][nb][3]};
  __syncthreads();
  constexpr int ITEMS = MT * BN / 8;  // 8 consecutive columns per item
  const bool vec = p.vec_store != 0;
  for (int it = tid; it < ITEMS; it += NW * 64) {
    const int m = it / (BN / 8), c8 = (it % (BN / 8)) * 8;
    if (m >= p.M) continue;
    float sum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const f32x4_t a = *(const f32x4_t*)(red + (w * MT + m) * BNP + c8);
      const f32x4_t b = *(const f32x4_t*)(red + (w * MT + m) * BNP + c8 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sum[e] += a[e];
        sum[e + 4] += b[e];
      }
    }
    const int gn = n0 + c8;
    if constexpr (ROW) {
      const float xv = p.xs[(int64_t)m * p.xs_m];
#pragma unroll
      for (int e = 0; e < 8; ++e) sum[e] = sum[e] * xv * p.ws[(int64_t)(gn + e) * p.ws_n];
    }
    using Op = MfmaOp<BF16>;
    const u32x4_t v{Op::pack2(sum[0], sum[1]), Op::pack2(sum[2], sum[3]), Op::pack2(sum[4], sum[5]),
                    Op::pack2(sum[6], sum[7])};
    store_row8(p.y + (int64_t)m * p.ldy + gn, gn, p.N, vec, v);
  }
}

template <typename C>
int launch_fp8_skinny(const Fp8Params& p, hipStream_t st) {
  const dim3 grid((unsigned)(p.N / C::BN)), block(C::NW_ * 64);
  hipLaunchKernelGGL((gemm_fp8_skinny_kernel<C>), grid, block, 0, st, p);
  return check_launch("gemm_fp8_skinny_kernel");
}

}  // namespace
}  // namespace kore

extern "C" int kore_gemm_a8w8_blockscale(const void* xq, int64_t ldx, const void* wq, int64_t ldw, const float* xs,
                                         int64_t xs_m, int64_t xs_k, const float* ws, int64_t ws_n, int64_t ws_k,
                                         void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  using namespace kore;
  if (!xq || !wq || !xs || !ws || !y) return set_error(KORE_EINVAL, "gemm_a8w8_blockscale: null pointer");
  if (M <= 0 || N <= 0 || K <= 0) return set_error(KORE_EINVAL, "gemm_a8w8_blockscale: M, N, K must be >= 1");
  if (K % 128 != 0 || N % 128 != 0)
    return set_error(KORE_EINVAL, "gemm_a8w8_blockscale: K and N must be multiples of 128 (K=%lld N=%lld)",
                     (long long)K, (long long)N);
  if (ldx < K || ldw < K || ldy < N) return set_error(KORE_EINVAL, "gemm_a8w8_blockscale: row stride smaller than row");
  if (ldx % 16 != 0 || ldw % 16 != 0 || !aligned16(xq) || !aligned16(wq))
    return set_error(KORE_EINVAL, "gemm_a8w8_blockscale: xq/wq rows must be 16-byte aligned");
  if (M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31))
    return set_error(KORE_EUNSUPPORTED, "gemm_a8w8_blockscale: dimension >= 2^31");
  constexpr int BM = 256, BN = 128;
  Fp8Params p{};
  p.xq = (const uint8_t*)xq;
  p.wq = (const uint8_t*)wq;
  p.xs = xs;
  p.ws = ws;
  p.y = (uint16_t*)y;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.xs_m = xs_m;
  p.xs_k = xs_k;
  p.ws_n = ws_n;
  p.ws_k = ws_k;
  p.tiles_m = (int)((M + BM - 1) / BM);
  p.tiles_n = (int)(N / BN);
  p.vec_store = (ldy % 8 == 0) && aligned16(y);
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  // the pipelined kernels address each tile through 32-bit buffer offsets
  const bool pipe_ok = 256 * ldx + K < (1ll << 31) && 256 * ldw + K < (1ll << 31) &&
                       (M * xs_m + K / 128 * xs_k) * 4 < (1ll << 31) && (N / 128 * ws_n + K / 128 * ws_k) * 4 < (1ll << 31);
  // the skinny kernel addresses X and a 32-row slab of W through 32-bit buffer offsets
  const bool skinny_ok = 128 * ldx + K < (1ll << 31) && 32 * ldw + K < (1ll << 31);
  if (M <= 128 && skinny_ok) {
    // weight streaming: every CU reads its own 32 columns of W once
    hipStream_t st = (hipStream_t)stream;
    if (M <= 16) return launch_fp8_skinny<SkinnyCfg<16, 8, 3>>(p, st);
    if (M <= 32) return launch_fp8_skinny<SkinnyCfg<32, 8, 2>>(p, st);
    if (M <= 64) return launch_fp8_skinny<SkinnyCfg<64, 4, 3>>(p, st);
    return launch_fp8_skinny<SkinnyCfg<128, 2, 2>>(p, st);  // 2 stages: 16.8 us at M=128 (3: 19.7)
  }
  if (pipe_ok) {
    // four K steps of scales per 16-byte load when scale rows are contiguous, 16-byte
    // aligned and K/128 is a multiple of 4 (so no load runs past a row)
    const bool xs4 = xs_k == 1 && xs_m % 4 == 0 && aligned16(xs) && ws_k == 1 && ws_n % 4 == 0 && aligned16(ws) &&
                     (K / 128) % 4 == 0;
    hipStream_t st = (hipStream_t)stream;
    // 256x256 tiles halve LDS and L2 traffic per MFMA but need enough of them to
    // occupy the 256 CUs; then 256x128 tiles (three LDS slots); with fewer than that,
    // 128x128 tiles on 4 waves (four slots) double the tile count again -- unless
    // those would need a second round on the CUs (M=768, N=7168: 128x128 41.0 us,
    // 256x128 28.2 us)
    const int64_t tiles256 = (M + 255) / 256 * (N / 256);
    const int64_t tiles256x128 = (M + 255) / 256 * (N / 128);
    const int64_t tiles128 = (M + 127) / 128 * (N / 128);
    // 256 x 224 tiles when they take fewer CU-rounds of tile area than 256 x 256 ones
    // (2048 x 7168: 256 tiles, one per CU, against 224 tiles on 256 CUs)
    const int64_t cus = device_cus();
    if (xs4 && M % 256 == 0 && N % 224 == 0 && (K / 128) % 4 == 0) {
      const int64_t t224 = (M / 256) * (N / 224);
      const int64_t cost224 = (t224 + cus - 1) / cus * 224;
      const int64_t cost256 = N % 256 == 0 ? (tiles256 + cus - 1) / cus * 256 : INT64_MAX;
      if (t224 >= cus / 2 && cost224 < cost256) return launch_fp8_wide(p, st);
    }
    if (N % 256 == 0 && tiles256 >= 192) {
      return xs4 ? launch_fp8_pipe<F8Cfg<256, 256, 8, 2, true>>(p, st)
                 : launch_fp8_pipe<F8Cfg<256, 256, 8, 2, false>>(p, st);
    }
    if (tiles256x128 >= 192 || tiles128 > cus) {
      return xs4 ? launch_fp8_pipe<F8Cfg<256, 128, 8, 3, true>>(p, st)
                 : launch_fp8_pipe<F8Cfg<256, 128, 8, 3, false>>(p, st);
    }
    // 128 x 128 tiles: with contiguous scales and at least three quarters of the CUs
    // covered, the K-split 8-wave kernel (two waves per SIMD) instead of the 4-wave one.
    // Same process: 512 x 7168 x 4096 24.3 -> 23.4 us, 384 x 7168 x 4096 (168 tiles) 23.5
    // -> 22.7 us, but 640 x 4096 x 4096 (160 tiles) 21.5 -> 23.1 us.  Both tiles take in
    // 64 bytes of operands per CU per MFMA-clock at full rate, above what a CU sustains
    // (about 40 B/clk from L2), so neither reaches the MFMA bound.
    if (xs4 && M % 128 == 0 && tiles128 >= 3 * cus / 4) return launch_fp8_ksplit(p, st);
    return xs4 ? launch_fp8_pipe<F8Cfg<128, 128, 4, 4, true>>(p, st)
               : launch_fp8_pipe<F8Cfg<128, 128, 4, 4, false>>(p, st);
  }
  hipLaunchKernelGGL((gemm_fp8_bs_kernel<BM, BN>), dim3((unsigned)blocks), dim3(kEngineThreads), 0,
                     (hipStream_t)stream, p);
  return check_launch("gemm_fp8_bs_kernel");
}

// ==============================================================================
// a8w8 GEMM with per-row activation and per-column weight scales (fp8 e4m3 or
// int8): Y[M,N] = bf16((sum_k xq[m,k] * wq[n,k]) * xs[m] * ws[n]).  The tiled and
// skinny kernels above run it in their row-scale modes (the K loop accumulates in
// the MFMA registers, scales are applied once in the epilogue); anything they cannot
// take (a K not a multiple of 128, strided or unaligned rows) runs a generic kernel.
// ==============================================================================
namespace kore {
namespace {

// OCP e4m3 byte -> fp32 from the format: sign bit 7, exponent bits 6..3 (bias 7),
// mantissa bits 2..0; exponent 0 is subnormal (m * 2^-9); 0x7f / 0xff are NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  const float mag = e == 0 ? (float)m * 0x1p-9f : __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  const float v = (e == 0xfu && m == 7u) ? __builtin_nanf("") : mag;
  return (c & 0x80u) ? -v : v;
}

struct A8GenericParams {
  const uint8_t* xq;
  const uint8_t* wq;
  const float* xs;
  const float* ws;
  uint16_t* y;
  int M, N, K;
  int64_t ldx_m, ldx_k, ldw_n, ldw_k, xs_st, ws_st, ldy;
};

// 64x64 output tile per workgroup (4x4 per thread), 32-wide K steps staged through
// LDS with bounds checks on every element.  int8 accumulates exactly in int32.
template <bool I8>
__global__ void __launch_bounds__(256) gemm_a8w8_generic_kernel(const A8GenericParams p) {
  using V = std::conditional_t<I8, int, float>;
  __shared__ V As[64][33];
  __shared__ V Bs[64][33];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = (int)blockIdx.y * 64, n0 = (int)blockIdx.x * 64;
  V acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0;
  auto decode = [](uint8_t c) -> V {
    if constexpr (I8) return (int)(int8_t)c;
    else return e4m3_to_f32(c);
  };
  for (int k0 = 0; k0 < p.K; k0 += 32) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int idx = tid + 256 * q, r = idx >> 5, kk = idx & 31, k = k0 + kk;
      const int m = m0 + r, n = n0 + r;
      As[r][kk] = (m < p.M && k < p.K) ? decode(p.xq[(int64_t)m * p.ldx_m + (int64_t)k * p.ldx_k]) : (V)0;
      Bs[r][kk] = (n < p.N && k < p.K) ? decode(p.wq[(int64_t)n * p.ldw_n + (int64_t)k * p.ldw_k]) : (V)0;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      V a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[ty * 4 + i][kk];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[tx * 4 + j][kk];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
  using Op = MfmaOp<BF16>;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= p.M) continue;
    const float xv = p.xs[(int64_t)m * p.xs_st];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n < p.N) {
        const float v = (float)acc[i][j] * xv * p.ws[(int64_t)n * p.ws_st];
        p.y[(int64_t)m * p.ldy + n] = (uint16_t)(Op::pack2(v, 0.0f) & 0xffffu);
      }
    }
  }
}

// a8w8 (per-token / per-channel scales) on the dense 4-wave tile (BufPipeEngine, as the bf16
// GEMM): 8-bit rows are 128-byte stage rows like the 16-bit ones (K = 128 per stage) and the
// accumulators stay in place in AGPRs.  int8: 16x16x64 MFMAs on the same 16-byte chunks as
// the 16x16x32 bf16 ones (mainloop16), int32 accumulators; fp8: 16x16x128 MFMAs on both
// chunks of a stage (mainloop_f8).  Epilogue as the row-scale pipe kernel: float(acc) *
// xs[m] * ws[n], one bf16 rounding.  Requires N % 256 == 0, K % 128 == 0, 16-byte aligned rows.
template <int MODE>
__global__ void __launch_bounds__(256) gemm_a8w8_buf_kernel(const Fp8Params p) {
  constexpr bool I8 = MODE == Q_ROW_I8;
  using E = BufPipeEngine<std::conditional_t<I8, INT8, FP8>, 256, 256, 2, 2, 1, B_KC, kCpolDefault, true, A_KC>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / E::WN, wn = wave % E::WN;
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int width = kFp8GroupM * p.tiles_n;
  const int grp = bid / width;
  const int first_m = grp * kFp8GroupM;
  const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
  const int tl = bid - grp * width;
  const int m0 = (first_m + tl % gsz) * 256, n0 = (tl / gsz) * 256;
  const int rows_a = min(256, p.M - m0);
  E eng;
  eng.ra = make_rsrc(p.xq + (int64_t)m0 * p.ldx, (uint32_t)((int64_t)(rows_a - 1) * p.ldx + p.K));
#pragma unroll
  for (int j = 0; j < E::AJ; ++j) {
    const int r = E::a_row(wave, lane, j);
    eng.a_voff[j] = (uint32_t)((int64_t)min(r, rows_a - 1) * p.ldx + 16 * E::chunk(r, lane));
  }
  eng.rb = make_rsrc(p.wq + (int64_t)n0 * p.ldw, (uint32_t)(255 * p.ldw + p.K));
#pragma unroll
  for (int j = 0; j < E::BJ; ++j) {
    const int r = E::b_row(wave, lane, j);
    eng.b_voff[j] = (uint32_t)((int64_t)r * p.ldw + 16 * E::chunk(r, lane));
  }
  f32x4_t acc[MI][NI][4];
  E::zero16(acc);
  if constexpr (I8) eng.mainloop16(lds, p.K / 2, acc);  // K in 16-bit units: 64 per 128-byte stage
  else eng.mainloop_f8(lds, p.K / 2, acc);

  using St = Stager<E::WROWS, E::WCOLS>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = lds + wave * (E::WROWS * E::WCOLS);
  const int mw0 = m0 + wm * E::WROWS, nw0 = n0 + wn * E::WCOLS;
  // the lane's scales, loaded together before the tile is converted: xs of its rows (MI
  // blocks x two 16-row halves), ws of its columns (NI blocks x two 16-column halves x 4).
  // Loaded per (j, g, i) inside the conversion loops instead (127 loads, each waited for
  // near its use), same process, bit-equal: fp8 4096^3 56.0 -> 52.0 us, 8192 x 4096 x
  // 4096 109.4 -> 101.9 us, cold 4096^3 60.9 -> 55.3 us; int8 4096^3 55.7 -> 54.9 us.
  float xrow[MI][2], wcol[NI][2][4];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      xrow[i][h] = p.xs[(int64_t)min(mw0 + acc_row<true>(i, 2 * h, lane), p.M - 1) * p.xs_m];
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) wcol[j][h][e] = p.ws[(int64_t)(nw0 + acc_col<true>(j, h, lane) + e) * p.ws_n];
#pragma unroll
  for (int j = 0; j < NI; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = acc_col<true>(j, g, lane);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int ml = acc_row<true>(i, g, lane);
        const float xr = xrow[i][g >> 1];
        float v[4];
        if constexpr (I8) {
          // reinterpret the whole 4-register tuple (casting single extracted elements of
          // an inline-asm AGPR result miscompiled: every element read the first register)
          const i32x4_t ai = __builtin_bit_cast(i32x4_t, acc[i][j][g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (float)ai[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][g][e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] * xr * wcol[j][g & 1][e];
        St::put(stg, ml, nl, u32x2_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3])});
      }
    }
  __syncthreads();
  const bool vec = p.vec_store != 0;
  St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
    const int gm = mw0 + row, gn = nw0 + col;
    if (gm < p.M) store_row8(p.y + (int64_t)gm * p.ldy + gn, gn, p.N, vec, v);
  });
}

template <int MODE>
int launch_a8w8_buf(Fp8Params p, hipStream_t st) {
  p.tiles_m = (p.M + 255) / 256;
  p.tiles_n = p.N / 256;
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm_a8w8: grid too large");
  hipLaunchKernelGGL((gemm_a8w8_buf_kernel<MODE>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return check_launch("gemm_a8w8_buf_kernel");
}

template <int MODE>
int launch_a8w8(const Fp8Params& p0, bool skinny, hipStream_t st) {
  Fp8Params p = p0;
  if (skinny) {
    // 16-column workgroups when 32-column ones would leave CUs idle (N < 8192)
    if (p.N / 32 < 256) {
      if (p.M <= 16) return launch_fp8_skinny<SkinnyCfg<16, 8, 3, MODE, 1>>(p, st);
      if (p.M <= 32) return launch_fp8_skinny<SkinnyCfg<32, 8, 3, MODE, 1>>(p, st);
      if (p.M <= 64) return launch_fp8_skinny<SkinnyCfg<64, 8, 2, MODE, 1>>(p, st);
      return launch_fp8_skinny<SkinnyCfg<128, 4, 2, MODE, 1>>(p, st);
    }
    if (p.M <= 16) return launch_fp8_skinny<SkinnyCfg<16, 8, 3, MODE>>(p, st);
    if (p.M <= 32) return launch_fp8_skinny<SkinnyCfg<32, 8, 2, MODE>>(p, st);
    if (p.M <= 64) return launch_fp8_skinny<SkinnyCfg<64, 4, 3, MODE>>(p, st);
    return launch_fp8_skinny<SkinnyCfg<128, 4, 2, MODE>>(p, st);
  }
  // tile choice as for the block-scale kernels
  const int64_t tiles256 = (int64_t)(p.M + 255) / 256 * (p.N / 256);
  const int64_t tiles256x128 = (int64_t)(p.M + 255) / 256 * (p.N / 128);
  const int64_t tiles128 = (int64_t)(p.M + 127) / 128 * (p.N / 128);
  // the dense 4-wave tile with the accumulators in AGPRs, where K is deep enough to carry
  // its prologue and its 4-wave epilogue (same process, bit-equal, against the 8-wave pipe
  // kernel).  int8: 4096^3 65.6 -> 56.6 us, 8192 x 4096 x 4096 128.4 -> 112.1 us,
  // 2048 x 7168 x 4096 58.5 -> 50.7 us, 4096 x 8192 x 2048 73.5 -> 68.3 us, 8192^2 x 1024
  // 83.1 -> 78.6 us, 4096^2 x 1024 23.2 -> 22.5 us.  fp8: 4096^3 55.6 -> 52.0 us, 4096^2 x
  // 3072 44.4 -> 41.0 us, 4096 x 8192 x 2048 61.8 -> 57.7 us, 4096^2 x 2048 32.7 -> 30.9 us;
  // at K = 1024 a tie (4096^2 21.4 either way, 3072 x 4096 19.3 against 19.6 us).
  const int kmin_buf = MODE == Q_ROW_I8 ? 1024 : 2048;
  if (p.N % 256 == 0 && tiles256 >= 192 && p.K >= kmin_buf) return launch_a8w8_buf<MODE>(p, st);
  if (p.N % 256 == 0 && tiles256 >= 192) return launch_fp8_pipe<F8Cfg<256, 256, 8, 2, false, MODE>>(p, st);
  if (tiles256x128 >= 192 || tiles128 > device_cus())
    return launch_fp8_pipe<F8Cfg<256, 128, 8, 3, false, MODE>>(p, st);
  return launch_fp8_pipe<F8Cfg<128, 128, 4, 4, false, MODE>>(p, st);
}

template <typename C>
int launch_fp8_grouped(Fp8Params p, int mblocks, hipStream_t st) {
  p.tiles_m = mblocks;
  p.tiles_n = p.N / C::BN;
  const dim3 grid((unsigned)((int64_t)p.tiles_m * p.tiles_n)), block(C::NW * 64);
  hipLaunchKernelGGL((gemm_fp8_pipe_kernel<C, false, true>), grid, block, 0, st, p);
  return check_launch("gemm_fp8_pipe_kernel(grouped)");
}

}  // namespace

int launch_grouped_a8w8(const GroupedA8Args& a, hipStream_t st) {
  Fp8Params p{};
  p.xq = (const uint8_t*)a.xq;
  p.wq = (const uint8_t*)a.wq;
  p.xs = a.xs;
  p.ws = a.ws;
  p.y = (uint16_t*)a.y;
  p.M = (int)a.M;
  p.N = (int)a.N;
  p.K = (int)a.K;
  p.ldx = a.ldx;
  p.ldw = a.K;
  p.ldy = a.ldy;
  p.xs_m = a.xs_stride;
  p.ws_n = 1;
  p.vec_store = a.ldy % 8 == 0 && ((uintptr_t)a.y & 15u) == 0;
  p.sorted = a.sorted;
  p.block_expert = a.block_expert;
  p.w_estride = a.N * a.K;
  p.ws_estride = a.N;
  const int mb = (int)(a.capacity / a.block_rows);
  if (a.block_rows == 256) return launch_fp8_grouped<F8Cfg<256, 256, 8, 2, false, Q_ROW_FP8>>(p, mb, st);
  if (a.block_rows == 128) return launch_fp8_grouped<F8Cfg<128, 128, 4, 4, false, Q_ROW_FP8>>(p, mb, st);
  return set_error(KORE_EINVAL, "grouped a8w8: block rows %d (128 or 256)", a.block_rows);
}

}  // namespace kore

extern "C" int kore_gemm_a8w8(int qtype, const void* xq, int64_t ldx_m, int64_t ldx_k, const void* wq, int64_t ldw_n,
                              int64_t ldw_k, const float* xs, int64_t xs_stride, const float* ws, int64_t ws_stride,
                              void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream) {
  using namespace kore;
  if (!xq || !wq || !xs || !ws || !y) return set_error(KORE_EINVAL, "gemm_a8w8: null pointer");
  if (qtype != KORE_Q_FP8 && qtype != KORE_Q_INT8) return set_error(KORE_EINVAL, "gemm_a8w8: unknown qtype %d", qtype);
  if (M <= 0 || N <= 0 || K <= 0) return set_error(KORE_EINVAL, "gemm_a8w8: M, N, K must be >= 1");
  if (ldy < N) return set_error(KORE_EINVAL, "gemm_a8w8: ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
  if (M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31))
    return set_error(KORE_EUNSUPPORTED, "gemm_a8w8: dimension >= 2^31");
  hipStream_t st = (hipStream_t)stream;
  const bool fast = ldx_k == 1 && ldw_k == 1 && K % 128 == 0 && N % 128 == 0 && ldx_m % 16 == 0 &&
                    ldw_n % 16 == 0 && aligned16(xq) && aligned16(wq) && 256 * ldx_m + K < (1ll << 31) &&
                    256 * ldw_n + K < (1ll << 31) && ldx_m >= K && ldw_n >= K;
  if (fast) {
    Fp8Params p{};
    p.xq = (const uint8_t*)xq;
    p.wq = (const uint8_t*)wq;
    p.xs = xs;
    p.ws = ws;
    p.y = (uint16_t*)y;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.ldx = ldx_m;
    p.ldw = ldw_n;
    p.ldy = ldy;
    p.xs_m = xs_stride;
    p.xs_k = 0;
    p.ws_n = ws_stride;
    p.ws_k = 0;
    p.tiles_m = p.tiles_n = 0;
    p.vec_store = (ldy % 8 == 0) && aligned16(y);
    const bool skinny = M <= 128;
    return qtype == KORE_Q_FP8 ? launch_a8w8<Q_ROW_FP8>(p, skinny, st) : launch_a8w8<Q_ROW_I8>(p, skinny, st);
  }
  A8GenericParams g{(const uint8_t*)xq, (const uint8_t*)wq, xs, ws, (uint16_t*)y, (int)M, (int)N, (int)K,
                    ldx_m, ldx_k, ldw_n, ldw_k, xs_stride, ws_stride, ldy};
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  if (grid.y > 65535) return set_error(KORE_EUNSUPPORTED, "gemm_a8w8: M too large for the generic kernel");
  if (qtype == KORE_Q_FP8) hipLaunchKernelGGL(gemm_a8w8_generic_kernel<false>, grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL(gemm_a8w8_generic_kernel<true>, grid, dim3(256), 0, st, g);
  return check_launch("gemm_a8w8_generic_kernel");
}
