// Fused top-k MoE with SiLU gated MLP (bf16) for gfx950.
//
// Pipeline (all on the caller's stream, no host synchronisation):
//  1. moe_align_chunk_kernel: expert histogram -> block-padded offsets -> stable,
//     expert-sorted slot list (slot s = t*topk + k) and the expert of every
//     BM-row block.  One workgroup per 256 slots, each computing the histogram it
//     needs itself; deterministic and ascending in slot order inside each expert.
//  2. moe_gateup_kernel: for every BM-row block of sorted slots (one expert e) and
//     every 128/BN-wide column tile of the intermediate dim, A rows are the gathered
//     tokens hidden[s/topk] and B rows are w1[e] gate and up rows interleaved so that
//     every wave owns gate and up for the same columns; the epilogue computes
//     h = silu(gate) * up in fp32 and writes it as two bf16 planes in sorted order,
//     Hhi = bf16(h) and Hlo = bf16(h - Hhi), so h survives to ~2^-17 relative.
//  3. moe_down_kernel: Y = (Hhi + Hlo)[block] @ w2[e]^T -- both planes multiply the
//     same w2 fragments (two MFMAs per fragment, w2 streamed once); the epilogue
//     scales each row by its router weight and writes fp32 rows Yw[slot, :] (padding
//     slots are skipped).
//  4. moe_combine_kernel: out[t] = bf16(sum_k Yw[t*topk + k]) in fixed k order over
//     the slots whose id is in [0, E): no atomics, bit-reproducible.
// Grids are sized for the worst case (every expert adds < 1 block of padding) and
// blocks past the real end exit after reading offsets[E].  Up to 128 slots per expert
// (decode and small batches) blocks are 32 or 128 rows and both GEMMs stream the expert
// weights once per block on a direct-to-LDS ring with non-temporal loads
// (moe_decode_kernel); padding rows of a block are zero-filled by the buffer range
// check at no memory cost.  Beyond 128 slots per expert: 256-row prefill tiles.
#include "../../include/kore_amd.h"
#include "kore_common.hpp"
#include "tile_engine.hpp"

#include <algorithm>

namespace kore {
namespace {

// ------------------------------------------------------------------------------
// 1. sort / align
// ------------------------------------------------------------------------------
constexpr int kAlignMaxE = 1024;

// Chunked sort / align: workgroup g owns R consecutive 256-slot sub-chunks of the slot
// list (R = 1 up to 65536 slots, so at most 256 workgroups), with no communication
// between workgroups.  Every workgroup reads all the ids (S ints, L2-resident) and
// builds in LDS the full expert histogram and the count of each expert in the slots
// before its range; a block-wide scan of the padded counts gives the expert starts.
// Slot c + t of a sub-chunk then goes to
//   start[e] + (slots of e before the sub-chunk) + (slots of e before it in the sub-chunk),
// the last term from per-wave expert counts and a scan of the wave's ids, so the order
// inside an expert is ascending slot order, as in the oracle.  The workgroups split the padding
// sentinels, the tail past the last expert and the block owners between them;
// workgroup 0 writes the offsets.  With zrows set (the top-1 grouped GEMMs, slot = output
// row) a slot whose id is outside [0, E) zeroes its output row (zcols bf16 values, a
// multiple of 8, 16-byte aligned rows), so the caller need not clear the whole output.
constexpr int kChunk = 256;

__global__ void __launch_bounds__(kChunk)
    moe_align_chunk_kernel(const int32_t* __restrict__ ids, int S, int E, int block, int R,
                           int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                           int32_t* __restrict__ block_expert, int cap, uint16_t* __restrict__ zrows,
                           int64_t ldz, int zcols) {
  __shared__ int hist[kAlignMaxE], pre[kAlignMaxE], base[kAlignMaxE];
  __shared__ int wcnt[kChunk / 64][kAlignMaxE];  // per-wave expert counts of a sub-chunk
  __shared__ __attribute__((aligned(16))) int cid[kChunk];
  __shared__ int wsum[kChunk / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = (int)blockIdx.x, G = (int)gridDim.x;
  const int first = g * R;  // first sub-chunk of this workgroup
  // this thread's slot of the first sub-chunk, loaded with the first histogram batch
  int my_e0 = first * kChunk + tid < S ? ids[first * kChunk + tid] : -1;
  for (int e = tid; e < E; e += kChunk) {
    hist[e] = pre[e] = 0;
#pragma unroll
    for (int w = 0; w < kChunk / 64; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  // histogram of every slot; sub-chunk i covers slots [256 i, 256 i + 256), all of
  // them before this workgroup's range when i < first.  Ids are loaded in batches of
  // kBatch sub-chunks so one memory latency covers the batch.
  constexpr int kBatch = 16;
  const int nsub = (S + kChunk - 1) / kChunk;
  for (int i0 = 0; i0 < nsub; i0 += kBatch) {
    int ev[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int sl = (i0 + u) * kChunk + tid;
      ev[u] = sl < S ? ids[sl] : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (ev[u] >= 0 && ev[u] < E) {
        atomicAdd(&hist[ev[u]], 1);
        if (i0 + u < first) atomicAdd(&pre[ev[u]], 1);
      }
    }
  }
  __syncthreads();
  // padded exclusive scan over experts: thread t owns experts [q t, q t + q)
  constexpr int Q = kAlignMaxE / kChunk;
  int local[Q], sum = 0;
#pragma unroll
  for (int k = 0; k < Q; ++k) {
    const int e = Q * tid + k;
    local[k] = e < E ? (hist[e] + block - 1) / block * block : 0;
    sum += local[k];
  }
  int incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kChunk / 64; ++w) {
    before += w < wave ? wsum[w] : 0;
    total += wsum[w];
  }
  int run = before + incl - sum;
#pragma unroll
  for (int k = 0; k < Q; ++k) {
    const int e = Q * tid + k;
    if (e < E) {
      base[e] = run;
      if (g == 0) offsets[e] = run;
    }
    run += local[k];
  }
  if (g == 0 && tid == 0) offsets[E] = total;
  // place the slots of each sub-chunk, stable: a slot's rank is the count of its expert
  // in the earlier waves of the sub-chunk (per-wave counts, LDS atomics) plus the count
  // among the earlier lanes of its wave (a scan of the wave's 64 ids in LDS); then the
  // per-expert counts advance past the sub-chunk
  for (int r = 0; r < R; ++r) {
    const int my_s = (first + r) * kChunk + tid;
    const int my_e = r == 0 ? my_e0 : (my_s < S ? ids[my_s] : -1);
    const bool valid = my_e >= 0 && my_e < E;
    if (!valid && zrows != nullptr && my_s < S) {
      uint4* row = (uint4*)(zrows + (int64_t)my_s * ldz);
      for (int c = 0; c < zcols / 8; ++c) row[c] = uint4{0u, 0u, 0u, 0u};
    }
    cid[tid] = my_e;
    if (valid) atomicAdd(&wcnt[wave][my_e], 1);
    __syncthreads();
    if (valid) {
      int rank = 0;
      const int4* c4 = (const int4*)(cid + wave * 64);
      int4 v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = c4[u];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        rank += (4 * u < lane && v[u].x == my_e) + (4 * u + 1 < lane && v[u].y == my_e) +
                (4 * u + 2 < lane && v[u].z == my_e) + (4 * u + 3 < lane && v[u].w == my_e);
      for (int w = 0; w < wave; ++w) rank += wcnt[w][my_e];
      sorted[base[my_e] + pre[my_e] + rank] = my_s;
    }
    __syncthreads();  // pre[], wcnt[] and cid[] are read: advance pre, clear this wave's counts
    if (valid) {
      atomicAdd(&pre[my_e], 1);
      wcnt[wave][my_e] = 0;
    }
  }
  // positions past the real slots: padding of every expert and the tail [total, cap)
  // get the sentinel S; the expert of a position (and of a block's first position) is
  // the last expert whose start is <= it, empty experts sharing the start of the next
  auto owner_of = [&](int pos) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (base[mid] <= pos) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  for (int i = g * kChunk + tid; i < cap; i += G * kChunk) {
    if (i >= total) {
      sorted[i] = S;
    } else {
      const int e = owner_of(i);
      if (i - base[e] >= hist[e]) sorted[i] = S;
    }
  }
  const int nblk = cap / block;
  for (int b = g * kChunk + tid; b < nblk; b += G * kChunk) block_expert[b] = b * block < total ? owner_of(b * block) : -1;
}

// ------------------------------------------------------------------------------
// 2/3. grouped GEMMs on the tile engine
// ------------------------------------------------------------------------------
struct MoeGemmParams {
  const uint16_t* x;      // gate_up: hidden [T, D] (row stride ldx); down: H [cap, I]
  const uint16_t* w;      // gate_up: w1 [E, 2I, D]; down: w2 [E, D, I]
  const int32_t* offsets;
  const int32_t* sorted;
  const int32_t* block_expert;
  const float* tw;        // [S] router weights (down)
  uint16_t* h;            // H high plane [cap, I] (gate_up output / down input)
  uint16_t* h_lo;         // H low plane [cap, I]
  float* yw;              // down output Yw [S, D]
  int64_t ldx;
  int E, S, topk, T;
  int K;                  // reduction length (D for gate_up, I for down)
  int Nout;               // output columns (I for gate_up, D for down)
  int64_t w_estride;      // elements between experts in w
  int64_t w_rstride;      // elements between rows of w[e]
  int max_mblocks, ntiles;
  int abm;                // rows per aligned block of the sorted slot list
  uint16_t* out;          // plain grouped GEMM: bf16 output rows, scattered by token
  int64_t ldo;
};

// GATEUP / DOWN: the two projections of the fused MoE.  PLAIN: a top-1 grouped GEMM
// out[t] = x[t] @ w[e]^T (gathered rows in, bf16 rows scattered back by token).
enum { MOE_GATEUP = 0, MOE_DOWN = 1, MOE_PLAIN = 2 };

// get(i, j, g, e): element 4g + e of the lane's accumulator of 32x32 tile (i, j), at
// wave-tile row acc_row<M16>(i, g, lane), column acc_col<M16>(j, g, lane) + e.
template <int MODE, int MI, int NI, int WROWS, int WCOLS, bool M16, typename Get>
__device__ __forceinline__ void moe_epilogue_at(Get&& get, uint16_t* lds, const MoeGemmParams& p, int pos0, int n0,
                                                int wm, int wn, int wave, int lane) {
  using Op = MfmaOp<BF16>;
  // a lane's rows in a 32-row block: one (32x32 layout: groups g = 0..3 share it) or two
  // (16x16 sub-tiles: g = 2 sm + sn, row set by sm)
  constexpr int NR = M16 ? 2 : 1, GPR = 4 / NR;
  if constexpr (MODE == MOE_GATEUP) {
    constexpr int HC = WCOLS / 2;  // h columns per wave
    using St = Stager<WROWS, HC>;
    uint16_t* stg_hi = lds + wave * (2 * WROWS * HC);
    uint16_t* stg_lo = stg_hi + WROWS * HC;
    // h = silu(gate) * up for 4 consecutive h columns, split into bf16 high/low planes
    auto put_h = [&](int row, int col, const float (&gt)[4], const float (&up)[4]) {
      float hi[4], lo[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float h = gt[q] * fast_sigmoid(gt[q]) * up[q];
        hi[q] = Op::to_f32((uint16_t)(Op::pack2(h, 0.0f) & 0xffffu));
        lo[q] = h - hi[q];  // exact in fp32
      }
      St::put(stg_hi, row, col, u32x2_t{Op::pack2(hi[0], hi[1]), Op::pack2(hi[2], hi[3])});
      St::put(stg_lo, row, col, u32x2_t{Op::pack2(lo[0], lo[1]), Op::pack2(lo[2], lo[3])});
    };
    if constexpr (NI == 1) {
      static_assert(!M16, "one 32-column block: the 32x32 layout");
      // one 32-row block: rows 0-15 are gate rows, 16-31 the matching up rows, so
      // register 4g+q (g < 2) holds a gate value and register 8+4g+q its up value
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float gt[4], up[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            gt[q] = get(i, 0, g, q);
            up[q] = get(i, 0, 2 + g, q);
          }
          put_h(out_row(i, lane), out_col(0, g, lane), gt, up);
        }
    } else {
      // 32-row blocks j < NI/2 are gate rows, block j + NI/2 the matching up rows
      constexpr int NH = NI / 2;
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NH; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float gt[4], up[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              gt[q] = get(i, j, g, q);
              up[q] = get(i, j + NH, g, q);
            }
            put_h(acc_row<M16>(i, g, lane), acc_col<M16>(j, g, lane), gt, up);
          }
    }
    __syncthreads();
    const int rw0 = pos0 + wm * WROWS, cw0 = n0 + wn * HC;
    St::drain(stg_hi, lane, [&](int row, int col, u32x4_t v) {
      *(u32x4_t*)(p.h + (int64_t)(rw0 + row) * p.Nout + cw0 + col) = v;
    });
    St::drain(stg_lo, lane, [&](int row, int col, u32x4_t v) {
      *(u32x4_t*)(p.h_lo + (int64_t)(rw0 + row) * p.Nout + cw0 + col) = v;
    });
  } else if constexpr (MODE == MOE_PLAIN) {
    // rows of this lane -> token (top-1: slot == token); bf16 8-byte stores of 4 columns
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int s = p.sorted[pos0 + wm * WROWS + acc_row<M16>(i, r * GPR, lane)];
        if (s >= p.S) continue;
        uint16_t* dst = p.out + (int64_t)s * p.ldo + n0 + wn * WCOLS;
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int g = r * GPR; g < (r + 1) * GPR; ++g)
            *(u32x2_t*)(dst + acc_col<M16>(j, g, lane)) =
                u32x2_t{Op::pack2(get(i, j, g, 0), get(i, j, g, 1)), Op::pack2(get(i, j, g, 2), get(i, j, g, 3))};
      }
  } else {
    // rows of this lane -> slot, scaled by its routing weight; fp32 16-byte stores
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int s = p.sorted[pos0 + wm * WROWS + acc_row<M16>(i, r * GPR, lane)];
        if (s >= p.S) continue;
        const float wgt = p.tw[s];
        float* dst = p.yw + (int64_t)s * p.Nout + n0 + wn * WCOLS;
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int g = r * GPR; g < (r + 1) * GPR; ++g) {
            const f32x4_t v = {get(i, j, g, 0) * wgt, get(i, j, g, 1) * wgt, get(i, j, g, 2) * wgt,
                               get(i, j, g, 3) * wgt};
            *(f32x4_t*)(dst + acc_col<M16>(j, g, lane)) = v;
          }
      }
  }
}

template <int MODE, int MI, int NI, int WROWS, int WCOLS>
__device__ __forceinline__ void moe_epilogue(f32x16_t (&acc)[MI][NI], uint16_t* lds, const MoeGemmParams& p, int pos0,
                                             int n0, int wm, int wn, int wave, int lane) {
  moe_epilogue_at<MODE, MI, NI, WROWS, WCOLS, false>([&](int i, int j, int g, int e) { return acc[i][j][4 * g + e]; },
                                                     lds, p, pos0, n0, wm, wn, wave, lane);
}
template <int MODE, int MI, int NI, int WROWS, int WCOLS>
__device__ __forceinline__ void moe_epilogue16(f32x4_t (&c4)[MI][NI][4], uint16_t* lds, const MoeGemmParams& p,
                                               int pos0, int n0, int wm, int wn, int wave, int lane) {
  moe_epilogue_at<MODE, MI, NI, WROWS, WCOLS, true>([&](int i, int j, int g, int e) { return c4[i][j][g][e]; }, lds,
                                                    p, pos0, n0, wm, wn, wave, lane);
}

template <int MODE, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(kEngineThreads)
    moe_gemm_kernel(const MoeGemmParams p) {
  using E = TileEngine<BF16, BM, BN, WM, WN, B_KC, MODE == MOE_DOWN ? 2 : 1>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int mb = bid % p.max_mblocks, nt = bid / p.max_mblocks;
  const int total = p.offsets[p.E];
  if (mb * BM >= total) return;  // uniform: the whole workgroup leaves
  const int e = p.block_expert[(mb * BM) / p.abm];  // BM divides abm
  const uint16_t* W = p.w + (int64_t)e * p.w_estride;
  const int pos0 = mb * BM;

  E eng;
  const int ch8 = (tid & 7) * 8;
#pragma unroll
  for (int j = 0; j < E::LA; ++j) {
    const int r = E::a_row_of(tid, j);
    int64_t row;
    if constexpr (MODE != MOE_DOWN) {
      const int s = p.sorted[pos0 + r];
      row = (s < p.S) ? s / p.topk : 0;  // padding rows read token 0; never stored
    } else {
      row = pos0 + r;
    }
    eng.a_src[j] = p.x + row * p.ldx + ch8;
    if constexpr (MODE == MOE_DOWN) eng.a2_src[j] = p.h_lo + row * p.ldx + ch8;
  }
  int n0;
  if constexpr (MODE == MOE_GATEUP) {
    // Tile covers BN/2 intermediate columns; inside each wave's WCOLS rows the first
    // half are gate rows and the second half the matching up rows.
    n0 = nt * (BN / 2);
    const int I = p.Nout;
#pragma unroll
    for (int j = 0; j < E::LB; ++j) {
      const int r = E::b_row_of(tid, j);
      const int q = r / E::WCOLS, within = r % E::WCOLS;
      const int half = within / (E::WCOLS / 2);
      const int col = n0 + q * (E::WCOLS / 2) + within % (E::WCOLS / 2);
      eng.b_src[j] = W + (int64_t)(half * I + col) * p.w_rstride + ch8;
    }
  } else {
    n0 = nt * BN;
#pragma unroll
    for (int j = 0; j < E::LB; ++j) eng.b_src[j] = W + (int64_t)(n0 + E::b_row_of(tid, j)) * p.w_rstride + ch8;
  }
  eng.ldb = 0;

  f32x16_t acc[MI][NI];
  E::zero(acc);
  eng.mainloop(lds, p.K, acc);

  moe_epilogue<MODE, MI, NI, E::WROWS, E::WCOLS>(acc, lds, p, pos0, n0, wm, wn, wave, lane);
}


// Prefill path on the buffer-load pipelined engine: A rows (gathered tokens for
// gate_up, H planes for down) and B rows (interleaved gate/up rows of w1[e], rows of
// w2[e]) become per-lane byte offsets of buffer resources, fixed for the whole K loop.
// 16x16x32 MFMAs on a 2 x 2 wave grid, one wave per SIMD, with the accumulators held in
// place in AGPRs (mma16_acc).  Fused MoE E=8 top-2 D=4096 I=14336, same process,
// bit-equal: T=4096 3.75 -> 3.58 ms against the former 2 x 4 grid of 8 waves (two per
// SIMD), which had itself replaced 4 waves of 32x32x16 MFMAs (T=4096 3.93 -> 3.83 ms);
// T=1024 within 1%.  The plain grouped GEMM: 117 us either way at M=4096, E=32, N=2048,
// K=4096 (jagged routing), 204.5 -> 202.2 us at 8192 x 16 x 1536 x 4096.
template <int MODE, int BM, int BN, int NWV>
__global__ void __launch_bounds__(64 * NWV)
    moe_buf_kernel(const MoeGemmParams p) {
  constexpr int AP = (MODE == MOE_DOWN) ? 2 : 1;
  // grouped (plain) GEMM: an expert's weight tile is read by that expert's row blocks
  // only, running side by side on one XCD (L2), so its loads are non-temporal
  using E = BufPipeEngine<BF16, BM, BN, 2, NWV / 2, AP, B_KC, MODE == MOE_PLAIN ? kCpolNT : kCpolDefault, true>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / E::WN, wn = wave % E::WN;

  int mb, nt;
  if constexpr (MODE == MOE_PLAIN) {
    const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    mb = bid % p.max_mblocks;
    nt = bid / p.max_mblocks;
  } else {
    // Expert-aligned raster: the row blocks of expert e ([offsets[e], offsets[e+1]) / BM)
    // are split into ng = ceil(nb / GMAX) groups of near-equal size, and a group's row
    // blocks sweep the column tiles together, so each group streams its expert's
    // weights once and xcd_remap keeps a group on one L2.  Logical ids past the last
    // block leave.  Against fixed groups of 1024 / BM blocks that straddle experts
    // (same process, bit-equal, E=8 top-2 D=4096 I=14336): T=4096 3.86 -> 3.72 ms,
    // T=1024 1.51 -> 1.47, T=8192 6.88 -> 6.78, T=16384 13.11 -> 13.08; gate_up groups
    // of up to 8 and down groups of up to 12 measured slower at T=16384 (13.44 ms).
    constexpr int GMAX = MODE == MOE_GATEUP ? 6 : 8;
    const int nT = p.ntiles;
    // The grid is sized for the largest possible slot list; the live tiles are the first
    // nreal logical ids.  They are spread over the XCDs by their own count (workgroup b
    // runs on XCD b % 8, so the first n8 workgroups take contiguous eighths of them);
    // remapped over the whole grid, the live ids filled the first XCDs' ranges and left
    // the last ones short.  Same process, bit-equal, E=8 top-2 D=4096 I=14336: T=1024
    // 1.472 -> 1.412 ms, T=2048 2.176 -> 2.035, T=4096 3.631 -> 3.601-3.634, T=8192
    // 6.579 -> 6.509, T=16384 12.68 -> 12.61.  Skipping the 128-row halves that hold only
    // padding (a per-workgroup scan of the experts' live blocks) measured slower: T=4096
    // 3.85 ms.
    const int nreal = (p.offsets[p.E] / BM) * nT;
    const int n8 = (nreal + 7) & ~7;
    if ((int)blockIdx.x >= n8) return;  // uniform: the whole workgroup leaves
    const int bid = xcd_remap((int)blockIdx.x, n8);
    if (bid >= nreal) return;
    int lo = 0, hi = p.E;  // largest e < E with offsets[e] / BM * nT <= bid (an expert with rows)
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((p.offsets[mid] / BM) * nT <= bid) lo = mid;
      else hi = mid;
    }
    const int b0 = p.offsets[lo] / BM, nb = p.offsets[lo + 1] / BM - b0;
    const int ng = (nb + GMAX - 1) / GMAX;
    const int local = bid - b0 * nT;
    int j = 0;
    while (j + 1 < ng && ((j + 1) * nb / ng) * nT <= local) ++j;
    const int gb = j * nb / ng, gsz = (j + 1) * nb / ng - gb;
    const int tl = local - gb * nT;
    mb = b0 + gb + tl % gsz;
    nt = tl / gsz;
  }
  const int total = p.offsets[p.E];
  if (mb * BM >= total) return;  // uniform: the whole workgroup leaves
  const int e = p.block_expert[(mb * BM) / p.abm];
  const int pos0 = mb * BM;

  E eng;
  // A: gathered token rows (gate_up, plain) or the H planes of this block (down)
  if constexpr (MODE != MOE_DOWN) {
    eng.ra = make_rsrc(p.x, (uint32_t)((int64_t)p.T * p.ldx * 2));
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int r = E::a_row(wave, lane, j);
      const int sl = p.sorted[pos0 + r];
      const int64_t row = (sl < p.S) ? sl / p.topk : 0;  // padding rows read token 0; never stored
      eng.a_voff[j] = (uint32_t)((row * p.ldx + 8 * E::chunk(r, lane)) * 2);
    }
  } else {
    const int64_t tile_bytes = (int64_t)BM * p.ldx * 2;
    eng.ra = make_rsrc(p.x + (int64_t)pos0 * p.ldx, (uint32_t)tile_bytes);
    eng.ra2 = make_rsrc(p.h_lo + (int64_t)pos0 * p.ldx, (uint32_t)tile_bytes);
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int r = E::a_row(wave, lane, j);
      eng.a_voff[j] = (uint32_t)(((int64_t)r * p.ldx + 8 * E::chunk(r, lane)) * 2);
    }
  }
  // B: interleaved gate/up rows of w1[e] (gate_up) or consecutive rows of w[e]
  int n0;
  if constexpr (MODE == MOE_GATEUP) {
    n0 = nt * (BN / 2);
    const int I = p.Nout;
    const uint16_t* W = p.w + (int64_t)e * p.w_estride;
    eng.rb = make_rsrc(W, (uint32_t)((int64_t)2 * I * p.w_rstride * 2));
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      const int r = E::b_row(wave, lane, j);
      const int q = r / E::WCOLS, within = r % E::WCOLS;
      const int half = within / (E::WCOLS / 2);
      const int col = n0 + q * (E::WCOLS / 2) + within % (E::WCOLS / 2);
      eng.b_voff[j] = (uint32_t)(((int64_t)(half * I + col) * p.w_rstride + 8 * E::chunk(r, lane)) * 2);
    }
  } else {
    n0 = nt * BN;
    const uint16_t* W = p.w + (int64_t)e * p.w_estride + (int64_t)n0 * p.w_rstride;
    eng.rb = make_rsrc(W, (uint32_t)((int64_t)BN * p.w_rstride * 2));
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      const int r = E::b_row(wave, lane, j);
      eng.b_voff[j] = (uint32_t)(((int64_t)r * p.w_rstride + 8 * E::chunk(r, lane)) * 2);
    }
  }

  f32x4_t acc[MI][NI][4];
  E::zero16(acc);
  eng.mainloop16(lds, p.K, acc);
  moe_epilogue16<MODE, MI, NI, E::WROWS, E::WCOLS>(acc, lds, p, pos0, n0, wm, wn, wave, lane);
}

// Down projection grid: workgroup b runs on XCD b % 8 (round-robin dispatch), so XCD x
// takes the blocks mb = x, x + 8, ... with all of their column tiles; each L2 then holds
// the H rows of an eighth of the blocks instead of every XCD streaming all of H, and the
// live blocks (the low mb) are spread evenly over the XCDs.  The grid is the block count
// rounded up to a multiple of 8 times ntiles.
__device__ __forceinline__ void down_coords(int b, int ntiles, int& mb, int& nt) {
  const int q = b >> 3;
  mb = (q / ntiles) * 8 + (b & 7);
  nt = q % ntiles;
}

// Weight-streaming path (32- and 128-row blocks) on the skinny ring engine.  Grid =
// ntiles x max_mblocks; a workgroup multiplies one BM-slot block by BN rows of its
// expert's weights over the whole K, so w1/w2 are streamed once per block, NSLOT-1
// stages in flight per workgroup, with the non-temporal load policy (each weight row is
// read by exactly one workgroup).
template <int MODE, int BN, int NSLOT, int BM>
__global__ void __launch_bounds__(256)
    moe_decode_kernel(const MoeGemmParams p) {
  constexpr int AP = (MODE == MOE_DOWN) ? 2 : 1;
  using E = SkinnyRingEngine<BF16, BN, AP, NSLOT, BM, kCpolNT>;  // each weight row is read by one workgroup
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  int mb, nt;
  if constexpr (MODE == MOE_DOWN) {
    down_coords((int)blockIdx.x, p.ntiles, mb, nt);
    if (mb >= p.max_mblocks) return;
  } else {
    const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    mb = bid % p.max_mblocks;
    nt = bid / p.max_mblocks;
  }
  const int total = p.offsets[p.E];
  if (mb * E::BM >= total) return;  // uniform: the whole workgroup leaves
  const int e = p.block_expert[(mb * E::BM) / p.abm];
  const int pos0 = mb * E::BM;

  E eng;
  // A: gathered token rows (gate_up, plain) or the H planes of this block (down).
  // A padding row (sorted slot >= S) gets the resource's byte size as its offset: the
  // buffer range check turns its loads into zeros with no memory traffic, and its
  // output row is never used (rows of an MFMA product are independent).
  if constexpr (MODE != MOE_DOWN) {
    const uint32_t bytes = (uint32_t)((int64_t)p.T * p.ldx * 2);
    eng.ra = make_rsrc(p.x, bytes);
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int ar = E::a_row(wave, lane, j);
      const int sl = p.sorted[pos0 + ar];
      eng.a_voff[j] = sl < p.S ? (uint32_t)(((int64_t)(sl / p.topk) * p.ldx + 8 * E::chunk(ar, lane)) * 2) : bytes;
    }
  } else {
    const uint32_t tile_bytes = (uint32_t)((int64_t)E::BM * p.ldx * 2);
    eng.ra = make_rsrc(p.x + (int64_t)pos0 * p.ldx, tile_bytes);
    eng.ra2 = make_rsrc(p.h_lo + (int64_t)pos0 * p.ldx, tile_bytes);
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int ar = E::a_row(wave, lane, j);
      eng.a_voff[j] = p.sorted[pos0 + ar] < p.S ? (uint32_t)(((int64_t)ar * p.ldx + 8 * E::chunk(ar, lane)) * 2)
                                                : tile_bytes;
    }
  }
  // B: interleaved gate/up rows of w1[e] (gate_up) or consecutive rows of w[e]
  int n0;
  if constexpr (MODE == MOE_GATEUP) {
    n0 = nt * (BN / 2);
    const int I = p.Nout;
    const uint16_t* W = p.w + (int64_t)e * p.w_estride;
    eng.rb = make_rsrc(W, (uint32_t)((int64_t)2 * I * p.w_rstride * 2));
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      // each wave's WCOLS rows: gate rows of its WCOLS/2 columns, then the up rows
      const int r = E::b_row(wave, lane, j);
      const int q = r / E::WCOLS, within = r % E::WCOLS;
      const int half = within / (E::WCOLS / 2);
      const int col = n0 + q * (E::WCOLS / 2) + within % (E::WCOLS / 2);
      eng.b_voff[j] = (uint32_t)(((int64_t)(half * I + col) * p.w_rstride + 8 * E::chunk(r, lane)) * 2);
    }
  } else {
    n0 = nt * BN;
    const uint16_t* W = p.w + (int64_t)e * p.w_estride + (int64_t)n0 * p.w_rstride;
    eng.rb = make_rsrc(W, (uint32_t)((int64_t)BN * p.w_rstride * 2));
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      const int r = E::b_row(wave, lane, j);
      eng.b_voff[j] = (uint32_t)(((int64_t)r * p.w_rstride + 8 * E::chunk(r, lane)) * 2);
    }
  }
  f32x16_t acc[MI][NI];
  E::zero(acc);
  eng.mainloop(lds, 0, p.K, acc);
  moe_epilogue<MODE, MI, NI, E::BM, E::WCOLS>(acc, lds, p, pos0, n0, 0, wave, wave, lane);
}

// ------------------------------------------------------------------------------
// 4. combine
// ------------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
    moe_combine_kernel(const float* __restrict__ yw, const int32_t* __restrict__ ids, uint16_t* __restrict__ out,
                       int T, int D, int topk, int E) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one thread per 4 outputs
  const int per_row = D / 4;
  if (idx >= (int64_t)T * per_row) return;
  const int t = (int)(idx / per_row), d0 = (int)(idx % per_row) * 4;
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
  // every row is loaded (a slot with an invalid id has an unwritten row) and selected
  // away, so the loads of all k are independent and go out together
#pragma unroll 8
  for (int k = 0; k < topk; ++k) {
    const int e = ids[t * topk + k];
    const bool ok = e >= 0 && e < E;
    const f32x4_t v = *(const f32x4_t*)(yw + ((int64_t)t * topk + k) * D + d0);
#pragma unroll
    for (int q = 0; q < 4; ++q) s[q] += ok ? v[q] : 0.0f;
  }
  using Op = MfmaOp<BF16>;
  *(u32x2_t*)(out + (int64_t)t * D + d0) = u32x2_t{Op::pack2(s[0], s[1]), Op::pack2(s[2], s[3])};
}

// ------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------
inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Worst-case padded length: every expert rounds up by < block rows.
inline int64_t align_capacity(int64_t S, int64_t E, int64_t block) {
  return align_up(S + E * (block - 1), block);
}

// Block size of the fused MoE GEMMs: skinny blocks when experts see few rows.
// Up to 16 slots per expert on average: 32-row blocks; up to 128: 128-row blocks, so
// nearly every expert's weights are streamed once (padding rows cost MFMA cycles, which
// are idle on these weight-bound shapes, but no memory traffic); beyond: 256.
inline int moe_block_rows(int64_t S, int64_t E) { return S <= 16 * E ? 32 : S <= 128 * E ? 128 : 256; }

struct MoeWorkspace {
  int32_t* offsets;
  int32_t* sorted;
  int32_t* block_expert;
  uint16_t* h;
  uint16_t* h_lo;
  float* yw;
  size_t bytes;
};

inline MoeWorkspace carve(void* base, int64_t T, int64_t topk, int64_t E, int64_t D, int64_t I) {
  const int64_t S = T * topk;
  const int BM = moe_block_rows(S, E);
  const int64_t cap = align_capacity(S, E, BM);
  MoeWorkspace w{};
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off = (size_t)align_up((int64_t)(off + n), 256);
    return o;
  };
  const size_t o_off = take(sizeof(int32_t) * (E + 1));
  const size_t o_sorted = take(sizeof(int32_t) * cap);
  const size_t o_blk = take(sizeof(int32_t) * (cap / BM));
  const size_t o_h = take(sizeof(uint16_t) * cap * I);
  const size_t o_hlo = take(sizeof(uint16_t) * cap * I);
  const size_t o_yw = take(sizeof(float) * S * D);
  char* b = (char*)base;
  w.offsets = (int32_t*)(b + o_off);
  w.sorted = (int32_t*)(b + o_sorted);
  w.block_expert = (int32_t*)(b + o_blk);
  w.h = (uint16_t*)(b + o_h);
  w.h_lo = (uint16_t*)(b + o_hlo);
  w.yw = (float*)(b + o_yw);
  w.bytes = off;
  return w;
}

template <int MODE, int BM, int BN, int WM, int WN>
int launch_moe_gemm(MoeGemmParams p, int64_t cap, hipStream_t st) {
  p.ntiles = (MODE == MOE_GATEUP) ? p.Nout / (BN / 2) : p.Nout / BN;
  p.max_mblocks = (int)(cap / BM);
  const int64_t blocks = (int64_t)p.max_mblocks * p.ntiles;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "fused_moe: grid too large");
  hipLaunchKernelGGL((moe_gemm_kernel<MODE, BM, BN, WM, WN>), dim3((unsigned)blocks), dim3(kEngineThreads), 0, st, p);
  return check_launch(MODE == MOE_GATEUP ? "moe_gateup_kernel" : "moe_down_kernel");
}


template <int MODE, int BN, int NSLOT, int BM = 32>
int launch_moe_decode(MoeGemmParams p, int64_t cap, hipStream_t st) {
  p.ntiles = (MODE == MOE_GATEUP) ? p.Nout / (BN / 2) : p.Nout / BN;
  p.max_mblocks = (int)(cap / BM);
  const int64_t mblocks = MODE == MOE_DOWN ? align_up(p.max_mblocks, 8) : p.max_mblocks;  // down_coords
  const int64_t blocks = mblocks * p.ntiles;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "fused_moe: grid too large");
  hipLaunchKernelGGL((moe_decode_kernel<MODE, BN, NSLOT, BM>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return check_launch(MODE == MOE_GATEUP ? "moe_gateup_decode_kernel" : "moe_down_decode_kernel");
}

template <int MODE, int BM, int BN>
int launch_moe_buf(MoeGemmParams p, int64_t cap, hipStream_t st) {
  p.ntiles = (MODE == MOE_GATEUP) ? p.Nout / (BN / 2) : p.Nout / BN;
  p.max_mblocks = (int)(cap / BM);
  const int64_t blocks = (int64_t)p.max_mblocks * p.ntiles;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "fused_moe: grid too large");
  constexpr int NWV = 4;
  hipLaunchKernelGGL((moe_buf_kernel<MODE, BM, BN, NWV>), dim3((unsigned)blocks), dim3(64 * NWV), 0, st, p);
  return check_launch(MODE == MOE_GATEUP ? "moe_gateup_buf_kernel" : "moe_down_buf_kernel");
}

}  // namespace
}  // namespace kore

namespace kore {
namespace {
// Test hook (kore_moe_test_force_generic): route the MoE GEMMs to the register-staged
// tile paths that operands beyond the 32-bit buffer range take, so tests reach them at
// small sizes.  Process-wide; off by default.
int g_force_generic = 0;

// Sort/align of S slots: the chunked kernel, one workgroup per 256 slots.
int launch_align(const int32_t* ids, int64_t S, int64_t E, int block, int32_t* offsets, int32_t* sorted,
                 int32_t* block_expert, int64_t cap, hipStream_t st, uint16_t* zrows = nullptr, int64_t ldz = 0,
                 int zcols = 0) {
  const int64_t chunks = std::max<int64_t>(1, (S + kChunk - 1) / kChunk);
  const int R = (int)((chunks + 255) / 256);  // sub-chunks per workgroup: at most 256 workgroups
  const int grid = (int)((chunks + R - 1) / R);
  hipLaunchKernelGGL(moe_align_chunk_kernel, dim3((unsigned)grid), dim3(kChunk), 0, st, ids, (int)S, (int)E, block, R,
                     offsets, sorted, block_expert, (int)cap, zrows, ldz, zcols);
  return check_launch("moe_align_chunk_kernel");
}
}  // namespace
}  // namespace kore

extern "C" int kore_moe_test_force_generic(int on) {
  const int prev = kore::g_force_generic;
  kore::g_force_generic = on != 0;
  return prev;
}

extern "C" int64_t kore_moe_align_capacity(int64_t T, int64_t topk, int64_t E, int64_t block) {
  if (T < 0 || topk <= 0 || E <= 0 || block <= 0) return -1;
  return kore::align_capacity(T * topk, E, block);
}

extern "C" int kore_moe_align(const int32_t* topk_ids, int64_t T, int64_t topk, int64_t E, int64_t block,
                              int32_t* offsets, int32_t* sorted_slots, int32_t* block_expert, int64_t cap,
                              void* stream) {
  using namespace kore;
  if (!topk_ids || !offsets || !sorted_slots || !block_expert) return set_error(KORE_EINVAL, "moe_align: null pointer");
  if (T < 0 || topk <= 0 || E <= 0 || block <= 0) return set_error(KORE_EINVAL, "moe_align: bad sizes");
  if (E > kAlignMaxE) return set_error(KORE_EUNSUPPORTED, "moe_align: E > %d", kAlignMaxE);
  if (T * topk >= (1ll << 30)) return set_error(KORE_EUNSUPPORTED, "moe_align: too many slots");
  if (cap < align_capacity(T * topk, E, block) || cap % block != 0)
    return set_error(KORE_EINVAL, "moe_align: cap %lld too small or not a multiple of block (need %lld)",
                     (long long)cap, (long long)align_capacity(T * topk, E, block));
  return launch_align(topk_ids, T * topk, E, (int)block, offsets, sorted_slots, block_expert, cap,
                      (hipStream_t)stream);
}

extern "C" size_t kore_fused_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t D, int64_t I) {
  if (T <= 0 || topk <= 0 || E <= 0 || D <= 0 || I <= 0) return 0;
  return kore::carve(nullptr, T, topk, E, D, I).bytes;
}

extern "C" int kore_fused_moe(const void* hidden, int64_t ldh, const void* w1, const void* w2,
                              const float* topk_weight, const int32_t* topk_ids, void* out, int64_t T, int64_t D,
                              int64_t I, int64_t E, int64_t topk, void* workspace, size_t workspace_bytes,
                              void* stream) {
  using namespace kore;
  if (!hidden || !w1 || !w2 || !topk_weight || !topk_ids || !out || !workspace)
    return set_error(KORE_EINVAL, "fused_moe: null pointer");
  if (T <= 0 || D <= 0 || I <= 0 || E <= 0 || topk <= 0) return set_error(KORE_EINVAL, "fused_moe: sizes must be >= 1");
  if (D % 128 != 0 || I % 128 != 0)
    return set_error(KORE_EUNSUPPORTED, "fused_moe: D and I must be multiples of 128 (D=%lld I=%lld)", (long long)D,
                     (long long)I);
  if (E > kAlignMaxE) return set_error(KORE_EUNSUPPORTED, "fused_moe: E > %d", kAlignMaxE);
  if (ldh < D || ldh % 8 != 0 || ((uintptr_t)hidden & 15u) || ((uintptr_t)w1 & 15u) || ((uintptr_t)w2 & 15u) ||
      ((uintptr_t)out & 15u))
    return set_error(KORE_EINVAL, "fused_moe: hidden/w1/w2/out must be 16-byte aligned with ldh %% 8 == 0");
  const int64_t S = T * topk;
  if (S >= (1ll << 30) || 2 * I * D >= (1ll << 40)) return set_error(KORE_EUNSUPPORTED, "fused_moe: problem too large");
  const MoeWorkspace ws = carve(workspace, T, topk, E, D, I);
  if (workspace_bytes < ws.bytes)
    return set_error(KORE_EWORKSPACE, "fused_moe: workspace %zu bytes < required %zu", workspace_bytes, ws.bytes);
  hipStream_t st = (hipStream_t)stream;
  const int BM = moe_block_rows(S, E);
  const int64_t cap = align_capacity(S, E, BM);
  int rc = launch_align(topk_ids, S, E, BM, ws.offsets, ws.sorted, ws.block_expert, cap, st);
  if (rc) return rc;

  MoeGemmParams p{};
  p.offsets = ws.offsets;
  p.sorted = ws.sorted;
  p.block_expert = ws.block_expert;
  p.tw = topk_weight;
  p.h = ws.h;
  p.h_lo = ws.h_lo;
  p.yw = ws.yw;
  p.abm = BM;
  p.E = (int)E;
  p.T = (int)T;
  p.S = (int)S;
  p.topk = (int)topk;
  // gate_up: x = hidden, K = D, outputs I columns of H
  p.x = (const uint16_t*)hidden;
  p.ldx = ldh;
  p.w = (const uint16_t*)w1;
  p.K = (int)D;
  p.Nout = (int)I;
  p.w_estride = 2 * I * D;
  p.w_rstride = D;
  // buffer-load engine needs operand byte ranges (plus a K step past a padding row's
  // offset) below 4 GiB and K % 64 == 0
  const bool buf_ok = T * ldh * 2 + 4 * D < (1ll << 32) && 2 * I * D * 2 < (1ll << 32) && D % 64 == 0 &&
                      I % 64 == 0 && !g_force_generic;
  // 128-row blocks without the buffer engine run 32-row tiles (four per aligned block)
  rc = (BM == 32 && buf_ok) ? launch_moe_decode<MOE_GATEUP, 128, 7>(p, cap, st)
       : (BM == 128 && buf_ok) ? launch_moe_decode<MOE_GATEUP, 128, 2, 128>(p, cap, st)
       : (BM <= 128) ? launch_moe_gemm<MOE_GATEUP, 32, 256, 1, 4>(p, cap, st)
       : buf_ok   ? launch_moe_buf<MOE_GATEUP, 256, 256>(p, cap, st)
                  : launch_moe_gemm<MOE_GATEUP, 256, 256, 2, 2>(p, cap, st);
  if (rc) return rc;
  // down: x = H, K = I, outputs D columns of Yw
  p.x = ws.h;
  p.ldx = I;
  p.w = (const uint16_t*)w2;
  p.K = (int)I;
  p.Nout = (int)D;
  p.w_estride = D * I;
  p.w_rstride = I;
  // two A planes double the A tile: prefill runs 128-row tiles (halves of a 256-row
  // aligned block) to stay inside the 160 KiB LDS budget.
  if (BM == 32 && buf_ok) {
    rc = launch_moe_decode<MOE_DOWN, 128, 6>(p, cap, st);
  } else if (BM == 128 && buf_ok) {
    rc = launch_moe_decode<MOE_DOWN, 128, 3, 128>(p, cap, st);
  } else if (BM <= 128) {
    rc = launch_moe_gemm<MOE_DOWN, 32, 128, 1, 4>(p, cap, st);
  } else if (buf_ok && D % 256 == 0) {
    rc = launch_moe_buf<MOE_DOWN, 128, 256>(p, cap, st);
  } else if (D % 256 == 0) {
    rc = launch_moe_gemm<MOE_DOWN, 128, 256, 2, 2>(p, cap, st);
  } else {
    rc = launch_moe_gemm<MOE_DOWN, 128, 128, 2, 2>(p, cap, st);
  }
  if (rc) return rc;
  const int64_t threads = T * (D / 4);
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, ws.yw, topk_ids,
                     (uint16_t*)out, (int)T, (int)D, (int)topk, (int)E);
  return check_launch("moe_combine_kernel");
}

// ==============================================================================
// Top-1 grouped (segmented) expert GEMM and the token permute (row gather).
// ==============================================================================
namespace kore {
namespace {

struct GroupedWorkspace {
  int32_t* offsets;
  int32_t* sorted;
  int32_t* block_expert;
  size_t bytes;
};

inline GroupedWorkspace carve_grouped(void* base, int64_t M, int64_t E, int BM) {
  const int64_t cap = align_capacity(M, E, BM);
  GroupedWorkspace w{};
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off = (size_t)align_up((int64_t)(off + n), 256);
    return o;
  };
  const size_t o_off = take(sizeof(int32_t) * (E + 1));
  const size_t o_sorted = take(sizeof(int32_t) * cap);
  const size_t o_blk = take(sizeof(int32_t) * (cap / BM));
  char* b = (char*)base;
  w.offsets = (int32_t*)(b + o_off);
  w.sorted = (int32_t*)(b + o_sorted);
  w.block_expert = (int32_t*)(b + o_blk);
  w.bytes = off;
  return w;
}

// Gather dst[i] = src[idx[i]] (an index outside [0, rows) writes a zero row) or, with
// SCATTER, dst[idx[i]] = src[i] (an index outside [0, rows) is skipped); 16-byte
// copies when every row start is 16-byte aligned.
template <bool SCATTER>
__global__ void __launch_bounds__(256)
    gather_rows_kernel(const uint8_t* __restrict__ src, int64_t ld_src, const int32_t* __restrict__ idx,
                       int64_t row_bytes, uint8_t* __restrict__ dst, int64_t ld_dst, int rows, int vec16) {
  const int i = (int)blockIdx.x;
  const int r = idx[i];
  const bool ok = r >= 0 && r < rows;
  if (SCATTER && !ok) return;
  const uint8_t* s = src + (SCATTER ? (int64_t)i : (int64_t)(ok ? r : 0)) * ld_src;
  uint8_t* d = dst + (SCATTER ? (int64_t)r : (int64_t)i) * ld_dst;
  if (vec16) {
    for (int64_t c = threadIdx.x; c < row_bytes / 16; c += 256)
      *(u32x4_t*)(d + 16 * c) = ok ? __builtin_nontemporal_load((const u32x4_t*)(s + 16 * c)) : u32x4_t{0u, 0u, 0u, 0u};
  } else {
    for (int64_t c = threadIdx.x; c < row_bytes; c += 256) d[c] = ok ? s[c] : (uint8_t)0;
  }
}

// Block rows of the fp8 grouped tiles: 256x256 when experts average >= 64 rows (one
// round of large tiles beats ~3 rounds of 128x128 tiles despite the padding).
inline int grouped_fp8_block_rows(int64_t M, int64_t E) { return M >= 64 * E ? 256 : 128; }

}  // namespace
}  // namespace kore

// One size serves the bf16 and fp8 grouped entries (every block size they use).
extern "C" size_t kore_moe_grouped_gemm_workspace_bytes(int64_t M, int64_t E) {
  if (M <= 0 || E <= 0) return 0;
  size_t b = 0;
  for (int bm : {32, 128, 256}) b = std::max(b, kore::carve_grouped(nullptr, M, E, bm).bytes);
  return b;
}

extern "C" int kore_moe_grouped_gemm(const void* x, int64_t ldx, const void* w, const int32_t* expert_ids, void* out,
                                     int64_t ldo, int64_t M, int64_t N, int64_t K, int64_t E, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  using namespace kore;
  if (!x || !w || !expert_ids || !out || !workspace) return set_error(KORE_EINVAL, "moe_grouped_gemm: null pointer");
  if (M <= 0 || N <= 0 || K <= 0 || E <= 0) return set_error(KORE_EINVAL, "moe_grouped_gemm: sizes must be >= 1");
  if (E > kAlignMaxE) return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm: E > %d", kAlignMaxE);
  if (N % 128 != 0 || K % 8 != 0)
    return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm: needs N %% 128 == 0 and K %% 8 == 0 (N=%lld K=%lld)",
                     (long long)N, (long long)K);
  if (ldx < K || ldx % 8 != 0 || ldo < N || ldo % 8 != 0 || ((uintptr_t)x & 15u) || ((uintptr_t)w & 15u) ||
      ((uintptr_t)out & 15u))
    return set_error(KORE_EINVAL, "moe_grouped_gemm: rows must be 16-byte aligned (ldx, ldo %% 8 == 0)");
  if (M >= (1ll << 30) || N * K >= (1ll << 40)) return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm: too large");
  const int BM = M <= 64 * E ? 32 : 256;  // the 32-row ring or 256-row tiles
  const GroupedWorkspace ws = carve_grouped(workspace, M, E, BM);
  if (workspace_bytes < kore_moe_grouped_gemm_workspace_bytes(M, E))
    return set_error(KORE_EWORKSPACE, "moe_grouped_gemm: workspace %zu bytes < required %zu", workspace_bytes,
                     kore_moe_grouped_gemm_workspace_bytes(M, E));
  hipStream_t st = (hipStream_t)stream;
  const int64_t cap = align_capacity(M, E, BM);
  int rc = launch_align(expert_ids, M, E, BM, ws.offsets, ws.sorted, ws.block_expert, cap, st, (uint16_t*)out, ldo,
                        (int)N);
  if (rc) return rc;
  MoeGemmParams p{};
  p.x = (const uint16_t*)x;
  p.ldx = ldx;
  p.w = (const uint16_t*)w;
  p.offsets = ws.offsets;
  p.sorted = ws.sorted;
  p.block_expert = ws.block_expert;
  p.E = (int)E;
  p.S = (int)M;
  p.T = (int)M;
  p.topk = 1;
  p.K = (int)K;
  p.Nout = (int)N;
  p.w_estride = N * K;
  p.w_rstride = K;
  p.abm = BM;
  p.out = (uint16_t*)out;
  p.ldo = ldo;
  const bool buf_ok =
      K % 64 == 0 && M * ldx * 2 + 4 * K < (1ll << 32) && N * K * 2 < (1ll << 32) && !g_force_generic;
  if (BM == 32) {
    rc = buf_ok ? launch_moe_decode<MOE_PLAIN, 128, 7>(p, cap, st) : launch_moe_gemm<MOE_PLAIN, 32, 128, 1, 4>(p, cap, st);
  } else if (buf_ok) {
    rc = N % 256 == 0 ? launch_moe_buf<MOE_PLAIN, 256, 256>(p, cap, st) : launch_moe_buf<MOE_PLAIN, 256, 128>(p, cap, st);
  } else {
    rc = N % 256 == 0 ? launch_moe_gemm<MOE_PLAIN, 256, 256, 2, 2>(p, cap, st)
                      : launch_moe_gemm<MOE_PLAIN, 256, 128, 2, 2>(p, cap, st);
  }
  return rc;
}

extern "C" int kore_moe_grouped_gemm_fp8(const void* xq, int64_t ldx, const void* wq, const float* xs,
                                         int64_t xs_stride, const float* ws, const int32_t* expert_ids, void* out,
                                         int64_t ldo, int64_t M, int64_t N, int64_t K, int64_t E, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  using namespace kore;
  if (!xq || !wq || !xs || !ws || !expert_ids || !out || !workspace)
    return set_error(KORE_EINVAL, "moe_grouped_gemm_fp8: null pointer");
  if (M <= 0 || N <= 0 || K <= 0 || E <= 0) return set_error(KORE_EINVAL, "moe_grouped_gemm_fp8: sizes must be >= 1");
  if (E > kAlignMaxE) return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm_fp8: E > %d", kAlignMaxE);
  if (N % 128 != 0 || K % 128 != 0)
    return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm_fp8: needs N %% 128 == 0 and K %% 128 == 0 (N=%lld K=%lld)",
                     (long long)N, (long long)K);
  if (ldx < K || ldx % 16 != 0 || ldo < N || ((uintptr_t)xq & 15u) || ((uintptr_t)wq & 15u))
    return set_error(KORE_EINVAL, "moe_grouped_gemm_fp8: rows must be 16-byte aligned (ldx %% 16 == 0)");
  if (M * ldx >= (1ll << 32) || 256 * K >= (1ll << 31) || M >= (1ll << 30) || N >= (1ll << 30))
    return set_error(KORE_EUNSUPPORTED, "moe_grouped_gemm_fp8: too large");
  if (workspace_bytes < kore_moe_grouped_gemm_workspace_bytes(M, E))
    return set_error(KORE_EWORKSPACE, "moe_grouped_gemm_fp8: workspace %zu bytes < required %zu", workspace_bytes,
                     kore_moe_grouped_gemm_workspace_bytes(M, E));
  const int BM = N % 256 == 0 ? grouped_fp8_block_rows(M, E) : 128;
  const GroupedWorkspace w = carve_grouped(workspace, M, E, BM);
  const int64_t cap = align_capacity(M, E, BM);
  hipStream_t st = (hipStream_t)stream;
  // rows of invalid ids are zeroed by the align kernel with 16-byte stores when out allows them
  const bool zok = ldo % 8 == 0 && ((uintptr_t)out & 15u) == 0;
  int rc = launch_align(expert_ids, M, E, BM, w.offsets, w.sorted, w.block_expert, cap, st,
                        zok ? (uint16_t*)out : nullptr, ldo, (int)N);
  if (rc) return rc;
  GroupedA8Args a{};
  a.xq = xq;
  a.ldx = ldx;
  a.wq = wq;
  a.xs = xs;
  a.xs_stride = xs_stride;
  a.ws = ws;
  a.sorted = w.sorted;
  a.block_expert = w.block_expert;
  a.y = out;
  a.ldy = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.capacity = cap;
  a.block_rows = BM;
  return launch_grouped_a8w8(a, st);
}

namespace kore {
namespace {
int launch_rows(bool scatter, const void* src, int64_t ld_src_bytes, const int32_t* idx, int64_t n, int64_t rows,
                int64_t row_bytes, void* dst, int64_t ld_dst_bytes, void* stream) {
  const char* what = scatter ? "scatter_rows" : "gather_rows";
  if (n == 0 || row_bytes == 0) return KORE_OK;
  if (!src || !idx || !dst) return set_error(KORE_EINVAL, "%s: null pointer", what);
  if (n < 0 || row_bytes < 0 || rows <= 0 || ld_src_bytes < row_bytes || ld_dst_bytes < row_bytes)
    return set_error(KORE_EINVAL, "%s: bad sizes", what);
  if (n >= (1ll << 31) || rows >= (1ll << 31)) return set_error(KORE_EUNSUPPORTED, "%s: too many rows", what);
  const int vec = row_bytes % 16 == 0 && ld_src_bytes % 16 == 0 && ld_dst_bytes % 16 == 0 &&
                  ((uintptr_t)src & 15u) == 0 && ((uintptr_t)dst & 15u) == 0;
  if (scatter)
    hipLaunchKernelGGL(gather_rows_kernel<true>, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, ld_src_bytes, idx, row_bytes, (uint8_t*)dst, ld_dst_bytes, (int)rows, vec);
  else
    hipLaunchKernelGGL(gather_rows_kernel<false>, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, ld_src_bytes, idx, row_bytes, (uint8_t*)dst, ld_dst_bytes, (int)rows, vec);
  return check_launch(what);
}
}  // namespace
}  // namespace kore

extern "C" int kore_gather_rows(const void* src, int64_t ld_src_bytes, int64_t src_rows, const int32_t* idx, int64_t n,
                                int64_t row_bytes, void* dst, int64_t ld_dst_bytes, void* stream) {
  return kore::launch_rows(false, src, ld_src_bytes, idx, n, src_rows, row_bytes, dst, ld_dst_bytes, stream);
}

extern "C" int kore_scatter_rows(const void* src, int64_t ld_src_bytes, const int32_t* idx, int64_t n, void* dst,
                                 int64_t dst_rows, int64_t row_bytes, int64_t ld_dst_bytes, void* stream) {
  return kore::launch_rows(true, src, ld_src_bytes, idx, n, dst_rows, row_bytes, dst, ld_dst_bytes, stream);
}
