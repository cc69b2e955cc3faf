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
// Pipelined kernel: direct-to-LDS buffer loads, three LDS slots.
//
// Per slot (one K step = one 128-wide scale block): A 256 rows x 128 B, B 128 rows x
// 128 B, the 256 activation scales of the tile rows and one copy per wave of the
// block's weight scale -- scales travel through the same DMA pipeline as the
// operands, so their waits are the operands' waits.  Rows are XOR-swizzled in 32-byte
// units, key 2*((row >> 1) & 3): a lane's 32 K-consecutive bytes stay adjacent (two
// ds_read_b128 at +0/+16) and the 8 rows read by 8 lanes land on distinct 16-byte
// bank groups.  Each wave owns 128 x 64 outputs as 4 x 2 tiles of 32x32.  A tile's
// two MFMAs (K 0..63, 64..127) accumulate into one of two rotating partials; the
// promotion acc += partial * (xs * ws) of tile t-1 is issued between the two MFMAs
// of tile t, so the VALU work runs under the matrix pipe.
//
// Slot lifecycle (stage s in slot s % 3): after the barrier in tile 6 of stage s
// every wave has finished reading slot s % 3 and stage s+1 has landed; the loads of
// stage s+3 go out in tiles 6-7 of stage s and tiles 0-4 of stage s+1, two per tile,
// so each load has between one and two stages to arrive.
// ------------------------------------------------------------------------------
constexpr int kF8BM = 256, kF8BN = 128, kF8Slots = 3;
constexpr int kF8ABytes = kF8BM * 128, kF8BBytes = kF8BN * 128;
constexpr int kF8XOff = kF8ABytes + kF8BBytes;           // 256 fp32 activation scales
constexpr int kF8WOff = kF8XOff + 1024;                   // 4 waves x 64 copies of ws
constexpr int kF8Slot = kF8WOff + 1024;
constexpr int kF8Loads = 14;  // per wave per stage: 8 A, 4 B, 1 xs, 1 ws

__device__ __forceinline__ void buf_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint8_t* lds_dst,
                                        int size) {
  if (size == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, (int)voff, (int)soff, 0, 0);
  else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 4, (int)voff, (int)soff, 0, 0);
}

__device__ __forceinline__ i32x8_t lds_frag32(const uint8_t* p) {
  const u32x4_t lo = *(const u32x4_t*)p;
  const u32x4_t hi = *(const u32x4_t*)(p + 16);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// FULL_M: every row of the M tile exists, so all A loads of a wave share one
// per-lane offset and differ by a scalar row offset; otherwise rows are clamped per load.
template <bool FULL_M>
__global__ void __launch_bounds__(256)
    gemm_fp8_pipe_kernel(const Fp8Params p) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kF8Slots * kF8Slot];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, hh = lane >> 5;

  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int width = kFp8GroupM * p.tiles_n;
  const int grp = bid / width;
  const int first_m = grp * kFp8GroupM;
  const int gsz = min(p.tiles_m - first_m, kFp8GroupM);
  const int tl = bid - grp * width;
  const int m0 = (first_m + tl % gsz) * kF8BM;
  const int n0 = (tl / gsz) * kF8BN;
  const int rows_a = min(p.M - m0, kF8BM);
  const int nk = p.K / 128;

  // ---- buffer resources (tile-based) and per-lane load offsets ----
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.xq + (int64_t)m0 * p.ldx, (uint32_t)(rows_a * p.ldx));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.wq + (int64_t)n0 * p.ldw, (uint32_t)(kF8BN * p.ldw));
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(p.xs + (int64_t)m0 * p.xs_m, (uint32_t)(((rows_a - 1) * p.xs_m + (nk - 1) * p.xs_k + 1) * 4));
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(p.ws + (int64_t)(n0 / 128) * p.ws_n, (uint32_t)(((nk - 1) * p.ws_k + 1) * 4));
  // 16-byte chunk this lane fetches: row (lane >> 3) of an 8-row group, position lane & 7.
  const int dchunk = (lane & 7) ^ (2 * ((lane >> 4) & 3));
  const int lrow = lane >> 3;
  uint32_t a_voff[FULL_M ? 1 : 8];
  if constexpr (FULL_M) {
    a_voff[0] = (uint32_t)((lrow + 8 * wave) * p.ldx + 16 * dchunk);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      a_voff[j] = (uint32_t)(min(lrow + 8 * (wave + 4 * j), rows_a - 1) * p.ldx + 16 * dchunk);
  }
  const uint32_t b_voff = (uint32_t)((lrow + 8 * wave) * p.ldw + 16 * dchunk);
  const uint32_t x_voff = (uint32_t)(min(64 * wave + lane, rows_a - 1) * p.xs_m * 4);
  const uint32_t a_rstep = (uint32_t)(32 * p.ldx), b_rstep = (uint32_t)(32 * p.ldw);
  const uint32_t xs_kstep = (uint32_t)(p.xs_k * 4), ws_kstep = (uint32_t)(p.ws_k * 4);

  // load q of stage kb (already clamped to nk - 1) into slot
  auto issue = [&](int slot, int kb, int q) {
    uint8_t* base = lds + slot * kF8Slot;
    if (q < 8) {
      const uint32_t v = FULL_M ? a_voff[0] : a_voff[FULL_M ? 0 : q];
      const uint32_t so = (uint32_t)kb * 128u + (FULL_M ? (uint32_t)q * a_rstep : 0u);
      buf_lds(ra, v, so, base + (wave + 4 * q) * 1024, 16);
    } else if (q < 12) {
      buf_lds(rb, b_voff, (uint32_t)kb * 128u + (uint32_t)(q - 8) * b_rstep, base + kF8ABytes + (wave + 4 * (q - 8)) * 1024,
              16);
    } else if (q == 12) {
      buf_lds(rx, x_voff, (uint32_t)kb * xs_kstep, base + kF8XOff + wave * 256, 4);
    } else {
      buf_lds(rw, 0u, (uint32_t)kb * ws_kstep, base + kF8WOff + wave * 256, 4);
    }
  };

  // ---- fragment read offsets: row lr of a 32-row block, K sub-step h ----
  const int key = 2 * ((lr >> 1) & 3);
  const int offh0 = lr * 128 + (((2 * hh) ^ key) << 4);
  const int offh1 = lr * 128 + (((4 + 2 * hh) ^ key) << 4);
  const int rowA0 = wm * 128, rowB0 = wn * 64;

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  f32x16_t part[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) part[1][r] = 0.0f;
  const f32x16_t zero = {};
  float sc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float xsv[4], wsv;
  i32x8_t af[2][2], bf[2][2];  // af[buffer][h], bf[j][h]

  // ---- prologue: stages 0 and 1 in flight, wait for 0, first fragments ----
#pragma unroll
  for (int q = 0; q < kF8Loads; ++q) issue(0, 0, q);
#pragma unroll
  for (int q = 0; q < kF8Loads; ++q) issue(1, min(1, nk - 1), q);
  wait_vmcnt<kF8Loads>();
  exec_barrier();
  {
    const uint8_t* cur = lds;
    af[0][0] = lds_frag32(cur + rowA0 * 128 + offh0);
    af[0][1] = lds_frag32(cur + rowA0 * 128 + offh1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf[j][0] = lds_frag32(cur + kF8ABytes + (rowB0 + 32 * j) * 128 + offh0);
      bf[j][1] = lds_frag32(cur + kF8ABytes + (rowB0 + 32 * j) * 128 + offh1);
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) issue(2, min(2, nk - 1), q);

  int slot = 0;
  for (int s = 0; s < nk; ++s) {
    const int slot1 = slot == 2 ? 0 : slot + 1;
    const int slot2 = slot1 == 2 ? 0 : slot1 + 1;
    const uint8_t* cur = lds + slot * kF8Slot;
    const uint8_t* nxt = lds + slot1 * kF8Slot;
    const int kb2 = min(s + 2, nk - 1), kb3 = min(s + 3, nk - 1);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int i = t >> 1, j = t & 1;
      if (t == 6) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<kF8Loads>();
        exec_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      part[j] = mma32_fp8(bf[j][0], af[i & 1][0], zero);
      __builtin_amdgcn_sched_barrier(0);
      if (t == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[q] = xsv[q] * wsv;
      }
      {
        // promote the previous tile (t == 0: tile 7 of the previous stage, whose
        // scale sc[3] is still live; zeros before the first stage)
        const int pt = (t + 7) & 7;
        const float f = sc[pt >> 1];
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[pt >> 1][pt & 1][r] = fmaf(part[j ^ 1][r], f, acc[pt >> 1][pt & 1][r]);
      }
      __builtin_amdgcn_sched_barrier(0);
      part[j] = mma32_fp8(bf[j][1], af[i & 1][1], part[j]);
      __builtin_amdgcn_sched_barrier(0);
      // LDS reads: scales of this stage, A of the next row block, B of the next stage
      if (t == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) xsv[q] = *(const float*)(cur + kF8XOff + (rowA0 + 32 * q + lr) * 4);
        wsv = *(const float*)(cur + kF8WOff + wave * 256 + lane * 4);
      }
      if (t < 6) {
        const uint8_t* src = cur + (rowA0 + 32 * (i + 1)) * 128 + (j ? offh1 : offh0);
        af[(i + 1) & 1][j] = lds_frag32(src);
      } else {
        const uint8_t* src = nxt + rowA0 * 128 + (j ? offh1 : offh0);
        af[0][j] = lds_frag32(src);
        bf[j][0] = lds_frag32(nxt + kF8ABytes + (rowB0 + 32 * j) * 128 + offh0);
        bf[j][1] = lds_frag32(nxt + kF8ABytes + (rowB0 + 32 * j) * 128 + offh1);
      }
      // direct loads: stage s+2 (tiles 0-4, loads 4..13), stage s+3 (tiles 6-7, loads 0..3)
      if (t <= 4) {
        issue(slot2, kb2, 4 + 2 * t);
        issue(slot2, kb2, 5 + 2 * t);
      } else if (t >= 6) {
        issue(slot, kb3, 2 * (t - 6));
        issue(slot, kb3, 2 * (t - 6) + 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    slot = slot1;
  }
  // promote the last tile of the last stage
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[3][1][r] = fmaf(part[1][r], sc[3], acc[3][1][r]);
  wait_vmcnt<0>();  // the clamped trailing loads must land before LDS is reused
  __syncthreads();

  // ---- epilogue: bf16 pack, stage per wave, 16-byte row stores ----
  using St = Stager<128, 64>;
  using Op = MfmaOp<BF16>;
  uint16_t* stg = (uint16_t*)lds + wave * (128 * 64);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
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
    if (gm < p.M) store_row8(p.y + (int64_t)gm * p.ldy + gn, gn, p.N, vec, v);
  });
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

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
  Fp8Params p;
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
  // the pipelined kernel addresses each tile through 32-bit buffer offsets
  const bool pipe_ok = 256 * ldx + K < (1ll << 31) && 128 * ldw + K < (1ll << 31) &&
                       (M * xs_m + K / 128 * xs_k) * 4 < (1ll << 31) && (K / 128 * ws_k) * 4 < (1ll << 31);
  if (pipe_ok) {
    if (M % BM == 0)
      hipLaunchKernelGGL((gemm_fp8_pipe_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
    else
      hipLaunchKernelGGL((gemm_fp8_pipe_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
    return check_launch("gemm_fp8_pipe_kernel");
  }
  hipLaunchKernelGGL((gemm_fp8_bs_kernel<BM, BN>), dim3((unsigned)blocks), dim3(kEngineThreads), 0,
                     (hipStream_t)stream, p);
  return check_launch("gemm_fp8_bs_kernel");
}
