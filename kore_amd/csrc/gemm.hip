// Dense and batched bf16/fp16 GEMM with fused bias + activation epilogue (gfx950).
//
// C[M,N] = act(A[M,K] @ B[K,N] + bias[N]) with fp32 accumulation, one RNE cast.
//
// Large grids (>= 192 tiles of 256x256, K % 64 == 0): gemm_buf_kernel on the buffer
// engine (BufPipeEngine, tile_engine.hpp).  Operands go straight from global memory into
// LDS with buffer_load ... lds (no VGPR staging), two 64-wide K stages in flight, one
// barrier per stage, 16x16x32 MFMAs.  K-contiguous B runs 4 waves (2 x 2, 128 x 128 each,
// one per SIMD, the accumulators held in place in AGPRs); an N-contiguous B (natural [K,N])
// or an M-contiguous A (a transposed view) runs 8 waves (2 x 4, 128 x 64 each, two per
// SIMD), staged as K-rows and read back with the LDS transpose read ds_read_b64_tr_b16.  LDS rows are 128 bytes with an XOR swizzle of the 16-byte chunks.
// The MFMA is issued with the B fragment as the first operand, so each lane holds 4
// N-consecutive outputs of one row; the epilogue applies bias and the activation in fp32,
// packs, stages the wave's tile in LDS and writes C with 16-byte row-contiguous stores.
//
// Mid-size grids run the deep ring engine (gemm_deep_kernel: several K stages in
// flight); decode-sized M splits K (gemm_splitk_kernel + a fixed-order reduction);
// 1024^3-like problems the skinny ring (gemm_ring_kernel); K tails and small K the
// register-staged tile engine (gemm_tile_kernel); batched K of 64 or 128 the persistent
// short-K kernel.  Generic path: any strides and any K, 128x128 MFMA tiles fed by
// bounds-checked element reads along the unit-stride index (gemm_generic_mfma_kernel).
#include "../../include/kore_amd.h"
#include "kore_common.hpp"
#include "tile_engine.hpp"

#include <algorithm>
#include <type_traits>

namespace kore {
namespace {

struct TileParams {
  const uint16_t* a;
  const uint16_t* b;
  const uint16_t* bias;
  uint16_t* c;
  int M, N, K;
  int64_t lda;  // A row stride (elements); A is K-contiguous
  int64_t ldb;  // B_KC: stride between n rows of B^T;  B_NC: stride between k rows of B
  int64_t ldc;  // C row stride; C is N-contiguous
  int64_t sa, sb, sc;  // batch strides (elements)
  int tiles_m, tiles_n, tiles_per_batch;
  int batch;  // number of batches (the persistent short-K kernel walks all of them)
  int kb;     // valid K-rows of an N-contiguous B on the direct-to-LDS engines (rows
              // from kb on fall outside the buffer resource and read as zero)
  int kreal;  // K-tail mode of the buffer engine: the true K (K is then rounded up to 64)
  int act;
  int vec_store;  // 16-byte C stores allowed (ldc % 8 == 0, aligned)
  int bias_vec;   // bias is 8-byte aligned: 4-wide bias loads allowed
};

constexpr int kGroupM = 4;

// Bias + activation in fp32, RNE pack, per-wave LDS staging, 16-byte row stores.
// Must be entered after a barrier that ends all reads of the K-loop buffers.
// get(i, j, g, e): element 4g + e of the lane's accumulator of 32x32 tile (i, j), whose
// output position is (acc_row<M16>(i, g), acc_col<M16>(j, g) + e).
template <typename T, int MI, int NI, int WROWS, int WCOLS, bool M16, typename Get>
__device__ __forceinline__ void dense_epilogue_at(Get&& get, uint16_t* lds, const TileParams& p, int m0, int n0, int wm,
                                                  int wn, int wave, int lane, uint16_t* C) {
  using Op = MfmaOp<T>;
  using St = Stager<WROWS, WCOLS>;
  const int M = p.M, N = p.N;
  uint16_t* stg = lds + wave * (WROWS * WCOLS);
  const int mw0 = m0 + wm * WROWS, nw0 = n0 + wn * WCOLS;
  auto epi = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nl = acc_col<M16>(j, g, lane);
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias != nullptr) {
          const int n = nw0 + nl;
          if (p.bias_vec && n + 4 <= N) {  // 4 consecutive bias values in one 8-byte load
            const u32x2_t w = *(const u32x2_t*)(p.bias + n);
            bv[0] = Op::to_f32((uint16_t)(w[0] & 0xffffu));
            bv[1] = Op::to_f32((uint16_t)(w[0] >> 16));
            bv[2] = Op::to_f32((uint16_t)(w[1] & 0xffffu));
            bv[3] = Op::to_f32((uint16_t)(w[1] >> 16));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = n + e < N ? Op::to_f32(p.bias[n + e]) : 0.0f;
          }
        }
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = apply_act<ACT>(get(i, j, g, e) + bv[e]);
          St::put(stg, acc_row<M16>(i, g, lane), nl, u32x2_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3])});
        }
      }
    }
  };
  switch (p.act) {
    case ACT_RELU: epi(std::integral_constant<int, ACT_RELU>{}); break;
    case ACT_GELU: epi(std::integral_constant<int, ACT_GELU>{}); break;
    case ACT_SILU: epi(std::integral_constant<int, ACT_SILU>{}); break;
    case ACT_TANH: epi(std::integral_constant<int, ACT_TANH>{}); break;
    case ACT_SIGMOID: epi(std::integral_constant<int, ACT_SIGMOID>{}); break;
    default: epi(std::integral_constant<int, ACT_NONE>{}); break;
  }
  __syncthreads();
  const bool vec = p.vec_store != 0;
  St::drain(stg, lane, [&](int row, int col, u32x4_t v) {
    const int gm = mw0 + row, gn = nw0 + col;
    if (gm < M) store_row8(C + (int64_t)gm * p.ldc + gn, gn, N, vec, v);
  });
}

template <typename T, int MI, int NI, int WROWS, int WCOLS>
__device__ __forceinline__ void dense_epilogue(f32x16_t (&acc)[MI][NI], uint16_t* lds, const TileParams& p, int m0,
                                               int n0, int wm, int wn, int wave, int lane, uint16_t* C) {
  dense_epilogue_at<T, MI, NI, WROWS, WCOLS, false>([&](int i, int j, int g, int e) { return acc[i][j][4 * g + e]; },
                                                    lds, p, m0, n0, wm, wn, wave, lane, C);
}
template <typename T, int MI, int NI, int WROWS, int WCOLS>
__device__ __forceinline__ void dense_epilogue16(f32x4_t (&c4)[MI][NI][4], uint16_t* lds, const TileParams& p, int m0,
                                                 int n0, int wm, int wn, int wave, int lane, uint16_t* C) {
  dense_epilogue_at<T, MI, NI, WROWS, WCOLS, true>([&](int i, int j, int g, int e) { return c4[i][j][g][e]; }, lds, p,
                                                   m0, n0, wm, wn, wave, lane, C);
}

// Tile coordinates: XCD-aware remap, then grouped raster per batch.
__device__ __forceinline__ void tile_coords(const TileParams& p, int BM, int BN, int& batch, int& m0, int& n0) {
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  batch = bid / p.tiles_per_batch;
  const int t = bid - batch * p.tiles_per_batch;
  const int width = kGroupM * p.tiles_n;
  const int grp = t / width;
  const int first_m = grp * kGroupM;
  const int gsz = min(p.tiles_m - first_m, kGroupM);
  const int tl = t - grp * width;
  m0 = (first_m + tl % gsz) * BM;
  n0 = (tl / gsz) * BN;
}

template <typename T, int BL, int BM, int BN>
__global__ void __launch_bounds__(kEngineThreads)
    gemm_tile_kernel(const TileParams p) {
  using E = TileEngine<T, BM, BN, 2, 2, BL>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  int batch, m0, n0;
  tile_coords(p, BM, BN, batch, m0, n0);

  const uint16_t* A = p.a + batch * p.sa;
  const uint16_t* B = p.b + batch * p.sb;
  uint16_t* C = p.c + batch * p.sc;
  const int M = p.M, N = p.N, K = p.K;

  E eng;
  const int ch8 = (tid & 7) * 8;
#pragma unroll
  for (int j = 0; j < E::LA; ++j) eng.a_src[j] = A + (int64_t)min(m0 + E::a_row_of(tid, j), M - 1) * p.lda + ch8;
  if constexpr (BL == B_KC) {
#pragma unroll
    for (int j = 0; j < E::LB; ++j) eng.b_src[j] = B + (int64_t)min(n0 + E::b_row_of(tid, j), N - 1) * p.ldb + ch8;
  } else {
#pragma unroll
    for (int j = 0; j < E::LB; ++j)
      eng.b_src[j] = B + (int64_t)(E::nc_kb(tid, j) * 8) * p.ldb + min(n0 + E::nc_nb(tid, j) * 8, N - 8);
  }
  eng.ldb = p.ldb;

  f32x16_t acc[MI][NI];
  E::zero(acc);
  eng.mainloop(lds, K, acc);

  dense_epilogue<T, MI, NI, E::WROWS, E::WCOLS>(acc, lds, p, m0, n0, wm, wn, wave, lane, C);
}


// Buffer resources and per-lane byte offsets of the direct-to-LDS engines.  Rows of A
// and of B^T past the tile's last valid row re-read that row; N-contiguous B is read
// as K-rows of the n0 column block whose chunks past N (N % 8 == 0) re-read the last
// chunk.  Either way the extra values only feed outputs that are never stored.
template <typename E, int BM, int BN, int BL>
__device__ __forceinline__ void setup_operands(E& eng, const TileParams& p, int batch, int m0, int n0, int wave,
                                               int lane) {
  const int rows_a = min(BM, p.M - m0), rows_b = min(BN, p.N - n0);
  const int kv = p.kreal > 0 ? p.kreal : p.K;  // K the operands hold
  if constexpr (E::AMC) {
    // M-contiguous A (element (m, k) at a[k * lda + m], M % 8 == 0): K-rows of the tile's
    // BM columns; chunks past M re-read the last one (their rows are never stored)
    const uint16_t* A = p.a + batch * p.sa + m0;
    eng.ra = make_rsrc(A, (uint32_t)(((int64_t)(p.K - 1) * p.lda + rows_a) * 2));
    eng.a_kstep = (uint32_t)(kBK * p.lda * 2);
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int kr = E::amc_krow(wave, lane, j);
      eng.a_voff[j] = (uint32_t)(((int64_t)kr * p.lda + min(8 * E::amc_chunk(kr, lane), rows_a - 8)) * 2);
    }
  } else {
    const uint16_t* A = p.a + batch * p.sa + (int64_t)m0 * p.lda;
    eng.ra = make_rsrc(A, (uint32_t)(((int64_t)(rows_a - 1) * p.lda + kv) * 2));
#pragma unroll
    for (int j = 0; j < E::AJ; ++j) {
      const int r = E::a_row(wave, lane, j);
      eng.a_voff[j] = (uint32_t)(((int64_t)min(r, rows_a - 1) * p.lda + 8 * E::chunk(r, lane)) * 2);
    }
  }
  if constexpr (BL == B_KC) {
    const uint16_t* B = p.b + batch * p.sb + (int64_t)n0 * p.ldb;
    eng.rb = make_rsrc(B, (uint32_t)(((int64_t)(rows_b - 1) * p.ldb + kv) * 2));
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      const int r = E::b_row(wave, lane, j);
      eng.b_voff[j] = (uint32_t)(((int64_t)min(r, rows_b - 1) * p.ldb + 8 * E::chunk(r, lane)) * 2);
    }
  } else {
    const uint16_t* B = p.b + batch * p.sb + n0;
    eng.rb = make_rsrc(B, (uint32_t)(((int64_t)(p.kb - 1) * p.ldb + rows_b) * 2));
    eng.b_kstep = (uint32_t)(kBK * p.ldb * 2);
#pragma unroll
    for (int j = 0; j < E::BJ; ++j) {
      const int kr = E::nc_krow(wave, lane, j);
      eng.b_voff[j] = (uint32_t)(((int64_t)kr * p.ldb + min(8 * E::nc_chunk(kr, lane), rows_b - 8)) * 2);
    }
  }
}

// Buffer-load pipelined variant for K-contiguous A, K % 64 == 0 and either B layout:
// K-contiguous B (the A.B^T / A.W^T layouts) or N-contiguous B (natural [K, N], N % 8 ==
// 0), whose fragments come out of LDS through transpose reads.
// 16x16x32 MFMAs.  NWV = 4 (K-contiguous B): 2 x 2 waves of 128 x 128, one per SIMD, the
// accumulators held in place in the 256 AGPRs (mma16_acc).  NWV = 8 (N-contiguous B): 2 x 4
// waves of 128 x 64, two per SIMD; an N-contiguous B reaches the 16x16 fragments through
// transpose reads with the nc_x16 chunk swizzle.  AL = A_MC: A is M-contiguous (a transposed
// view) and read like an N-contiguous B (8 waves only).  KT: K tails (K % 64 != 0) read in
// place (mainloop16<true>).
template <typename T, int BM, int BN, int BL, int NWV, int AL, bool KT = false>
__global__ void __launch_bounds__(64 * NWV)
    gemm_buf_kernel(const TileParams p) {
  using E = BufPipeEngine<T, BM, BN, 2, NWV / 2, 1, BL, kCpolDefault, NWV == 8 || BL == B_KC, AL>;
  constexpr int MI = E::MI, NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / E::WN, wn = wave % E::WN;
  int batch, m0, n0;
  tile_coords(p, BM, BN, batch, m0, n0);
  E eng;
  setup_operands<E, BM, BN, BL>(eng, p, batch, m0, n0, wave, lane);
  if constexpr (KT) {  // last stage at K - 64 (bytes along a row / over N-contiguous K-rows)
    eng.a_klast = (uint32_t)((p.kreal - kBK) * 2);
    eng.b_klast = BL == B_NC ? (uint32_t)((int64_t)(p.kreal - kBK) * p.ldb * 2) : eng.a_klast;
    eng.kdup = p.K - p.kreal;
  }
  if constexpr (E::M16) {
    f32x4_t acc[MI][NI][4];
    E::zero16(acc);
    eng.template mainloop16<KT>(lds, p.K, acc);
    dense_epilogue16<T, MI, NI, E::WROWS, E::WCOLS>(acc, lds, p, m0, n0, wm, wn, wave, lane, p.c + batch * p.sc);
  } else {
    static_assert(!KT, "K tails run on the 16x16 engine");
    f32x16_t acc[MI][NI];
    E::zero(acc);
    eng.mainloop(lds, p.K, acc);
    dense_epilogue<T, MI, NI, E::WROWS, E::WCOLS>(acc, lds, p, m0, n0, wm, wn, wave, lane, p.c + batch * p.sc);
  }
}

// Mid-size problems (a few hundred tiles, long K) on the deep ring engine: NSLOT - 1
// K stages in flight per CU instead of one or two.  Either B layout, K % 64 == 0 (KT:
// K tails read in place, the ring engine's K-tail mode).
template <typename T, int BM, int BN, int WM, int WN, int NSLOT, int BL, bool KT = false>
__global__ void __launch_bounds__(256) gemm_deep_kernel(const TileParams p) {
  using E = RingEngine<T, BM, BN, WM, WN, NSLOT, BL>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int batch, m0, n0;
  tile_coords(p, BM, BN, batch, m0, n0);
  E eng;
  setup_operands<E, BM, BN, BL>(eng, p, batch, m0, n0, wave, lane);
  if constexpr (KT) {  // last stage at K - 64 (bytes along a row / over N-contiguous K-rows)
    eng.a_klast = (uint32_t)((p.kreal - kBK) * 2);
    eng.b_klast = BL == B_NC ? (uint32_t)((int64_t)(p.kreal - kBK) * p.ldb * 2) : eng.a_klast;
    eng.kdup = p.K - p.kreal;
  }
  f32x16_t acc[E::MI][E::NI];
  E::zero(acc);
  eng.template mainloop<KT>(lds, p.K, acc);
  dense_epilogue<T, E::MI, E::NI, E::WROWS, E::WCOLS>(acc, lds, p, m0, n0, wave / WN, wave % WN, wave, lane,
                                                      p.c + batch * p.sc);
}

// ---------------------------------------------------------------------------------
// Split-K for small problems with a long K (decode-sized M: 1x4096x4096 has 32 tiles of
// 32x128 for 256 CUs).  Workgroup (tile, s) runs the 32x128 deep ring over K slice s and
// writes its fp32 partial tile to part[s]; splitk_reduce_kernel then sums the slices in
// a fixed order (deterministic), applies bias and activation and stores C.
// ---------------------------------------------------------------------------------
template <typename T, int BL, int BM, int BN, int WM, int WN, int NSLOT>
__global__ void __launch_bounds__(256) gemm_splitk_kernel(const TileParams p, float* part, int splits, int kper) {
  using E = RingEngine<T, BM, BN, WM, WN, NSLOT, BL, kCpolNT>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = (int)blockIdx.x % splits, t = (int)blockIdx.x / splits;
  const int m0 = (t % p.tiles_m) * BM, n0 = (t / p.tiles_m) * BN;
  const int k_begin = s * kper, k_end = min(p.K, k_begin + kper);
  E eng;
  setup_operands<E, BM, BN, BL>(eng, p, 0, m0, n0, wave, lane);
  f32x16_t acc[E::MI][E::NI];
  E::zero(acc);
  eng.mainloop_range(lds, k_begin, k_end, acc);
  float* dst = part + (int64_t)s * p.M * p.N;
  const int mw = m0 + (wave / WN) * E::WROWS, nw = n0 + (wave % WN) * E::WCOLS;
#pragma unroll
  for (int i = 0; i < E::MI; ++i) {
    const int m = mw + out_row(i, lane);
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < E::NI; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nw + out_col(j, g, lane);
        float* q = dst + (int64_t)m * p.N + n;
        if ((p.N & 3) == 0 && n + 4 <= p.N) {
          *(f32x4_t*)q = f32x4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.N) q[e] = acc[i][j][4 * g + e];
        }
      }
  }
}

// Fixed-order sum of the split-K partials (slice 0, 1, ...), then bias, activation and
// the store.  CW columns per thread: 4 with 16-byte partial loads when N % 4 == 0 -- the
// loads of four slices go out before their adds, so their latencies overlap (a decode
// GEMM reduces one row on a handful of workgroups) -- otherwise 8 scalar columns.
template <typename T, int CW>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* part, int splits, int M, int N,
                                                            const uint16_t* bias, int act, uint16_t* C, int64_t ldc,
                                                            int vec) {
  using Op = MfmaOp<T>;
  const int nc = (N + CW - 1) / CW;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * nc) return;
  const int m = (int)(idx / nc), n = (int)(idx % nc) * CW;
  float v[CW];
#pragma unroll
  for (int e = 0; e < CW; ++e) v[e] = 0.0f;
  if constexpr (CW == 4) {
    const float* q = part + (int64_t)m * N + n;
    const int64_t slice = (int64_t)M * N;
    int s = 0;
    for (; s + 4 <= splits; s += 4) {
      f32x4_t a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = *(const f32x4_t*)(q + (s + u) * slice);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += a[u][e];
    }
    for (; s < splits; ++s) {
      const f32x4_t a = *(const f32x4_t*)(q + s * slice);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += a[e];
    }
  } else {
    for (int s = 0; s < splits; ++s) {
      const float* q = part + ((int64_t)s * M + m) * N + n;
#pragma unroll
      for (int e = 0; e < CW; ++e)
        if (n + e < N) v[e] += q[e];
    }
  }
  if (bias != nullptr) {
#pragma unroll
    for (int e = 0; e < CW; ++e)
      if (n + e < N) v[e] += Op::to_f32(bias[n + e]);
  }
  auto fin = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int e = 0; e < CW; ++e) v[e] = apply_act<ACT>(v[e]);
  };
  switch (act) {
    case ACT_RELU: fin(std::integral_constant<int, ACT_RELU>{}); break;
    case ACT_GELU: fin(std::integral_constant<int, ACT_GELU>{}); break;
    case ACT_SILU: fin(std::integral_constant<int, ACT_SILU>{}); break;
    case ACT_TANH: fin(std::integral_constant<int, ACT_TANH>{}); break;
    case ACT_SIGMOID: fin(std::integral_constant<int, ACT_SIGMOID>{}); break;
    default: break;
  }
  uint16_t* out = C + (int64_t)m * ldc + n;
  if (vec && n + CW <= N) {
    if constexpr (CW == 4)
      *(u32x2_t*)out = u32x2_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3])};
    else
      *(u32x4_t*)out = u32x4_t{Op::pack2(v[0], v[1]), Op::pack2(v[2], v[3]), Op::pack2(v[4], v[5]),
                               Op::pack2(v[6], v[7])};
  } else {
#pragma unroll
    for (int e = 0; e < CW; ++e)
      if (n + e < N) out[e] = (uint16_t)(Op::pack2(v[e], 0.0f) & 0xffffu);
  }
}

// ---------------------------------------------------------------------------------
// Small problems (fewer than 128 tiles of 128x128, e.g. 1024^3 with 64): the time is
// load latency, not MFMA work (a 64x64 tile with a register double buffer waits one
// full memory round trip per 64-wide K step).  32 x BN tiles on the skinny ring
// engine instead: four times the tiles of 64x64 at BN = 128 (256 for 1024^3, one per
// CU) and an NSLOT-deep ring of direct-to-LDS K stages, NSLOT - 1 of them in flight
// per CU.  Waves sit side by side over N (32 x BN/4 each); the epilogue is the dense
// one (bias, activation, 16-byte row stores).  K % 64 == 0, A and B K-contiguous.
// ---------------------------------------------------------------------------------
template <typename T, int BN, int NSLOT>
__global__ void __launch_bounds__(256) gemm_ring_kernel(const TileParams p) {
  using E = SkinnyRingEngine<T, BN, 1, NSLOT>;
  constexpr int NI = E::NI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[E::LDS_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int batch, m0, n0;
  tile_coords(p, E::BM, BN, batch, m0, n0);
  const uint16_t* A = p.a + batch * p.sa + (int64_t)m0 * p.lda;
  const uint16_t* B = p.b + batch * p.sb + (int64_t)n0 * p.ldb;
  const int rows_a = min(E::BM, p.M - m0), rows_b = min(BN, p.N - n0);
  E eng;
  eng.ra = make_rsrc(A, (uint32_t)(((int64_t)(rows_a - 1) * p.lda + p.K) * 2));
  eng.rb = make_rsrc(B, (uint32_t)(((int64_t)(rows_b - 1) * p.ldb + p.K) * 2));
  const int ar = E::a_row(wave, lane);
  eng.a_voff[0] = (uint32_t)(((int64_t)min(ar, rows_a - 1) * p.lda + 8 * E::chunk(ar, lane)) * 2);
#pragma unroll
  for (int j = 0; j < E::BJ; ++j) {
    const int r = E::b_row(wave, lane, j);
    eng.b_voff[j] = (uint32_t)(((int64_t)min(r, rows_b - 1) * p.ldb + 8 * E::chunk(r, lane)) * 2);
  }
  f32x16_t acc[1][NI];
  E::zero(acc);
  eng.mainloop(lds, 0, p.K, acc);
  dense_epilogue<T, 1, NI, E::BM, E::WCOLS>(acc, lds, p, m0, n0, 0, wave, wave, lane, p.c + batch * p.sc);
}

// ---------------------------------------------------------------------------------
// Persistent short-K kernel (K = 64 * NKS, NKS = 1 or 2; A K-contiguous).
//
// With K = 128 a 128x128 tile is 4 MFLOP against 32 KiB of output, so the time is the
// output stream.  A store instruction stalls its wave while the memory system pushes
// back, so a wave that both multiplies and stores serialises the two (measured with
// s_memtime: ~1.5 us of every ~2.3 us per tile went to issuing the stores while no
// other work ran).  Here one workgroup per CU has two roles, one wave of each per SIMD:
//  * waves 0-3 (compute) load A, multiply and pack: wave w owns rows 32w .. 32w + 31
//    and all 128 columns, and packs its finished rows into the LDS it read its own A
//    rows from (so no other wave's operands are overwritten);
//  * waves 4-7 (store) write the previous tile from LDS to memory with 16-byte
//    row-contiguous buffer stores and never wait on vmcnt, so the output stream runs
//    while the next tile is multiplied, and a compute wave's vmcnt counts its loads only.
// Each tile walks three LDS slots: A rows (loaded two tiles ahead, direct-to-LDS), then
// the packed output, then free.  One workgroup walks "segments": runs of up to SEG tiles
// down one column of the output (one batch, one 128-column block of B, consecutive
// 128-row blocks of A); the B block is loaded once per segment (K-contiguous B by direct
// loads, N-contiguous B -- the B.transpose(1, 2) view of a [B, K, N] tensor -- through
// registers, 8 K-rows x 8 columns per thread, transposed with v_perm into the same
// K-contiguous layout).  Rows past M and columns past N get an offset beyond the buffer
// size, which the hardware drops.
//
// Segment order: u = (batch * nseg + seg) * tiles_n + n-block, so consecutive segments
// share their A blocks; when the grid and the segment count are multiples of 8, XCD x
// (the workgroups g with g % 8 == x, dispatched round-robin) owns the x-th eighth of the
// segments and its 32 CUs read the same A blocks from its L2 at the same time.  Tiles
// past the last row block (when SEG does not divide it) load the last block again and
// store nothing.
// ---------------------------------------------------------------------------------

template <typename T, int NKS, int BL>
__global__ void __launch_bounds__(512) gemm_shortk_kernel(const TileParams p, const int seg) {
  using Op = MfmaOp<T>;
  constexpr int BM = 128, BN = 128, NW = 4, WROWS = 32, NI = 4, NA = 3;
  constexpr int A_ELEMS = BM * kBK, B_ELEMS = BN * kBK;  // one 64-wide K stage
  // a slot holds the tile's A rows, then its packed output (rows of 256 bytes)
  constexpr int A_BUF = NKS * A_ELEMS > BM * BN ? NKS * A_ELEMS : BM * BN;
  constexpr int HALF = A_BUF / 2;                 // 16 KiB: the second K stage / rows 16..31
  constexpr int B_OFF = NA * A_BUF;
  constexpr bool NC = BL == B_NC;
  constexpr int AJ = BM / 8 / NW, BJ = BN / 8 / NW;
  constexpr int NQ = NKS * 4;                     // 16-wide K sub-steps
  // sub-steps whose B fragments stay in registers for the whole segment: N-contiguous B
  // keeps none (its segment-start transposes need those registers; 256 VGPRs at most)
  constexpr int NQR = NC ? 0 : (NQ < 4 ? NQ : 4);
  constexpr int L = NKS * AJ;                     // A loads per compute wave per tile
  constexpr int NCBLK = (NKS * kBK / 8) * (BN / 8);  // 8x8 blocks of an N-contiguous B tile
  static_assert(NCBLK <= 256, "one 8x8 block per compute thread");
  static_assert(HALF == 16 * 128 * 4, "a wave's 16 output rows (4 KiB) per half slot");
  __shared__ __attribute__((aligned(1024))) uint16_t lds[NA * A_BUF + NKS * B_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool storer = wave >= NW;
  const int w = wave & 3, ctid = tid & 255;
  const int lr = lane & 31, hh = lane >> 5;
  const int rowA0 = w * WROWS;

  // ---- this workgroup's segments u = first + k * step, k < nsegs ----
  const int nseg = (p.tiles_m + seg - 1) / seg;
  const int total = p.batch * nseg * p.tiles_n;
  const int G = (int)gridDim.x, g = (int)blockIdx.x;
  int first, step, nsegs;
  if ((G & 7) == 0 && (total & 7) == 0) {
    const int per = total >> 3, c = g >> 3, gx = G >> 3;
    first = (g & 7) * per + c;
    step = gx;
    nsegs = c < per ? (per - c + gx - 1) / gx : 0;
  } else {
    first = g;
    step = G;
    nsegs = g < total ? (total - g + G - 1) / G : 0;
  }
  const int count = nsegs * seg;
  // tile i of this workgroup: batch, row block mb (live if < tiles_m), column n0
  auto tile_of = [&](int i, int& batch, int& mb, int& n0) {
    const int k = i / seg;
    const int u = first + k * step;
    const int bs = u / p.tiles_n;
    n0 = (u - bs * p.tiles_n) * BN;
    batch = bs / nseg;
    mb = (bs - batch * nseg) * seg + (i - k * seg);
  };

  // ---- (compute waves) A rows of tile i into slot `slot`, direct-to-LDS, all of K ----
  auto issue_a = [&](int i, int slot) {
    int batch, mb, n0;
    tile_of(i, batch, mb, n0);
    const int m0 = min(mb, p.tiles_m - 1) * BM;
    const int rows_a = min(BM, p.M - m0);
    const uint16_t* A = p.a + (int64_t)batch * p.sa + (int64_t)m0 * p.lda;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)(((int64_t)(rows_a - 1) * p.lda + p.K) * 2));
    uint16_t* base = lds + slot * A_BUF;
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      const int r = (w + NW * j) * 8 + (lane >> 3);
      const uint32_t v = (uint32_t)((min(r, rows_a - 1) * (int)p.lda + 8 * ((lane & 7) ^ swz8(r))) * 2);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        buf_lds16(ra, v, (uint32_t)ks * (kBK * 2), base + ks * A_ELEMS + (w + NW * j) * 8 * kBK);
    }
  };

  // ---- (compute waves) the B block of tile i's column into LDS; complete (for this
  // wave) on return ----
  auto load_b = [&](int i) {
    int batch, mb, n0;
    tile_of(i, batch, mb, n0);
    uint16_t* sB = lds + B_OFF;
    if constexpr (!NC) {
      const int rows_b = min(BN, p.N - n0);
      const uint16_t* B = p.b + (int64_t)batch * p.sb + (int64_t)n0 * p.ldb;
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)(((int64_t)(rows_b - 1) * p.ldb + p.K) * 2));
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const int r = (w + NW * j) * 8 + (lane >> 3);
        const uint32_t v = (uint32_t)((min(r, rows_b - 1) * (int)p.ldb + 8 * ((lane & 7) ^ swz8(r))) * 2);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          buf_lds16(rb, v, (uint32_t)ks * (kBK * 2), sB + ks * B_ELEMS + (w + NW * j) * 8 * kBK);
      }
      wait_vmcnt<0>();
    } else {
      // compute thread t owns block (kb, nb) = (t / 16, t % 16); N % 8 == 0, so a block is
      // wholly inside or past N, and blocks past N re-read the last one (never stored)
      const int kb = ctid / (BN / 8), nb = ctid % (BN / 8);
      if (ctid < NCBLK) {
        const uint16_t* src = p.b + (int64_t)batch * p.sb + (int64_t)(8 * kb) * p.ldb + min(n0 + 8 * nb, p.N - 8);
        u32x4_t rows[8], tr[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) rows[r] = ld16(src + (int64_t)r * p.ldb);
        transpose8x8(rows, tr);
        uint16_t* dst = sB + (kb >> 3) * B_ELEMS;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int n = 8 * nb + jj;
          *(u32x4_t*)(dst + n * kBK + (((kb & 7) ^ swz8(n)) << 3)) = tr[jj];
        }
      }
    }
  };

  // Packed output of compute wave w in a slot: its rows 0..15 at w * 4 KiB, rows 16..31
  // at HALF + w * 4 KiB (exactly where its own A rows of K stages 0 and 1 were);
  // 256-byte rows whose 16-byte chunk c sits at c ^ (row % 16).
  auto out_addr = [&](uint16_t* slotp, int ww, int row, int chunk) -> uint16_t* {
    return slotp + (row >> 4) * HALF + ww * 2048 + (row & 15) * 128 + ((chunk ^ (row & 15)) << 3);
  };

  // ---- (store waves) write the packed tile i of slot `slot` ----
  auto store_tile = [&](int i, int slot) {
    int batch, mb, n0;
    tile_of(i, batch, mb, n0);
    const int rows_c = mb < p.tiles_m ? min(BM, p.M - mb * BM) : 0, cols_c = min(BN, p.N - n0);
    uint16_t* Cb = p.c + (int64_t)batch * p.sc + (int64_t)min(mb, p.tiles_m - 1) * BM * p.ldc + n0;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(Cb, (uint32_t)(((int64_t)(BM - 1) * p.ldc + cols_c) * 2));
    uint16_t* slotp = lds + slot * A_BUF;
    // store wave w writes compute wave w's 32 rows: 4 rows of 16 chunks per instruction
#pragma unroll
    for (int it = 0; it < WROWS / 4; ++it) {
      const int row = it * 4 + (lane >> 4), chunk = lane & 15;
      const u32x4_t v = *(const u32x4_t*)out_addr(slotp, w, row, chunk);
      const int r = rowA0 + row, c = chunk * 8;
      const bool ok = r < rows_c && c < cols_c;  // N % 8 == 0: 8 columns wholly in or out
      const uint32_t voff = ok ? (uint32_t)((r * (int)p.ldc + c) * 2) : 0xfffffff0u;
      __builtin_amdgcn_raw_buffer_store_b128(v, rc, voff, 0, 2);  // nt: C is written once
    }
  };

  // fragment row R + lr (R % 32 == 0): swz8(R + lr) = (lr & 7) ^ (lr >> 3) ^ (4 * ((R / 32) & 1))
  int off[2][4];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int sw = ((lr & 7) ^ (lr >> 3) ^ (4 * par)) & 7;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) off[par][kk] = lr * kBK + (((2 * kk + hh) ^ sw) << 3);
  }

  if (count == 0) return;  // uniform per workgroup, before any barrier
  if (!storer) {
    issue_a(0, 0);
    if (count > 1) issue_a(1, 1);
  }
  // (compute waves) B fragments of the segment's first NQR sub-steps, held in registers;
  // the rest are read from LDS per tile (all of them would exceed 256 VGPRs)
  u32x4_t bq[NQR > 0 ? NQR : 1][NI];
  int slot = 0;
  for (int i = 0; i < count; ++i) {
    const int pslot = slot == 0 ? NA - 1 : slot - 1;  // slot of tile i - 1, then of tile i + 2
    if (i % seg == 0) {
      // a new segment: every compute wave finished its B reads before the last barrier
      if (!storer) load_b(i);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      exec_barrier();
      if (!storer) {
#pragma unroll
        for (int q = 0; q < NQR; ++q)
#pragma unroll
          for (int b = 0; b < NI; ++b)
            bq[q][b] = *(const u32x4_t*)(lds + B_OFF + (q >> 2) * B_ELEMS + b * 32 * kBK + off[b & 1][q & 3]);
      }
    }
    if (!storer) {
      // A loads issued after tile i's: tile i + 1's (B loads were waited for completely)
      if (i + 1 < count) wait_vmcnt<L>();
      else wait_vmcnt<0>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    exec_barrier();

    if (!storer) {
      uint16_t* slotp = lds + slot * A_BUF;
      f32x16_t acc[NI];
#pragma unroll
      for (int b = 0; b < NI; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[b][r] = 0.0f;
      // fragments of sub-step q + 1 (A, and B past the registered ones) are read before
      // the MFMAs of sub-step q
      const uint16_t* sA = slotp + rowA0 * kBK;
      const int par = w & 1;
      u32x4_t af[2], bl[2][NI];
      auto frags = [&](int q, u32x4_t& fa, u32x4_t (&fb)[NI]) {
        fa = *(const u32x4_t*)(sA + (q >> 2) * A_ELEMS + off[par][q & 3]);
        if (q >= NQR) {
#pragma unroll
          for (int b = 0; b < NI; ++b)
            fb[b] = *(const u32x4_t*)(lds + B_OFF + (q >> 2) * B_ELEMS + b * 32 * kBK + off[b & 1][q & 3]);
        }
      };
      frags(0, af[0], bl[0]);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if (q + 1 < NQ) frags(q + 1, af[(q + 1) & 1], bl[(q + 1) & 1]);
#pragma unroll
        for (int b = 0; b < NI; ++b) acc[b] = Op::mma32(q < NQR ? bq[q < NQR ? q : 0][b] : bl[q & 1][b], af[q & 1], acc[b]);
      }
      // pack into this wave's own A rows (its reads of them have completed)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int b = 0; b < NI; ++b)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int col = out_col(b, gq, lane);
          *(u32x2_t*)(out_addr(slotp, w, lr, col >> 3) + (col & 7)) =
              u32x2_t{Op::pack2(acc[b][4 * gq], acc[b][4 * gq + 1]), Op::pack2(acc[b][4 * gq + 2], acc[b][4 * gq + 3])};
        }
    } else if (i >= 1) {
      store_tile(i - 1, pslot);
    }
    // the packed tile i is complete; tile i - 1's slot has been read by the store waves
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    exec_barrier();
    if (!storer && i + 2 < count) issue_a(i + 2, pslot);
    slot = slot + 1 == NA ? 0 : slot + 1;
  }
  // the last packed tile (its slot: the one before `slot`)
  if (storer) store_tile(count - 1, slot == 0 ? NA - 1 : slot - 1);
}

// Arguments of the generic MFMA kernel below (any strides / K / alignment).
struct GenericParams {
  const uint16_t* a;
  const uint16_t* b;
  const uint16_t* bias;
  uint16_t* c;
  int M, N, K;
  int64_t sam, sak, sbk, sbn, scm;
  int64_t sa, sb, sc;
  int act;
};

// ---------------------------------------------------------------------------------
// Generic MFMA kernel: any strides, any K (layouts the engines cannot read, when the
// problem is too small for a pack pass).  128x128 tiles,
// 4 waves of 64x64, K steps of 32.  Operands are read element by element, 16 per thread
// per operand and step, along whichever index is unit-stride (so a wave reads 128
// contiguous bytes), every read bounds-checked (zero outside); the next step is loaded
// into registers while the current one is multiplied.  LDS rows of 32 values with a
// stride of 40 (80 bytes): a 16-byte fragment read by 8 consecutive rows covers all 32
// banks once.
// ---------------------------------------------------------------------------------
constexpr int kGenBK = 32, kGenLd = 40;

template <typename T>
__global__ void __launch_bounds__(256) gemm_generic_mfma_kernel(const GenericParams p) {
  using Op = MfmaOp<T>;
  __shared__ __attribute__((aligned(16))) uint16_t sA[128 * kGenLd];
  __shared__ __attribute__((aligned(16))) uint16_t sB[128 * kGenLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = (int)blockIdx.y * 128, n0 = (int)blockIdx.x * 128, z = (int)blockIdx.z;
  const uint16_t* A = p.a + (int64_t)z * p.sa;
  const uint16_t* B = p.b + (int64_t)z * p.sb;
  uint16_t* C = p.c + (int64_t)z * p.sc;
  // element e (0..15) of a thread: tile row and K index; the unit-stride index runs
  // fastest across the lanes
  const bool a_rows = p.sak != 1 && p.sam == 1;  // A's M index is the unit-stride one
  const bool b_rows = p.sbk != 1 && p.sbn == 1;  // B's N index is the unit-stride one
  auto a_idx = [&](int e, int& r, int& k) {
    const int q = e * 256 + tid;  // 0 .. 4095
    if (a_rows) { r = q & 127; k = q >> 7; } else { k = q & 31; r = q >> 5; }
  };
  auto b_idx = [&](int e, int& r, int& k) {
    const int q = e * 256 + tid;
    if (b_rows) { r = q & 127; k = q >> 7; } else { k = q & 31; r = q >> 5; }
  };
  uint16_t ra[16], rb[16];
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      int r, k;
      a_idx(e, r, k);
      const int gm = m0 + r, gk = k0 + k;
      ra[e] = (gm < p.M && gk < p.K) ? A[(int64_t)gm * p.sam + (int64_t)gk * p.sak] : (uint16_t)0;
      b_idx(e, r, k);
      const int gn = n0 + r, gkb = k0 + k;
      rb[e] = (gn < p.N && gkb < p.K) ? B[(int64_t)gkb * p.sbk + (int64_t)gn * p.sbn] : (uint16_t)0;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      int r, k;
      a_idx(e, r, k);
      sA[r * kGenLd + k] = ra[e];
      b_idx(e, r, k);
      sB[r * kGenLd + k] = rb[e];
    }
  };
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const int lr = lane & 31, hh = lane >> 5;
  load(0);
  for (int k0 = 0; k0 < p.K; k0 += kGenBK) {
    __syncthreads();  // the previous step's fragment reads are done
    store();
    __syncthreads();
    if (k0 + kGenBK < p.K) load(k0 + kGenBK);
#pragma unroll
    for (int ks = 0; ks < kGenBK / 16; ++ks) {
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const u32x4_t*)(sA + (wm * 64 + 32 * i + lr) * kGenLd + 16 * ks + 8 * hh);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *(const u32x4_t*)(sB + (wn * 64 + 32 * j + lr) * kGenLd + 16 * ks + 8 * hh);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = Op::mma32(bf[j], af[i], acc[i][j]);
    }
  }
  auto epi = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gm = m0 + wm * 64 + out_row(i, lane);
      if (gm >= p.M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int gn = n0 + wn * 64 + out_col(j, g, lane) + e;
            if (gn >= p.N) continue;
            const float v = apply_act<ACT>(acc[i][j][4 * g + e] + (p.bias ? Op::to_f32(p.bias[gn]) : 0.0f));
            C[(int64_t)gm * p.scm + gn] = (uint16_t)(Op::pack2(v, 0.0f) & 0xffffu);
          }
    }
  };
  switch (p.act) {
    case ACT_RELU: epi(std::integral_constant<int, ACT_RELU>{}); break;
    case ACT_GELU: epi(std::integral_constant<int, ACT_GELU>{}); break;
    case ACT_SILU: epi(std::integral_constant<int, ACT_SILU>{}); break;
    case ACT_TANH: epi(std::integral_constant<int, ACT_TANH>{}); break;
    case ACT_SIGMOID: epi(std::integral_constant<int, ACT_SIGMOID>{}); break;
    default: epi(std::integral_constant<int, ACT_NONE>{}); break;
  }
}

// ---------------------------------------------------------------------------------
// Operand packing for transposed or strided layouts the direct-to-LDS engines cannot
// read in place (K-contiguous rows that are only misaligned go to repitch16_kernel):
// out[b][r][k] = in[b * sbat + r * sr + k * sk] for k < K and 0 for K <= k < Kp, with
// out rows of Kp (a multiple of 64) elements.  64 x 64 tiles through LDS; the loads
// walk whichever of r and k is unit-stride so they coalesce, the stores are 16-byte
// row chunks.
// ---------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pack16_kernel(const uint16_t* in, int64_t sr, int64_t sk, int64_t sbat,
                                                     uint16_t* out, int64_t obat, int R, int K, int Kp) {
  __shared__ uint16_t t[64][66];  // [r][k]
  const int tid = threadIdx.x;
  const int r0 = (int)blockIdx.y * 64, k0 = (int)blockIdx.x * 64;
  const uint16_t* src = in + (int64_t)blockIdx.z * sbat;
  uint16_t* dst = out + (int64_t)blockIdx.z * obat;
  const bool r_unit = sr == 1 && sk != 1;
  if (r_unit && sk % 8 == 0 && ((uintptr_t)src & 15u) == 0) {
    // R-contiguous with 16-byte aligned K-rows (a transposed view): 8 rows per 16-byte load
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int idx = tid + 256 * q, k = idx >> 3, ch = idx & 7;
      const int gk = k0 + k, gr = r0 + 8 * ch;
      uint16_t v[8];
      if (gk < K && gr + 8 <= R) {
        const u32x4_t w = *(const u32x4_t*)(src + (int64_t)gk * sk + gr);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (gk < K && gr + e < R) ? src[(int64_t)gk * sk + gr + e] : (uint16_t)0;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) t[8 * ch + e][k] = v[e];
    }
  } else {
    // each wave instruction reads 64 consecutive elements along the unit-stride index
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int u = tid & 63, v = 4 * i + (tid >> 6);
      const int r = r_unit ? u : v, k = r_unit ? v : u;
      const int gr = r0 + r, gk = k0 + k;
      t[r][k] = (gr < R && gk < K) ? src[(int64_t)gr * sr + (int64_t)gk * sk] : (uint16_t)0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = tid + 256 * q, r = idx >> 3, ch = idx & 7;
    if (r0 + r >= R) continue;
    u32x4_t v;
#pragma unroll
    for (int w = 0; w < 4; ++w) v[w] = (uint32_t)t[r][8 * ch + 2 * w] | ((uint32_t)t[r][8 * ch + 2 * w + 1] << 16);
    *(u32x4_t*)(dst + (int64_t)(r0 + r) * Kp + k0 + 8 * ch) = v;
  }
}

// The common packing case, K-contiguous rows whose element stride leaves them unaligned
// (K = 4095): out[b][r][k] = in[b * sbat + r * sr + k] for k < K, 0 for K <= k < Kp.
// One thread per 16-byte output chunk of 8 elements, built from the naturally aligned
// dwords that cover it (five when the chunk starts at a 2 mod 4 byte address, shifted
// into place with alignbyte); the row's last partial chunk and the zero tail go element
// by element.  Each wave streams 1 KiB of a row, so this is a straight copy at HBM rate
// instead of pack16_kernel's 2-byte loads and LDS round trip.
__global__ void __launch_bounds__(256) repitch16_kernel(const uint16_t* in, int64_t sr, int64_t sbat,
                                                        uint16_t* out, int64_t obat, int R, int K, int Kp) {
  const int cpr = Kp / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)R * cpr) return;
  const int r = (int)(idx / cpr), k0 = (int)(idx % cpr) * 8;
  const uint16_t* src = in + (int64_t)blockIdx.y * sbat + (int64_t)r * sr + k0;
  u32x4_t v;
  if (k0 + 8 < K) {
    // elements k0 .. k0 + 8 exist, so the covering dwords stay inside the row
    const uintptr_t addr = (uintptr_t)src;
    const uint32_t* p = (const uint32_t*)(addr & ~(uintptr_t)3);
    const bool odd = (addr & 2) != 0;
    const uint32_t d0 = p[0], d1 = p[1], d2 = p[2], d3 = p[3], d4 = p[odd ? 4 : 3];
    v = odd ? u32x4_t{__builtin_amdgcn_alignbyte(d1, d0, 2), __builtin_amdgcn_alignbyte(d2, d1, 2),
                      __builtin_amdgcn_alignbyte(d3, d2, 2), __builtin_amdgcn_alignbyte(d4, d3, 2)}
            : u32x4_t{d0, d1, d2, d3};
  } else {
    uint32_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = k0 + j < K ? (uint32_t)src[j] : 0u;
    v = u32x4_t{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
  }
  *(u32x4_t*)(out + (int64_t)blockIdx.y * obat + (int64_t)r * Kp + k0) = v;
}

int launch_pack16(const uint16_t* in, int64_t sr, int64_t sk, int64_t sbat, uint16_t* out, int64_t obat, int64_t R,
                  int64_t K, int64_t Kp, int64_t batch, hipStream_t stream) {
  if (sk == 1) {
    const int64_t chunks = R * (Kp / 8);
    hipLaunchKernelGGL(repitch16_kernel, dim3((unsigned)((chunks + 255) / 256), (unsigned)batch), dim3(256), 0, stream,
                       in, sr, sbat, out, obat, (int)R, (int)K, (int)Kp);
    return check_launch("repitch16_kernel");
  }
  hipLaunchKernelGGL(pack16_kernel, dim3((unsigned)(Kp / 64), (unsigned)((R + 63) / 64), (unsigned)batch), dim3(256), 0,
                     stream, in, sr, sk, sbat, out, obat, (int)R, (int)K, (int)Kp);
  return check_launch("pack16_kernel");
}

// ---------------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------------
struct GemmDesc {
  int dtype, act;
  const void *a, *b, *bias;
  void* c;
  int64_t M, N, K, batch;
  int64_t sam, sak, sbk, sbn, scm;  // element strides; B given as (k, n)
  int64_t sa, sb, sc;               // batch strides
  int64_t kvalid = 0;               // > 0: K-rows of an N-contiguous B that exist (K is padded)
};

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T, int BL, int BM, int BN>
int launch_tile(const GemmDesc& d, hipStream_t stream) {
  TileParams p{};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.lda = d.sam;
  p.ldb = (BL == B_KC) ? d.sbn : d.sbk;
  p.ldc = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.tiles_m = (int)((d.M + BM - 1) / BM);
  p.tiles_n = (int)((d.N + BN - 1) / BN);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = (int)d.batch;
  p.act = d.act;
  p.vec_store = (d.scm % 8 == 0) && aligned16(d.c) && (d.sc % 8 == 0);
  p.bias_vec = d.bias != nullptr && ((uintptr_t)d.bias & 7u) == 0;
  const int64_t blocks = (int64_t)p.tiles_per_batch * d.batch;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm: grid too large");
  hipLaunchKernelGGL((gemm_tile_kernel<T, BL, BM, BN>), dim3((unsigned)blocks), dim3(kEngineThreads), 0, stream, p);
  return check_launch("gemm_tile_kernel");
}


// KT: K % 64 != 0, rows of any 2-byte alignment, read in place (K-tail mode of the
// 16x16 engine: the loop runs over K rounded up to 64, the last stage starts at K - 64).
template <typename T, int BM, int BN, int BL, int AL = A_KC, bool KT = false>
int launch_buf(const GemmDesc& d, hipStream_t stream) {
  TileParams p{};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.kb = (int)(d.kvalid > 0 ? d.kvalid : d.K);
  p.lda = AL == A_MC ? d.sak : d.sam;
  p.ldb = (BL == B_KC) ? d.sbn : d.sbk;
  p.ldc = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.tiles_m = (int)((d.M + BM - 1) / BM);
  p.tiles_n = (int)((d.N + BN - 1) / BN);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = (int)d.batch;
  p.act = d.act;
  p.vec_store = (d.scm % 8 == 0) && aligned16(d.c) && (d.sc % 8 == 0);
  p.bias_vec = d.bias != nullptr && ((uintptr_t)d.bias & 7u) == 0;
  const int64_t blocks = (int64_t)p.tiles_per_batch * d.batch;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm: grid too large");
  if constexpr (AL == A_MC) {
    hipLaunchKernelGGL((gemm_buf_kernel<T, BM, BN, BL, 8, A_MC>), dim3((unsigned)blocks), dim3(512), 0, stream, p);
    return check_launch("gemm_buf_kernel");
  }
  // K-contiguous B: 4 waves of 128 x 128 with the accumulators in place in AGPRs (one
  // wave per SIMD; same process, bit-equal, against the 8-wave tile: 4096^3 bf16 95.8 ->
  // 91.9 us, fp16 + bias + gelu 109.2 -> 106.1 us, 8192 x 4096 x 4096 189.9 -> 184.0 us).
  // N-contiguous B: 8 waves on 16x16x32 MFMAs.  Over more than one round of the CUs it
  // used to keep the 4-wave 32x32x16 tile, 1-4% faster cold than the 8-wave one of that
  // time; with the 16-row swizzle and the full-stage load lead the 8-wave tile wins there
  // too (same process, bit-equal, cold: 8192 x 8192 x 4096 429.9 -> 409.6 us, 8192 x 4096 x
  // 4096 223.4 -> 215.2 us; warm 418.3 -> 392.8, 211.9 -> 199.3).
  // K tails keep 8 waves for both layouts (3072 x 4096 x 1000 with K-contiguous B: 34.8 us
  // against 36.5 us on 4 waves; 4096 x 4096 x 4095 within 1%).
  if constexpr (KT) {
    p.kreal = (int)d.K;
    p.K = (int)((d.K + kBK - 1) / kBK * kBK);
    hipLaunchKernelGGL((gemm_buf_kernel<T, BM, BN, BL, 8, A_KC, true>), dim3((unsigned)blocks), dim3(512), 0, stream, p);
    return check_launch("gemm_buf_kernel");
  }
  constexpr int NWV = BL == B_KC ? 4 : 8;
  hipLaunchKernelGGL((gemm_buf_kernel<T, BM, BN, BL, NWV, A_KC>), dim3((unsigned)blocks), dim3(64 * NWV), 0, stream,
                     p);
  return check_launch("gemm_buf_kernel");
}

template <typename T, int BM, int BN, int WM, int WN, int NSLOT, int BL, bool KT = false>
int launch_deep(const GemmDesc& d, hipStream_t stream) {
  TileParams p{};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.kb = (int)(d.kvalid > 0 ? d.kvalid : d.K);
  p.lda = d.sam;
  p.ldb = (BL == B_KC) ? d.sbn : d.sbk;
  p.ldc = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.tiles_m = (int)((d.M + BM - 1) / BM);
  p.tiles_n = (int)((d.N + BN - 1) / BN);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = (int)d.batch;
  p.act = d.act;
  p.vec_store = (d.scm % 8 == 0) && aligned16(d.c) && (d.sc % 8 == 0);
  p.bias_vec = d.bias != nullptr && ((uintptr_t)d.bias & 7u) == 0;
  const int64_t blocks = (int64_t)p.tiles_per_batch * d.batch;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm: grid too large");
  if constexpr (KT) {  // the loop over K rounded up to 64; the true K for the last stage
    p.kreal = (int)d.K;
    p.K = (int)((d.K + kBK - 1) / kBK * kBK);
  }
  hipLaunchKernelGGL((gemm_deep_kernel<T, BM, BN, WM, WN, NSLOT, BL, KT>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     p);
  return check_launch("gemm_deep_kernel");
}

// Persistent short-K launch: one 128 KiB-LDS workgroup per CU, at most one per tile.
template <typename T, int BL>
int launch_shortk(const GemmDesc& d, hipStream_t stream) {
  TileParams p{};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = nullptr;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.lda = d.sam;
  p.ldb = (BL == B_KC) ? d.sbn : d.sbk;
  p.ldc = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.tiles_m = (int)((d.M + 127) / 128);
  p.tiles_n = (int)((d.N + 127) / 128);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = (int)d.batch;
  p.act = KORE_ACT_NONE;
  p.vec_store = 0;
  p.bias_vec = 0;
  const int64_t tiles = (int64_t)p.tiles_per_batch * d.batch;
  // segment length: about the tiles per CU, at most one column
  const int64_t per_cu = tiles / device_cus();
  const int seg = (int)std::max<int64_t>(1, std::min<int64_t>(p.tiles_m, per_cu));
  const int64_t nseg = (p.tiles_m + seg - 1) / seg;
  const int64_t total = nseg * p.tiles_n * d.batch;
  if (total > 0x7fffffff || total * seg > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm: grid too large");
  const int grid = (int)std::min<int64_t>(total, device_cus());
  const dim3 gr((unsigned)grid), blk(512);
  if (BL == B_KC && d.K == 64) hipLaunchKernelGGL((gemm_shortk_kernel<T, 1, B_KC>), gr, blk, 0, stream, p, seg);
  if (BL == B_KC && d.K == 128) hipLaunchKernelGGL((gemm_shortk_kernel<T, 2, B_KC>), gr, blk, 0, stream, p, seg);
  if (BL == B_NC && d.K == 64) hipLaunchKernelGGL((gemm_shortk_kernel<T, 1, B_NC>), gr, blk, 0, stream, p, seg);
  if (BL == B_NC && d.K == 128) hipLaunchKernelGGL((gemm_shortk_kernel<T, 2, B_NC>), gr, blk, 0, stream, p, seg);
  return check_launch("gemm_shortk_kernel");
}

template <typename T>
int launch_ring(const GemmDesc& d, hipStream_t stream) {
  constexpr int BM = 32, BN = 128, NSLOT = 7;
  TileParams p{};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.lda = d.sam;
  p.ldb = d.sbn;
  p.ldc = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.tiles_m = (int)((d.M + BM - 1) / BM);
  p.tiles_n = (int)((d.N + BN - 1) / BN);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = (int)d.batch;
  p.act = d.act;
  p.vec_store = (d.scm % 8 == 0) && aligned16(d.c) && (d.sc % 8 == 0);
  p.bias_vec = d.bias != nullptr && ((uintptr_t)d.bias & 7u) == 0;
  const int64_t blocks = (int64_t)p.tiles_per_batch * d.batch;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm: grid too large");
  hipLaunchKernelGGL((gemm_ring_kernel<T, BN, NSLOT>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
  return check_launch("gemm_ring_kernel");
}

template <typename T>
int launch_generic(const GemmDesc& d, hipStream_t stream) {
  GenericParams p;
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.sam = d.sam;
  p.sak = d.sak;
  p.sbk = d.sbk;
  p.sbn = d.sbn;
  p.scm = d.scm;
  p.sa = d.sa;
  p.sb = d.sb;
  p.sc = d.sc;
  p.act = d.act;
  if (d.batch > 65535) return set_error(KORE_EUNSUPPORTED, "gemm: batch > 65535 on the generic path");
  dim3 grid((unsigned)((d.N + 127) / 128), (unsigned)((d.M + 127) / 128), (unsigned)d.batch);
  hipLaunchKernelGGL(gemm_generic_mfma_kernel<T>, grid, dim3(256), 0, stream, p);
  return check_launch("gemm_generic_mfma_kernel");
}

// Split-K launch (batch 1): `splits` slices of `kper` (a multiple of 64) K elements on
// BM x BN ring tiles.
template <typename T, int BL, int BM, int BN, int WM, int WN, int NSLOT>
int launch_splitk(const GemmDesc& d, int splits, int kper, Ws& ws, hipStream_t stream) {
  const size_t bytes = (size_t)splits * d.M * d.N * sizeof(float);
  float* part = (float*)ws.take(bytes);
  if (ws.plan) return KORE_OK;
  if (part == nullptr)
    return set_error(KORE_EWORKSPACE, "gemm: split-K needs %zu workspace bytes (got %zu)", ws_bytes(bytes), ws.bytes);
  TileParams p = {};
  p.a = (const uint16_t*)d.a;
  p.b = (const uint16_t*)d.b;
  p.bias = (const uint16_t*)d.bias;
  p.c = (uint16_t*)d.c;
  p.M = (int)d.M;
  p.N = (int)d.N;
  p.K = (int)d.K;
  p.kb = (int)(d.kvalid > 0 ? d.kvalid : d.K);
  p.lda = d.sam;
  p.ldb = (BL == B_KC) ? d.sbn : d.sbk;
  p.ldc = d.scm;
  p.tiles_m = (int)((d.M + BM - 1) / BM);
  p.tiles_n = (int)((d.N + BN - 1) / BN);
  p.tiles_per_batch = p.tiles_m * p.tiles_n;
  p.batch = 1;
  p.act = d.act;
  hipLaunchKernelGGL((gemm_splitk_kernel<T, BL, BM, BN, WM, WN, NSLOT>), dim3((unsigned)(p.tiles_per_batch * splits)),
                     dim3(256), 0, stream, p, part, splits, kper);
  int rc = check_launch("gemm_splitk_kernel");
  if (rc == KORE_OK) {
    if (d.N % 4 == 0) {  // 16-byte partial loads (the workspace is 256-byte aligned)
      const int vec = (d.scm % 4 == 0) && ((uintptr_t)d.c & 7u) == 0;
      const int64_t threads = d.M * (d.N / 4);
      hipLaunchKernelGGL((splitk_reduce_kernel<T, 4>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                         (const float*)part, splits, (int)d.M, (int)d.N, (const uint16_t*)d.bias, d.act,
                         (uint16_t*)d.c, d.scm, vec);
    } else {
      const int vec = (d.scm % 8 == 0) && aligned16(d.c);
      const int64_t threads = d.M * ((d.N + 7) / 8);
      hipLaunchKernelGGL((splitk_reduce_kernel<T, 8>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                         (const float*)part, splits, (int)d.M, (int)d.N, (const uint16_t*)d.bias, d.act,
                         (uint16_t*)d.c, d.scm, vec);
    }
    rc = check_launch("splitk_reduce_kernel");
  }
  return rc;
}

// Tile shape for the direct-to-LDS engines.  Every CU runs one tile at a time, so a
// launch costs about (rounds of tiles over the CUs) x (time of one tile); a tile's time
// is its area over its engine's efficiency (the 256x256 pipelined engine is best;
// narrower ring tiles move more bytes per MFMA).  Small problems that fill less
// than half the chip even with 64x128 tiles take 32x128 tiles.
enum TileShape { TILE_256x256, TILE_256x128, TILE_128x128, TILE_64x128, TILE_32x128 };

inline TileShape pick_tile(const GemmDesc& d) {
  const int64_t cus = device_cus();
  struct Opt {
    TileShape t;
    int bm, bn;
    double cost_per_round;  // tile area / efficiency, in 64x128 units
  } opts[] = {// efficiencies from one full round at K = 4096 each: 4096^3 (256x256,
              // 111 us), 1536x4096 (256x128, 71 us), 2048^2 x 4096-equivalent (128x128),
              // 512x4096 (64x128, 32 us), relative to the 256x256 engine
              {TILE_256x256, 256, 256, 8.0 / 1.0},
              {TILE_256x128, 256, 128, 4.0 / 0.79},
              {TILE_128x128, 128, 128, 2.0 / 0.55},
              {TILE_64x128, 64, 128, 1.0 / 0.43}};
  TileShape best = TILE_32x128;
  double best_cost = 1e300;
  for (const Opt& o : opts) {
    const int64_t tiles = ((d.M + o.bm - 1) / o.bm) * ((d.N + o.bn - 1) / o.bn) * d.batch;
    if (tiles * 2 < cus) continue;  // leaves most of the chip idle
    const double cost = (double)((tiles + cus - 1) / cus) * o.cost_per_round;
    if (cost < best_cost) {
      best_cost = cost;
      best = o.t;
    }
  }
  return best;
}

// Direct-to-LDS engine for an already conforming problem (A and B K-contiguous or B
// N-contiguous, 16-byte rows, K % 64 == 0, buffer ranges checked by the caller).
template <typename T, int BL>
int launch_engine(const GemmDesc& d, hipStream_t stream) {
  switch (pick_tile(d)) {
    case TILE_256x256: return launch_buf<T, 256, 256, BL>(d, stream);
    case TILE_256x128: return launch_deep<T, 256, 128, 2, 2, 3, BL>(d, stream);
    case TILE_128x128: return launch_deep<T, 128, 128, 2, 2, 4, BL>(d, stream);
    case TILE_64x128: return launch_deep<T, 64, 128, 2, 2, 6, BL>(d, stream);
    default: return launch_deep<T, 32, 128, 1, 4, 7, BL>(d, stream);
  }
}

// K tails on the deep ring (tile shapes below 256x256), read in place.
template <typename T, int BL>
int launch_deep_kt(const GemmDesc& d, hipStream_t stream) {
  switch (pick_tile(d)) {
    case TILE_256x128: return launch_deep<T, 256, 128, 2, 2, 3, BL, true>(d, stream);
    case TILE_128x128: return launch_deep<T, 128, 128, 2, 2, 4, BL, true>(d, stream);
    case TILE_64x128: return launch_deep<T, 64, 128, 2, 2, 6, BL, true>(d, stream);
    default: return launch_deep<T, 32, 128, 1, 4, 7, BL, true>(d, stream);
  }
}

// Layouts the engines cannot read in place (rows not 16-byte aligned, e.g. K = 4095;
// transposed or strided operands): A, and B unless it is N-contiguous with aligned
// K-rows, are packed K-contiguous with the K tail zero-padded to a multiple of 64
// into the caller's workspace.
// An N-contiguous B is read in place: its buffer resource ends at the last real
// K-row, so the padded rows read as zero.  The caller checks padded_fits first.
inline bool padded_b_inplace(const GemmDesc& d) {
  return d.sbn == 1 && d.sbk % 8 == 0 && aligned16(d.b) && d.sb % 8 == 0 && d.N % 8 == 0 &&
         d.sbk * 2 * d.K + d.N * 2 < (1ll << 31);
}
inline bool padded_fits(const GemmDesc& d) {
  const int64_t Kp = (d.K + 63) / 64 * 64;
  return d.M < (1ll << 31) && d.N < (1ll << 31) && Kp * 2 * 256 + Kp * 2 < (1ll << 31) && d.batch <= 65535;
}
template <typename T>
int launch_padded(const GemmDesc& d, Ws& ws, hipStream_t stream) {
  const int64_t Kp = (d.K + 63) / 64 * 64;
  const bool b_nc = padded_b_inplace(d);
  const size_t a_bytes = (size_t)(d.batch * d.M * Kp * 2 + 255) / 256 * 256;
  const size_t b_bytes = b_nc ? 0 : (size_t)(d.batch * d.N * Kp * 2);
  void* buf = ws.take(a_bytes + b_bytes);
  if (ws.plan) return KORE_OK;
  if (buf == nullptr)
    return set_error(KORE_EWORKSPACE, "gemm: packing the operands needs %zu workspace bytes (got %zu)",
                     ws_bytes(a_bytes + b_bytes), ws.bytes);
  uint16_t* ap = (uint16_t*)buf;
  uint16_t* bp = (uint16_t*)((char*)buf + a_bytes);
  int rc = launch_pack16((const uint16_t*)d.a, d.sam, d.sak, d.sa, ap, d.M * Kp, d.M, d.K, Kp, d.batch, stream);
  GemmDesc q = d;
  q.a = ap;
  q.sam = Kp;
  q.sak = 1;
  q.sa = d.M * Kp;
  q.K = Kp;
  if (rc == KORE_OK && !b_nc) {
    // B^T rows (n) with K-contiguous, zero-padded K
    rc = launch_pack16((const uint16_t*)d.b, d.sbn, d.sbk, d.sb, bp, d.N * Kp, d.N, d.K, Kp, d.batch, stream);
    q.b = bp;
    q.sbk = 1;
    q.sbn = Kp;
    q.sb = d.N * Kp;
  }
  if (rc == KORE_OK) {
    if (b_nc) {
      q.kvalid = d.K;
      rc = launch_engine<T, B_NC>(q, stream);
    } else {
      rc = launch_engine<T, B_KC>(q, stream);
    }
  }
  return rc;
}

// Picks the kernel path for d and launches it; in plan mode (ws.plan) it launches
// nothing and only records the workspace that path needs.
template <typename T>
int dispatch_typed(const GemmDesc& d, Ws& ws, hipStream_t stream) {
  // Fast-path preconditions: A K-contiguous with 16-byte aligned rows, K % 8 == 0,
  // B K- or N-contiguous with 16-byte aligned rows, C N-contiguous.
  const bool a_ok = d.sak == 1 && d.sam % 8 == 0 && aligned16(d.a) && d.sa % 8 == 0 && d.K % 8 == 0;
  const bool b_kc = d.sbk == 1 && d.sbn % 8 == 0 && aligned16(d.b) && d.sb % 8 == 0;
  const bool b_nc = d.sbn == 1 && d.sbk % 8 == 0 && aligned16(d.b) && d.sb % 8 == 0 && d.N % 8 == 0;
  const bool fits32 = d.M < (1ll << 31) && d.N < (1ll << 31) && d.K < (1ll << 31);
  // M-contiguous A (a transposed view, e.g. dY^T of the backward) on the 256x256 buffer
  // engine, read in place through LDS transpose reads; smaller grids pack A instead.
  const bool a_mc = d.sam == 1 && d.sak % 8 == 0 && aligned16(d.a) && d.sa % 8 == 0 && d.M % 8 == 0 &&
                    d.K % 64 == 0 && d.K > 256 && d.sak * 2 * d.K + 512 < (1ll << 31);
  // K tails (K % 64 != 0, e.g. 4095) on the 256x256 grid: the 16x16 engine reads A and B
  // in place -- direct-to-LDS loads take rows at any 2-byte alignment -- and its last
  // stage starts at K - 64, with the columns it repeats zeroed in LDS (mainloop16<true>),
  // instead of a pack pass over A (4096 x 4096 x 4095 with the task's [K,N] B: 16 us).
  if (d.K % 64 != 0 && d.K > 64 && d.sak == 1 && fits32 && pick_tile(d) == TILE_256x256 &&
      d.sam * 2 * 256 + d.K * 2 < (1ll << 31)) {
    const bool kc = d.sbk == 1 && d.sbn * 2 * 256 + d.K * 2 < (1ll << 31);
    const bool nc = d.sbn == 1 && d.sbk % 8 == 0 && aligned16(d.b) && d.sb % 8 == 0 && d.N % 8 == 0 &&
                    d.sbk * 2 * d.K + d.N * 2 < (1ll << 31);
    if (kc || nc) {
      if (ws.plan) return KORE_OK;
      return kc ? launch_buf<T, 256, 256, B_KC, A_KC, true>(d, stream)
                : launch_buf<T, 256, 256, B_NC, A_KC, true>(d, stream);
    }
  }
  // The same for mid-size grids (at least 128 tiles of 128x128, K >= 256) on the deep
  // ring engine's K-tail mode, at the tile shape pick_tile chooses.
  if (d.K % 64 != 0 && d.K >= 256 && d.sak == 1 && fits32 && d.sam * 2 * 256 + d.K * 2 < (1ll << 31) &&
      ((d.M + 127) / 128) * ((d.N + 127) / 128) * d.batch >= 128) {
    const bool kc = d.sbk == 1 && d.sbn * 2 * 256 + d.K * 2 < (1ll << 31);
    const bool nc = d.sbn == 1 && d.sbk % 8 == 0 && aligned16(d.b) && d.sb % 8 == 0 && d.N % 8 == 0 &&
                    d.sbk * 2 * d.K + d.N * 2 < (1ll << 31);
    if (kc || nc) {
      if (ws.plan) return KORE_OK;
      return kc ? launch_deep_kt<T, B_KC>(d, stream) : launch_deep_kt<T, B_NC>(d, stream);
    }
  }
  if (a_mc && fits32 && pick_tile(d) == TILE_256x256 &&
      ((b_kc && d.sbn * 2 * 256 + d.K * 2 < (1ll << 31)) || (b_nc && d.sbk * 2 * d.K + d.N * 2 < (1ll << 31)))) {
    if (ws.plan) return KORE_OK;
    return b_kc ? launch_buf<T, 256, 256, B_KC, A_MC>(d, stream) : launch_buf<T, 256, 256, B_NC, A_MC>(d, stream);
  }
  if (a_ok && (b_kc || b_nc) && fits32) {
    // Macro tile: 256x256 when it still gives >= ~1 wave of tiles, else 128x128.
    const int64_t big_tiles = ((d.M + 255) / 256) * ((d.N + 255) / 256) * d.batch;
    const bool big = big_tiles >= 192;
    // Buffer-load engine: each operand tile must span < 4 GiB of bytes.
    const bool buf_ok = d.K % 64 == 0 && d.sam * 2 * 256 + d.K * 2 < (1ll << 31) &&
                        d.sbn * 2 * 256 + d.K * 2 < (1ll << 31);
    // Short K (a few K steps per tile, e.g. the batched K=128 shape) is bound by the
    // output stores: 128x128 tiles (64 KiB LDS) let two workgroups share a CU, so one
    // tile's epilogue overlaps the next tile's loads.  Fewer than 128 tiles of 128x128
    // (1024^3 has 64) leave most CUs idle: 64x64 tiles then.
    const int64_t mid_tiles = ((d.M + 127) / 128) * ((d.N + 127) / 128) * d.batch;
    const bool short_k = d.K <= 256;
    const bool small = mid_tiles < 128;
    // N-contiguous B on the direct-to-LDS engines: B bytes from the tile's first column
    // through the last K-row must fit the 32-bit buffer offsets.
    const bool buf_nc_ok = d.K % 64 == 0 && d.sam * 2 * 256 + d.K * 2 < (1ll << 31) &&
                           d.sbk * 2 * d.K + d.N * 2 < (1ll << 31);
    const bool deep_ok = (b_kc ? buf_ok : buf_nc_ok) && d.K >= 256;
    // Long K and enough tiles to fill half the chip: the direct-to-LDS engines at the
    // tile shape with the fewest weighted rounds (small problems, under 128 tiles of
    // 128x128, keep their latency-bound paths below: split-K, the 32x128 rings).
    if (deep_ok && !small && pick_tile(d) != TILE_32x128) {
      if (ws.plan) return KORE_OK;
      return b_kc ? launch_engine<T, B_KC>(d, stream) : launch_engine<T, B_NC>(d, stream);
    }
    // K of one or two 64-wide steps, no epilogue, enough 128x128 tiles to give every
    // CU several: the persistent short-K kernel (16-byte buffer stores need N % 8 == 0
    // and 16-byte aligned C rows; per-tile byte offsets must stay below 2^31).
    const bool shortk = (d.K == 64 || d.K == 128) && d.act == KORE_ACT_NONE && d.bias == nullptr &&
                        d.N % 8 == 0 && d.scm % 8 == 0 && d.sc % 8 == 0 && aligned16(d.c) &&
                        d.sam * 2 * 128 + d.K * 2 < (1ll << 31) && (b_nc || d.sbn * 2 * 128 + d.K * 2 < (1ll << 31)) &&
                        d.scm * 2 * 128 < (1ll << 31) && mid_tiles >= 4 * (int64_t)device_cus();
    if (shortk) {
      if (ws.plan) return KORE_OK;
      return b_kc ? launch_shortk<T, B_KC>(d, stream) : launch_shortk<T, B_NC>(d, stream);
    }
    // Few 32x128 tiles for the CUs and a long K (decode-sized M): split K.
    const int64_t t32 = ((d.M + 31) / 32) * ((d.N + 127) / 128);
    if (d.batch == 1 && (b_kc ? buf_ok : buf_nc_ok) && d.K >= 1024 && t32 * 2 <= device_cus()) {
      const int nk = (int)(d.K / 64);
      const int want = (int)std::min<int64_t>(device_cus() / t32, nk / 4);
      const int per = (nk + want - 1) / want, splits = (nk + per - 1) / per;
      return b_kc ? launch_splitk<T, B_KC, 32, 128, 1, 4, 7>(d, splits, per * 64, ws, stream)
                  : launch_splitk<T, B_NC, 32, 128, 1, 4, 7>(d, splits, per * 64, ws, stream);
    }
    if (ws.plan) return KORE_OK;
    // few tiles and a long K: the latency-bound case, on the deep direct-to-LDS ring
    if (b_kc && small && buf_ok && d.K >= 512) return launch_ring<T>(d, stream);
    if (!b_kc && small && buf_nc_ok && d.K >= 512) return launch_deep<T, 32, 128, 1, 4, 7, B_NC>(d, stream);
    if (b_kc) {
      if (big && !short_k) return launch_tile<T, B_KC, 256, 256>(d, stream);
      return small ? launch_tile<T, B_KC, 64, 64>(d, stream) : launch_tile<T, B_KC, 128, 128>(d, stream);
    }
    if (big && !short_k) return launch_tile<T, B_NC, 256, 256>(d, stream);
    return small ? launch_tile<T, B_NC, 64, 64>(d, stream) : launch_tile<T, B_NC, 128, 128>(d, stream);
  }
  // Large problems in other layouts: pack, then the engines (small ones are cheaper on
  // the generic kernel than a pack pass).
  if (d.M * d.N * d.K >= (1ll << 27) && d.K >= 64 && padded_fits(d)) return launch_padded<T>(d, ws, stream);
  if (ws.plan) return KORE_OK;
  return launch_generic<T>(d, stream);
}

int run_gemm(const GemmDesc& d, Ws& ws, void* stream) {
  if (d.c == nullptr || (d.K > 0 && (d.a == nullptr || d.b == nullptr)))
    return set_error(KORE_EINVAL, "gemm: null pointer");
  if (d.M <= 0 || d.N <= 0 || d.K < 0 || d.batch <= 0)
    return set_error(KORE_EINVAL, "gemm: need M, N, batch >= 1 and K >= 0 (M=%lld N=%lld K=%lld batch=%lld)", (long long)d.M,
                     (long long)d.N, (long long)d.K, (long long)d.batch);
  if (d.act < KORE_ACT_NONE || d.act > KORE_ACT_SIGMOID) return set_error(KORE_EINVAL, "gemm: unknown act %d", d.act);
  if (d.scm < d.N) return set_error(KORE_EINVAL, "gemm: ldc_m (%lld) < N (%lld)", (long long)d.scm, (long long)d.N);
  hipStream_t s = (hipStream_t)stream;
  if (d.dtype == KORE_DT_BF16) return dispatch_typed<BF16>(d, ws, s);
  if (d.dtype == KORE_DT_FP16) return dispatch_typed<F16>(d, ws, s);
  if (d.dtype == KORE_DT_FP32) {
    if (d.batch != 1) return set_error(KORE_EUNSUPPORTED, "gemm: fp32 is not batched");
    GemmF32Args f{d.a, d.b, d.bias, d.c, d.M, d.N, d.K, d.sam, d.sak, d.sbk, d.sbn, d.scm, d.act};
    return launch_gemm_f32(f, ws, s);
  }
  return set_error(KORE_EINVAL, "gemm: unsupported dtype code %d", d.dtype);
}

}  // namespace
}  // namespace kore

extern "C" size_t kore_gemm_workspace_bytes(int dtype, int act, const void* a, int64_t lda_m, int64_t lda_k,
                                            const void* b, int64_t ldb_k, int64_t ldb_n, const void* bias, void* c,
                                            int64_t ldc_m, int64_t M, int64_t N, int64_t K) {
  kore::GemmDesc d{dtype, act, a, b, bias, c, M, N, K, 1, lda_m, lda_k, ldb_k, ldb_n, ldc_m, 0, 0, 0};
  kore::Ws ws;
  ws.plan = true;
  if (kore::run_gemm(d, ws, nullptr) != KORE_OK) return 0;  // the call itself reports the error
  return kore::ws_bytes(ws.need);
}

extern "C" int kore_gemm(int dtype, int act, const void* a, int64_t lda_m, int64_t lda_k, const void* b,
                         int64_t ldb_k, int64_t ldb_n, const void* bias, void* c, int64_t ldc_m, int64_t M,
                         int64_t N, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  kore::GemmDesc d{dtype, act, a, b, bias, c, M, N, K, 1, lda_m, lda_k, ldb_k, ldb_n, ldc_m, 0, 0, 0};
  kore::Ws ws;
  ws.ptr = workspace;
  ws.bytes = workspace ? workspace_bytes : 0;
  return kore::run_gemm(d, ws, stream);
}

extern "C" size_t kore_batched_gemm_workspace_bytes(int dtype, const void* a, int64_t sa_b, int64_t sa_m,
                                                    int64_t sa_k, const void* b, int64_t sb_b, int64_t sb_n,
                                                    int64_t sb_k, void* c, int64_t sc_b, int64_t sc_m, int64_t batch,
                                                    int64_t M, int64_t N, int64_t K) {
  kore::GemmDesc d{dtype, KORE_ACT_NONE, a, b, nullptr, c, M, N, K, batch, sa_m, sa_k, sb_k, sb_n, sc_m,
                   sa_b, sb_b, sc_b};
  kore::Ws ws;
  ws.plan = true;
  if (kore::run_gemm(d, ws, nullptr) != KORE_OK) return 0;
  return kore::ws_bytes(ws.need);
}

extern "C" int kore_batched_gemm(int dtype, const void* a, int64_t sa_b, int64_t sa_m, int64_t sa_k, const void* b,
                                 int64_t sb_b, int64_t sb_n, int64_t sb_k, void* c, int64_t sc_b, int64_t sc_m,
                                 int64_t batch, int64_t M, int64_t N, int64_t K, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  // C[i] = A[i] @ B[i]^T: B[i] is [N,K], i.e. the (k, n) strides are (sb_k, sb_n).
  kore::GemmDesc d{dtype, KORE_ACT_NONE, a, b, nullptr, c, M, N, K, batch, sa_m, sa_k, sb_k, sb_n, sc_m,
                   sa_b, sb_b, sc_b};
  kore::Ws ws;
  ws.ptr = workspace;
  ws.bytes = workspace ? workspace_bytes : 0;
  return kore::run_gemm(d, ws, stream);
}

// Linear-layer backward for Y = X @ W^T: dX = dY @ W and dW = dY^T @ X, two run_gemm
// calls.  dY, W and X are read in place: W and X as N-contiguous B operands (LDS
// transpose reads), dY^T as an M-contiguous A view of dY on the 8-wave buffer tiles.
// Only grids too small for those tiles pack dY^T into the caller's workspace.
namespace kore {
namespace {
// The two GEMMs of the backward.
GemmDesc bwd_dx(int dtype, const void* w, int64_t ldw, const void* dy, int64_t lddy, void* dx, int64_t lddx,
                int64_t M, int64_t N, int64_t K) {
  // dX[M,K] = dY[M,N] @ W[N,K]: W read in place as an N-contiguous B (element (n, k) at
  // w[n*ldw + k]); the engines stage it through LDS transpose reads
  return GemmDesc{dtype, KORE_ACT_NONE, dy, w, nullptr, dx, M, K, N, 1, lddy, 1, ldw, 1, lddx, 0, 0, 0};
}
GemmDesc bwd_dw(int dtype, const void* x, int64_t ldx, const void* dy, int64_t lddy, void* dw, int64_t lddw,
                int64_t M, int64_t N, int64_t K) {
  // dW[N,K] = dY^T[N,M] @ X[M,K]: dY^T is the transposed view of dY (element (n, m) at
  // dy[m*lddy + n], an M-contiguous A) and X an N-contiguous B (element (m, k) at
  // x[m*ldx + k]), both read in place by the buffer engine or packed by the dispatch
  return GemmDesc{dtype, KORE_ACT_NONE, dy, x, nullptr, dw, N, K, M, 1, 1, lddy, ldx, 1, lddw, 0, 0, 0};
}
int bwd_check(int dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, const void* dy, int64_t lddy,
              const void* dx, int64_t lddx, const void* dw, int64_t lddw, int64_t M, int64_t N, int64_t K) {
  if (dtype != KORE_DT_BF16 && dtype != KORE_DT_FP16)
    return set_error(KORE_EINVAL, "gemm_backward: dtype must be bf16 or fp16 (got %d)", dtype);
  if (!x || !w || !dy || !dx || !dw) return set_error(KORE_EINVAL, "gemm_backward: null pointer");
  if (M <= 0 || N <= 0 || K <= 0) return set_error(KORE_EINVAL, "gemm_backward: M, N, K must be >= 1");
  if (ldx < K || ldw < K || lddy < N || lddx < K || lddw < K)
    return set_error(KORE_EINVAL, "gemm_backward: row stride smaller than row");
  if (M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31))
    return set_error(KORE_EUNSUPPORTED, "gemm_backward: dimension >= 2^31");
  return KORE_OK;
}
}  // namespace
}  // namespace kore

// Workspace: the scratch of the two GEMMs (they run one after the other, so they share
// it); none when both run on the buffer engine in place.
extern "C" size_t kore_gemm_backward_workspace_bytes(int dtype, const void* x, int64_t ldx, const void* w,
                                                     int64_t ldw, const void* dy, int64_t lddy, const void* dx,
                                                     int64_t lddx, const void* dw, int64_t lddw, int64_t M,
                                                     int64_t N, int64_t K) {
  using namespace kore;
  if (bwd_check(dtype, x, ldx, w, ldw, dy, lddy, dx, lddx, dw, lddw, M, N, K) != KORE_OK) return 0;
  Ws ws;
  ws.plan = true;
  GemmDesc gx = bwd_dx(dtype, w, ldw, dy, lddy, (void*)dx, lddx, M, N, K);
  GemmDesc gw = bwd_dw(dtype, x, ldx, dy, lddy, (void*)dw, lddw, M, N, K);
  if (run_gemm(gx, ws, nullptr) != KORE_OK || run_gemm(gw, ws, nullptr) != KORE_OK) return 0;
  return ws_bytes(ws.need);
}

extern "C" int kore_gemm_backward(int dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, const void* dy,
                                  int64_t lddy, void* dx, int64_t lddx, void* dw, int64_t lddw, int64_t M, int64_t N,
                                  int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace kore;
  int rc = bwd_check(dtype, x, ldx, w, ldw, dy, lddy, dx, lddx, dw, lddw, M, N, K);
  if (rc != KORE_OK) return rc;
  const size_t need = kore_gemm_backward_workspace_bytes(dtype, x, ldx, w, ldw, dy, lddy, dx, lddx, dw, lddw, M, N, K);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(KORE_EWORKSPACE, "gemm_backward: needs %zu workspace bytes (got %zu)", need,
                     workspace ? workspace_bytes : (size_t)0);
  hipStream_t st = (hipStream_t)stream;
  Ws ws;  // the two GEMMs run one after the other and share the scratch
  ws.ptr = workspace;
  ws.bytes = workspace_bytes;
  GemmDesc gx = bwd_dx(dtype, w, ldw, dy, lddy, dx, lddx, M, N, K);
  rc = run_gemm(gx, ws, st);
  if (rc != KORE_OK) return rc;
  GemmDesc gw = bwd_dw(dtype, x, ldx, dy, lddy, dw, lddw, M, N, K);
  return run_gemm(gw, ws, st);
}

// ---------------------------------------------------------------------------------
// kore_gemm_noalloc: kore_gemm for callers that cannot allocate device memory.  The
// scratch of its packed and split-K paths is a file-scope device array: each GPU the
// library runs on holds one copy (kNoAllocScratchBytes) from the library's first use on
// it until the process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol); the address hipGetSymbolAddress returns for
// the current device is looked up once per device and used instead.  Every call on a
// GPU shares that GPU's array: calls that overlap on one GPU (different streams, or
// host threads) race.  The packed operands and split-K partials are written in full
// before they are read, so nothing has to start at zero.
// ---------------------------------------------------------------------------------
#include <mutex>

namespace kore {

constexpr size_t kNoAllocScratchBytes = 64ull << 20;  // 64 MiB per GPU
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
void* g_scratch_ptr[64] = {};
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (resolved once per device).
int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return set_error(KORE_EHIP, "gemm_noalloc: no current HIP device (%s)", hipGetErrorString(e));
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return set_error(KORE_EHIP, "gemm_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                       hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KORE_OK;
}
}  // namespace
}  // namespace kore

extern "C" size_t kore_gemm_noalloc_scratch_bytes(void) { return kore::kNoAllocScratchBytes; }

extern "C" int kore_gemm_noalloc(int dtype, int act, const void* a, int64_t lda_m, int64_t lda_k, const void* b,
                                 int64_t ldb_k, int64_t ldb_n, const void* bias, void* c, int64_t ldc_m, int64_t M,
                                 int64_t N, int64_t K, void* stream) {
  using namespace kore;
  GemmDesc d{dtype, act, a, b, bias, c, M, N, K, 1, lda_m, lda_k, ldb_k, ldb_n, ldc_m, 0, 0, 0};
  void* base = nullptr;
  int rc = noalloc_scratch(&base);
  if (rc != KORE_OK) return rc;
  Ws plan;
  plan.plan = true;
  rc = run_gemm(d, plan, nullptr);
  if (rc != KORE_OK) return rc;
  if (plan.need > kNoAllocScratchBytes)
    return set_error(KORE_EWORKSPACE,
                     "gemm_noalloc: this call needs %zu bytes of scratch, more than the %zu-byte static scratch "
                     "(use kore_gemm with a workspace)",
                     plan.need, kNoAllocScratchBytes);
  Ws ws;
  ws.ptr = base;
  ws.bytes = kNoAllocScratchBytes;
  return run_gemm(d, ws, stream);
}
