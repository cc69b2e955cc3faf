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
  hipLaunchKernelGGL((gemm_fp8_bs_kernel<BM, BN>), dim3((unsigned)blocks), dim3(kEngineThreads), 0,
                     (hipStream_t)stream, p);
  return check_launch("gemm_fp8_bs_kernel");
}
