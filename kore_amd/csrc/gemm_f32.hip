// fp32 GEMM with fused bias + activation on the fp32 matrix cores (gfx950).
//
// C[M,N] = act(A[M,K] @ B[K,N] + bias[N]), fp32 in, fp32 out, v_mfma_f32_32x32x2_f32
// (full fp32 products, fp32 accumulation).  One such MFMA is 4096 FLOP and occupies the
// matrix core for 64 cycles, so the kernel is MFMA-bound with a register-staged double
// buffer and one barrier per K step, provided a K step's MFMAs outlast the global load
// latency of the next step: K steps are 64 values (a 64x32 wave tile issues 64 MFMAs,
// ~4000 cycles, per step; 32-value steps measured 20% slower at one tile per CU).
//
// 4 waves in a 2x2 grid, each (BM/2) x (BN/2) as 32x32 blocks; K step 64 floats.
//  A tile in LDS: BM rows of 64 floats (256 bytes), 16-byte chunk c of row r stored at
//    c ^ (r % 16), so a fragment read (16 rows per pass, one chunk each) is
//    conflict-free.  Lane l reads chunk 2q + l/32 of its row: 4 K values that feed 4
//    MFMAs (K slot l/32 of MFMA j holds k = 8q + 4(l/32) + j; B uses the same map).
//  B, K-contiguous ([N,K] rows, the W.t() view): the same layout as A.
//  B, N-contiguous ([K,N] rows): 64 rows of BN floats, row stride BN + 8 so the two
//    half-waves (rows k and k+4) fall on different banks; a lane reads the 4 K values
//    of its column with 4 ds_read_b32.
// The B fragment is the first MFMA operand, so lane l owns output row l % 32 and four
// N-consecutive columns per register group: 16-byte stores straight from registers.
//
// Any other layout, K % 32 != 0 or unaligned rows: large problems are packed into the
// caller's workspace first; small ones run a bounds-checked generic MFMA kernel.
#include "../../include/kore_amd.h"
#include "kore_common.hpp"
#include "tile_engine.hpp"

#include <type_traits>

namespace kore {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

struct F32Params {
  const float* a;
  const float* b;
  const float* bias;
  float* c;
  int M, N, K;
  int64_t lda, ldb, ldc;  // ldb: between n rows (B_KC) or k rows (B_NC)
  int tiles_m, tiles_n;
  int act;
  int vec_store;
  int kb;  // ring kernel, N-contiguous B: K-rows that exist (rows from kb on read as 0)
  int kreal;  // ring kernel K-tail mode: the true K (K is then rounded up to 32)
};

constexpr int kF32BK = 64;          // K values per stage
constexpr int kF32CH = kF32BK / 4;   // 16-byte chunks per staged row

// 16-byte chunk position of chunk c in row r: XOR with r % 16, so the 16 rows a
// 16-lane pass of ds_read_b128 touches land on 16 distinct chunk columns (64 banks).
__device__ __forceinline__ int f32_pos(int r, int c) { return c ^ (r & (kF32CH - 1)); }

// M16: 16x16x4 MFMAs (lane l: row l % 16, K slot l / 16) instead of 32x32x2 (row l % 32,
// K slot l / 32); the N-contiguous B row stride then puts the four K-slot row groups
// (rows 4 apart) on distinct banks with BN + 4.
template <int BM, int BN, bool BNC, bool M16>
struct F32Cfg {
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int BS = M16 ? 16 : 32;  // MFMA block edge
  static constexpr int MI = WM / BS, NI = WN / BS;
  static_assert(MI >= 1 && NI >= 1, "wave tile");
  static constexpr int A_FLOATS = BM * kF32BK;
  static constexpr int B_STRIDE = BNC ? BN + (M16 ? 4 : 8) : kF32BK;
  static constexpr int B_FLOATS = BNC ? kF32BK * B_STRIDE : BN * kF32BK;
  static constexpr int STAGE = A_FLOATS + B_FLOATS;
  static constexpr int AL = BM * kF32CH / 256;  // 16-byte A chunks per thread
  static constexpr int BL = BN * kF32CH / 256;  // 16-byte B chunks per thread
  static_assert(AL * 256 == BM * kF32CH && BL * 256 == BN * kF32CH, "loads cover the tile");
  static_assert(2 * STAGE * 4 <= 160 * 1024, "LDS budget");
};

template <int ACT>
__device__ __forceinline__ void f32_store(const F32Params& p, float (&v)[4], int m, int n) {
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.bias != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[e] = n + e < p.N ? p.bias[n + e] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = apply_act<ACT>(v[e] + bv[e]);
  float* dst = p.c + (int64_t)m * p.ldc + n;
  if (p.vec_store && n + 4 <= p.N) {
    *(f32x4v*)dst = f32x4v{v[0], v[1], v[2], v[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < p.N) dst[e] = v[e];
  }
}

template <int BM, int BN, bool BNC, bool M16>
__global__ void __launch_bounds__(256) gemm_f32_kernel(const F32Params p) {
  using C = F32Cfg<BM, BN, BNC, M16>;
  using AccT = std::conditional_t<M16, f32x4_t, f32x16_t>;
  constexpr int BS = C::BS, NACC = M16 ? 4 : 16, KPF = M16 ? 16 : 8;  // K values per fragment group
  constexpr int MI = C::MI, NI = C::NI, AL = C::AL, BL = C::BL;
  __shared__ __attribute__((aligned(16))) float lds[2 * C::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = M16 ? (lane & 15) : (lane & 31), hh = M16 ? (lane >> 4) : (lane >> 5);
  const int bid = (int)blockIdx.x;
  const int m0 = (bid % p.tiles_m) * BM, n0 = (bid / p.tiles_m) * BN;
  const int nk = p.K / kF32BK;

  // ---- global -> register sources (rows clamped; their results are never stored) ----
  const float* a_src[AL];
  int a_dst[AL];
#pragma unroll
  for (int j = 0; j < AL; ++j) {
    const int q = tid + 256 * j, r = q / kF32CH, ch = q % kF32CH;
    a_src[j] = p.a + (int64_t)min(m0 + r, p.M - 1) * p.lda + 4 * ch;
    a_dst[j] = r * kF32BK + 4 * f32_pos(r, ch);
  }
  const float* b_src[BL];
  int b_dst[BL];
#pragma unroll
  for (int j = 0; j < BL; ++j) {
    const int q = tid + 256 * j;
    if constexpr (BNC) {
      // row k = q / (BN/4), 4 columns at (q % (BN/4)) * 4; N % 4 == 0 so a clamped
      // chunk only ever lands in columns >= N
      const int k = q / (BN / 4), c4 = (q % (BN / 4)) * 4;
      b_src[j] = p.b + (int64_t)k * p.ldb + min(n0 + c4, p.N - 4);
      b_dst[j] = C::A_FLOATS + k * C::B_STRIDE + c4;
    } else {
      const int r = q / kF32CH, ch = q % kF32CH;
      b_src[j] = p.b + (int64_t)min(n0 + r, p.N - 1) * p.ldb + 4 * ch;
      b_dst[j] = C::A_FLOATS + r * kF32BK + 4 * f32_pos(r, ch);
    }
  }
  const int64_t b_kstep = BNC ? (int64_t)kF32BK * p.ldb : kF32BK;

  f32x4v ra[AL], rb[BL];
  auto load = [&](int kt) {
#pragma unroll
    for (int j = 0; j < AL; ++j) ra[j] = *(const f32x4v*)(a_src[j] + (int64_t)kt * kF32BK);
#pragma unroll
    for (int j = 0; j < BL; ++j) rb[j] = *(const f32x4v*)(b_src[j] + (int64_t)kt * b_kstep);
  };
  auto store = [&](int buf) {
    float* s = lds + buf * C::STAGE;
#pragma unroll
    for (int j = 0; j < AL; ++j) *(f32x4v*)(s + a_dst[j]) = ra[j];
#pragma unroll
    for (int j = 0; j < BL; ++j) *(f32x4v*)(s + b_dst[j]) = rb[j];
  };

  AccT acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < NACC; ++r) acc[i][j][r] = 0.0f;

  const int rowA0 = wm * C::WM, rowB0 = wn * C::WN;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load(kt + 1);
    const float* s = lds + (kt & 1) * C::STAGE;
    // fragments of K group q (KPF K values): A chunk (KPF/4) q + hh of each block's row,
    // and B's matching 4 K values of each block's column
    f32x4v af[2][MI], bf[2][NI];
    auto frags = [&](int q, f32x4v (&fa)[MI], f32x4v (&fb)[NI]) {
      const int chunk = (KPF / 4) * q + hh;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = rowA0 + BS * i + lr;
        fa[i] = *(const f32x4v*)(s + r * kF32BK + 4 * f32_pos(r, chunk));
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = rowB0 + BS * j + lr;
        if constexpr (BNC) {
          const float* col = s + C::A_FLOATS + (KPF * q + 4 * hh) * C::B_STRIDE + n;
          fb[j] = f32x4v{col[0], col[C::B_STRIDE], col[2 * C::B_STRIDE], col[3 * C::B_STRIDE]};
        } else {
          fb[j] = *(const f32x4v*)(s + C::A_FLOATS + n * kF32BK + 4 * f32_pos(n, chunk));
        }
      }
    };
    // group q + 1's LDS reads are issued before group q's MFMAs, so their latency hides
    // under 4*MI*NI MFMAs (the compiler otherwise reads each group right before use)
    frags(0, af[0], bf[0]);
#pragma unroll
    for (int q = 0; q < kF32BK / KPF; ++q) {
      if (q + 1 < kF32BK / KPF) frags(q + 1, af[(q + 1) & 1], bf[(q + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j) {
            if constexpr (M16)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[q & 1][j][e], af[q & 1][i][e], acc[i][j], 0, 0, 0);
            else
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[q & 1][j][e], af[q & 1][i][e], acc[i][j], 0, 0, 0);
          }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (kt + 1 < nk) store((kt + 1) & 1);
    __syncthreads();
  }

  auto epi = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = m0 + rowA0 + BS * i + lr;
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int g = 0; g < NACC / 4; ++g) {
          float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          // 32x32: register group g holds columns 8g + 4hh ..; 16x16: columns 4hh ..
          f32_store<ACT>(p, v, m, n0 + rowB0 + BS * j + (M16 ? 4 * hh : 8 * g + 4 * hh));
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

// Any strides, any K: 64x64 tile, BK 16, fp32 FMA.
struct F32GenericParams {
  const float* a;
  const float* b;
  const float* bias;
  float* c;
  int M, N, K;
  int64_t sam, sak, sbk, sbn, scm;
  int act;
};

// Generic fp32 kernel on the fp32 matrix cores: any strides, any K (layouts the MFMA
// kernels cannot read when the problem is too small for a pack pass).  128x128 tiles, 4 waves of 64x64, K steps of
// 16; operands read element by element along whichever index is unit-stride (a wave
// reads 256 contiguous bytes), every read bounds-checked, the next step prefetched into
// registers.  LDS rows of 16 floats at a stride of 20: a 16-byte fragment read by 8
// consecutive rows covers all 32 banks once.  K group q: lane half hh holds
// k = 8q + 4hh + e, which MFMA e consumes (the same map for A and B).
constexpr int kF32GK = 16, kF32GLd = 20;

__global__ void __launch_bounds__(256) gemm_f32_generic_kernel(const F32GenericParams p) {
  __shared__ __attribute__((aligned(16))) float sA[128 * kF32GLd];
  __shared__ __attribute__((aligned(16))) float sB[128 * kF32GLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, hh = lane >> 5;
  const int m0 = (int)blockIdx.y * 128, n0 = (int)blockIdx.x * 128;
  const bool a_rows = p.sak != 1 && p.sam == 1;  // A's M index is the unit-stride one
  const bool b_rows = p.sbk != 1 && p.sbn == 1;  // B's N index is the unit-stride one
  auto idx = [&](bool rows, int e, int& r, int& k) {
    const int q = e * 256 + tid;  // 0 .. 2047
    if (rows) { r = q & 127; k = q >> 7; } else { k = q & 15; r = q >> 4; }
  };
  float ra[8], rb[8];
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int r, k;
      idx(a_rows, e, r, k);
      const int gm = m0 + r, gka = k0 + k;
      ra[e] = (gm < p.M && gka < p.K) ? p.a[(int64_t)gm * p.sam + (int64_t)gka * p.sak] : 0.0f;
      idx(b_rows, e, r, k);
      const int gn = n0 + r, gkb = k0 + k;
      rb[e] = (gn < p.N && gkb < p.K) ? p.b[(int64_t)gkb * p.sbk + (int64_t)gn * p.sbn] : 0.0f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int r, k;
      idx(a_rows, e, r, k);
      sA[r * kF32GLd + k] = ra[e];
      idx(b_rows, e, r, k);
      sB[r * kF32GLd + k] = rb[e];
    }
  };
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  load(0);
  for (int k0 = 0; k0 < p.K; k0 += kF32GK) {
    __syncthreads();  // the previous step's fragment reads are done
    store();
    __syncthreads();
    if (k0 + kF32GK < p.K) load(k0 + kF32GK);
#pragma unroll
    for (int q = 0; q < kF32GK / 8; ++q) {
      f32x4v af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const f32x4v*)(sA + (wm * 64 + 32 * i + lr) * kF32GLd + 8 * q + 4 * hh);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *(const f32x4v*)(sB + (wn * 64 + 32 * j + lr) * kF32GLd + 8 * q + 4 * hh);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[j][e], af[i][e], acc[i][j], 0, 0, 0);
    }
  }
  auto epi = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gm = m0 + wm * 64 + 32 * i + lr;
      if (gm >= p.M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int gn = n0 + wn * 64 + 32 * j + 8 * g + 4 * hh + e;
            if (gn >= p.N) continue;
            p.c[(int64_t)gm * p.scm + gn] = apply_act<ACT>(acc[i][j][4 * g + e] + (p.bias ? p.bias[gn] : 0.0f));
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

inline bool al16(const void* q) { return ((uintptr_t)q & 15u) == 0; }

// Transposed or strided operands the MFMA kernel cannot read (K-contiguous rows go to
// repitch32_kernel below): out[r][k] = in[r * sr + k * sk] for k < K, 0 for
// K <= k < Kp (a multiple of 64), rows of Kp floats.  64 x 64 tiles through LDS, loads
// along whichever index is unit-stride, 16-byte row stores.
__global__ void __launch_bounds__(256) pack32_kernel(const float* in, int64_t sr, int64_t sk, float* out, int R, int K,
                                                     int Kp) {
  __shared__ float t[64][65];  // [r][k]
  const int tid = threadIdx.x;
  const int r0 = (int)blockIdx.y * 64, k0 = (int)blockIdx.x * 64;
  const bool r_unit = sr == 1 && sk != 1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int u = tid & 63, v = 4 * i + (tid >> 6);
    const int r = r_unit ? u : v, k = r_unit ? v : u;
    const int gr = r0 + r, gk = k0 + k;
    t[r][k] = (gr < R && gk < K) ? in[(int64_t)gr * sr + (int64_t)gk * sk] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int idx = tid + 256 * q, r = idx >> 4, ch = idx & 15;
    if (r0 + r >= R) continue;
    *(f32x4v*)(out + (int64_t)(r0 + r) * Kp + k0 + 4 * ch) =
        f32x4v{t[r][4 * ch], t[r][4 * ch + 1], t[r][4 * ch + 2], t[r][4 * ch + 3]};
  }
}

// K-contiguous rows (any row stride, e.g. K = 4095): out[r][k] = in[r * sr + k] for k < K,
// 0 for K <= k < Kp.  One thread per 16-byte output chunk of 4 floats (dword loads, the
// row's last partial chunk and the zero tail element by element): a straight copy at HBM
// rate instead of pack32_kernel's LDS round trip.
__global__ void __launch_bounds__(256) repitch32_kernel(const float* in, int64_t sr, float* out, int R, int K,
                                                        int Kp) {
  const int cpr = Kp / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)R * cpr) return;
  const int r = (int)(idx / cpr), k0 = (int)(idx % cpr) * 4;
  const float* src = in + (int64_t)r * sr + k0;
  f32x4v v;
  if (k0 + 4 <= K) {
    v = f32x4v{src[0], src[1], src[2], src[3]};
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = k0 + j < K ? src[j] : 0.0f;
  }
  *(f32x4v*)(out + (int64_t)r * Kp + k0) = v;
}

int launch_pack32(const float* in, int64_t sr, int64_t sk, float* out, int64_t R, int64_t K, int64_t Kp,
                  hipStream_t st) {
  if (sk == 1) {
    const int64_t chunks = R * (Kp / 4);
    hipLaunchKernelGGL(repitch32_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, in, sr, out, (int)R,
                       (int)K, (int)Kp);
    return check_launch("repitch32_kernel");
  }
  hipLaunchKernelGGL(pack32_kernel, dim3((unsigned)(Kp / 64), (unsigned)((R + 63) / 64)), dim3(256), 0, st, in, sr, sk,
                     out, (int)R, (int)K, (int)Kp);
  return check_launch("pack32_kernel");
}

// ---------------------------------------------------------------------------------
// Deep-ring fp32 kernel.  The register-staged kernel above stalls once per K step on
// its LDS stores and the barrier, with one step of loads in flight.  Here an NSLOT-deep
// ring of 32-float K stages is filled by direct-to-LDS buffer loads NSLOT - 1 stages
// ahead of the MFMAs (one barrier per stage).  A and K-contiguous B use 128-byte rows
// with the swz8 chunk swizzle (source side); N-contiguous B is staged as 32 K-rows of
// BN floats and a lane reads the 4 K values of its column with 4 ds_read_b32.  Wave
// tile (BM/2) x (BN/2) as 32x32 blocks; within a stage, K group q+1's fragments are
// read under group q's MFMAs.
// ---------------------------------------------------------------------------------
constexpr int kF32RK = 32;  // K floats per ring stage

// KT: K % 32 != 0 read in place (rows at 4-byte alignment): the loop runs over K rounded
// up to 32, the last stage is read from K - 32 (no load passes K), and the columns it
// shares with the stage before are zeroed in LDS in both operands once it has landed.
template <int BM, int BN, int NSLOT, bool BNC, bool KT = false>
__global__ void __launch_bounds__(256) gemm_f32_ring_kernel(const F32Params p) {
  constexpr int WM = BM / 2, WN = BN / 2, MI = WM / 32, NI = WN / 32;
  static_assert(MI >= 1 && NI >= 1, "wave tile");
  constexpr int A_FL = BM * kF32RK, STAGE = (BM + BN) * kF32RK;  // floats
  constexpr int AJ = BM / 32, BJ = BN / 32;                       // 1 KiB loads per wave per stage
  constexpr int LPS = AJ + BJ;
  constexpr int NCR = 256 / BN, NCH = BN / 4;  // N-contiguous B: K-rows and chunks per load
  static_assert((NSLOT - 2) * LPS <= 63, "vmcnt range");
  static_assert(NSLOT * STAGE * 4 <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) float lds[NSLOT * STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, hh = lane >> 5;
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int m0 = (bid % p.tiles_m) * BM, n0 = (bid / p.tiles_m) * BN;
  const int rows_a = min(BM, p.M - m0), rows_b = min(BN, p.N - n0);
  const int nk = p.K / kF32RK;
  const int kv = KT ? p.kreal : p.K;  // K the operands hold

  // buffer resources and per-lane byte offsets (rows past the tile re-read its last row,
  // chunks past N re-read the last chunk: they only feed outputs that are never stored)
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(p.a + (int64_t)m0 * p.lda, (uint32_t)(((int64_t)(rows_a - 1) * p.lda + kv) * 4));
  const __amdgpu_buffer_rsrc_t rb =
      BNC ? make_rsrc(p.b + n0, (uint32_t)(((int64_t)(p.kb - 1) * p.ldb + rows_b) * 4))
          : make_rsrc(p.b + (int64_t)n0 * p.ldb, (uint32_t)(((int64_t)(rows_b - 1) * p.ldb + kv) * 4));
  uint32_t a_voff[AJ], b_voff[BJ];
#pragma unroll
  for (int j = 0; j < AJ; ++j) {
    const int r = (wave + 4 * j) * 8 + (lane >> 3);
    a_voff[j] = (uint32_t)(((int64_t)min(r, rows_a - 1) * p.lda + 4 * ((lane & 7) ^ swz8(r))) * 4);
  }
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    if constexpr (BNC) {
      const int kr = (wave + 4 * j) * NCR + lane / NCH;
      b_voff[j] = (uint32_t)(((int64_t)kr * p.ldb + min(4 * (lane % NCH), rows_b - 4)) * 4);
    } else {
      const int r = (wave + 4 * j) * 8 + (lane >> 3);
      b_voff[j] = (uint32_t)(((int64_t)min(r, rows_b - 1) * p.ldb + 4 * ((lane & 7) ^ swz8(r))) * 4);
    }
  }
  const uint32_t b_kstep = BNC ? (uint32_t)(kF32RK * p.ldb * 4) : (uint32_t)(kF32RK * 4);
  // K tail: the last stage's scalar offsets (from K - 32) and its columns [0, kdup)
  const uint32_t a_klast = (uint32_t)((kv - kF32RK) * 4);
  const uint32_t b_klast = BNC ? (uint32_t)((int64_t)(kv - kF32RK) * p.ldb * 4) : a_klast;
  const int kdup = p.K - kv;
  auto issue = [&](int slot, int stage) {
    const int st = min(stage, nk - 1);  // past the end: re-load the last stage into a free slot
    const bool last = KT && st == nk - 1;
    const uint32_t sa_off = last ? a_klast : (uint32_t)st * (kF32RK * 4);
    const uint32_t sb_off = last ? b_klast : (uint32_t)st * b_kstep;
    float* base = lds + slot * STAGE;
#pragma unroll
    for (int j = 0; j < AJ; ++j) buf_lds16(ra, a_voff[j], sa_off, (uint16_t*)(base + (wave + 4 * j) * 256));
#pragma unroll
    for (int j = 0; j < BJ; ++j) buf_lds16(rb, b_voff[j], sb_off, (uint16_t*)(base + A_FL + (wave + 4 * j) * 256));
  };
  // zero K columns [0, kdup) of both operands of the stage in slot sl (rows of 32 floats
  // hold chunk c at position c ^ swz8(row); an N-contiguous B stages whole K-rows)
  auto zero_dup = [&](int sl) {
    float* base = lds + sl * STAGE;
    for (int idx = tid; idx < BM * kdup; idx += 256) {
      const int r = idx / kdup, k = idx - r * kdup;
      base[r * kF32RK + 4 * ((k >> 2) ^ swz8(r)) + (k & 3)] = 0.0f;
    }
    if constexpr (BNC) {
      for (int idx = tid; idx < kdup * BN; idx += 256) base[A_FL + idx] = 0.0f;
    } else {
      for (int idx = tid; idx < BN * kdup; idx += 256) {
        const int r = idx / kdup, k = idx - r * kdup;
        base[A_FL + r * kF32RK + 4 * ((k >> 2) ^ swz8(r)) + (k & 3)] = 0.0f;
      }
    }
  };

  // fragment offsets: row R + lr of a 32-row block (R % 32 == 0) has
  // swz8(R + lr) = (lr & 7) ^ (lr >> 3) ^ (4 * ((R / 32) & 1))
  const int rowA0 = wm * WM, rowB0 = wn * WN;
  int offA[2][4], offB[2][4];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int swa = ((lr & 7) ^ (lr >> 3) ^ (4 * ((wm * MI + par) & 1))) & 7;
    const int swb = ((lr & 7) ^ (lr >> 3) ^ (4 * ((wn * NI + par) & 1))) & 7;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      offA[par][q] = lr * kF32RK + 4 * ((2 * q + hh) ^ swa);
      offB[par][q] = lr * kF32RK + 4 * ((2 * q + hh) ^ swb);
    }
  }

  f32x16_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
  for (int st = 0; st < NSLOT - 1; ++st) issue(st, st);
  int slot = 0;
  for (int s = 0; s < nk; ++s) {
    wait_vmcnt<(NSLOT - 2) * LPS>();
    exec_barrier();
    if constexpr (KT) {
      if (s == nk - 1) {  // the last stage has landed: zero its repeated columns before any read
        zero_dup(slot);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        exec_barrier();
      }
    }
    issue(slot == 0 ? NSLOT - 1 : slot - 1, s + NSLOT - 1);
    const float* sa = lds + slot * STAGE + rowA0 * kF32RK;
    const float* sb = lds + slot * STAGE + A_FL;
    // K group q (8 K values): lane half hh holds k = 8q + 4hh + e for e = 0..3
    auto frags = [&](int q, f32x4v (&fa)[MI], f32x4v (&fb)[NI]) {
#pragma unroll
      for (int i = 0; i < MI; ++i) fa[i] = *(const f32x4v*)(sa + i * 32 * kF32RK + offA[i & 1][q]);
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        if constexpr (BNC) {
          const float* col = sb + (8 * q + 4 * hh) * BN + rowB0 + 32 * j + lr;
          fb[j] = f32x4v{col[0], col[BN], col[2 * BN], col[3 * BN]};
        } else {
          fb[j] = *(const f32x4v*)(sb + (rowB0 + 32 * j) * kF32RK + offB[j & 1][q]);
        }
      }
    };
    f32x4v af[2][MI], bf[2][NI];
    frags(0, af[0], bf[0]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q + 1 < 4) frags(q + 1, af[(q + 1) & 1], bf[(q + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[q & 1][j][e], af[q & 1][i][e], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    slot = slot + 1 == NSLOT ? 0 : slot + 1;
  }
  wait_vmcnt<0>();  // the clamped trailing loads must land before the kernel ends

  auto epi = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = m0 + rowA0 + 32 * i + lr;
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < NI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
          f32_store<ACT>(p, v, m, n0 + rowB0 + 32 * j + 8 * g + 4 * hh);
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

template <int BM, int BN, int NSLOT, bool BNC, bool KT = false>
int launch_f32_ring(F32Params p, hipStream_t st) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm fp32: grid too large");
  hipLaunchKernelGGL((gemm_f32_ring_kernel<BM, BN, NSLOT, BNC, KT>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return check_launch("gemm_f32_ring_kernel");
}

constexpr bool kF32M16 = false;

template <int BM, int BN, bool BNC>
int launch_f32(F32Params p, hipStream_t st) {
  p.tiles_m = (p.M + BM - 1) / BM;
  p.tiles_n = (p.N + BN - 1) / BN;
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > 0x7fffffff) return set_error(KORE_EUNSUPPORTED, "gemm fp32: grid too large");
  hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BNC, kF32M16>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return check_launch("gemm_f32_kernel");
}

template <bool BNC>
int pick_f32(const F32Params& p, hipStream_t st) {
  // the largest tile that still gives every CU a tile; the deep ring whenever its
  // 32-float stages tile K and the buffer offsets fit 32 bits
  const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
  const int64_t t12864 = (int64_t)((p.M + 127) / 128) * ((p.N + 63) / 64);
  const bool ring = p.K % kF32RK == 0 && (int64_t)p.lda * 4 * 128 + (int64_t)p.K * 4 < (1ll << 31) &&
                    (BNC ? (int64_t)p.ldb * 4 * p.K + (int64_t)p.N * 4 < (1ll << 31)
                         : (int64_t)p.ldb * 4 * 128 + (int64_t)p.K * 4 < (1ll << 31));
  if (ring) {
    // 64x64 tiles on a 3-stage ring (48 KiB): up to three workgroups share a CU, so
    // one's LDS reads and barriers overlap another's MFMAs (as fast as 128x128 tiles
    // at 4096^3 and faster below); few tiles: one deeper ring per CU
    if (t12864 >= 200) return launch_f32_ring<64, 64, 3, BNC>(p, st);
    return launch_f32_ring<64, 64, 8, BNC>(p, st);
  }
  if (t128 >= 240) return launch_f32<128, 128, BNC>(p, st);
  if (t12864 >= 200) return launch_f32<128, 64, BNC>(p, st);
  return launch_f32<64, 64, BNC>(p, st);
}

}  // namespace

int launch_gemm_f32(const GemmF32Args& d, Ws& ws, hipStream_t st) {
  const bool fits = d.M < (1ll << 31) && d.N < (1ll << 31) && d.K < (1ll << 31);
  const bool a_ok = d.sak == 1 && d.sam % 4 == 0 && al16(d.a) && d.sam >= d.K;
  const bool b_kc = d.sbk == 1 && d.sbn % 4 == 0 && al16(d.b) && d.sbn >= d.K;
  const bool b_nc = d.sbn == 1 && d.sbk % 4 == 0 && al16(d.b) && d.N % 4 == 0 && d.sbk >= d.N;
  if (fits && d.K % kF32BK == 0 && d.K > 0 && a_ok && (b_kc || b_nc)) {
    F32Params p{};
    p.a = (const float*)d.a;
    p.b = (const float*)d.b;
    p.bias = (const float*)d.bias;
    p.c = (float*)d.c;
    p.M = (int)d.M;
    p.N = (int)d.N;
    p.K = (int)d.K;
    p.lda = d.sam;
    p.ldb = b_kc ? d.sbn : d.sbk;
    p.ldc = d.scm;
    p.act = d.act;
    p.vec_store = d.scm % 4 == 0 && al16(d.c);
    p.kb = p.K;
    if (ws.plan) return KORE_OK;
    return b_kc ? pick_f32<false>(p, st) : pick_f32<true>(p, st);
  }
  if (!fits) return set_error(KORE_EUNSUPPORTED, "gemm fp32: dimension >= 2^31");
  // Large K tails (K % 64 != 0, e.g. 4095) with K-contiguous A and a K-contiguous or an
  // aligned N-contiguous B: the ring kernel reads the rows in place (direct-to-LDS loads
  // take any 4-byte offset) and starts its last 32-float stage at K - 32, the columns it
  // shares with the stage before zeroed in LDS (KT); no pack pass.
  const bool b_ktc = d.sbk == 1 && d.sbn >= d.K && d.sbn * 4 * 64 + d.K * 4 < (1ll << 31);
  const bool b_ktn = b_nc && d.sbk * 4 * d.K + d.N * 4 < (1ll << 31);
  if (d.K % kF32BK != 0 && d.K > kF32RK && d.sak == 1 && d.sam >= d.K && d.sam * 4 * 64 + d.K * 4 < (1ll << 31) &&
      (b_ktc || b_ktn) && d.M * d.N * d.K >= (1ll << 26)) {
    if (ws.plan) return KORE_OK;
    F32Params p{};
    p.a = (const float*)d.a;
    p.b = (const float*)d.b;
    p.bias = (const float*)d.bias;
    p.c = (float*)d.c;
    p.M = (int)d.M;
    p.N = (int)d.N;
    p.K = (int)((d.K + kF32RK - 1) / kF32RK * kF32RK);
    p.kreal = (int)d.K;
    p.kb = (int)d.K;
    p.lda = d.sam;
    p.ldb = b_ktn ? d.sbk : d.sbn;
    p.ldc = d.scm;
    p.act = d.act;
    p.vec_store = d.scm % 4 == 0 && al16(d.c);
    const bool many = (d.M + 127) / 128 * ((d.N + 63) / 64) >= 200;
    if (b_ktn) return many ? launch_f32_ring<64, 64, 3, true, true>(p, st) : launch_f32_ring<64, 64, 8, true, true>(p, st);
    return many ? launch_f32_ring<64, 64, 3, false, true>(p, st) : launch_f32_ring<64, 64, 8, false, true>(p, st);
  }
  // Large problems in other layouts: pack A to [M, Kp] and B to [N, Kp] (K-contiguous,
  // zero K tail) in the caller's workspace, then the MFMA kernel.
  const int64_t Kp = (d.K + kF32BK - 1) / kF32BK * kF32BK;
  if (d.M * d.N * d.K >= (1ll << 26) && d.K >= kF32BK) {
    // an N-contiguous B with aligned K-rows is read in place by the ring kernel, its
    // buffer resource ending at the last real K-row (the padded rows read as zero)
    const bool b_inplace = b_nc && Kp * 4 * 128 + Kp * 4 < (1ll << 31) && d.sbk * 4 * Kp + d.N * 4 < (1ll << 31);
    const size_t a_bytes = (size_t)(d.M * Kp * 4 + 255) / 256 * 256;
    const size_t total = a_bytes + (b_inplace ? 0 : (size_t)d.N * Kp * 4);
    float* buf = (float*)ws.take(total);
    if (ws.plan) return KORE_OK;
    if (buf == nullptr)
      return set_error(KORE_EWORKSPACE, "gemm fp32: packing the operands needs %zu workspace bytes (got %zu)",
                       ws_bytes(total), ws.bytes);
    {
      float* ap = buf;
      float* bp = (float*)((char*)buf + a_bytes);
      int rc = launch_pack32((const float*)d.a, d.sam, d.sak, ap, d.M, d.K, Kp, st);
      if (rc == KORE_OK && b_inplace) {
        F32Params p{};
        p.a = ap;
        p.b = (const float*)d.b;
        p.bias = (const float*)d.bias;
        p.c = (float*)d.c;
        p.M = (int)d.M;
        p.N = (int)d.N;
        p.K = (int)Kp;
        p.kb = (int)d.K;
        p.lda = Kp;
        p.ldb = d.sbk;
        p.ldc = d.scm;
        p.act = d.act;
        p.vec_store = d.scm % 4 == 0 && al16(d.c);
        const int64_t t12864 = (d.M + 127) / 128 * ((d.N + 63) / 64);
        rc = t12864 >= 200 ? launch_f32_ring<64, 64, 3, true>(p, st) : launch_f32_ring<64, 64, 8, true>(p, st);
        return rc;
      }
      if (rc == KORE_OK) {
        // rows of B^T: element (n, k) at b[k * sbk + n * sbn]
        rc = launch_pack32((const float*)d.b, d.sbn, d.sbk, bp, d.N, d.K, Kp, st);
      }
      if (rc == KORE_OK) {
        F32Params p{};
        p.a = ap;
        p.b = bp;
        p.bias = (const float*)d.bias;
        p.c = (float*)d.c;
        p.M = (int)d.M;
        p.N = (int)d.N;
        p.K = (int)Kp;
        p.lda = Kp;
        p.ldb = Kp;
        p.ldc = d.scm;
        p.act = d.act;
        p.vec_store = d.scm % 4 == 0 && al16(d.c);
        p.kb = p.K;
        rc = pick_f32<false>(p, st);
      }
      return rc;
    }
  }
  if (ws.plan) return KORE_OK;
  F32GenericParams g{};
  g.a = (const float*)d.a;
  g.b = (const float*)d.b;
  g.bias = (const float*)d.bias;
  g.c = (float*)d.c;
  g.M = (int)d.M;
  g.N = (int)d.N;
  g.K = (int)d.K;
  g.sam = d.sam;
  g.sak = d.sak;
  g.sbk = d.sbk;
  g.sbn = d.sbn;
  g.scm = d.scm;
  g.act = d.act;
  dim3 grid((unsigned)((d.N + 127) / 128), (unsigned)((d.M + 127) / 128));
  hipLaunchKernelGGL(gemm_f32_generic_kernel, grid, dim3(256), 0, st, g);
  return check_launch("gemm_f32_generic_kernel");
}

}  // namespace kore
