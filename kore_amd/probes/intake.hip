// LDS intake microbenchmark (measurement tool, not part of libkore_amd.so).
//
// One workgroup per CU streams 32 stages of 64 KiB into a two-slot LDS ring with
// direct-to-LDS buffer loads (the GEMM tiles' staging), one barrier pair per stage, and
// optionally reads the landed slot back with ds_read_b128 (the tiles' fragment reads),
// so the per-CU rates of the two LDS clients can be measured alone and together.
//   MODE 0: each 1 KiB load instruction covers 8 rows x 128 B (rows `rs` bytes apart,
//           +128 B per stage): the tiles' operand shape.
//   MODE 1: each load instruction covers 1 KiB of contiguous memory.
//   reads > 0: per stage each wave issues `reads` ds_read_b128 (4 independent chains);
//   reads < 0: the same reads with no loads at all.
// Every address stays inside `bytes` of `src` (16 tiles of 2 MiB, rows of 4 KiB), and
// the buffer range check drops anything beyond; LDS offsets stay inside the 128 KiB ring.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void bar() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int NW, int MODE>
__global__ void __launch_bounds__(NW * 64)
    intake_kernel(const uint8_t* src, uint32_t bytes, int rs, int nstage, int reads, uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * 65536];
  constexpr int L = 64 / NW;  // load instructions per wave and stage
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t base = (uint32_t)(blockIdx.x % 16) * (2u << 20);
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), (short)0, (int)bytes, 0x00020000);
  auto issue = [&](int s, int slot) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const int q = wave + NW * i;
      uint32_t voff, soff;
      if (MODE == 0) {
        voff = base + (uint32_t)((8 * q + (lane >> 3)) * rs + 16 * (lane & 7));
        soff = (uint32_t)s * 128u;
      } else {
        voff = base + (uint32_t)(q * 1024 + 16 * lane);
        soff = (uint32_t)s * 65536u;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(lds + slot * 65536 + q * 1024), 16, (int)voff,
                                               (int)soff, 0, 0);
    }
  };
  const bool dma = reads >= 0;
  if (reads < 0) reads = -reads;
  uint32_t acc = 0;
  if (dma) issue(0, 0);
  if (dma && nstage > 1) issue(1, 1);
  for (int s = 0; s < nstage; ++s) {
    if (s + 1 < nstage) wait_vm<L>();
    else wait_vm<0>();
    bar();
    const uint8_t* sl = lds + (s & 1) * 65536;
    u32x4_t a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0;
    for (int i = 0; i < reads; i += 4) {
      a0 ^= *(const u32x4_t*)(sl + (((i + 0) * 1024 + wave * 4096 + lane * 16) & 65535));
      a1 ^= *(const u32x4_t*)(sl + (((i + 1) * 1024 + wave * 4096 + lane * 16) & 65535));
      a2 ^= *(const u32x4_t*)(sl + (((i + 2) * 1024 + wave * 4096 + lane * 16) & 65535));
      a3 ^= *(const u32x4_t*)(sl + (((i + 3) * 1024 + wave * 4096 + lane * 16) & 65535));
    }
    const u32x4_t ax = a0 ^ a1 ^ a2 ^ a3;
    acc ^= ax[0] ^ ax[1] ^ ax[2] ^ ax[3];
    bar();
    if (dma && s + 2 < nstage) issue(s + 2, s & 1);
  }
  wait_vm<0>();
  if (acc == 0x12345678u) out[blockIdx.x] = acc;  // keeps the reads live
}

// Launch on `stream`: nw in {4, 8}, mode in {0, 1}; `reads` a multiple of 4 (negative:
// reads without loads).  Returns the HIP error code of the launch.
extern "C" int kore_probe_intake(int nw, int mode, const void* src, uint32_t bytes, int rs, int nstage, int reads,
                                 void* out, void* stream) {
  if (bytes < (32u << 20) || rs > 4096 || nstage < 1 || nstage > 32 || reads % 4 != 0) return (int)hipErrorInvalidValue;
  const dim3 g(256), b((unsigned)(nw * 64));
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s = (const uint8_t*)src;
  uint32_t* o = (uint32_t*)out;
  if (nw == 4 && mode == 0) hipLaunchKernelGGL((intake_kernel<4, 0>), g, b, 0, st, s, bytes, rs, nstage, reads, o);
  else if (nw == 4 && mode == 1) hipLaunchKernelGGL((intake_kernel<4, 1>), g, b, 0, st, s, bytes, rs, nstage, reads, o);
  else if (nw == 8 && mode == 0) hipLaunchKernelGGL((intake_kernel<8, 0>), g, b, 0, st, s, bytes, rs, nstage, reads, o);
  else if (nw == 8 && mode == 1) hipLaunchKernelGGL((intake_kernel<8, 1>), g, b, 0, st, s, bytes, rs, nstage, reads, o);
  else return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}
