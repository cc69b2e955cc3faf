// Shared device/host helpers for the gfx950 (CDNA4) GEMM-family kernels.
//
// Lane layouts used throughout (verified on MI355X with an in-bounds probe of the
// compiler builtins):
//   v_mfma_f32_32x32x16_{bf16,f16}: lane l holds 8 K-consecutive values of row
//     (l % 32) of each operand, K offset 8*(l/32); output register i of lane l is
//     D[8*(i/4) + 4*(l/32) + (i%4)][l % 32].
//   v_mfma_f32_32x32x64_f8f6f4 (e4m3): lane l holds 32 K-consecutive bytes of row
//     (l % 32), K offset 32*(l/32); same output layout.
//   v_mfma_f32_16x16x32_bf16: lane l holds 8 K values of row (l % 16) at K offset
//     8*(l/16); output register i is D[4*(l/16) + i][l % 16].
//   v_mfma_f32_16x16x128_f8f6f4, v_mfma_i32_{32x32x32,16x16x64}_i8: row (l % 32) or
//     (l % 16) per lane, output layouts as above (pinned by the GPU parity tests
//     of the kernels that use them).
// Only the pairing of A and B K-slots matters for a product, and both operands are
// always staged with the same K mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kore {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Element tags: the 16-bit float types share all staging code and differ only in
// the MFMA opcode and the final conversion.
struct BF16 {};
struct F16 {};
struct INT8 {};  // int8 operands (a8w8): bytes staged like the 16-bit ones, i32 accumulators
struct FP8 {};   // fp8 (OCP e4m3) operands on the same byte layout (BufPipeEngine::mainloop_f8)

template <typename T> struct MfmaOp;
template <> struct MfmaOp<BF16> {
  static __device__ __forceinline__ f32x16_t mma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t mma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // Two fp32 -> two packed bf16 (round to nearest even, overflow -> inf, NaN kept).
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    __bf16 a = (__bf16)x, b = (__bf16)y;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  }
  static __device__ __forceinline__ float to_f32(uint16_t v) {
    return __builtin_bit_cast(float, (uint32_t)v << 16);
  }
};
// 16x16x32 MFMA accumulating in place in AGPRs (inline asm: srcC and vdst are the same
// registers).  With 256 AGPRs of accumulators (one wave per SIMD, 128 x 128 wave tiles)
// the builtin's separate result lets the register allocator rotate every accumulator
// through fresh AGPRs and copy it back once per stage (about 500 v_accvgpr moves per
// 128 MFMAs); the tied form keeps each tile in place.  The compiler does not see these
// as MFMAs, so the caller provides the wait states around them: the first product of each
// accumulator is mma16_acc0 (no VALU write precedes it), and at least 7 wait states
// separate the last of these from any VALU read of the accumulators (mma16_acc_fence
// below gives 24).
template <typename T> __device__ __forceinline__ void mma16_acc(f32x4_t& c, u32x4_t a, u32x4_t b);
template <> __device__ __forceinline__ void mma16_acc<BF16>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
template <> __device__ __forceinline__ void mma16_acc<F16>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// int8 on the same layout: v_mfma_i32_16x16x64_i8 takes 16 bytes per lane (row l % 16, K
// bytes 16 (l / 16) .. + 15 of a 64-byte sub-step, the chunks the 16-bit engines read) and
// accumulates int32 bit patterns in the f32x4_t registers.
template <> __device__ __forceinline__ void mma16_acc<INT8>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// First product of an accumulator: the same MFMA with an inline-constant zero for srcC, so
// no VALU instruction writes the accumulators before the MFMAs read them.
template <typename T> __device__ __forceinline__ void mma16_acc0(f32x4_t& c, u32x4_t a, u32x4_t b);
template <> __device__ __forceinline__ void mma16_acc0<BF16>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}
template <> __device__ __forceinline__ void mma16_acc0<F16>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}
template <> __device__ __forceinline__ void mma16_acc0<INT8>(f32x4_t& c, u32x4_t a, u32x4_t b) {
  asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}
// fp8 (OCP e4m3) 16x16x128 on AGPR accumulators in place, 32 bytes per lane (two 16-byte
// chunks); first product with a zero srcC, as above.
__device__ __forceinline__ void mma16_f8_acc(f32x4_t& c, i32x8_t a, i32x8_t b) {
  asm("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mma16_f8_acc0(f32x4_t& c, i32x8_t a, i32x8_t b) {
  asm("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
}
// Wait states around a run of mma16_acc (scheduling fences keep other instructions from
// moving across).
__device__ __forceinline__ void mma16_acc_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <> struct MfmaOp<F16> {
  static __device__ __forceinline__ f32x16_t mma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4_t mma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    _Float16 a = (_Float16)x, b = (_Float16)y;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  }
  static __device__ __forceinline__ float to_f32(uint16_t v) {
    return (float)__builtin_bit_cast(_Float16, v);
  }
};

// fp8 (OCP e4m3) 32x32x64 MFMA with unit scales.  The scaled builtin with zero
// scale operands lowers to the unscaled v_mfma_f32_32x32x64_f8f6f4 opcode.
__device__ __forceinline__ f32x16_t mma32_fp8(i32x8_t a, i32x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mma16_fp8(i32x8_t a, i32x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// int8 MFMAs (int32 accumulate): 16 K-bytes per lane, the same row-per-lane layout and
// output layout as the 16-bit shapes of the same M x N.
__device__ __forceinline__ i32x16_t mma32_i8(u32x4_t a, u32x4_t b, i32x16_t c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, a), __builtin_bit_cast(i32x4_t, b), c, 0,
                                               0, 0);
}
__device__ __forceinline__ i32x4_t mma16_i8(u32x4_t a, u32x4_t b, i32x4_t c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a), __builtin_bit_cast(i32x4_t, b), c, 0,
                                               0, 0);
}

// Epilogue activations (fp32), KORE act codes, built on the hardware exp2 and
// reciprocal (v_exp_f32 / v_rcp_f32, ~1 ulp): e^x = 2^(x*log2(e)).
//   sigmoid(x) = 1 / (1 + e^-x)
//   silu(x)    = x * sigmoid(x)
//   gelu(x)    = x * sigmoid(2u), u = sqrt(2/pi)*(x + 0.044715 x^3), which equals
//                0.5x(1 + tanh(u)) (tanh approximation of GELU)
//   tanh(x)    = 2 * sigmoid(2x) - 1
// Saturation is exact: e^-x -> inf gives rcp(inf) = 0, e^-x -> 0 gives 1, so
// gelu(-inf-like) = -0, gelu(+large) = x and no NaN appears for finite x.
enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2, ACT_SILU = 3, ACT_TANH = 4, ACT_SIGMOID = 5 };

__device__ __forceinline__ float fast_sigmoid(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

template <int ACT>
__device__ __forceinline__ float apply_act(float x) {
  if constexpr (ACT == ACT_RELU) {
    return x < 0.0f ? 0.0f : x;  // NaN passes through like torch.relu
  } else if constexpr (ACT == ACT_GELU) {
    const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return x * fast_sigmoid(2.0f * u);
  } else if constexpr (ACT == ACT_SILU) {
    return x * fast_sigmoid(x);
  } else if constexpr (ACT == ACT_TANH) {
    return 2.0f * fast_sigmoid(2.0f * x) - 1.0f;
  } else if constexpr (ACT == ACT_SIGMOID) {
    return fast_sigmoid(x);
  } else {
    return x;
  }
}

// XOR swizzle of 16-byte chunks inside a 128-byte LDS row, for the 32-row fragment
// shape (32x32 MFMAs: lane l reads row l % 32 at chunk c(l / 32)).  Measured with an
// in-bounds ds_read_b128 probe on MI355X (8 waves per CU, 1 KiB per wave instruction):
// that read pattern runs at the contiguous rate, 4 cycles per instruction per CU
// (256 bytes per clock).
__device__ __forceinline__ int swz8(int r) { return (r ^ (r >> 3)) & 7; }

// Swizzle key for the 16-row fragment shape (16x16 MFMAs: lane l reads row l % 16 of a
// 16-row group at chunk c0 + l / 16).  With swz8 that pattern took 8 cycles per
// instruction in the same probe (a 2-way bank conflict, also seen as rocprof's
// SQ_LDS_BANK_CONFLICT in the kernels that used it), with this key 4, the contiguous rate.  Only r % 16 matters: any XOR that
// is constant over a 16-row group moves every lane's chunk alike.
__device__ __forceinline__ int swz16(int r) {
  return ((((r >> 2) & 3) << 1) ^ ((r & 3) << 1) ^ (r & 1)) & 7;
}

// XCD-aware remap of a 1-D launch: workgroups are dispatched round-robin over the
// 8 XCDs, so consecutive tile ids are handed to one XCD (one L2) when possible.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  if ((nblocks & 7) != 0) return bid;
  const int per = nblocks >> 3;
  return (bid & 7) * per + (bid >> 3);
}

__device__ __forceinline__ void lds_fence_barrier() { __syncthreads(); }

}  // namespace kore

// ---- host-side error plumbing (defined in status.cpp) ----
namespace kore {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus();

// Device scratch of one call: the caller's workspace (the library allocates none).
// In plan mode nothing is launched: the dispatch only records in `need` the bytes
// the path it picks would take, which is what the *_workspace_bytes queries return.
struct Ws {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool plan = false;
  size_t need = 0;
  // Scratch of `n` bytes (256-byte aligned start) for the chosen path: nullptr in
  // plan mode (after recording the need) or when the workspace is too small.
  void* take(size_t n) {
    if (plan) {
      if (n > need) need = n;
      return nullptr;
    }
    const uintptr_t base = ((uintptr_t)ptr + 255) & ~(uintptr_t)255;
    if (ptr == nullptr || base - (uintptr_t)ptr + n > bytes) return nullptr;
    return (void*)base;
  }
};
// Bytes a workspace must hold so that take(n) succeeds whatever its alignment.
inline size_t ws_bytes(size_t need) { return need == 0 ? 0 : need + 256; }

// Top-1 grouped fp8 a8w8 GEMM over an expert-sorted token order (tiles of
// gemm_fp8_blockscale.hip, called by the grouped entry in moe.hip): xq[M,K] (row
// stride ldx), wq[E,N,K] and ws[E,N] contiguous, xs[m * xs_stride]; sorted/block_expert
// come from the align kernel with block `block_rows` (128 or 256) and `capacity` slots.
struct GroupedA8Args {
  const void* xq;
  int64_t ldx;
  const void* wq;
  const float* xs;
  int64_t xs_stride;
  const float* ws;
  const int32_t* sorted;
  const int32_t* block_expert;
  void* y;
  int64_t ldy;
  int64_t M, N, K, capacity;
  int block_rows;
};
int launch_grouped_a8w8(const GroupedA8Args& a, hipStream_t st);

// fp32 GEMM + bias + activation (gemm_f32.hip, called by kore_gemm for KORE_DT_FP32):
// A (m, k) at a[m*sam + k*sak], B (k, n) at b[k*sbk + n*sbn], C[m*scm + n], bias[N].
struct GemmF32Args {
  const void* a;
  const void* b;
  const void* bias;
  void* c;
  int64_t M, N, K;
  int64_t sam, sak, sbk, sbn, scm;
  int act;
};
int launch_gemm_f32(const GemmF32Args& d, Ws& ws, hipStream_t st);
}  // namespace kore
