// kore_amd._C: the PyTorch-ROCm host layer over the C ABI of libkore_amd.so.
//
// Each operator validates its tensors, allocates the output (and any workspace the C
// ABI asks for) with the tensor allocator of the input's device, and calls the C entry
// point on the current HIP stream of that device -- the stream the reference drivers
// time with events (kore/tasks/gemm_bf16/driver.py:87-93).  The operators are registered
// as torch.ops.korehip.* (TORCH_LIBRARY) and bound directly for the Python host
// (kore_amd/ops.py), so a call costs one C++ entry rather than Python-side checks and a
// ctypes marshalling.  Status codes of the C ABI become Python exceptions the way the
// reference drivers expect (a raised exception is a failing verdict,
// kore/tasks/gemm_bf16/driver.py:115-118): KORE_EINVAL / KORE_EWORKSPACE -> ValueError,
// KORE_EUNSUPPORTED -> NotImplementedError, KORE_EHIP -> RuntimeError.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>
#include <torch/library.h>

#include <optional>
#include <tuple>

#include "kore_amd.h"

namespace {

void check_rc(int rc) {
  if (rc == KORE_OK) return;
  const char* msg = kore_last_error();
  TORCH_CHECK_NOT_IMPLEMENTED(rc != KORE_EUNSUPPORTED, "kore_amd error ", rc, ": ", msg);
  TORCH_CHECK(rc != KORE_EHIP, "kore_amd error ", rc, ": ", msg);
  TORCH_CHECK_VALUE(false, "kore_amd error ", rc, ": ", msg);
}

void* stream_of(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Every tensor is a HIP device tensor on one device.
void require_hip(std::initializer_list<std::reference_wrapper<const at::Tensor>> ts) {
  const at::Tensor* first = nullptr;
  for (const at::Tensor& t : ts) {
    TORCH_CHECK_VALUE(t.defined(), "kore_amd: undefined tensor");
    TORCH_CHECK_VALUE(t.is_cuda(), "kore_amd operators need HIP device tensors (got ", t.device(), ")");
    if (first == nullptr) first = &t;
    TORCH_CHECK_VALUE(t.device() == first->device(), "tensors on different devices: ", first->device(), " vs ",
                      t.device());
  }
}

// Device scratch of one call (none when the path needs none); torch's allocator owns
// it, so under graph capture it comes from the graph's private pool.
at::Tensor workspace(size_t nbytes, const at::Tensor& like) {
  if (nbytes == 0) return at::Tensor();
  return at::empty({(int64_t)nbytes}, like.options().dtype(at::kByte));
}
void* ptr_or_null(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }
size_t bytes_of(const at::Tensor& t) { return t.defined() ? (size_t)t.numel() : 0; }

int dt_code(at::ScalarType s) {
  switch (s) {
    case at::kBFloat16: return KORE_DT_BF16;
    case at::kHalf: return KORE_DT_FP16;
    case at::kFloat: return KORE_DT_FP32;
    default: return -1;
  }
}

// ---- dense GEMM + fused epilogue (kore/tasks/gemm_bf16/seed_triton.py:64-86,
// kore/tasks/_genops.py:715-731) ----
at::Tensor gemm_fused(const at::Tensor& a, const at::Tensor& b, const std::optional<at::Tensor>& bias, int64_t act) {
  require_hip({a, b});
  TORCH_CHECK_VALUE(a.dim() == 2 && b.dim() == 2, "gemm expects 2-D operands, got ", a.sizes(), " and ", b.sizes());
  TORCH_CHECK_VALUE(a.size(1) == b.size(0), "incompatible dims: a ", a.sizes(), " @ b ", b.sizes());
  const int dt = dt_code(a.scalar_type());
  TORCH_CHECK_VALUE(dt >= 0 && b.scalar_type() == a.scalar_type(),
                    "gemm supports bf16/fp16/fp32 operands of one dtype (got ", a.scalar_type(), ", ",
                    b.scalar_type(), ")");
  TORCH_CHECK_VALUE(act >= KORE_ACT_NONE && act <= KORE_ACT_SIGMOID, "unknown activation code ", act);
  const int64_t M = a.size(0), K = a.size(1), N = b.size(1);
  at::Tensor bc;
  if (bias.has_value() && bias->defined()) {
    require_hip({a, *bias});
    TORCH_CHECK_VALUE(bias->dim() == 1 && bias->size(0) == N && bias->scalar_type() == a.scalar_type(),
                      "bias must be [", N, "] ", a.scalar_type(), " (got ", bias->sizes(), " ", bias->scalar_type(),
                      ")");
    bc = bias->contiguous();
  }
  const c10::DeviceGuard guard(a.device());
  at::Tensor c = at::empty({M, N}, a.options());
  if (M == 0 || N == 0) return c;
  const void* bp = ptr_or_null(bc);
  const size_t need = kore_gemm_workspace_bytes(dt, (int)act, a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(),
                                                b.stride(0), b.stride(1), bp, c.data_ptr(), c.stride(0), M, N, K);
  at::Tensor ws = workspace(need, a);
  check_rc(kore_gemm(dt, (int)act, a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1), bp,
                     c.data_ptr(), c.stride(0), M, N, K, ptr_or_null(ws), bytes_of(ws), stream_of(a)));
  return c;
}

at::Tensor gemm(const at::Tensor& a, const at::Tensor& b) {
  TORCH_CHECK_VALUE(a.scalar_type() == at::kBFloat16 && b.scalar_type() == at::kBFloat16,
                    "gemm (gemm_bf16 task) takes bf16 operands (got ", a.scalar_type(), ", ", b.scalar_type(), ")");
  return gemm_fused(a, b, std::nullopt, KORE_ACT_NONE);
}

// ---- batched GEMM C[i] = A[i] @ B[i]^T (kore/tasks/vendor_ops.py:914-920) ----
at::Tensor batched_gemm(const at::Tensor& a, const at::Tensor& b) {
  require_hip({a, b});
  TORCH_CHECK_VALUE(a.dim() == 3 && b.dim() == 3 && a.size(0) == b.size(0) && a.size(2) == b.size(2),
                    "batched_gemm expects a[B,M,K], b[B,N,K] (got ", a.sizes(), ", ", b.sizes(), ")");
  TORCH_CHECK_VALUE((a.scalar_type() == at::kBFloat16 || a.scalar_type() == at::kHalf) &&
                        b.scalar_type() == a.scalar_type(),
                    "batched_gemm supports bf16/fp16 (got ", a.scalar_type(), ", ", b.scalar_type(), ")");
  const int64_t B = a.size(0), M = a.size(1), K = a.size(2), N = b.size(1);
  const c10::DeviceGuard guard(a.device());
  at::Tensor c = at::empty({B, M, N}, a.options());
  if (B == 0 || M == 0 || N == 0) return c;
  const int dt = dt_code(a.scalar_type());
  const size_t need = kore_batched_gemm_workspace_bytes(dt, a.data_ptr(), a.stride(0), a.stride(1), a.stride(2),
                                                        b.data_ptr(), b.stride(0), b.stride(1), b.stride(2),
                                                        c.data_ptr(), c.stride(0), c.stride(1), B, M, N, K);
  at::Tensor ws = workspace(need, a);
  check_rc(kore_batched_gemm(dt, a.data_ptr(), a.stride(0), a.stride(1), a.stride(2), b.data_ptr(), b.stride(0),
                             b.stride(1), b.stride(2), c.data_ptr(), c.stride(0), c.stride(1), B, M, N, K,
                             ptr_or_null(ws), bytes_of(ws), stream_of(a)));
  return c;
}

// ---- GEMM backward of Y = X @ W^T (kore/tasks/gemm_backward_bf16/seed_triton.py:74-86) ----
std::tuple<at::Tensor, at::Tensor> gemm_backward(const at::Tensor& x_, const at::Tensor& w_, const at::Tensor& dy_) {
  require_hip({x_, w_, dy_});
  TORCH_CHECK_VALUE(x_.dim() == 2 && w_.dim() == 2 && dy_.dim() == 2, "gemm_backward expects 2-D x[M,K], w[N,K], dy[M,N]");
  const int64_t M = x_.size(0), K = x_.size(1), N = w_.size(0);
  TORCH_CHECK_VALUE(w_.size(1) == K && dy_.size(0) == M && dy_.size(1) == N, "incompatible shapes x", x_.sizes(), " w",
                    w_.sizes(), " dy", dy_.sizes());
  TORCH_CHECK_VALUE((x_.scalar_type() == at::kBFloat16 || x_.scalar_type() == at::kHalf) &&
                        w_.scalar_type() == x_.scalar_type() && dy_.scalar_type() == x_.scalar_type(),
                    "gemm_backward takes bf16/fp16 tensors of one dtype (got ", x_.scalar_type(), ", ",
                    w_.scalar_type(), ", ", dy_.scalar_type(), ")");
  const at::Tensor x = x_.stride(1) == 1 ? x_ : x_.contiguous();
  const at::Tensor w = w_.stride(1) == 1 ? w_ : w_.contiguous();
  const at::Tensor dy = dy_.stride(1) == 1 ? dy_ : dy_.contiguous();
  const c10::DeviceGuard guard(x.device());
  at::Tensor dx = at::empty({M, K}, x.options()), dw = at::empty({N, K}, x.options());
  if (M == 0 || N == 0 || K == 0) return {dx.zero_(), dw.zero_()};
  const int dt = dt_code(x.scalar_type());
  const size_t need = kore_gemm_backward_workspace_bytes(dt, x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                                         dy.data_ptr(), dy.stride(0), dx.data_ptr(), dx.stride(0),
                                                         dw.data_ptr(), dw.stride(0), M, N, K);
  at::Tensor ws = workspace(need, x);
  check_rc(kore_gemm_backward(dt, x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), dy.data_ptr(), dy.stride(0),
                              dx.data_ptr(), dx.stride(0), dw.data_ptr(), dw.stride(0), M, N, K, ptr_or_null(ws),
                              bytes_of(ws), stream_of(x)));
  return {dx, dw};
}

// ---- fp8 a8w8 block-scaled GEMM (kore/tasks/gemm_fp8_a8w8_blockscale/seed_triton.py:49-60) ----
at::Tensor gemm_a8w8_blockscale(const at::Tensor& xq_, const at::Tensor& wq_, const at::Tensor& xs,
                                const at::Tensor& ws) {
  require_hip({xq_, wq_, xs, ws});
  TORCH_CHECK_VALUE(xq_.scalar_type() == at::kFloat8_e4m3fn && wq_.scalar_type() == at::kFloat8_e4m3fn,
                    "xq/wq must be torch.float8_e4m3fn (got ", xq_.scalar_type(), ", ", wq_.scalar_type(), ")");
  TORCH_CHECK_VALUE(xs.scalar_type() == at::kFloat && ws.scalar_type() == at::kFloat, "scales must be fp32");
  TORCH_CHECK_VALUE(xq_.dim() == 2 && wq_.dim() == 2 && xq_.size(1) == wq_.size(1), "expected xq[M,K], wq[N,K] (got ",
                    xq_.sizes(), ", ", wq_.sizes(), ")");
  const int64_t M = xq_.size(0), K = xq_.size(1), N = wq_.size(0);
  TORCH_CHECK_VALUE(K % 128 == 0 && N % 128 == 0, "block-scale needs K % 128 == 0 and N % 128 == 0 (got N=", N, ", K=",
                    K, ")");
  TORCH_CHECK_VALUE(xs.dim() == 2 && xs.size(0) == M && xs.size(1) == K / 128 && ws.dim() == 2 &&
                        ws.size(0) == N / 128 && ws.size(1) == K / 128,
                    "scale shapes must be [", M, ",", K / 128, "] and [", N / 128, ",", K / 128, "] (got ", xs.sizes(),
                    ", ", ws.sizes(), ")");
  const bool rows_ok = xq_.stride(1) == 1 && wq_.stride(1) == 1;
  const at::Tensor xq = rows_ok ? xq_ : xq_.contiguous();
  const at::Tensor wq = rows_ok ? wq_ : wq_.contiguous();
  const c10::DeviceGuard guard(xq.device());
  at::Tensor y = at::empty({M, N}, xq.options().dtype(at::kBFloat16));
  if (M == 0) return y;
  check_rc(kore_gemm_a8w8_blockscale(xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0), xs.data_ptr<float>(),
                                     xs.stride(0), xs.stride(1), ws.data_ptr<float>(), ws.stride(0), ws.stride(1),
                                     y.data_ptr(), y.stride(0), M, N, K, stream_of(xq)));
  return y;
}

// A [n,1] / [1,n] / [n] fp32 scale: its element stride along n.
int64_t scale_stride(const at::Tensor& s, int64_t n, const char* what) {
  TORCH_CHECK_VALUE(s.scalar_type() == at::kFloat, what, " must be fp32 (got ", s.scalar_type(), ")");
  TORCH_CHECK_VALUE(s.numel() == n && (s.dim() == 1 || (s.dim() == 2 && (s.size(0) == 1 || s.size(1) == 1))), what,
                    " must hold ", n, " values as [", n, ",1], [1,", n, "] or [", n, "] (got ", s.sizes(), ")");
  const bool along0 = s.dim() == 1 || s.size(0) == n;
  return along0 ? s.stride(0) : s.stride(1);
}

// ---- a8w8 GEMM with per-row / per-column scales (kore/tasks/gemm_fp8_a8w8*/seed_triton.py,
// kore/tasks/gemm_int8_a8w8/seed_triton.py, kore/tasks/vendor_ops.py:697-760) ----
at::Tensor gemm_a8w8(const at::Tensor& xq, const at::Tensor& wq, const at::Tensor& xs, const at::Tensor& ws) {
  require_hip({xq, wq, xs, ws});
  const bool fp8 = xq.scalar_type() == at::kFloat8_e4m3fn, i8 = xq.scalar_type() == at::kChar;
  TORCH_CHECK_VALUE((fp8 || i8) && wq.scalar_type() == xq.scalar_type(),
                    "xq/wq must both be float8_e4m3fn or both int8 (got ", xq.scalar_type(), ", ", wq.scalar_type(),
                    ")");
  TORCH_CHECK_VALUE(xq.dim() == 2 && wq.dim() == 2 && xq.size(1) == wq.size(1), "expected xq[M,K], wq[N,K] (got ",
                    xq.sizes(), ", ", wq.sizes(), ")");
  const int64_t M = xq.size(0), K = xq.size(1), N = wq.size(0);
  const int64_t xs_st = scale_stride(xs, M, "x_scale"), ws_st = scale_stride(ws, N, "w_scale");
  const c10::DeviceGuard guard(xq.device());
  at::Tensor y = at::empty({M, N}, xq.options().dtype(at::kBFloat16));
  if (M == 0 || N == 0) return y;
  if (K == 0) return y.zero_();
  check_rc(kore_gemm_a8w8(fp8 ? KORE_Q_FP8 : KORE_Q_INT8, xq.data_ptr(), xq.stride(0), xq.stride(1), wq.data_ptr(),
                          wq.stride(0), wq.stride(1), xs.data_ptr<float>(), xs_st, ws.data_ptr<float>(), ws_st,
                          y.data_ptr(), y.stride(0), M, N, K, stream_of(xq)));
  return y;
}

// ---- MoE sort/align (kore/tasks/breadth/moe_ext.py:617-621) ----
std::tuple<at::Tensor, at::Tensor, at::Tensor> moe_align(const at::Tensor& topk_ids, int64_t num_experts,
                                                         int64_t block) {
  require_hip({topk_ids});
  TORCH_CHECK_VALUE(topk_ids.dim() == 2 && topk_ids.scalar_type() == at::kInt, "topk_ids must be int32 [T, topk]");
  const at::Tensor ids = topk_ids.contiguous();
  const int64_t T = ids.size(0), topk = ids.size(1);
  const int64_t cap = kore_moe_align_capacity(T, topk, num_experts, block);
  TORCH_CHECK_VALUE(cap >= 0, "bad moe_align sizes (T=", T, ", topk=", topk, ", E=", num_experts, ", block=", block, ")");
  const c10::DeviceGuard guard(ids.device());
  at::Tensor offsets = at::empty({num_experts + 1}, ids.options());
  at::Tensor sorted = at::empty({std::max<int64_t>(cap, 1)}, ids.options());
  at::Tensor owner = at::empty({std::max<int64_t>(cap / block, 1)}, ids.options());
  check_rc(kore_moe_align(ids.data_ptr<int32_t>(), T, topk, num_experts, block, offsets.data_ptr<int32_t>(),
                          sorted.data_ptr<int32_t>(), owner.data_ptr<int32_t>(), cap, stream_of(ids)));
  return {offsets, sorted.narrow(0, 0, cap), owner.narrow(0, 0, cap / block)};
}

// ---- fused top-k MoE SiLU gated MLP (kore/tasks/fused_moe_silu_bf16/seed_triton.py:69-86) ----
at::Tensor fused_moe(const at::Tensor& hidden, const at::Tensor& w1_, const at::Tensor& w2_, const at::Tensor& tw_,
                     const at::Tensor& ti_) {
  require_hip({hidden, w1_, w2_, tw_, ti_});
  TORCH_CHECK_VALUE(hidden.scalar_type() == at::kBFloat16 && w1_.scalar_type() == at::kBFloat16 &&
                        w2_.scalar_type() == at::kBFloat16,
                    "fused_moe takes bf16 hidden/w1/w2");
  TORCH_CHECK_VALUE(hidden.dim() == 2 && w1_.dim() == 3 && w2_.dim() == 3, "expected hidden[T,D], w1[E,2I,D], w2[E,D,I]");
  const int64_t T = hidden.size(0), D = hidden.size(1), E = w1_.size(0), twoI = w1_.size(1), I = twoI / 2;
  TORCH_CHECK_VALUE(w1_.size(2) == D && twoI == 2 * I && w2_.size(0) == E && w2_.size(1) == D && w2_.size(2) == I,
                    "shape mismatch: hidden ", hidden.sizes(), ", w1 ", w1_.sizes(), ", w2 ", w2_.sizes());
  TORCH_CHECK_VALUE(ti_.dim() == 2 && ti_.size(0) == T && tw_.sizes() == ti_.sizes(),
                    "topk_weight/topk_ids must both be [T, topk]");
  const int64_t topk = ti_.size(1);
  const at::Tensor tw = tw_.to(at::kFloat).contiguous(), ti = ti_.to(at::kInt).contiguous();
  const at::Tensor x = hidden.stride(1) == 1 ? hidden : hidden.contiguous();
  const at::Tensor w1 = w1_.contiguous(), w2 = w2_.contiguous();
  const c10::DeviceGuard guard(x.device());
  at::Tensor out = at::empty({T, D}, x.options());
  if (T == 0 || topk == 0) return out.zero_();
  at::Tensor ws = workspace(kore_fused_moe_workspace_bytes(T, topk, E, D, I), x);
  check_rc(kore_fused_moe(x.data_ptr(), x.stride(0), w1.data_ptr(), w2.data_ptr(), tw.data_ptr<float>(),
                          ti.data_ptr<int32_t>(), out.data_ptr(), T, D, I, E, topk, ptr_or_null(ws), bytes_of(ws),
                          stream_of(x)));
  return out;
}

// ---- top-1 grouped expert GEMMs (kore/tasks/moe_grouped_gemm_bf16 / _fp8); the
// zero-padding of shapes the kernels do not take stays in the Python host.  Every
// shape, dtype and length is checked here, before any data pointer is taken, so a
// direct torch.ops.korehip call with mismatched tensors raises instead of reading
// past the ids, weights or scales on the device. ----

// expert_ids: int32 with exactly M ids (any shape), returned as a contiguous [M].
at::Tensor expert_ids_of(const at::Tensor& ids, int64_t M) {
  TORCH_CHECK_VALUE(ids.defined(), "expert_ids: undefined tensor");
  TORCH_CHECK_VALUE(ids.scalar_type() == at::kInt, "expert_ids must be int32 (got ", ids.scalar_type(), ")");
  TORCH_CHECK_VALUE(ids.numel() == M, "expert_ids must hold one id per row: ", M, " (got ", ids.sizes(), ")");
  return ids.reshape({M}).contiguous();
}

at::Tensor grouped_gemm(const at::Tensor& x_, const at::Tensor& w_, const at::Tensor& ids_) {
  TORCH_CHECK_VALUE(x_.defined() && w_.defined(), "grouped_gemm: undefined tensor");
  TORCH_CHECK_VALUE(x_.dim() == 2 && w_.dim() == 3 && w_.size(2) == x_.size(1),
                    "grouped_gemm expects hidden[M,K], w[E,N,K] (got ", x_.sizes(), ", ", w_.sizes(), ")");
  TORCH_CHECK_NOT_IMPLEMENTED(x_.scalar_type() == at::kBFloat16 && w_.scalar_type() == at::kBFloat16,
                              "grouped_gemm runs bf16 operands (got ", x_.scalar_type(), ", ", w_.scalar_type(), ")");
  const int64_t M = x_.size(0), K = x_.size(1), E = w_.size(0), N = w_.size(1);
  const at::Tensor ids = expert_ids_of(ids_, M);
  require_hip({x_, w_, ids});
  const at::Tensor x = x_.stride(1) == 1 && x_.stride(0) % 8 == 0 ? x_ : x_.contiguous();
  const at::Tensor w = w_.contiguous();
  const c10::DeviceGuard guard(x.device());
  // the library zeroes the rows of ids outside [0, E); every other row is written
  at::Tensor out = at::empty({M, N}, x.options());
  if (M == 0 || N == 0 || K == 0 || E == 0) return out.zero_();
  at::Tensor ws = workspace(kore_moe_grouped_gemm_workspace_bytes(M, E), x);
  check_rc(kore_moe_grouped_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), ids.data_ptr<int32_t>(), out.data_ptr(),
                                 out.stride(0), M, N, K, E, ptr_or_null(ws), bytes_of(ws), stream_of(x)));
  return out;
}

at::Tensor grouped_gemm_fp8(const at::Tensor& xq_, const at::Tensor& wq_, const at::Tensor& xs, const at::Tensor& wsc_,
                            const at::Tensor& ids_) {
  TORCH_CHECK_VALUE(xq_.defined() && wq_.defined() && xs.defined() && wsc_.defined(), "grouped_gemm_fp8: undefined tensor");
  TORCH_CHECK_VALUE(xq_.dim() == 2 && wq_.dim() == 3 && wq_.size(2) == xq_.size(1),
                    "grouped_gemm_fp8 expects xq[M,K], wq[E,N,K] (got ", xq_.sizes(), ", ", wq_.sizes(), ")");
  TORCH_CHECK_NOT_IMPLEMENTED(xq_.scalar_type() == at::kFloat8_e4m3fn && wq_.scalar_type() == at::kFloat8_e4m3fn,
                              "grouped_gemm_fp8 runs float8_e4m3fn operands (got ", xq_.scalar_type(), ", ",
                              wq_.scalar_type(), ")");
  const int64_t M = xq_.size(0), K = xq_.size(1), E = wq_.size(0), N = wq_.size(1);
  const int64_t xs_st = scale_stride(xs, M, "x_scale");
  TORCH_CHECK_VALUE(wsc_.scalar_type() == at::kFloat, "w_scale must be fp32 (got ", wsc_.scalar_type(), ")");
  TORCH_CHECK_VALUE((wsc_.dim() == 2 && wsc_.size(0) == E && wsc_.size(1) == N) ||
                        (wsc_.dim() == 3 && wsc_.size(0) == E && wsc_.size(1) == N && wsc_.size(2) == 1),
                    "w_scale must be [", E, ",", N, ",1] or [", E, ",", N, "] (got ", wsc_.sizes(), ")");
  const at::Tensor ids = expert_ids_of(ids_, M);
  require_hip({xq_, wq_, xs, wsc_, ids});
  const at::Tensor xq = xq_.stride(1) == 1 && xq_.stride(0) % 16 == 0 ? xq_ : xq_.contiguous();
  const at::Tensor wq = wq_.contiguous();
  const at::Tensor wsc = wsc_.reshape({E, N}).contiguous();
  const c10::DeviceGuard guard(xq.device());
  // contiguous bf16 rows (N % 128 == 0 here): the library zeroes the rows of ids outside
  // [0, E) and writes every other row
  at::Tensor out = at::empty({M, N}, xq.options().dtype(at::kBFloat16));
  if (M == 0 || N == 0 || K == 0 || E == 0) return out.zero_();
  at::Tensor ws = workspace(kore_moe_grouped_gemm_workspace_bytes(M, E), xq);
  check_rc(kore_moe_grouped_gemm_fp8(xq.data_ptr(), xq.stride(0), wq.data_ptr(), xs.data_ptr<float>(), xs_st,
                                     wsc.data_ptr<float>(), ids.data_ptr<int32_t>(), out.data_ptr(), out.stride(0), M,
                                     N, K, E, ptr_or_null(ws), bytes_of(ws), stream_of(xq)));
  return out;
}

// ---- token permute / unpermute as row copies (kore/tasks/moe_permute_bf16/reference.py:56-59,
// kore/tasks/breadth/moe_ext.py:546-571).  Row indices outside the table are
// range-checked by the kernel (a gathered row reads zero, a scattered row is
// dropped); the number of rows read is checked here. ----

// idx: int32 1-D, returned contiguous.
at::Tensor row_index_of(const at::Tensor& idx) {
  TORCH_CHECK_VALUE(idx.defined(), "row index: undefined tensor");
  TORCH_CHECK_VALUE(idx.dim() == 1 && idx.scalar_type() == at::kInt, "row index must be int32 [n] (got ",
                    idx.sizes(), " ", idx.scalar_type(), ")");
  return idx.contiguous();
}

at::Tensor gather_rows(const at::Tensor& src_, const at::Tensor& idx_) {
  TORCH_CHECK_VALUE(src_.defined() && src_.dim() == 2, "gather_rows expects src[rows, D] (got ",
                    src_.defined() ? src_.sizes() : at::IntArrayRef{}, ")");
  const at::Tensor idx = row_index_of(idx_);
  require_hip({src_, idx});
  const at::Tensor src = src_.stride(1) == 1 ? src_ : src_.contiguous();
  const int64_t eb = src.element_size();
  const c10::DeviceGuard guard(src.device());
  at::Tensor out = at::empty({idx.numel(), src.size(1)}, src.options());
  if (idx.numel() && src.size(1) && src.size(0))
    check_rc(kore_gather_rows(src.data_ptr(), src.stride(0) * eb, src.size(0), idx.data_ptr<int32_t>(), idx.numel(),
                              src.size(1) * eb, out.data_ptr(), out.stride(0) * eb, stream_of(src)));
  else if (idx.numel())
    out.zero_();
  return out;
}

at::Tensor scatter_rows(const at::Tensor& src_, const at::Tensor& idx_) {
  TORCH_CHECK_VALUE(src_.defined() && src_.dim() == 2, "scatter_rows expects src[rows, D] (got ",
                    src_.defined() ? src_.sizes() : at::IntArrayRef{}, ")");
  const at::Tensor idx = row_index_of(idx_);
  TORCH_CHECK_VALUE(idx.numel() <= src_.size(0), "scatter_rows reads one src row per index: ", idx.numel(),
                    " indices for ", src_.size(0), " rows");
  require_hip({src_, idx});
  const at::Tensor src = src_.stride(1) == 1 ? src_ : src_.contiguous();
  const int64_t eb = src.element_size();
  const c10::DeviceGuard guard(src.device());
  at::Tensor out = at::zeros_like(src, at::MemoryFormat::Contiguous);
  if (idx.numel() && src.size(1))
    check_rc(kore_scatter_rows(src.data_ptr(), src.stride(0) * eb, idx.data_ptr<int32_t>(), idx.numel(),
                               out.data_ptr(), src.size(0), src.size(1) * eb, out.stride(0) * eb, stream_of(src)));
  return out;
}

}  // namespace

TORCH_LIBRARY(korehip, m) {
  m.def("gemm(Tensor a, Tensor b) -> Tensor");
  m.def("gemm_fused(Tensor a, Tensor b, Tensor? bias, int act) -> Tensor");
  m.def("batched_gemm(Tensor a, Tensor b) -> Tensor");
  m.def("gemm_backward(Tensor x, Tensor w, Tensor dy) -> (Tensor, Tensor)");
  m.def("gemm_a8w8_blockscale(Tensor xq, Tensor wq, Tensor x_scale, Tensor w_scale) -> Tensor");
  m.def("gemm_a8w8(Tensor xq, Tensor wq, Tensor x_scale, Tensor w_scale) -> Tensor");
  m.def("moe_align(Tensor topk_ids, int num_experts, int block) -> (Tensor, Tensor, Tensor)");
  m.def("fused_moe(Tensor hidden, Tensor w1, Tensor w2, Tensor topk_weight, Tensor topk_ids) -> Tensor");
  m.def("grouped_gemm(Tensor hidden, Tensor w, Tensor expert_ids) -> Tensor");
  m.def("grouped_gemm_fp8(Tensor xq, Tensor wq, Tensor x_scale, Tensor w_scale, Tensor expert_ids) -> Tensor");
  m.def("gather_rows(Tensor src, Tensor idx) -> Tensor");
  m.def("scatter_rows(Tensor src, Tensor idx) -> Tensor");
}

// CompositeExplicitAutograd: the operators take any device and check for HIP tensors
// themselves, so a CPU tensor reaches the check (ValueError) instead of a missing kernel.
TORCH_LIBRARY_IMPL(korehip, CompositeExplicitAutograd, m) {
  m.impl("gemm", &gemm);
  m.impl("gemm_fused", &gemm_fused);
  m.impl("batched_gemm", &batched_gemm);
  m.impl("gemm_backward", &gemm_backward);
  m.impl("gemm_a8w8_blockscale", &gemm_a8w8_blockscale);
  m.impl("gemm_a8w8", &gemm_a8w8);
  m.impl("moe_align", &moe_align);
  m.impl("fused_moe", &fused_moe);
  m.impl("grouped_gemm", &grouped_gemm);
  m.impl("grouped_gemm_fp8", &grouped_gemm_fp8);
  m.impl("gather_rows", &gather_rows);
  m.impl("scatter_rows", &scatter_rows);
}

PYBIND11_MODULE(_C, m) {
  m.doc() = "kore_amd host operators over the libkore_amd.so C ABI (also registered as torch.ops.korehip)";
  m.def("gemm", &gemm);
  m.def("gemm_fused", &gemm_fused, py::arg("a"), py::arg("b"), py::arg("bias"), py::arg("act"));
  m.def("batched_gemm", &batched_gemm);
  m.def("gemm_backward", &gemm_backward);
  m.def("gemm_a8w8_blockscale", &gemm_a8w8_blockscale);
  m.def("gemm_a8w8", &gemm_a8w8);
  m.def("moe_align", &moe_align);
  m.def("fused_moe", &fused_moe);
  m.def("grouped_gemm", &grouped_gemm);
  m.def("grouped_gemm_fp8", &grouped_gemm_fp8);
  m.def("gather_rows", &gather_rows);
  m.def("scatter_rows", &scatter_rows);
}
