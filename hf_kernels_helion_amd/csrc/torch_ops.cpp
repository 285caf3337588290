// PyTorch-ROCm custom ops over the C ABI of libfp8_blockwise.so.
//
// Registers, in the namespace _finegrained_fp8_helion_rocm_mi355x (the
// kernel-builder scheme of finegrained-fp8-helion/build/torch-cuda/_ops.py:21-30):
//   w8a8_block_fp8_matmul(A, B, As, Bs, block_n, block_k) -> fp32 Tensor
//       (schema of finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-11)
//   w8a8_block_fp8_matmul_dtype(..., ScalarType output_dtype) -> Tensor
//   act_quant(x, block_size) -> (q, s)   (x float32, bfloat16 or float16)
//   silu_and_mul(Tensor(a!) out, x) -> ()
//       (schema of activation-helion/.../torch-ext/activation_helion/op.py:15-18)
//   silu_and_mul_quant(x, block_size) -> (q, s)
//   gate_up_silu_quant(A, B, As, Bs) -> (q, s)   (gate/up weights interleaved)
//   act_quant_matmul(x, B, Bs, block_n, block_k, ScalarType output_dtype) -> Tensor
//       (act_quant then w8a8_block_fp8_matmul in one op, the same bits: one
//       kernel that quantises inside the GEMM on small-M plans, else two
//       launches)
//   weight_quant(W, block_n, block_k) -> (Wq, Bs)   (128x128 blocks)
// and, in _deep_gemm_helion_rocm_mi355x (deep-gemm-helion's op,
// deep-gemm-helion/deep-gemm-helion/torch-ext/deep_gemm_helion/op.py:7-14):
//   gemm_fp8_fp8_bf16_nt(A, B, As, Bs, block_k) -> bf16 Tensor
//       (per-row weight scales Bs [N, K/block_k]: block_n = 1)
// Each op validates its tensors (TORCH_CHECK -> RuntimeError), allocates its
// outputs and any split-K workspace from torch's caching allocator, and calls
// one C-ABI entry point on torch's current HIP stream. CPU tensors raise: the
// path has no CPU implementation.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "../../include/fp8_blockwise.h"
#include "torch_ops.h"

namespace fp8b_torch {

using at::Tensor;

void* current_stream(const Tensor& t) {
  return (void*)at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_status(int st, const char* what) {
  TORCH_CHECK(st == FP8B_OK, what, " failed (status ", st, "): ", fp8b_last_error());
}

void check_gpu(const Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a tensor on a ROCm GPU (got ", t.device(),
              "); this package has no CPU implementation");
}

// A 2-D operand the kernels can read in place: unit stride along the last
// dimension and rows at least a row apart (no overlap). Anything else (an
// expanded row with stride 0, an unfold view, a transposed tensor) is copied
// to a contiguous tensor first, so the row stride passed down is always
// >= the row length.
Tensor rows_apart(const Tensor& t) {
  const int64_t rows = t.size(0), len = t.size(1);
  const bool unit_k = len <= 1 || t.stride(1) == 1;
  const bool apart = rows <= 1 || t.stride(0) >= std::max<int64_t>(len, 1);
  return (unit_k && apart) ? t : t.contiguous();
}

// Row stride to pass for a tensor returned by rows_apart.
int64_t row_stride(const Tensor& t) {
  return t.size(0) > 1 ? std::max<int64_t>(t.stride(0), t.size(1)) : t.size(1);
}

int out_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return FP8B_F32;
    case at::kBFloat16: return FP8B_BF16;
    case at::kHalf: return FP8B_F16;
    default: TORCH_CHECK(false, "unsupported output_dtype ", t, " (float32, bfloat16, float16)");
  }
  return -1;
}

Tensor matmul_impl(const Tensor& A_in, const Tensor& B_in, const Tensor& As, const Tensor& Bs,
                   int64_t block_n, int64_t block_k, at::ScalarType out_dtype) {
  check_gpu(A_in, "A");
  check_gpu(B_in, "B");
  check_gpu(As, "As");
  check_gpu(Bs, "Bs");
  TORCH_CHECK(A_in.dim() == 2 && B_in.dim() == 2, "A and B must be 2-D ([M,K] and [N,K])");
  const Tensor A = rows_apart(A_in), B = rows_apart(B_in);
  TORCH_CHECK(A.scalar_type() == at::kFloat8_e4m3fn, "A must be float8_e4m3fn, got ",
              A.scalar_type());
  TORCH_CHECK(B.scalar_type() == at::kFloat8_e4m3fn, "B must be float8_e4m3fn, got ",
              B.scalar_type());
  TORCH_CHECK(As.scalar_type() == at::kFloat, "As must be float32, got ", As.scalar_type());
  TORCH_CHECK(Bs.scalar_type() == at::kFloat, "Bs must be float32, got ", Bs.scalar_type());
  const int64_t M = A.size(0), K = A.size(1), N = B.size(0);
  TORCH_CHECK(B.size(1) == K, "A is [M,K]=[", M, ",", K, "] but B is [N,K]=[", N, ",",
              B.size(1), "]");
  TORCH_CHECK(block_n > 0 && block_k > 0, "block_size entries must be positive");
  const int64_t kb = (K + block_k - 1) / block_k, nb = (N + block_n - 1) / block_n;
  TORCH_CHECK(As.dim() == 2 && As.size(0) >= M && As.size(1) >= kb,
              "As must be [M, ceil(K/block_k)] = [", M, ",", kb, "], got ", As.sizes());
  TORCH_CHECK(Bs.dim() == 2 && Bs.size(0) >= nb && Bs.size(1) >= kb,
              "Bs must be [ceil(N/block_n), ceil(K/block_k)] = [", nb, ",", kb, "], got ",
              Bs.sizes());
  TORCH_CHECK(B.device() == A.device() && As.device() == A.device() && Bs.device() == A.device(),
              "all tensors must be on one device");
  const int code = out_code(out_dtype);
  at::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
  Tensor out = at::empty({M, N}, A.options().dtype(out_dtype));
  if (M == 0 || N == 0) return out;
  const size_t ws_bytes = fp8b_gemm_workspace_size(M, N, K, block_n, block_k);
  Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, A.options().dtype(at::kByte));
  const int64_t lda = row_stride(A), ldb = row_stride(B);
  const int st = fp8b_w8a8_block_matmul(
      A.data_ptr(), lda, B.data_ptr(), ldb, As.data_ptr<float>(), As.stride(0), As.stride(1),
      Bs.data_ptr<float>(), Bs.stride(0), Bs.stride(1), out.data_ptr(), N, code, M, N, K,
      block_n, block_k, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, current_stream(A));
  check_status(st, "w8a8_block_fp8_matmul");
  return out;
}

Tensor w8a8_block_fp8_matmul(const Tensor& A, const Tensor& B, const Tensor& As,
                             const Tensor& Bs, int64_t block_n, int64_t block_k) {
  return matmul_impl(A, B, As, Bs, block_n, block_k, at::kFloat);
}

Tensor w8a8_block_fp8_matmul_dtype(const Tensor& A, const Tensor& B, const Tensor& As,
                                   const Tensor& Bs, int64_t block_n, int64_t block_k,
                                   at::ScalarType output_dtype) {
  return matmul_impl(A, B, As, Bs, block_n, block_k, output_dtype);
}

Tensor act_quant_matmul(const Tensor& x_in, const Tensor& B_in, const Tensor& Bs,
                        int64_t block_n, int64_t block_k, at::ScalarType output_dtype) {
  check_gpu(x_in, "x");
  check_gpu(B_in, "B");
  check_gpu(Bs, "Bs");
  TORCH_CHECK(x_in.dim() == 2 && B_in.dim() == 2, "x and B must be 2-D ([M,K] and [N,K])");
  const Tensor x = rows_apart(x_in), B = rows_apart(B_in);
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16, got ", x.scalar_type());
  TORCH_CHECK(B.scalar_type() == at::kFloat8_e4m3fn, "B must be float8_e4m3fn, got ",
              B.scalar_type());
  TORCH_CHECK(Bs.scalar_type() == at::kFloat, "Bs must be float32, got ", Bs.scalar_type());
  TORCH_CHECK(block_n == 128 && block_k == 128, "act_quant_matmul supports block_size "
              "[128, 128] (1x128 activation groups), got [", block_n, ",", block_k, "]");
  const int64_t M = x.size(0), K = x.size(1), N = B.size(0);
  TORCH_CHECK(B.size(1) == K, "x is [M,K]=[", M, ",", K, "] but B is [N,K]=[", N, ",",
              B.size(1), "]");
  TORCH_CHECK(K % 128 == 0, "K must be a multiple of 128, got ", K);
  const int64_t kb = K / 128, nb = (N + 127) / 128;
  TORCH_CHECK(Bs.dim() == 2 && Bs.size(0) >= nb && Bs.size(1) >= kb,
              "Bs must be [ceil(N/128), K/128] = [", nb, ",", kb, "], got ", Bs.sizes());
  TORCH_CHECK(B.device() == x.device() && Bs.device() == x.device(),
              "all tensors must be on one device");
  const int code = out_code(output_dtype);
  at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  Tensor out = at::empty({M, N}, x.options().dtype(output_dtype));
  if (M == 0 || N == 0) return out;
  const size_t ws_bytes = fp8b_act_quant_matmul_workspace_size(M, N, K);
  Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
  const int64_t ldx = row_stride(x), ldb = row_stride(B);
  const int st = fp8b_act_quant_matmul(
      x.data_ptr(), ldx, B.data_ptr(), ldb, Bs.data_ptr<float>(), Bs.stride(0), Bs.stride(1),
      out.data_ptr(), N, code, M, N, K, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
      current_stream(x));
  check_status(st, "act_quant_matmul");
  return out;
}

std::tuple<Tensor, Tensor> weight_quant(const Tensor& W_in, int64_t block_n, int64_t block_k) {
  check_gpu(W_in, "W");
  TORCH_CHECK(W_in.dim() == 2, "W must be 2-D [N,K]");
  const Tensor W = rows_apart(W_in);
  TORCH_CHECK(W.scalar_type() == at::kFloat || W.scalar_type() == at::kBFloat16,
              "W must be float32 or bfloat16, got ", W.scalar_type());
  TORCH_CHECK(block_n == 128 && block_k == 128, "weight_quant supports 128x128 blocks, got [",
              block_n, ",", block_k, "]");
  const int64_t N = W.size(0), K = W.size(1);
  at::hip::HIPGuardMasqueradingAsCUDA guard(W.device());
  const int64_t kp = (K + 1) / 2 * 2;  // even row stride for the 2-byte stores
  Tensor qbuf = at::empty({N, kp}, W.options().dtype(at::kFloat8_e4m3fn));
  Tensor q = qbuf.narrow(1, 0, K);
  Tensor s = at::empty({(N + 127) / 128, (K + 127) / 128}, W.options().dtype(at::kFloat));
  if (N == 0 || K == 0) return {q, s};
  const int64_t ldw = row_stride(W);
  const int st = fp8b_weight_quant(W.data_ptr(), ldw,
                                   W.scalar_type() == at::kFloat ? FP8B_F32 : FP8B_BF16,
                                   q.data_ptr(), kp, s.data_ptr<float>(), s.stride(0),
                                   s.stride(1), N, K, current_stream(W));
  check_status(st, "weight_quant");
  return {kp == K ? qbuf : q.contiguous(), s};
}

Tensor gemm_fp8_fp8_bf16_nt(const Tensor& A, const Tensor& B, const Tensor& As,
                            const Tensor& Bs, int64_t block_k) {
  return matmul_impl(A, B, As, Bs, 1, block_k, at::kBFloat16);
}

void check_group(int64_t g) {
  TORCH_CHECK(g == 32 || g == 64 || g == 128 || g == 256,
              "group size must be 32, 64, 128 or 256, got ", g);
}

std::tuple<Tensor, Tensor> act_quant(const Tensor& x, int64_t block_size) {
  check_gpu(x, "x");
  const at::ScalarType xt = x.scalar_type();
  TORCH_CHECK(xt == at::kBFloat16 || xt == at::kHalf || xt == at::kFloat,
              "x must be bfloat16, float16 or float32, got ", xt);
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dimension");
  check_group(block_size);
  const int64_t K = x.size(-1);
  const int64_t groups = (K + block_size - 1) / block_size;
  auto lead = x.sizes().vec();
  lead.pop_back();
  Tensor x2 = x.reshape({-1, K});
  if (x2.numel() > 0) x2 = rows_apart(x2);
  const int64_t M = x2.size(0);
  at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  Tensor q = at::empty({M, K}, x.options().dtype(at::kFloat8_e4m3fn));
  Tensor s = at::empty({M, groups}, x.options().dtype(at::kFloat));
  if (M > 0 && K > 0) {
    const int64_t ldx = row_stride(x2);
    const int st = fp8b_act_quant_typed(x2.data_ptr(), ldx, out_code(xt), q.data_ptr(), K,
                                        s.data_ptr<float>(), groups, 1, M, K, block_size,
                                        current_stream(x));
    check_status(st, "act_quant");
  }
  auto qshape = lead;
  qshape.push_back(K);
  auto sshape = lead;
  sshape.push_back(groups);
  return {q.view(qshape), s.view(sshape)};
}

// out = silu(x[..., :d]) * x[..., d:] for x and out of float32, bfloat16 or
// float16 (any pair), leading dimensions flattened as op.py:9-12 does with
// reshape. x may have any strides (copied when its rows are not 2-D
// addressable); out is written in place when it flattens to rows with a unit
// inner stride, else through a contiguous temporary copied back into it (the
// reference's reshape would write a copy and leave out untouched).
void silu_and_mul(Tensor& out, const Tensor& x) {
  check_gpu(x, "x");
  check_gpu(out, "out");
  TORCH_CHECK(x.dim() >= 1 && out.dim() >= 1, "x and out must have at least one dimension");
  const int xt = out_code(x.scalar_type()), ot = out_code(out.scalar_type());
  const int64_t d = out.size(-1);
  TORCH_CHECK(x.size(-1) == 2 * d, "x last dim must be 2*d = ", 2 * d, ", got ", x.size(-1));
  const int64_t M = d > 0 ? out.numel() / d : 0;
  TORCH_CHECK(d == 0 || x.numel() / (2 * d) == M, "x and out must have the same leading shape");
  if (M == 0 || d == 0) return;
  at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  Tensor x2 = rows_apart(x.reshape({M, 2 * d}));
  // out itself when it is contiguous or 2-D rows with a unit inner stride
  // (e.g. a slice out[:, :d] of a wider buffer), else a contiguous temporary
  const bool direct = out.is_contiguous() ||
                      (out.dim() == 2 && out.stride(1) == 1 && out.stride(0) >= d);
  Tensor tmp = direct ? Tensor() : at::empty({M, d}, out.options());
  Tensor o2 = !direct ? tmp : (out.is_contiguous() ? out.view({M, d}) : out);
  const int64_t ldo = o2.size(0) > 1 ? o2.stride(0) : d;
  const int st = fp8b_silu_and_mul_typed(x2.data_ptr(), row_stride(x2), xt, o2.data_ptr(), ldo,
                                         ot, M, d, current_stream(x));
  check_status(st, "silu_and_mul");
  if (!direct) out.copy_(tmp.view(out.sizes()));
}

std::tuple<Tensor, Tensor> silu_and_mul_quant(const Tensor& x, int64_t block_size) {
  check_gpu(x, "x");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16, got ", x.scalar_type());
  check_group(block_size);
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) % 2 == 0, "x last dim must be even");
  const int64_t d = x.size(-1) / 2;
  const int64_t groups = (d + block_size - 1) / block_size;
  auto lead = x.sizes().vec();
  lead.pop_back();
  Tensor x2 = x.reshape({-1, 2 * d}).contiguous();
  const int64_t M = x2.size(0);
  at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  Tensor q = at::empty({M, d}, x.options().dtype(at::kFloat8_e4m3fn));
  Tensor s = at::empty({M, groups}, x.options().dtype(at::kFloat));
  if (M > 0 && d > 0) {
    const int st = fp8b_silu_and_mul_quant(x2.data_ptr(), 2 * d, q.data_ptr(), d,
                                           s.data_ptr<float>(), groups, 1, M, d, block_size,
                                           current_stream(x));
    check_status(st, "silu_and_mul_quant");
  }
  auto qshape = lead;
  qshape.push_back(d);
  auto sshape = lead;
  sshape.push_back(groups);
  return {q.view(qshape), s.view(sshape)};
}

// Gate/up GEMM with SiLU(gate)*up and group-128 quantisation in its
// epilogue; B/Bs hold gate and up interleaved in 128-row blocks
// (interleave_gate_up in finegrained_fp8_helion/mlp.py).
std::tuple<Tensor, Tensor> gate_up_silu_quant(const Tensor& A_in, const Tensor& B_in,
                                              const Tensor& As, const Tensor& Bs) {
  check_gpu(A_in, "A");
  check_gpu(B_in, "B");
  check_gpu(As, "As");
  check_gpu(Bs, "Bs");
  TORCH_CHECK(A_in.dim() == 2 && B_in.dim() == 2, "A and B must be 2-D ([M,K] and [2I,K])");
  const Tensor A = rows_apart(A_in), B = rows_apart(B_in);
  TORCH_CHECK(A.scalar_type() == at::kFloat8_e4m3fn && B.scalar_type() == at::kFloat8_e4m3fn,
              "A and B must be float8_e4m3fn");
  TORCH_CHECK(As.scalar_type() == at::kFloat && Bs.scalar_type() == at::kFloat,
              "As and Bs must be float32");
  const int64_t M = A.size(0), K = A.size(1), N = B.size(0);
  TORCH_CHECK(B.size(1) == K, "A is [M,K]=[", M, ",", K, "] but B is [2I,K]=[", N, ",",
              B.size(1), "]");
  TORCH_CHECK(N % 256 == 0, "B must have 2I rows with I a multiple of 128, got ", N);
  TORCH_CHECK(As.dim() == 2 && As.size(0) >= M && As.size(1) >= K / 128,
              "As must be [M, K/128], got ", As.sizes());
  TORCH_CHECK(Bs.dim() == 2 && Bs.size(0) >= N / 128 && Bs.size(1) >= K / 128,
              "Bs must be [2I/128, K/128], got ", Bs.sizes());
  TORCH_CHECK(K % 128 == 0 && K > 0, "K must be a positive multiple of 128, got ", K);
  const int64_t I = N / 2;
  at::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
  Tensor q = at::empty({M, I}, A.options());
  Tensor s = at::empty({M, I / 128}, As.options());
  if (M > 0) {
    const int st = fp8b_gate_up_silu_quant(
        A.data_ptr(), row_stride(A), B.data_ptr(), row_stride(B), As.data_ptr<float>(),
        As.stride(0), As.stride(1), Bs.data_ptr<float>(), Bs.stride(0), Bs.stride(1), q.data_ptr(), I,
        s.data_ptr<float>(), I / 128, 1, M, I, K, current_stream(A));
    check_status(st, "gate_up_silu_quant");
  }
  return {q, s};
}

// CPU tensors reach these: raise instead of computing anything.
[[noreturn]] void no_cpu(const char* op) {
  TORCH_CHECK(false, op, ": tensors must be on a ROCm GPU; this package has no CPU "
              "implementation");
}
Tensor matmul_cpu(const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t, int64_t) {
  no_cpu("w8a8_block_fp8_matmul");
}
Tensor matmul_dtype_cpu(const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t,
                        int64_t, at::ScalarType) {
  no_cpu("w8a8_block_fp8_matmul_dtype");
}
std::tuple<Tensor, Tensor> act_quant_cpu(const Tensor&, int64_t) { no_cpu("act_quant"); }
Tensor act_quant_matmul_cpu(const Tensor&, const Tensor&, const Tensor&, int64_t, int64_t,
                            at::ScalarType) {
  no_cpu("act_quant_matmul");
}
std::tuple<Tensor, Tensor> weight_quant_cpu(const Tensor&, int64_t, int64_t) {
  no_cpu("weight_quant");
}
Tensor gemm_nt_cpu(const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t) {
  no_cpu("gemm_fp8_fp8_bf16_nt");
}
void silu_and_mul_cpu(Tensor&, const Tensor&) { no_cpu("silu_and_mul"); }
std::tuple<Tensor, Tensor> silu_and_mul_quant_cpu(const Tensor&, int64_t) {
  no_cpu("silu_and_mul_quant");
}
std::tuple<Tensor, Tensor> gate_up_silu_quant_cpu(const Tensor&, const Tensor&, const Tensor&,
                                                  const Tensor&) {
  no_cpu("gate_up_silu_quant");
}

}  // namespace fp8b_torch

using namespace fp8b_torch;

TORCH_LIBRARY(_finegrained_fp8_helion_rocm_mi355x, m) {
  m.def("w8a8_block_fp8_matmul(Tensor A, Tensor B, Tensor As, Tensor Bs, int block_n, "
        "int block_k) -> Tensor");
  m.def("w8a8_block_fp8_matmul_dtype(Tensor A, Tensor B, Tensor As, Tensor Bs, int block_n, "
        "int block_k, ScalarType output_dtype) -> Tensor");
  m.def("act_quant(Tensor x, int block_size) -> (Tensor, Tensor)");
  m.def("silu_and_mul(Tensor(a!) out, Tensor x) -> ()");
  m.def("silu_and_mul_quant(Tensor x, int block_size) -> (Tensor, Tensor)");
  m.def("gate_up_silu_quant(Tensor A, Tensor B, Tensor As, Tensor Bs) -> (Tensor, Tensor)");
  m.def("act_quant_matmul(Tensor x, Tensor B, Tensor Bs, int block_n, int block_k, "
        "ScalarType output_dtype) -> Tensor");
  m.def("weight_quant(Tensor W, int block_n, int block_k) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(_finegrained_fp8_helion_rocm_mi355x, CUDA, m) {
  m.impl("w8a8_block_fp8_matmul", &w8a8_block_fp8_matmul);
  m.impl("w8a8_block_fp8_matmul_dtype", &w8a8_block_fp8_matmul_dtype);
  m.impl("act_quant", &act_quant);
  m.impl("silu_and_mul", &silu_and_mul);
  m.impl("silu_and_mul_quant", &silu_and_mul_quant);
  m.impl("gate_up_silu_quant", &gate_up_silu_quant);
  m.impl("act_quant_matmul", &act_quant_matmul);
  m.impl("weight_quant", &weight_quant);
}

TORCH_LIBRARY_IMPL(_finegrained_fp8_helion_rocm_mi355x, CPU, m) {
  m.impl("w8a8_block_fp8_matmul", &matmul_cpu);
  m.impl("w8a8_block_fp8_matmul_dtype", &matmul_dtype_cpu);
  m.impl("act_quant", &act_quant_cpu);
  m.impl("silu_and_mul", &silu_and_mul_cpu);
  m.impl("silu_and_mul_quant", &silu_and_mul_quant_cpu);
  m.impl("gate_up_silu_quant", &gate_up_silu_quant_cpu);
  m.impl("act_quant_matmul", &act_quant_matmul_cpu);
  m.impl("weight_quant", &weight_quant_cpu);
}

TORCH_LIBRARY(_deep_gemm_helion_rocm_mi355x, m) {
  m.def("gemm_fp8_fp8_bf16_nt(Tensor A, Tensor B, Tensor As, Tensor Bs, int block_k) -> Tensor");
}

TORCH_LIBRARY_IMPL(_deep_gemm_helion_rocm_mi355x, CUDA, m) {
  m.impl("gemm_fp8_fp8_bf16_nt", &gemm_fp8_fp8_bf16_nt);
}

TORCH_LIBRARY_IMPL(_deep_gemm_helion_rocm_mi355x, CPU, m) {
  m.impl("gemm_fp8_fp8_bf16_nt", &gemm_nt_cpu);
}
