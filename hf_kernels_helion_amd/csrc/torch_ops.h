// The op implementations of torch_ops.cpp (each validates its tensors,
// allocates its outputs and calls one C-ABI entry point on torch's current
// HIP stream), shared by the TORCH_LIBRARY registrations there and the
// direct Python bindings of torch_fast.cpp.
#pragma once

#include <ATen/ATen.h>

#include <tuple>

namespace fp8b_torch {

at::Tensor w8a8_block_fp8_matmul(const at::Tensor& A, const at::Tensor& B, const at::Tensor& As,
                                 const at::Tensor& Bs, int64_t block_n, int64_t block_k);
at::Tensor w8a8_block_fp8_matmul_dtype(const at::Tensor& A, const at::Tensor& B,
                                       const at::Tensor& As, const at::Tensor& Bs,
                                       int64_t block_n, int64_t block_k,
                                       at::ScalarType output_dtype);
at::Tensor act_quant_matmul(const at::Tensor& x, const at::Tensor& B, const at::Tensor& Bs,
                            int64_t block_n, int64_t block_k, at::ScalarType output_dtype);
at::Tensor gemm_fp8_fp8_bf16_nt(const at::Tensor& A, const at::Tensor& B, const at::Tensor& As,
                                const at::Tensor& Bs, int64_t block_k);
std::tuple<at::Tensor, at::Tensor> act_quant(const at::Tensor& x, int64_t block_size);
void silu_and_mul(at::Tensor& out, const at::Tensor& x);
std::tuple<at::Tensor, at::Tensor> silu_and_mul_quant(const at::Tensor& x, int64_t block_size);

}  // namespace fp8b_torch
