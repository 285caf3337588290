"""MI355X drop-in for deep-gemm-helion's blockwise fp8 GEMM.

Public surface of deep-gemm-helion/deep-gemm-helion/torch-ext/deep_gemm_helion/
__init__.py:6-11: ``gemm_fp8_fp8_bf16_nt(A, B, As, Bs, block_size=128)`` computes
(A*As) @ (B*Bs)^T in bf16 with per-row weight scales Bs [N, K/block_size]
(fp8.py:13-29), the finegrained-fp8 formula with block_n = 1. The op runs the
same gfx950 kernels as w8a8_block_fp8_matmul (per-row scale folding in the
128x128 pipelined and decode kernels for block_size 128; the generic kernel
otherwise).
"""
from __future__ import annotations

import torch

from ..finegrained_fp8_helion import op as _load_ops  # loads the op library and bindings
from ._ops import add_op_namespace_prefix, ops


@torch.library.register_fake(add_op_namespace_prefix("gemm_fp8_fp8_bf16_nt"))
def _(A, B, As, Bs, block_k):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=torch.bfloat16)


def gemm_fp8_fp8_bf16_nt(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor,
                         Bs: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """DeepGEMM-style blockwise fp8 GEMM (NT layout): (A*As) @ (B*Bs)^T -> bf16.

    A [M,K] e4m3fn, B [N,K] e4m3fn, As fp32 [M, K//block_size], Bs fp32
    [N, K//block_size] (one scale per weight row and K-block)."""
    if not torch.compiler.is_compiling():
        out = _load_ops.fast.gemm_fp8_fp8_bf16_nt(A, B, As, Bs, int(block_size))
        if out is not None:
            return out
    return ops.gemm_fp8_fp8_bf16_nt(A, B, As, Bs, int(block_size))


__all__ = ["gemm_fp8_fp8_bf16_nt"]
