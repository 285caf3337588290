"""MI355X-native drop-in for the finegrained-fp8-helion package.

Public surface of finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/
__init__.py:7-17 (``w8a8_block_fp8_matmul`` with the same signature, block_size
unpacking and output_dtype default) plus the activation quantiser that feeds
it, the gated SiLU of the FP8 MLP chain and their fused form.
"""
from __future__ import annotations

import torch

from ._ops import ops
from . import op as _op  # registers the custom ops
from .mlp import fp8_mlp, gate_up_silu_quant, interleave_gate_up

_DIRECT_OUT = (torch.float32, torch.bfloat16, torch.float16)
# Plain eager calls go through _op.fast (direct bindings of the same C++ op
# functions, ~2 us less host time per call); while torch.compile traces, and
# whenever a binding returns None (tensor subclasses, autograd, dispatch or
# torch-function modes, functorch), the call takes torch.ops.
_fast = _op.fast
_compiling = torch.compiler.is_compiling


def w8a8_block_fp8_matmul(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor,
                          Bs: torch.Tensor, block_size, output_dtype=torch.float32):
    """C = A @ B.T with blockwise scales (reference __init__.py:7-14).

    A: [M,K] float8_e4m3fn, B: [N,K] float8_e4m3fn, As: [M, K//bk] fp32,
    Bs: [N//bn, K//bk] fp32, block_size = [block_n, block_k].
    Returns [M,N] in output_dtype. float32/bfloat16/float16 are written by the
    kernel's epilogue; other dtypes are cast from the fp32 result.
    """
    block_n, block_k = int(block_size[0]), int(block_size[1])
    if output_dtype in _DIRECT_OUT:
        if not _compiling():
            out = _fast.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, block_n, block_k, output_dtype)
            if out is not None:
                return out
        return ops.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, block_n, block_k, output_dtype)
    out = ops.w8a8_block_fp8_matmul(A, B, As, Bs, block_n, block_k)
    return out.to(output_dtype)


def act_quant(x: torch.Tensor, block_size: int = 128):
    """Quantise activations per 1 x block_size group to float8_e4m3fn.

    x is bfloat16, float16 or float32. Returns (q, s): q has x's shape, s is
    fp32 [..., ceil(K/block_size)] with s = max(amax, 1e-10) / 448 and
    q = e4m3fn(x / s), both divisions in fp32. The pair is the (A, As)
    operand of w8a8_block_fp8_matmul.
    """
    if not _compiling():
        r = _fast.act_quant(x, int(block_size))
        if r is not None:
            return r
    return ops.act_quant(x, int(block_size))


def per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128):
    """Alias of act_quant under the name serving stacks use for it."""
    return act_quant(x, group_size)


def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """out = silu(x[..., :d]) * x[..., d:], written into ``out``
    (activation-helion/activation-helion/torch-ext/activation_helion/__init__.py:7-10).
    x and out may each be float32, bfloat16 or float16, with the rounding
    points of act.py:25-28; leading dimensions are flattened (op.py:9-12)."""
    if _compiling() or _fast.silu_and_mul(out, x) is None:
        ops.silu_and_mul(out, x)
    return out


def silu_and_mul_quant(x: torch.Tensor, block_size: int = 128):
    """act_quant(silu_and_mul(x)) in one pass; returns (q, s)."""
    if not _compiling():
        r = _fast.silu_and_mul_quant(x, int(block_size))
        if r is not None:
            return r
    return ops.silu_and_mul_quant(x, int(block_size))


def act_quant_w8a8_block_fp8_matmul(x: torch.Tensor, B: torch.Tensor, Bs: torch.Tensor,
                                    block_size=(128, 128), output_dtype=torch.float32):
    """w8a8_block_fp8_matmul(*act_quant(x, 128), B, Bs, block_size, output_dtype),
    bit for bit, as one op. On decode-sized M (up to 32 rows on the split-K
    decode plan, up to 8 on the skinny and small-grid plans; 16-byte aligned
    rows) one kernel reads the bf16 rows and quantises them inside the GEMM;
    otherwise the quantiser writes (q, s) into the op's workspace and the
    GEMM reads them (two launches on the current stream).
    x: [M,K] bfloat16, K % 128 == 0; block_size must be [128, 128]."""
    block_n, block_k = int(block_size[0]), int(block_size[1])
    if output_dtype in _DIRECT_OUT:
        if not _compiling():
            out = _fast.act_quant_matmul(x, B, Bs, block_n, block_k, output_dtype)
            if out is not None:
                return out
        return ops.act_quant_matmul(x, B, Bs, block_n, block_k, output_dtype)
    return ops.act_quant_matmul(x, B, Bs, block_n, block_k, torch.float32).to(output_dtype)


def quantize_weight(W: torch.Tensor, block_size=(128, 128)):
    """Offline 128x128 block quantisation of a float32/bfloat16 weight [N,K]:
    returns (Wq e4m3fn [N,K], Bs fp32 [ceil(N/128), ceil(K/128)]) with
    Bs = max(block amax, 1e-10) / 448 and Wq = e4m3fn(W / Bs) -- the (B, Bs)
    operands of w8a8_block_fp8_matmul and the weight/weight_scale_inv pair of
    FP8 checkpoints."""
    return ops.weight_quant(W, int(block_size[0]), int(block_size[1]))


__all__ = [
    "w8a8_block_fp8_matmul",
    "quantize_weight",
    "act_quant_w8a8_block_fp8_matmul",
    "act_quant",
    "per_token_group_quant_fp8",
    "silu_and_mul",
    "silu_and_mul_quant",
    "fp8_mlp",
    "interleave_gate_up",
    "gate_up_silu_quant",
]
