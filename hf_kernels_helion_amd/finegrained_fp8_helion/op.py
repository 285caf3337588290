"""Loads the torch custom-op library and registers the ops' fake (meta) kernels.

The ops themselves are C++ (hf_kernels_helion_amd/csrc/torch_ops.cpp): each
validates its tensors, takes torch's current HIP stream and calls one C-ABI
entry point of libfp8_blockwise.so. There is no CPU or eager fallback: CPU
tensors and a missing library raise RuntimeError.

Mirrors finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-16
(the matmul op: functional, fp32 result, fake impl for tracing) and
activation-helion/activation-helion/torch-ext/activation_helion/op.py:15-23
(silu_and_mul: mutates ``out``).
"""
from __future__ import annotations

import importlib.util
from pathlib import Path

import torch

from ._ops import add_op_namespace_prefix

_LIB = Path(__file__).resolve().parent.parent / "_lib" / "libfp8_torch_ops.so"
_FAST = _LIB.parent / "_fp8_fast.so"


def _load():
    """Load the op library, then the direct bindings of its hot ops (module
    _fp8_fast: the same C++ functions without the dispatcher, for plain eager
    calls; each returns None when the call must take torch.ops)."""
    for f in (_LIB, _FAST):
        if not f.exists():
            raise RuntimeError(
                f"{f} is missing: build the HIP kernels and op library first "
                "(python -m hf_kernels_helion_amd.build)")
    torch.ops.load_library(str(_LIB))
    spec = importlib.util.spec_from_file_location("_fp8_fast", _FAST)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


fast = _load()


@torch.library.register_fake(add_op_namespace_prefix("w8a8_block_fp8_matmul"))
def _(A, B, As, Bs, block_n, block_k):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=torch.float32)


@torch.library.register_fake(add_op_namespace_prefix("w8a8_block_fp8_matmul_dtype"))
def _(A, B, As, Bs, block_n, block_k, output_dtype):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=output_dtype)


@torch.library.register_fake(add_op_namespace_prefix("act_quant"))
def _(x, block_size):
    K = x.shape[-1]
    groups = -(-K // block_size)
    return (x.new_empty(x.shape, dtype=torch.float8_e4m3fn),
            x.new_empty((*x.shape[:-1], groups), dtype=torch.float32))


@torch.library.register_fake(add_op_namespace_prefix("silu_and_mul"))
def _(out, x):
    return None


@torch.library.register_fake(add_op_namespace_prefix("silu_and_mul_quant"))
def _(x, block_size):
    d = x.shape[-1] // 2
    groups = -(-d // block_size)
    return (x.new_empty((*x.shape[:-1], d), dtype=torch.float8_e4m3fn),
            x.new_empty((*x.shape[:-1], groups), dtype=torch.float32))


@torch.library.register_fake(add_op_namespace_prefix("gate_up_silu_quant"))
def _(A, B, As, Bs):
    i = B.shape[0] // 2
    return (A.new_empty((A.shape[0], i), dtype=torch.float8_e4m3fn),
            As.new_empty((A.shape[0], i // 128), dtype=torch.float32))


@torch.library.register_fake(add_op_namespace_prefix("act_quant_matmul"))
def _(x, B, Bs, block_n, block_k, output_dtype):
    return x.new_empty((x.shape[0], B.shape[0]), dtype=output_dtype)


@torch.library.register_fake(add_op_namespace_prefix("weight_quant"))
def _(W, block_n, block_k):
    N, K = W.shape
    return (W.new_empty((N, K), dtype=torch.float8_e4m3fn),
            W.new_empty((-(-N // block_n), -(-K // block_k)), dtype=torch.float32))
