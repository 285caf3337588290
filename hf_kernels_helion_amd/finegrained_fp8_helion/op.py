"""torch custom ops over the gfx950 HIP library.

Every op validates its tensors, takes torch's current HIP stream and calls one
C-ABI entry point of libfp8_blockwise.so through ctypes. There is no CPU or
eager fallback: a tensor that is not on a ROCm GPU, or a missing library,
raises RuntimeError.

Mirrors finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-16
(the matmul op: functional, fp32 result, fake impl for tracing) and
activation-helion/activation-helion/torch-ext/activation_helion/op.py:15-23
(silu_and_mul: mutates ``out``).
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _native
from ._ops import add_op_namespace_prefix

_FP8 = torch.float8_e4m3fn
_OUT_CODES = {torch.float32: _native.F32, torch.bfloat16: _native.BF16,
              torch.float16: _native.F16}


def _require_gpu(name: str, t: torch.Tensor) -> None:
    if t.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(
            f"{name} must be a tensor on a ROCm GPU (got device {t.device}); "
            "this package has no CPU implementation")


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_matmul_args(A, B, As, Bs, block_n, block_k):
    for name, t in (("A", A), ("B", B), ("As", As), ("Bs", Bs)):
        _require_gpu(name, t)
    _require(A.dim() == 2 and B.dim() == 2, "A and B must be 2-D ([M,K] and [N,K])")
    _require(A.dtype == _FP8, f"A must be float8_e4m3fn, got {A.dtype}")
    _require(B.dtype == _FP8, f"B must be float8_e4m3fn, got {B.dtype}")
    _require(As.dtype == torch.float32, f"As must be float32, got {As.dtype}")
    _require(Bs.dtype == torch.float32, f"Bs must be float32, got {Bs.dtype}")
    M, K = A.shape
    N, K2 = B.shape
    _require(K == K2, f"A is [M,K]=[{M},{K}] but B is [N,K]=[{N},{K2}]")
    _require(block_n > 0 and block_k > 0, "block_size entries must be positive")
    kb = -(-K // block_k)
    nb = -(-N // block_n)
    _require(As.dim() == 2 and As.shape[0] >= M and As.shape[1] >= kb,
             f"As must be [M, ceil(K/block_k)] = [{M},{kb}], got {list(As.shape)}")
    _require(Bs.dim() == 2 and Bs.shape[0] >= nb and Bs.shape[1] >= kb,
             f"Bs must be [ceil(N/block_n), ceil(K/block_k)] = [{nb},{kb}], got {list(Bs.shape)}")
    _require(A.stride(1) == 1 or K <= 1, "A must have unit stride along K")
    _require(B.stride(1) == 1 or K <= 1, "B must have unit stride along K")
    dev = A.device
    _require(all(t.device == dev for t in (B, As, Bs)), "all tensors must be on one device")
    return M, N, K


def _matmul_into(out, A, B, As, Bs, block_n, block_k):
    M, N, K = out.shape[0], out.shape[1], A.shape[1]
    lib = _native.load()
    ws_bytes = lib.fp8b_gemm_workspace_size(M, N, K, block_n, block_k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=A.device) if ws_bytes else None
    lda = A.stride(0) if M > 1 else max(K, 1)
    ldb = B.stride(0) if N > 1 else max(K, 1)
    ldc = out.stride(0) if M > 1 else max(N, 1)
    # Single-row tensors can report any row stride; only K bytes are read.
    lda = max(lda, K)
    ldb = max(ldb, K)
    with torch.cuda.device(A.device):
        st = lib.fp8b_w8a8_block_matmul(
            A.data_ptr(), lda, B.data_ptr(), ldb,
            As.data_ptr(), As.stride(0), As.stride(1),
            Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
            out.data_ptr(), ldc, _OUT_CODES[out.dtype],
            M, N, K, block_n, block_k,
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream(A))
    _native.check(st, "w8a8_block_fp8_matmul")
    return out


@torch.library.custom_op(add_op_namespace_prefix("w8a8_block_fp8_matmul"), mutates_args=())
def w8a8_block_fp8_matmul(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor,
                          Bs: torch.Tensor, block_n: int, block_k: int) -> torch.Tensor:
    """fp32 [M,N] = blockwise-scaled A @ B.T (reference op.py:8-11)."""
    M, N, _ = _check_matmul_args(A, B, As, Bs, block_n, block_k)
    out = torch.empty((M, N), dtype=torch.float32, device=A.device)
    return _matmul_into(out, A, B, As, Bs, block_n, block_k)


@w8a8_block_fp8_matmul.register_fake
def _(A, B, As, Bs, block_n, block_k):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=torch.float32)


@torch.library.custom_op(add_op_namespace_prefix("w8a8_block_fp8_matmul_dtype"),
                         mutates_args=())
def w8a8_block_fp8_matmul_dtype(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor,
                                Bs: torch.Tensor, block_n: int, block_k: int,
                                output_dtype: torch.dtype) -> torch.Tensor:
    """As w8a8_block_fp8_matmul, but the epilogue writes ``output_dtype``
    (float32, bfloat16 or float16) directly: the fp32 accumulator is rounded
    once, to nearest even, exactly as ``fp32_result.to(output_dtype)``."""
    M, N, _ = _check_matmul_args(A, B, As, Bs, block_n, block_k)
    _require(output_dtype in _OUT_CODES, f"unsupported output_dtype {output_dtype}")
    out = torch.empty((M, N), dtype=output_dtype, device=A.device)
    return _matmul_into(out, A, B, As, Bs, block_n, block_k)


@w8a8_block_fp8_matmul_dtype.register_fake
def _(A, B, As, Bs, block_n, block_k, output_dtype):
    return A.new_empty((A.shape[0], B.shape[0]), dtype=output_dtype)


def _check_group(group: int) -> None:
    _require(group in (32, 64, 128, 256), f"group size must be 32, 64, 128 or 256, got {group}")


@torch.library.custom_op(add_op_namespace_prefix("act_quant"), mutates_args=())
def act_quant(x: torch.Tensor, block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token-group fp8 quantisation of bf16 x[..., K]: returns
    (q float8_e4m3fn [..., K], s float32 [..., ceil(K/block_size)])."""
    _require_gpu("x", x)
    _require(x.dtype == torch.bfloat16, f"x must be bfloat16, got {x.dtype}")
    _require(x.dim() >= 1, "x must have at least one dimension")
    _check_group(block_size)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.numel() > 0 and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    groups = -(-K // block_size)
    q = torch.empty((M, K), dtype=_FP8, device=x.device)
    s = torch.empty((M, groups), dtype=torch.float32, device=x.device)
    if M > 0 and K > 0:
        lib = _native.load()
        ldx = max(x2.stride(0), K) if M > 1 else K
        with torch.cuda.device(x.device):
            st = lib.fp8b_act_quant(x2.data_ptr(), ldx, q.data_ptr(), K, s.data_ptr(), groups, 1,
                                    M, K, block_size, _stream(x))
        _native.check(st, "act_quant")
    return q.reshape(*lead, K), s.reshape(*lead, groups)


@act_quant.register_fake
def _(x, block_size):
    K = x.shape[-1]
    groups = -(-K // block_size)
    return (x.new_empty(x.shape, dtype=_FP8),
            x.new_empty((*x.shape[:-1], groups), dtype=torch.float32))


def _flat2d(out: torch.Tensor, x: torch.Tensor):
    """Flatten leading dims to [rows, d] / [rows, 2d] (reference op.py:9-12)."""
    d = out.shape[-1]
    return out.reshape(-1, d), x.reshape(-1, x.shape[-1])


@torch.library.custom_op(add_op_namespace_prefix("silu_and_mul"), mutates_args={"out"})
def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """out = silu(x[..., :d]) * x[..., d:] in bf16 (reference act.py:20-28)."""
    _require_gpu("x", x)
    _require_gpu("out", out)
    _require(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16,
             "silu_and_mul supports bfloat16 x and out")
    d = out.shape[-1]
    _require(x.shape[-1] == 2 * d, f"x last dim must be 2*d = {2 * d}, got {x.shape[-1]}")
    _require(out.is_contiguous() and x.is_contiguous(), "x and out must be contiguous")
    o2, x2 = _flat2d(out, x)
    _require(o2.shape[0] == x2.shape[0], "x and out must have the same leading shape")
    M = o2.shape[0]
    if M == 0 or d == 0:
        return
    lib = _native.load()
    with torch.cuda.device(x.device):
        st = lib.fp8b_silu_and_mul(x2.data_ptr(), 2 * d, o2.data_ptr(), d, M, d, _stream(x))
    _native.check(st, "silu_and_mul")


@silu_and_mul.register_fake
def _(out, x):
    pass


@torch.library.custom_op(add_op_namespace_prefix("silu_and_mul_quant"), mutates_args=())
def silu_and_mul_quant(x: torch.Tensor, block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """act_quant(silu_and_mul(x), block_size) without materialising the bf16
    intermediate; bit-identical to the two-op sequence."""
    _require_gpu("x", x)
    _require(x.dtype == torch.bfloat16, f"x must be bfloat16, got {x.dtype}")
    _check_group(block_size)
    _require(x.shape[-1] % 2 == 0, "x last dim must be even")
    d = x.shape[-1] // 2
    lead = x.shape[:-1]
    x2 = x.reshape(-1, 2 * d).contiguous()
    M = x2.shape[0]
    groups = -(-d // block_size)
    q = torch.empty((M, d), dtype=_FP8, device=x.device)
    s = torch.empty((M, groups), dtype=torch.float32, device=x.device)
    if M > 0 and d > 0:
        lib = _native.load()
        with torch.cuda.device(x.device):
            st = lib.fp8b_silu_and_mul_quant(x2.data_ptr(), 2 * d, q.data_ptr(), d, s.data_ptr(),
                                             groups, 1, M, d, block_size, _stream(x))
        _native.check(st, "silu_and_mul_quant")
    return q.reshape(*lead, d), s.reshape(*lead, groups)


@silu_and_mul_quant.register_fake
def _(x, block_size):
    d = x.shape[-1] // 2
    groups = -(-d // block_size)
    return (x.new_empty((*x.shape[:-1], d), dtype=_FP8),
            x.new_empty((*x.shape[:-1], groups), dtype=torch.float32))
