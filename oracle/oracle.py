"""numpy/ctypes front end of oracle/fp8_oracle.c -- TEST INFRASTRUCTURE ONLY.

Arrays in and out are numpy: bf16 tensors travel as uint16 bit patterns,
float8_e4m3fn as uint8 codes. The C library is built by oracle/Makefile (or
__graft_entry__.build()) into oracle/_build/libfp8_oracle.so.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "_build" / "libfp8_oracle.so"
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int64


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_e4m3fn_from_f32.restype = ctypes.c_uint8
        lib.oracle_e4m3fn_from_f32.argtypes = [ctypes.c_float]
        lib.oracle_e4m3fn_to_f32.restype = ctypes.c_float
        lib.oracle_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        lib.oracle_act_quant.argtypes = [_P, _I, _I, _I, _I, _P, _P]
        lib.oracle_act_quant_f32.argtypes = [_P, _I, _I, _I, _I, _P, _P]
        lib.oracle_block_gemm.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]
        lib.oracle_dequant_matmul.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]
        lib.oracle_silu_and_mul.argtypes = [_P, _I, _I, _P]
        lib.oracle_quant_weight_block.argtypes = [_P, _I, _I, _I, _I, _P, _P]
        for f in ("oracle_act_quant", "oracle_act_quant_f32", "oracle_block_gemm",
                  "oracle_dequant_matmul",
                  "oracle_silu_and_mul", "oracle_quant_weight_block"):
            getattr(lib, f).restype = None
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def bf16_bits(x_f32: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(x_f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) & 0x8000).astype(np.uint16) | 0x7FC0
    return r


def e4m3fn_from_f32(x: np.ndarray) -> np.ndarray:
    lib = load()
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.fromiter((lib.oracle_e4m3fn_from_f32(float(v)) for v in flat), dtype=np.uint8,
                      count=flat.size)
    return out.reshape(np.shape(x))


def e4m3fn_to_f32(codes: np.ndarray) -> np.ndarray:
    lib = load()
    lut = np.array([lib.oracle_e4m3fn_to_f32(i) for i in range(256)], dtype=np.float32)
    return lut[np.asarray(codes, dtype=np.uint8)]


def act_quant(x_bits: np.ndarray, group: int = 128):
    """x_bits: uint16 bf16 patterns [M, K] -> (q uint8 [M,K], s fp32 [M, ceil(K/group)])."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x.shape
    G = -(-K // group)
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, G), dtype=np.float32)
    load().oracle_act_quant(_ptr(x), M, K, K, group, _ptr(q), _ptr(s))
    return q, s


def act_quant_f32(x: np.ndarray, group: int = 128):
    """x: fp32 values [M, K] (fp16 inputs widened to fp32, which is exact) ->
    (q uint8 [M,K], s fp32 [M, ceil(K/group)]), the act_quant contract."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    G = -(-K // group)
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, G), dtype=np.float32)
    load().oracle_act_quant_f32(_ptr(x), M, K, K, group, _ptr(q), _ptr(s))
    return q, s


def _gemm(fn, A, B, As, Bs, block_size):
    A = np.ascontiguousarray(A, dtype=np.uint8)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    M, K = A.shape
    N = B.shape[0]
    bn, bk = int(block_size[0]), int(block_size[1])
    KB, NB = -(-K // bk), -(-N // bn)
    As = np.ascontiguousarray(np.asarray(As, dtype=np.float32)[:M, :KB])
    Bs = np.ascontiguousarray(np.asarray(Bs, dtype=np.float32)[:NB, :KB])
    C = np.empty((M, N), dtype=np.float32)
    fn(_ptr(A), _ptr(B), _ptr(As), _ptr(Bs), M, N, K, bn, bk, _ptr(C))
    return C


def block_gemm(A, B, As, Bs, block_size=(128, 128)) -> np.ndarray:
    """fp32 [M,N]: the reference kernel's blockwise arithmetic (fp8.py:28-38)."""
    return _gemm(load().oracle_block_gemm, A, B, As, Bs, block_size)


def dequant_matmul(A, B, As, Bs, block_size=(128, 128)) -> np.ndarray:
    """fp32 [M,N]: (A*As) @ (B*Bs)^T (bench.py:11-14 with 2-D Bs)."""
    return _gemm(load().oracle_dequant_matmul, A, B, As, Bs, block_size)


def silu_and_mul(x_bits: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, D2 = x.shape
    d = D2 // 2
    out = np.empty((M, d), dtype=np.uint16)
    load().oracle_silu_and_mul(_ptr(x), M, d, _ptr(out))
    return out


def _round_to(v: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded (to nearest even) to bf16, fp16 or fp32, as fp32."""
    v = np.asarray(v, dtype=np.float32)
    if dtype == "float32":
        return v
    if dtype == "float16":
        with np.errstate(over="ignore"):
            return v.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return (bf16_bits(v).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(dtype)


def silu_and_mul_typed(x: np.ndarray, x_dtype: str, out_dtype: str) -> np.ndarray:
    """activation-helion/.../act.py:20-28 for any element types: x holds
    x_dtype values as fp32 [M, 2d]; returns out_dtype values as fp32 [M, d]:
    out = out_dtype(x_dtype(x_dtype(silu(a)) * b)), silu(a) = a * sigmoid(a)
    in fp32 (sigmoid = 1 / (1 + exp(-a))), each product formed in fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[1] // 2
    a, b = x[:, :d], x[:, d:]
    with np.errstate(over="ignore"):
        sig = np.float32(1) / (np.float32(1) + np.exp(-a))
    silu = (a * sig).astype(np.float32)
    h = _round_to(_round_to(silu, x_dtype) * b, x_dtype)
    return _round_to(h, out_dtype)


def quant_weight_block(W: np.ndarray, block=(128, 128)):
    W = np.ascontiguousarray(W, dtype=np.float32)
    N, K = W.shape
    bn, bk = int(block[0]), int(block[1])
    Wq = np.empty((N, K), dtype=np.uint8)
    Bs = np.empty((-(-N // bn), -(-K // bk)), dtype=np.float32)
    load().oracle_quant_weight_block(_ptr(W), N, K, bn, bk, _ptr(Wq), _ptr(Bs))
    return Wq, Bs
