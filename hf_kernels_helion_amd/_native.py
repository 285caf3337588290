"""ctypes binding of libfp8_blockwise.so (the C ABI in include/fp8_blockwise.h).

The library is built in-tree by ``hf_kernels_helion_amd.build``. There is no
fallback: if the library is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libfp8_blockwise.so"

# fp8b_status codes (include/fp8_blockwise.h).
STATUS_NAMES = {
    0: "FP8B_OK",
    1: "FP8B_ERR_NULL",
    2: "FP8B_ERR_DIMS",
    3: "FP8B_ERR_ALIGN",
    4: "FP8B_ERR_BLOCK",
    5: "FP8B_ERR_DTYPE",
    6: "FP8B_ERR_WORKSPACE",
    7: "FP8B_ERR_LAUNCH",
}

# fp8b_dtype codes.
F32, BF16, F16 = 0, 1, 2


class PlanInfo(ctypes.Structure):
    """fp8b_plan_info: what fp8b_w8a8_block_matmul launches for one call."""
    _fields_ = [
        ("kernel", ctypes.c_int),
        ("tile_m", ctypes.c_int),
        ("tile_n", ctypes.c_int),
        ("splits", ctypes.c_int),
        ("kb_per_split", ctypes.c_int),
        ("waves", ctypes.c_int),
        ("ring", ctypes.c_int),
        ("workgroups", ctypes.c_int64),
        ("tail_kernel", ctypes.c_int),
        ("tail_tile_m", ctypes.c_int),
        ("tail_tile_n", ctypes.c_int),
        ("tail_workgroups", ctypes.c_int64),
        ("reduce", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
        ("cu_count", ctypes.c_int),
    ]

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "fp8b_version": (ctypes.c_int, []),
    "fp8b_last_error": (ctypes.c_char_p, []),
    "fp8b_act_quant": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "fp8b_act_quant_typed": (
        ctypes.c_int, [_vp, _i64, ctypes.c_int, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "fp8b_w8a8_block_matmul": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, ctypes.c_int,
         _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp],
    ),
    "fp8b_gemm_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "fp8b_gemm_plan": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i64, ctypes.c_int,
                                      ctypes.POINTER(PlanInfo)]),
    "fp8b_kernel_name": (ctypes.c_char_p, [ctypes.c_int]),
    "fp8b_gate_up_plan": (ctypes.c_int, [_i64, _i64, _i64, ctypes.c_int,
                                         ctypes.POINTER(PlanInfo)]),
    "fp8b_act_quant_matmul_plan": (ctypes.c_int, [_i64, _i64, _i64, ctypes.c_int,
                                                  ctypes.POINTER(PlanInfo)]),
    "fp8b_w8a8_block_matmul_noalloc": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, ctypes.c_int,
         _i64, _i64, _i64, _i64, _i64, _vp],
    ),
    "fp8b_act_quant_matmul": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, ctypes.c_int,
         _i64, _i64, _i64, _vp, _sz, _vp],
    ),
    "fp8b_act_quant_matmul_workspace_size": (_sz, [_i64, _i64, _i64]),
    "fp8b_weight_quant": (
        ctypes.c_int,
        [_vp, _i64, ctypes.c_int, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp],
    ),
    "fp8b_silu_and_mul": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "fp8b_silu_and_mul_typed": (
        ctypes.c_int, [_vp, _i64, ctypes.c_int, _vp, _i64, ctypes.c_int, _i64, _i64, _vp]),
    "fp8b_silu_and_mul_quant": (
        ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "fp8b_gate_up_silu_quant": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
         _i64, _i64, _i64, _vp],
    ),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP kernels first "
                    "(python -m hf_kernels_helion_amd.build)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def gemm_plan(M: int, N: int, K: int, block_n: int = 128, block_k: int = 128,
              cu_count: int = 0) -> dict:
    """The launches of one fp8b_w8a8_block_matmul call for contiguous, aligned
    operands (fp8b_gemm_plan), with kernel codes turned into names.
    cu_count <= 0 asks the current device; a positive count makes no GPU call."""
    lib = load()
    info = PlanInfo()
    check(lib.fp8b_gemm_plan(M, N, K, block_n, block_k, cu_count, ctypes.byref(info)),
          "fp8b_gemm_plan")
    return _plan_dict(lib, info)


def act_quant_matmul_plan(M: int, N: int, K: int, cu_count: int = 0) -> dict:
    """The GEMM launch of one fp8b_act_quant_matmul call for a contiguous,
    aligned x (fp8b_act_quant_matmul_plan): gemm_decode_quant_kernel when one
    kernel quantises and multiplies, else the GEMM after the act-quant launch."""
    lib = load()
    info = PlanInfo()
    check(lib.fp8b_act_quant_matmul_plan(M, N, K, cu_count, ctypes.byref(info)),
          "fp8b_act_quant_matmul_plan")
    return _plan_dict(lib, info)


def gate_up_plan(M: int, I: int, K: int, cu_count: int = 0) -> dict:
    """The launch of one fp8b_gate_up_silu_quant call (fp8b_gate_up_plan)."""
    lib = load()
    info = PlanInfo()
    check(lib.fp8b_gate_up_plan(M, I, K, cu_count, ctypes.byref(info)), "fp8b_gate_up_plan")
    return _plan_dict(lib, info)


def _plan_dict(lib, info) -> dict:
    out = {name: getattr(info, name) for name, _ in PlanInfo._fields_}
    for key in ("kernel", "tail_kernel"):
        out[key] = lib.fp8b_kernel_name(out[key]).decode()
    return out


def check(status: int, what: str) -> None:
    """Turn a non-zero fp8b_status into RuntimeError with the library's text."""
    if status != 0:
        msg = load().fp8b_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {STATUS_NAMES.get(status, status)}: {msg}")
