"""torch.ops namespace of the deep-gemm drop-in (same kernel-builder naming
scheme as the finegrained-fp8 package: ``_<kernel_name>_<backend>_<id>``)."""
import torch

KERNEL_NAME = "deep_gemm_helion"
BACKEND = "rocm"
UNIQUE_ID = "mi355x"

_OPS_NAME = f"_{KERNEL_NAME}_{BACKEND}_{UNIQUE_ID}"


def add_op_namespace_prefix(op_name: str) -> str:
    return f"{_OPS_NAME}::{op_name}"


ops = getattr(torch.ops, _OPS_NAME)
