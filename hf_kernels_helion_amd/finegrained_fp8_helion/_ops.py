"""torch.ops namespace of this package.

Same naming scheme as the kernel-builder glue of the reference
(finegrained-fp8-helion/build/torch-cuda/_ops.py:21-36): the namespace is
``_<kernel_name>_<backend>_<unique_id>``; the backend is always "rocm" here
because the only implementation is the gfx950 HIP library.
"""
import torch

KERNEL_NAME = "finegrained_fp8_helion"
BACKEND = "rocm"
UNIQUE_ID = "mi355x"

_OPS_NAME = f"_{KERNEL_NAME}_{BACKEND}_{UNIQUE_ID}"


def add_op_namespace_prefix(op_name: str) -> str:
    """Prefix op by namespace (reference: _ops.py:32-36)."""
    return f"{_OPS_NAME}::{op_name}"


ops = getattr(torch.ops, _OPS_NAME)
