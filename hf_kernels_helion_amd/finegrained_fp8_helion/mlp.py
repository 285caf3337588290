"""Block-FP8 gated MLP: the chain the finegrained-fp8 GEMM serves in a model.

    x bf16 [M, H]
      -> act_quant (1x128 groups)                    -> xq, xs
      -> w8a8 GEMM with gate/up weight [2I, H]       -> h bf16 [M, 2I]
      -> silu(h[:, :I]) * h[:, I:], act_quant fused  -> hq, hs
      -> w8a8 GEMM with down weight [H, I]           -> y bf16 [M, H]

The gate/up GEMM's output columns are [gate | up], the layout silu_and_mul
consumes (activation-helion/.../act.py:20-28).
"""
from __future__ import annotations

import torch

from ._ops import ops


def fp8_mlp(x: torch.Tensor, w_gate_up: torch.Tensor, s_gate_up: torch.Tensor,
            w_down: torch.Tensor, s_down: torch.Tensor, block_size=(128, 128),
            fuse_quant: bool = True) -> torch.Tensor:
    """y = down(silu(gate(x)) * up(x)) with e4m3fn weights and 128x128 block
    scales. ``fuse_quant=False`` runs silu_and_mul and act_quant as two ops
    (bit-identical result, one more bf16 round trip through HBM)."""
    bn, bk = int(block_size[0]), int(block_size[1])
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    xq, xs = ops.act_quant(x2, bk)
    h = ops.w8a8_block_fp8_matmul_dtype(xq, w_gate_up, xs, s_gate_up, bn, bk, torch.bfloat16)
    if fuse_quant:
        hq, hs = ops.silu_and_mul_quant(h, bk)
    else:
        a = torch.empty((h.shape[0], h.shape[1] // 2), dtype=torch.bfloat16, device=h.device)
        ops.silu_and_mul(a, h)
        hq, hs = ops.act_quant(a, bk)
    y = ops.w8a8_block_fp8_matmul_dtype(hq, w_down, hs, s_down, bn, bk, torch.bfloat16)
    return y.reshape(*lead, y.shape[-1])
