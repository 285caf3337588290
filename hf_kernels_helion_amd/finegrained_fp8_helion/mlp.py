"""Block-FP8 gated MLP: the chain the finegrained-fp8 GEMM serves in a model.

    x bf16 [M, H]
      -> act_quant (1x128 groups)                    -> xq, xs
      -> w8a8 GEMM with gate/up weight [2I, H]       -> h bf16 [M, 2I]
      -> silu(h[:, :I]) * h[:, I:], act_quant fused  -> hq, hs
      -> w8a8 GEMM with down weight [H, I]           -> y bf16 [M, H]

The gate/up GEMM's output columns are [gate | up], the layout silu_and_mul
consumes (activation-helion/.../act.py:20-28).

With the gate/up weight interleaved once in 128-row blocks
(``interleave_gate_up``), every 256-column tile of the gate/up GEMM holds a
gate block and its matching up block, and the GEMM's epilogue forms
silu(gate) * up and quantises it itself (``gate_up_silu_quant``): the bf16
h [M, 2I] is never written. Same bits as the three-step chain whenever its
GEMM runs unsplit. Below FUSED_GATE_UP_MIN_ROWS rows the fused kernel's
256-row tiles would leave most of the GPU idle, so those run the chain
itself on the interleaved weights (each 256-column block of h is one
gate | up pair).
"""
from __future__ import annotations

import torch

from ._ops import ops


def interleave_gate_up(w_gate_up: torch.Tensor, s_gate_up: torch.Tensor):
    """Reorder a [gate; up] weight [2I, H] and its block scales [2I/128, H/128]
    into 128-row blocks [gate 0, up 0, gate 1, up 1, ...] (a one-time weight
    preparation for ``gate_up_silu_quant``). I must be a multiple of 128."""
    n2, h = w_gate_up.shape
    if n2 % 256 != 0:
        raise ValueError(f"gate/up weight must have 2I rows with I % 128 == 0, got {n2}")
    nb = n2 // 256
    w = w_gate_up.reshape(2, nb, 128, h).transpose(0, 1).reshape(n2, h).contiguous()
    s = s_gate_up.reshape(2, nb, s_gate_up.shape[-1]).transpose(0, 1)
    return w, s.reshape(2 * nb, s_gate_up.shape[-1]).contiguous()


# Rows from which the fused gate/up kernel beats the GEMM + silu_and_mul_quant
# chain (H = 4096, I = 14336, weights streamed from HBM: M = 256 98.7 us
# fused against 95.3 for the chain, M = 512 126.1 against 127.5, M = 32
# 76.5 against 49.9).
FUSED_GATE_UP_MIN_ROWS = 512


def gate_up_silu_quant(xq: torch.Tensor, xs: torch.Tensor, w_il: torch.Tensor,
                       s_il: torch.Tensor):
    """act_quant(silu_and_mul(w8a8 GEMM(xq, w, xs, s) in bf16), 128) with
    (w_il, s_il) from ``interleave_gate_up``: from FUSED_GATE_UP_MIN_ROWS
    rows one kernel (bit-identical to the chain whenever the chain's GEMM
    runs unsplit), below that the chain's two ops on the interleaved layout.
    Needs block_size (128, 128) and H % 128 == 0. Returns (q [M, I] e4m3fn,
    s [M, I/128] fp32)."""
    m = xq.shape[0]
    if m >= FUSED_GATE_UP_MIN_ROWS or m == 0:
        return ops.gate_up_silu_quant(xq, w_il, xs, s_il)
    # the fused kernel's shape contract, for both routes
    if xq.dim() != 2 or w_il.dim() != 2 or w_il.shape[0] % 256 != 0 or \
            xq.shape[1] % 128 != 0 or xq.shape[1] == 0:
        raise RuntimeError("gate_up_silu_quant: I must be a multiple of 128 and K a positive "
                           f"multiple of 128 (A {tuple(xq.shape)}, B {tuple(w_il.shape)})")
    i = w_il.shape[0] // 2
    h = ops.w8a8_block_fp8_matmul_dtype(xq, w_il, xs, s_il, 128, 128, torch.bfloat16)
    # rows of 256 columns: gate block | up block
    hq, hs = ops.silu_and_mul_quant(h.view(m * (i // 128), 256), 128)
    return hq.view(m, i), hs.view(m, i // 128)


def fp8_mlp(x: torch.Tensor, w_gate_up: torch.Tensor, s_gate_up: torch.Tensor,
            w_down: torch.Tensor, s_down: torch.Tensor, block_size=(128, 128),
            fuse_quant: bool = True, gate_up_interleaved: bool = False) -> torch.Tensor:
    """y = down(silu(gate(x)) * up(x)) with e4m3fn weights and 128x128 block
    scales. ``fuse_quant=False`` runs silu_and_mul and act_quant as two ops
    (bit-identical result, one more bf16 round trip through HBM).
    ``gate_up_interleaved=True``: (w_gate_up, s_gate_up) come from
    ``interleave_gate_up`` and the gate/up GEMM, SiLU·up and its quantisation
    run as one kernel from FUSED_GATE_UP_MIN_ROWS rows (the same bits as the
    default chain whenever its gate/up GEMM runs unsplit; below that many
    rows the default chain's ops on the interleaved layout, the same bits)."""
    bn, bk = int(block_size[0]), int(block_size[1])
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    xq, xs = ops.act_quant(x2, bk)
    if gate_up_interleaved:
        if (bn, bk) != (128, 128):
            raise ValueError("gate_up_interleaved needs block_size (128, 128)")
        hq, hs = gate_up_silu_quant(xq, xs, w_gate_up, s_gate_up)
        y = ops.w8a8_block_fp8_matmul_dtype(hq, w_down, hs, s_down, bn, bk, torch.bfloat16)
        return y.reshape(*lead, y.shape[-1])
    h = ops.w8a8_block_fp8_matmul_dtype(xq, w_gate_up, xs, s_gate_up, bn, bk, torch.bfloat16)
    if fuse_quant:
        hq, hs = ops.silu_and_mul_quant(h, bk)
    else:
        a = torch.empty((h.shape[0], h.shape[1] // 2), dtype=torch.bfloat16, device=h.device)
        ops.silu_and_mul(a, h)
        hq, hs = ops.act_quant(a, bk)
    y = ops.w8a8_block_fp8_matmul_dtype(hq, w_down, hs, s_down, bn, bk, torch.bfloat16)
    return y.reshape(*lead, y.shape[-1])
