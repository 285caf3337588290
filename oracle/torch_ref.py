"""The reference's PyTorch CPU dequantise-then-matmul path -- TEST/BASELINE ONLY.

Restates finegrained-fp8-helion/bench.py:11-14 with the weight scales
expanded over both N and K (the finegrained layout Bs[N/bn, K/bk]), plus the
CPU act-quant for configurations that quantise activations in-op. bench.py
times these on the GPU box's host cores as the reported CPU baseline; tests
use them as a second, independent formulation.
"""
from __future__ import annotations

import torch


def expand_scales(As: torch.Tensor, Bs: torch.Tensor, M: int, N: int, K: int,
                  block_n: int, block_k: int):
    saf = As[:M].repeat_interleave(block_k, dim=1)[:, :K]
    sbf = Bs.repeat_interleave(block_n, dim=0)[:N].repeat_interleave(block_k, dim=1)[:, :K]
    return saf, sbf


def dequant_matmul(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor, Bs: torch.Tensor,
                   block_size=(128, 128), out_dtype=torch.bfloat16) -> torch.Tensor:
    """((A.float()*As) @ (B.float()*Bs).T).to(out_dtype) on whatever device A is on."""
    M, K = A.shape
    N = B.shape[0]
    bn, bk = int(block_size[0]), int(block_size[1])
    saf, sbf = expand_scales(As, Bs, M, N, K, bn, bk)
    return ((A.float() * saf) @ (B.float() * sbf).T).to(out_dtype)


def act_quant(x: torch.Tensor, group: int = 128):
    """CPU per-token-group quantiser: s = max(amax,1e-10)/448, q = e4m3fn(x/s).
    Finite inputs only (the baseline workloads are finite)."""
    M, K = x.shape
    G = -(-K // group)
    pad = G * group - K
    xf = x.float()
    if pad:
        xf = torch.nn.functional.pad(xf, (0, pad))
    xg = xf.view(M, G, group)
    amax = xg.abs().amax(dim=-1).clamp_min(1e-10)
    s = amax / 448.0
    q = (xg / s.unsqueeze(-1)).to(torch.float8_e4m3fn).view(M, G * group)[:, :K]
    return q.contiguous(), s


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    d = x.shape[-1] // 2
    a = x[..., :d].float()
    return (torch.nn.functional.silu(a).to(x.dtype) * x[..., d:]).to(x.dtype)

