"""Seeded synthetic inputs for the block-FP8 configurations.

All tensors are drawn on the CPU with torch.Generator so a CPU baseline and a
GPU run see identical bits; callers move them to the device.

Distributions:
  activations  bf16 ~ N(0,1); optional outliers: ceil(frac*K) seeded columns
               per row multiplied by `outlier_scale`;
  weights      fp32 ~ N(0, 0.02), quantised per block_n x block_k block:
               Bs = max(amax, 1e-10)/448, Wq = e4m3fn(W / Bs);
  harness      the reference harness's operands (scripts/rebench_llm.py:128-131):
               A, B = (randn*0.3).to(e4m3fn), As, Bs ~ U(0.5, 1.0).
"""
from __future__ import annotations

import torch

SEED_A = 1234
SEED_W = 5678


def activations(M: int, K: int, seed: int = SEED_A, outlier_frac: float = 0.0,
                outlier_scale: float = 20.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outlier_frac > 0.0:
        n_out = max(1, int(-(-outlier_frac * K // 1)))
        idx = torch.stack([torch.randperm(K, generator=g)[:n_out] for _ in range(M)])
        rows = torch.arange(M).unsqueeze(1).expand_as(idx)
        x[rows, idx] *= outlier_scale
    return x.to(torch.bfloat16)


def quantize_weight_blockwise(W: torch.Tensor, block_n: int = 128, block_k: int = 128):
    """fp32 [N,K] -> (e4m3fn [N,K], fp32 [ceil(N/bn), ceil(K/bk)]) with torch ops."""
    N, K = W.shape
    NB, KB = -(-N // block_n), -(-K // block_k)
    Wp = torch.nn.functional.pad(W.float(), (0, KB * block_k - K, 0, NB * block_n - N))
    blocks = Wp.view(NB, block_n, KB, block_k)
    amax = blocks.abs().amax(dim=(1, 3)).clamp_min(1e-10)
    Bs = amax / 448.0
    q = (blocks / Bs[:, None, :, None]).to(torch.float8_e4m3fn)
    Wq = q.view(NB * block_n, KB * block_k)[:N, :K].contiguous()
    return Wq, Bs.contiguous()


def weights(N: int, K: int, seed: int = SEED_W, std: float = 0.02, block_n: int = 128,
            block_k: int = 128):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(N, K, generator=g) * std
    return quantize_weight_blockwise(W, block_n, block_k)


def harness_operands(M: int, N: int, K: int, seed: int = 0, block_n: int = 128,
                     block_k: int = 128):
    g = torch.Generator().manual_seed(seed)
    A = (torch.randn(M, K, generator=g) * 0.3).to(torch.float8_e4m3fn)
    B = (torch.randn(N, K, generator=g) * 0.3).to(torch.float8_e4m3fn)
    As = torch.rand(M, -(-K // block_k), generator=g) * 0.5 + 0.5
    Bs = torch.rand(-(-N // block_n), -(-K // block_k), generator=g) * 0.5 + 0.5
    return A, B, As, Bs
