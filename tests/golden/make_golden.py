"""Writes the golden fixtures under tests/golden/ from library routines.

The reference (finegrained-fp8-helion) ships no golden vectors or known-answer
tests for this path, and its kernel cannot run here (it needs helion/Triton on
an NVIDIA GPU). The fixtures therefore come from torch's own float8_e4m3fn
cast -- the routine the reference's harness uses to build its fp8 operands
(scripts/rebench_llm.py:130) -- and from float64 numpy arithmetic:

  e4m3fn_cast_table.npz
    enc : uint8[65536]  torch's e4m3fn code of every bf16 bit pattern
    dec : float32[256]  torch's fp32 value of every e4m3fn code
  gemm_fp64_small.npz
    a tiny block-scaled GEMM (M=5, N=131, K=256, blocks 128x128) whose
    expected output is the float64 matmul of the dequantised operands.

Run: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def cast_table():
    bits = np.arange(65536, dtype=np.uint32)
    f = (bits << 16).view(np.float32)
    enc = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    codes = torch.arange(256, dtype=torch.uint8)
    dec = codes.view(torch.float8_e4m3fn).float().numpy()
    np.savez_compressed(OUT / "e4m3fn_cast_table.npz", enc=enc, dec=dec)


def gemm_small():
    g = torch.Generator().manual_seed(20240601)
    M, N, K, bn, bk = 5, 131, 256, 128, 128
    A = (torch.randn(M, K, generator=g) * 0.3).to(torch.float8_e4m3fn)
    B = (torch.randn(N, K, generator=g) * 0.3).to(torch.float8_e4m3fn)
    As = torch.rand(M, K // bk, generator=g) * 0.5 + 0.5
    Bs = torch.rand(-(-N // bn), K // bk, generator=g) * 0.5 + 0.5
    a = A.float().double().numpy() * np.repeat(As.double().numpy(), bk, axis=1)
    sb = np.repeat(np.repeat(Bs.double().numpy(), bn, axis=0)[:N], bk, axis=1)
    b = B.float().double().numpy() * sb
    C = a @ b.T
    np.savez_compressed(OUT / "gemm_fp64_small.npz", A=A.view(torch.uint8).numpy(),
                        B=B.view(torch.uint8).numpy(), As=As.numpy(), Bs=Bs.numpy(),
                        C=C, block=np.array([bn, bk]))


if __name__ == "__main__":
    cast_table()
    gemm_small()
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))
