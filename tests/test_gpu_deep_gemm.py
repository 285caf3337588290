"""GPU parity of the per-row weight-scale GEMM (deep-gemm-helion's
gemm_fp8_fp8_bf16_nt, deep-gemm-helion/.../deep_gemm_helion/fp8.py:13-29:
(A*As) @ (B*Bs)^T with Bs [N, K/128]) against the oracle's blockwise formula
with block_n = 1, within the north-star tolerance (1e-2 relative, 1e-3
absolute of the bf16 result). Covers the decode kernel (M <= 64), the
small-grid kernel, the 128x128, 256x128 and 256x256 pipelined kernels,
split-K, the generic fallback (column-major As) and ragged edges."""
import pytest
import torch

import oracle
from hf_kernels_helion_amd import deep_gemm_helion as dg
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


def _operands(M, N, K, seed):
    x = synthetic.activations(M, K, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    W = torch.randn(N, K, generator=g) * 0.02
    Wq, Bs = synthetic.quantize_weight_blockwise(W, 1, 128)  # one scale per row and K-block
    return x, Wq, Bs


@pytest.mark.parametrize("M,N,K", [(1, 256, 256), (16, 4096, 14336), (32, 2048, 14336),
                                   (48, 640, 1024),
                                   (64, 512, 1024), (300, 700, 1536), (128, 2048, 8192)])
def test_deep_gemm_vs_oracle(M, N, K, dev):
    print(f"deep-gemm per-row M={M} N={N} K={K}", flush=True)
    x, Wq, Bs = _operands(M, N, K, seed=M + N)
    q, s = fp8.act_quant(x.to(dev), 128)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wq.to(dev), s, Bs.to(dev), 128)
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)
    rows = torch.arange(M) if M <= 64 else torch.tensor([0, 1, M // 2, M - 1])
    ref = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(Wq), s.cpu()[rows].numpy(), Bs.numpy(),
                            (1, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


def test_per_row_full_check_and_fp32(dev):
    """Every row against torch's fp32 dequant-matmul; the fp32 output of the
    finegrained API with block_size [1, 128] gives the same bf16 after
    rounding."""
    M, N, K = 1024, 1536, 2048
    x, Wq, Bs = _operands(M, N, K, seed=3)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    f32 = fp8.w8a8_block_fp8_matmul(q, Wd, s, Bsd, [1, 128], torch.float32)
    assert torch.equal(f32.to(torch.bfloat16), out)


@pytest.mark.parametrize("M,N,K,splits", [(32, 7168, 8192, 4), (16, 12800, 8192, 2),
                                          (8, 18432, 8192, 1), (64, 4096, 14336, 8),
                                          (50, 6144, 8192, 5), (64, 8192, 8192, 4),
                                          (48, 36864, 1024, 1), (17, 33024, 4224, 1),
                                          (48, 28672, 2048, 1), (33, 16384, 4096, 2)])
def test_per_row_decode_split_plans(M, N, K, splits, dev):
    """The per-row decode plan splits K as often as keeps one workgroup per
    CU (its four-stage ring holds one per CU): 56 column tiles x 4, 100 x 2
    (32 K-blocks per split), 144 unsplit; with 49..64 rows (64 activation
    rows per workgroup) 32 x 8, 48 x 5 and 64 x 4; past one workgroup per CU
    (288 and 258 column tiles, unsplit) two share a CU on the three-stage
    ring; 17..48 rows on 224 and 128 column tiles take it over the small-grid
    kernel. Every element against torch's
    fp32 dequant-matmul, sampled rows against the oracle."""
    from hf_kernels_helion_amd import _native
    print(f"deep-gemm per-row decode split plan M={M} N={N} K={K}", flush=True)
    ws = _native.load().fp8b_gemm_workspace_size(M, N, K, 1, 128)
    assert ws == (splits * M * N * 4 if splits > 1 else 0)
    x, Wq, Bs = _operands(M, N, K, seed=N + 11)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor([0, M // 2, M - 1])
    ref = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(Wq), s.cpu()[rows].numpy(), Bs.numpy(),
                            (1, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(2999, 4000, 1536), (4096, 4096, 8192), (1500, 13900, 512)])
def test_per_row_256_tiles(M, N, K, dev):
    """Grids that get 256x256 tiles: a partial wave with ragged edges and a
    K-block count (12) that leaves the second 8-block scale window half
    empty, the full 4096-square wave, and a grid whose last partial wave (74
    of 330 tiles) runs as 256x128 halves, one of them past N. Every element
    against torch's fp32 dequant-matmul."""
    print(f"deep-gemm per-row 256x256 tiles M={M} N={N} K={K}", flush=True)
    x, Wq, Bs = _operands(M, N, K, seed=7)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 2048), (1000, 7000, 1536), (256, 28672, 1024),
                                   (1537, 4096, 512)])
def test_per_row_256x128_tiles(M, N, K, dev):
    """Grids whose 256x128 tiles fit one wave of workgroups while 128x128
    tiles need two or more: the per-row 256x128 kernel, with ragged edges, a
    K-block count (12) that leaves the second scale window half empty and a
    last tile row of one row. Every element against torch's fp32
    dequant-matmul, and bit for bit against row slices on the unsplit
    per-row 128x128 kernel."""
    from hf_kernels_helion_amd import _native
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    t = lambda bm, bn: -(-M // bm) * -(-N // bn)
    if not t(128, 128) > cus >= t(256, 128):
        pytest.skip(f"{M}x{N} is not a 256x128 grid on {cus} CUs")
    print(f"deep-gemm per-row 256x128 tiles M={M} N={N} K={K}", flush=True)
    x, Wq, Bs = _operands(M, N, K, seed=13)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    lib = _native.load()
    h = 128 * (cus // -(-N // 128))
    slices = [(r0, r0 + h) for r0 in range(0, M - h, h)] + [(M - h, M)]
    for r0, r1 in slices:
        assert lib.fp8b_gemm_workspace_size(r1 - r0, N, K, 1, 128) == 0
        part = dg.gemm_fp8_fp8_bf16_nt(q[r0:r1], Wd, s[r0:r1], Bsd)
        assert torch.equal(out[r0:r1], part)


def test_per_row_generic_fallback(dev):
    """Column-major As: the pipelined kernel's scale windows need K-contiguous
    scales, so the generic kernel runs; same tolerance."""
    M, N, K = 96, 384, 1024
    x, Wq, Bs = _operands(M, N, K, seed=5)
    q, s = fp8.act_quant(x.to(dev), 128)
    s_t = s.T.contiguous().T
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wq.to(dev), s_t, Bs.to(dev))
    ref = oracle.block_gemm(_u8(q), _u8(Wq), s.cpu().numpy(), Bs.numpy(), (1, 128))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (1024, 512, 7168), (768, 768, 4096),
                                   (2048, 1024, 2048), (32, 14336, 4096), (1, 8192, 4096),
                                   (64, 4096, 4096), (300, 700, 1536), (1024, 2048, 4096),
                                   (960, 1024, 4096), (32, 4096, 4096), (16, 4096, 7168)])
def test_per_row_small_grid_tiles(M, N, K, dev):
    """Small grids run gemm_tiny_kernel with per-row weight scales (8, 4, 2
    and 1 waves per 32x32 tile, decode-sized M, ragged edges): every element
    against torch's fp32 dequant-matmul, sampled rows against the oracle,
    no workspace, the same bits on a second call. With one wave per tile the
    fold order is that of the unsplit per-row plans, so the same rows inside
    a 32768-row grid give the same bits."""
    from hf_kernels_helion_amd import _native
    print(f"deep-gemm per-row small grid M={M} N={N} K={K}", flush=True)
    lib = _native.load()
    assert lib.fp8b_gemm_workspace_size(M, N, K, 1, 128) == 0
    x, Wq, Bs = _operands(M, N, K, seed=M + 3 * N)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor(sorted({r for r in (0, 31, 32, M // 2, M - 1) if r < M}))
    ref = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(Wq), s.cpu()[rows].numpy(), Bs.numpy(),
                            (1, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    assert torch.equal(dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd), out)
    t64 = -(-M // 64) * -(-N // 64)
    kb = K // 128
    band64 = M > 64 and 16 <= kb <= 64 and (
        (t64 == 512 and kb <= 32) or (256 < t64 < 512 and 24 <= kb <= 48 and N <= 16 * M) or (224 <= t64 <= 256 and (kb <= 32 or N <= 16 * M)))
    if not band64 and ((M + 31) // 32) * ((N + 31) // 32) > 4 * 256:
        big = 32768
        reps = (big + M - 1) // M
        qb = q.repeat(reps, 1)[:big].contiguous()
        sb = s.repeat(reps, 1)[:big].contiguous()
        assert lib.fp8b_gemm_workspace_size(big, N, K, 1, 128) == 0
        assert torch.equal(dg.gemm_fp8_fp8_bf16_nt(qb, Wd, sb, Bsd)[:M], out)


@pytest.mark.parametrize("M,N,K", [(128, 4096, 32768), (1024, 2048, 14336), (3000, 1000, 2048)])
def test_per_row_128_tiles_split_and_unsplit(M, N, K, dev):
    """Grids past the small-grid range on the per-row 128x128 kernel: split
    along K (128 rows, 8 splits; 1024 x 2048 x 14336, 2 splits) and unsplit (3000 x
    1000: 192 tiles). Every element against torch's fp32 dequant-matmul."""
    from hf_kernels_helion_amd import _native
    print(f"deep-gemm per-row 128x128 tiles M={M} N={N} K={K}", flush=True)
    need = _native.load().fp8b_gemm_workspace_size(M, N, K, 1, 128)
    assert (need > 0) == (M <= 1024)
    x, Wq, Bs = _operands(M, N, K, seed=11)
    q, s = fp8.act_quant(x.to(dev), 128)
    Wd, Bsd = Wq.to(dev), Bs.to(dev)
    out = dg.gemm_fp8_fp8_bf16_nt(q, Wd, s, Bsd)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (Wd.float() * Bsd.repeat_interleave(
        128, 1)).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
