"""GPU parity of the block-FP8 GEMM against the CPU oracle.

Tolerance: the bf16 output within 1e-2 relative /
1e-3 absolute of the oracle's result of the reference formula
(finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/fp8.py:28-38),
itself checked against the fp32 dequant-matmul oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _u8(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.uint8).numpy()


def _operands(M, N, K, seed, kind="model", outliers=0.0):
    if kind == "harness":
        return synthetic.harness_operands(M, N, K, seed=seed)
    x = synthetic.activations(M, K, seed=seed, outlier_frac=outliers)
    xg = x.cuda()
    q, s = fp8.act_quant(xg, 128)
    W, Bs = synthetic.weights(N, K, seed=seed + 1)
    return q.cpu(), W, s.cpu(), Bs


def _check(out_gpu, A, B, As, Bs, block=(128, 128), rows=None):
    ref = oracle.block_gemm(_u8(A), _u8(B), As.numpy(), Bs.numpy(), block)
    got = out_gpu.float().cpu()
    if rows is not None:
        got = got[rows]
    ref_t = torch.from_numpy(ref)
    if out_gpu.dtype != torch.float32:
        ref_t = ref_t.to(out_gpu.dtype).float()
    torch.testing.assert_close(got, ref_t, rtol=RTOL, atol=ATOL)
    return ref


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (128, 256, 1024), (57, 200, 384),
                                   (1, 128, 128), (300, 640, 512), (32, 4096, 1024),
                                   (64, 512, 2048), (257, 384, 256), (3, 1000, 640),
                                   (48, 130, 256), (65, 384, 512), (8, 4096, 14336)])
@pytest.mark.parametrize("kind", ["model", "harness"])
def test_gemm_bf16_vs_oracle(M, N, K, kind, dev):
    print(f"gemm bf16 {kind} M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=M + N + K, kind=kind)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128],
                                    torch.bfloat16)
    assert out.dtype == torch.bfloat16 and out.shape == (M, N)
    _check(out, A, B, As, Bs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.float64])
@pytest.mark.parametrize("M", [96, 17])
def test_gemm_output_dtypes(dtype, M, dev):
    print(f"gemm out dtype {dtype} M={M}", flush=True)
    N, K = 384, 1024
    A, B, As, Bs = _operands(M, N, K, seed=5)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128],
                                    dtype)
    assert out.dtype == dtype
    _check(out.float() if dtype == torch.float64 else out, A, B, As, Bs)


def test_gemm_default_output_is_fp32(dev):
    A, B, As, Bs = _operands(64, 128, 256, seed=1)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), (128, 128))
    assert out.dtype == torch.float32


def test_gemm_bf16_is_rne_of_fp32(dev):
    """The bf16 epilogue equals the fp32 op's result rounded by torch."""
    M, N, K = 200, 512, 2048
    A, B, As, Bs = [t.to(dev) for t in _operands(M, N, K, seed=8)]
    f32 = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.float32)
    b16 = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
    assert torch.equal(f32.to(torch.bfloat16), b16)


def test_gemm_exact_small_integers(dev):
    """As = Bs = 1 and small-integer fp8 operands: every partial sum is an
    integer below 2^24, so the result is exact and must match bit for bit."""
    print("gemm exact integers", flush=True)
    g = torch.Generator().manual_seed(3)
    M, N, K = 160, 256, 1024
    A = torch.randint(-4, 5, (M, K), generator=g).float().to(torch.float8_e4m3fn)
    B = torch.randint(-4, 5, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    As = torch.ones(M, K // 128)
    Bs = torch.ones(N // 128, K // 128)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128])
    exact = A.double() @ B.double().T
    assert torch.equal(out.cpu().double(), exact)


def test_gemm_one_hot_rows_select_weight_rows(dev):
    M, N, K = 64, 256, 512
    A = torch.zeros(M, K)
    cols = torch.arange(M) * 7 % K
    A[torch.arange(M), cols] = 1.0
    A = A.to(torch.float8_e4m3fn)
    W, Bs = synthetic.weights(N, K, seed=4)
    As = torch.full((M, K // 128), 2.0)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), W.to(dev), As.to(dev), Bs.to(dev), [128, 128])
    sbf = Bs.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]
    expect = (W.float() * sbf)[:, cols].T * 2.0
    assert torch.equal(out.cpu(), expect)


def test_gemm_generic_block_sizes(dev):
    """Block sizes other than 128x128 and ragged K run the generic kernel."""
    for (M, N, K, bn, bk) in [(33, 70, 200, 64, 64), (16, 96, 256, 32, 128), (40, 130, 300, 128, 128)]:
        print(f"gemm generic M={M} N={N} K={K} bn={bn} bk={bk}", flush=True)
        A, B, As, Bs = synthetic.harness_operands(M, N, K, seed=M, block_n=bn, block_k=bk)
        out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [bn, bk],
                                        torch.float32)
        _check(out, A, B, As, Bs, block=(bn, bk))


def test_gemm_strided_scales_and_operands(dev):
    """Non-contiguous A (row stride > K) and transposed-storage As."""
    M, N, K = 100, 256, 1024
    A, B, As, Bs = _operands(M, N, K, seed=12)
    Abig = torch.zeros(M, K + 256, dtype=torch.uint8)
    Abig[:, :K] = A.view(torch.uint8)
    Av = Abig.to(dev).view(torch.float8_e4m3fn)[:, :K]
    As_t = As.T.contiguous().to(dev).T  # column-major storage
    out = fp8.w8a8_block_fp8_matmul(Av, B.to(dev), As_t, Bs.to(dev), [128, 128], torch.bfloat16)
    _check(out, A, B, As, Bs)


def test_gemm_empty_shapes(dev):
    A = torch.empty(0, 256, dtype=torch.float8_e4m3fn, device=dev)
    B = torch.zeros(128, 256, dtype=torch.float8_e4m3fn, device=dev)
    out = fp8.w8a8_block_fp8_matmul(A, B, torch.ones(0, 2, device=dev),
                                    torch.ones(1, 2, device=dev), [128, 128], torch.bfloat16)
    assert out.shape == (0, 128)


@pytest.mark.parametrize("N", [4096, 2048])
def test_gemm_decode_shape(N, dev):
    """M=32, K=14336 on the split-K decode kernel and its sum (32 column
    tiles x 8 splits for the decode config, 16 x 16 for N = 2048), against
    the oracle on all rows."""
    print(f"gemm decode 32x{N}x14336", flush=True)
    A, B, As, Bs = _operands(32, N, 14336, seed=21)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128],
                                    torch.bfloat16)
    _check(out, A, B, As, Bs)


@pytest.mark.parametrize("M,N,K,splits", [(32, 7168, 8192, 4), (16, 12800, 8192, 3),
                                          (8, 18432, 8192, 1), (32, 28672, 4096, 1),
                                          (24, 9216, 11264, 3), (48, 28672, 2048, 1),
                                          (48, 16384, 4096, 2), (1, 28672, 2048, 1),
                                          (16, 32768, 1536, 1), (20, 4000, 14336, 8),
                                          (33, 4096, 14336, 8), (13, 8100, 8192, 4)])
def test_gemm_decode_split_plans(M, N, K, splits, dev):
    """The decode plan's split counts: as many splits as keep one workgroup
    per CU (56 column tiles x 4; 144 and 224 tiles unsplit, no sum kernel;
    72 tiles x 3), and one split more, past the CU count on the three-stage
    ring two workgroups per CU, where that would leave 32 K-blocks per split
    (100 tiles x 3: 300 workgroups); 17..48 rows on 224 and 128 column tiles,
    and 1..16 rows on more than 128 with short K, take it over the
    small-grid kernel. Split sums over column-tile counts that are
    multiples of 8 run XCD-local (rows past M in a block of 8, a ragged last
    column tile: 20x4000, 33x4096, 13x8100), the others in row order. Every
    element against torch's fp32 dequant-matmul, sampled rows against the
    oracle."""
    from hf_kernels_helion_amd import _native
    print(f"gemm decode split plan M={M} N={N} K={K} splits={splits}", flush=True)
    ws = _native.load().fp8b_gemm_workspace_size(M, N, K, 128, 128)
    assert ws == (splits * M * N * 4 if splits > 1 else 0)
    A, B, As, Bs = _operands(M, N, K, seed=N + K, outliers=0.01)
    Ad, Bd, Asd, Bsd = A.to(dev), B.to(dev), As.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16)
    full = (Ad.float() * Asd.repeat_interleave(128, 1)) @ (
        Bd.float() * Bsd.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor([0, M // 2, M - 1])
    _check(out, A[rows], B, As[rows], Bs, rows=rows)
    assert torch.equal(fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16),
                       out)


@pytest.mark.parametrize("M,N,K,outliers", [(2048, 2048, 4096, 0.01), (4096, 4096, 8192, 0.0)])
def test_gemm_large_sampled_rows(M, N, K, outliers, dev):
    """Benchmark sizes: every row checked against torch's fp32 dequant-matmul
    on the GPU; a seeded sample of rows checked against the oracle."""
    print(f"gemm large M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=M, outliers=outliers)
    Ad, Bd, Asd, Bsd = A.to(dev), B.to(dev), As.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(1))[:8]
    ref = oracle.block_gemm(_u8(A[rows]), _u8(B), As[rows].numpy(), Bs.numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    saf = Asd.repeat_interleave(128, 1)[:, :K]
    sbf = Bsd.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]
    full = (Ad.float() * saf) @ (Bd.float() * sbf).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 2048), (4096, 2048, 4096), (8192, 4096, 8192),
                                   (8192, 8192, 8192)])
def test_gemm_reference_tuning_shapes(M, N, K, dev):
    """The reference's fp8 tuning shapes not covered above
    (scripts/aot_tune.py:134-136) on its own operand recipe (:139-146: A, B =
    e4m3fn(randn * 0.3), As, Bs ~ U(0.5, 1)), bf16 out as it requests: every
    row against torch's fp32 dequant-matmul, a seeded sample of rows against
    the oracle. 8192x4096x8192 and 8192x8192x8192 are two and four full
    waves of 256x256 tiles."""
    print(f"gemm tuning shape M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=M + 2 * N + 3 * K, kind="harness")
    Ad, Bd, Asd, Bsd = A.to(dev), B.to(dev), As.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16)
    _full_check(out, Ad, Bd, Asd, Bsd)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(M))[:8]
    _check(out, A[rows], B, As[rows], Bs, rows=rows)


def _full_check(out, Ad, Bd, Asd, Bsd):
    """Every row against torch's fp32 dequant-matmul on the GPU."""
    M, K = Ad.shape
    N = Bd.shape[0]
    saf = Asd.repeat_interleave(128, 1)[:, :K]
    sbf = Bsd.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]
    full = (Ad.float() * saf) @ (Bd.float() * sbf).T
    if out.dtype != torch.float32:
        full = full.to(out.dtype)
    torch.testing.assert_close(out.float(), full.float(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 512), (4096, 4096, 1024), (4000, 4200, 1536),
                                   (4096, 4352, 2560), (3001, 5000, 2048),
                                   (4096, 4096, 384), (4096, 4096, 1152), (3001, 4096, 8192)])
def test_gemm_large_tile_kernels(M, N, K, dev):
    """Grids of at least one 256x256 tile per CU: the pipelined kernel (K-block
    counts that are multiples of 4; windows of 8 K-blocks, full and half) and
    K-block counts 3 and 9 (scale windows by 4-byte lanes), with ragged M
    and N edges; 3001x4096x8192 is a partial wave of 256x256 tiles
    (192 tiles, chosen over three waves of 128x128 tiles for long K). Every row against torch's fp32 dequant-matmul, a
    sample of rows against the oracle."""
    print(f"gemm large-tile M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=K + M)
    Ad, Bd, Asd, Bsd = A.to(dev), B.to(dev), As.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16)
    _full_check(out, Ad, Bd, Asd, Bsd)
    rows = torch.cat([torch.tensor([0, M - 1]),
                      torch.randperm(M, generator=torch.Generator().manual_seed(2))[:4]])
    ref = oracle.block_gemm(_u8(A[rows]), _u8(B), As[rows].numpy(), Bs.numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 4096), (1000, 3000, 3072), (130, 4096, 14336),
                                   (3001, 4096, 14336), (200, 640, 1536)])
def test_gemm_mid_tile_kernels(M, N, K, dev):
    """Grids below one 256x256 tile per CU: 128x128 tiles with and without
    split-K (split sizes rounded to whole half-windows of 4 K-blocks),
    ragged M and N. Every row against torch's fp32 dequant-matmul, a sample
    of rows against the oracle."""
    print(f"gemm mid-tile M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=K + N)
    Ad, Bd, Asd, Bsd = A.to(dev), B.to(dev), As.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(Ad, Bd, Asd, Bsd, [128, 128], torch.bfloat16)
    _full_check(out, Ad, Bd, Asd, Bsd)
    rows = torch.tensor([0, M // 2, M - 1])
    ref = oracle.block_gemm(_u8(A[rows]), _u8(B), As[rows].numpy(), Bs.numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


def test_gemm_large_tile_exact_and_fp32(dev):
    """Pipelined kernel with small-integer operands and unit scales (exact
    result), fp32 output; and with column-major As (4-byte window lanes)."""
    print("gemm large-tile exact", flush=True)
    g = torch.Generator().manual_seed(5)
    M, N, K = 4096, 4096, 512
    A = torch.randint(-4, 5, (M, K), generator=g).float().to(torch.float8_e4m3fn).to(dev)
    B = torch.randint(-4, 5, (N, K), generator=g).float().to(torch.float8_e4m3fn).to(dev)
    As = torch.ones(M, K // 128, device=dev)
    Bs = torch.ones(N // 128, K // 128, device=dev)
    out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.float32)
    exact = A.double() @ B.double().T
    assert torch.equal(out.double(), exact)
    A2, B2, As2, Bs2 = [t.to(dev) for t in _operands(M, N, 1024, seed=9)]
    As2_t = As2.T.contiguous().T
    out2 = fp8.w8a8_block_fp8_matmul(A2, B2, As2_t, Bs2, [128, 128], torch.float32)
    _full_check(out2, A2, B2, As2, Bs2)


# Grids of the pipelined kernels whose scale windows take 4-byte DMA lanes:
# K-block counts (and split sizes) that are not multiples of 4 (K = 11008:
# LLaMA-2's intermediate size; 1152, 1408), for block scales and per-row
# weight scales, with the tails of partial waves.
WIN4_CASES = [
    (4096, 4096, 1408, 128, "gemm_pipe256_kernel"),
    (4224, 4096, 1152, 128, "gemm_pipe256_kernel"),      # + 128x128 quarters
    (4096, 6144, 1408, 128, "gemm_pipe256_kernel"),      # + 256x128 halves
    (3001, 4096, 1408, 128, "gemm_pipe192_kernel"),
    (2048, 4096, 1408, 128, "gemm_pipe256x128_kernel"),
    (2048, 2048, 1408, 128, "gemm_pipe128_kernel"),
    (512, 4096, 11008, 128, "gemm_pipe128_kernel"),      # 2 splits of 43 K-blocks
    (128, 4096, 11008, 128, "gemm_pipe128_kernel"),      # 8 splits of 11
    (4096, 4096, 1408, 1, "gemm_pipe256_kernel"),
    (4224, 4096, 1152, 1, "gemm_pipe256_kernel"),
    (2048, 4096, 1408, 1, "gemm_pipe256x128_kernel"),
    (512, 4096, 11008, 1, "gemm_pipe256x128_kernel"),    # 4 splits of 22
    (2048, 2048, 1408, 1, "gemm_pipe128_kernel"),
    (128, 4096, 11008, 1, "gemm_pipe128_kernel"),
]


@pytest.mark.parametrize("M,N,K,block_n,kernel", WIN4_CASES)
def test_gemm_pipelined_any_k_block_count(M, N, K, block_n, kernel, dev):
    """The pipelined kernels with K-block counts or split sizes that are not
    multiples of 4 (scale windows by 4-byte lanes): every row against
    torch's fp32 dequant-matmul, a sample of rows against the oracle."""
    from hf_kernels_helion_amd import _native
    print(f"gemm any-KB M={M} N={N} K={K} block_n={block_n}", flush=True)
    plan = _native.gemm_plan(M, N, K, block_n=block_n)
    if plan["cu_count"] == 256:
        assert plan["kernel"] == kernel, plan
    x = synthetic.activations(M, K, seed=M + K)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + K, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], torch.bfloat16)
    saf = s.repeat_interleave(128, 1)[:, :K]
    sbf = (Bs if block_n == 1 else Bs.repeat_interleave(128, 0)[:N]).repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor([0, M // 2, M - 1])
    ref = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy(), (block_n, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K,block_n", [(4096, 4096, 1024, 128), (2048, 2048, 2048, 128),
                                           (3001, 4096, 1024, 128), (512, 4096, 8192, 128),
                                           (4096, 4096, 1024, 1), (2048, 4096, 2048, 1),
                                           (4096, 4096, 1408, 128)])
def test_gemm_scale_layouts_same_bits(M, N, K, block_n, dev):
    """Scales that are not K-contiguous 16-byte aligned rows (column-major,
    or rows padded to an odd stride) take the 4-byte window lanes on the same
    plan: the result bits equal those of contiguous scales."""
    print(f"gemm scale layouts M={M} N={N} K={K} block_n={block_n}", flush=True)
    x = synthetic.activations(M, K, seed=3 * M + K)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 2 * K, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    ref = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], torch.bfloat16)
    KB = s.shape[1]
    s_cm = s.T.contiguous().T                                   # column-major As
    s_pad = torch.zeros(M, KB + 1, device=dev)[:, :KB].copy_(s)  # row stride KB + 1
    Bs_cm = Bs.T.contiguous().T
    for As_, Bs_ in ((s_cm, Bs), (s_pad, Bs), (s, Bs_cm), (s_cm, Bs_cm)):
        out = fp8.w8a8_block_fp8_matmul(q, W, As_, Bs_, [block_n, 128], torch.bfloat16)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def _random_layout_cases(n, seed):
    """Random shapes on the pipelined grids (M 129..4096, N 129..8192, any
    K-block count 1..96), block or per-row weight scales, and a random scale
    layout: contiguous, column-major, or rows padded to an odd stride."""
    g = torch.Generator().manual_seed(seed)
    cases = []
    for i in range(n):
        M = int(torch.randint(129, 4097, (1,), generator=g))
        N = int(torch.randint(129, 8193, (1,), generator=g))
        KB = int(torch.randint(1, 97, (1,), generator=g))
        block_n = 1 if i % 3 == 0 else 128
        layout = ["contiguous", "colmajor", "padded"][i % 3 if block_n == 128 else (i // 3) % 3]
        cases.append((M, N, 128 * KB, block_n, layout))
    return cases


@pytest.mark.parametrize("M,N,K,block_n,layout", _random_layout_cases(18, 31))
def test_gemm_random_shapes_and_scale_layouts(M, N, K, block_n, layout, dev):
    """Every element against torch's fp32 dequant-matmul, within the
    north-star tolerance, for random shapes with any K-block count and
    scales in any of three layouts."""
    print(f"gemm random layout M={M} N={N} K={K} block_n={block_n} {layout}", flush=True)
    x = synthetic.activations(M, K, seed=M + 3 * N + K)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + K, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)

    def lay(t):
        if layout == "colmajor":
            return t.T.contiguous().T
        if layout == "padded":
            return torch.zeros(t.shape[0], t.shape[1] + 1, device=dev)[:, :t.shape[1]].copy_(t)
        return t
    out = fp8.w8a8_block_fp8_matmul(q, W, lay(s), lay(Bs), [block_n, 128], torch.bfloat16)
    saf = s.repeat_interleave(128, 1)[:, :K]
    sbf = (Bs if block_n == 1 else Bs.repeat_interleave(128, 0)[:N]).repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)


def test_gemm_golden_fixture(dev):
    """Float64 golden output; the fp8 MFMA sums a 128-long K-block with less
    than fp32 precision (measured ~2^-15 relative to the block's dot), so the
    bound is 1e-4 absolute on outputs of magnitude ~1."""
    import pathlib
    z = np.load(pathlib.Path(__file__).parent / "golden" / "gemm_fp64_small.npz")
    A = torch.from_numpy(z["A"]).view(torch.float8_e4m3fn)
    B = torch.from_numpy(z["B"]).view(torch.float8_e4m3fn)
    As, Bs = torch.from_numpy(z["As"]), torch.from_numpy(z["Bs"])
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev),
                                    z["block"].tolist(), torch.float32)
    np.testing.assert_allclose(out.cpu().numpy(), z["C"], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 1024), (512, 512, 2048), (32, 4096, 14336),
                                   (32, 4096, 4096), (3001, 4096, 4096), (2048, 2048, 4096)])
def test_gemm_power_of_two_row_scaling(M, N, K, dev):
    """Scaling the activation scales of one row by 2^k scales that fp32
    output row by exactly 2^k and leaves every other row bit-identical, on
    each kernel family (256x256 pipelined, small-grid 32x32 and 32x16 tiles,
    split-K decode, partial-wave 256x256, 128x128 pipelined)."""
    print(f"gemm 2^k row scaling M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = [t.to(dev) for t in _operands(M, N, K, seed=7 + M, kind="harness")]
    out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.float32)
    rows = torch.tensor([0, M // 3, M - 1], device=dev)
    As2 = As.clone()
    As2[rows] *= 8.0
    out2 = fp8.w8a8_block_fp8_matmul(A, B, As2, Bs, [128, 128], torch.float32)
    assert torch.equal(out2[rows], out[rows] * 8.0)
    keep = torch.ones(M, dtype=torch.bool, device=dev)
    keep[rows] = False
    assert torch.equal(out2[keep], out[keep])


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 1024), (300, 640, 2048), (32, 4096, 14336)])
def test_gemm_k_block_permutation(M, N, K, dev):
    """Permuting the K-blocks of A and B together with their scale columns
    changes only the order of the fp32 sums: the result stays within the
    tolerance of the unpermuted one."""
    print(f"gemm K-block permutation M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = [t.to(dev) for t in _operands(M, N, K, seed=11 + M)]
    KB = K // 128
    perm = torch.randperm(KB, generator=torch.Generator().manual_seed(KB)).to(dev)
    cols = (perm[:, None] * 128 + torch.arange(128, device=dev)[None, :]).reshape(-1)
    Ap = A.view(torch.uint8)[:, cols].contiguous().view(torch.float8_e4m3fn)
    Bp = B.view(torch.uint8)[:, cols].contiguous().view(torch.float8_e4m3fn)
    out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
    outp = fp8.w8a8_block_fp8_matmul(Ap, Bp, As[:, perm].contiguous(), Bs[:, perm].contiguous(),
                                     [128, 128], torch.bfloat16)
    torch.testing.assert_close(outp.float(), out.float(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(1, 1, 128), (5, 15, 384), (70, 1, 1024), (33, 17, 14336)])
def test_gemm_tiny_n(M, N, K, dev):
    """Weight row counts below one 16-row fragment (rows past N clamped on
    load, masked on store) on the skinny, decode and tiled paths."""
    print(f"gemm tiny N M={M} N={N} K={K}", flush=True)
    A, B, As, Bs = _operands(M, N, K, seed=M * 7 + N)
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128],
                                    torch.bfloat16)
    assert out.shape == (M, N)
    _check(out, A, B, As, Bs)


def test_gemm_zero_k_gives_zeros(dev):
    """K = 0: the reference kernel's accumulator starts at zero and no
    K-block is added (fp8.py:29-38), so the output is all zeros."""
    A = torch.empty(4, 0, dtype=torch.float8_e4m3fn, device=dev)
    B = torch.empty(8, 0, dtype=torch.float8_e4m3fn, device=dev)
    out = fp8.w8a8_block_fp8_matmul(A, B, torch.empty(4, 0, device=dev),
                                    torch.empty(1, 0, device=dev), [128, 128], torch.float32)
    assert out.shape == (4, 8) and torch.equal(out, torch.zeros_like(out))


def test_gemm_skinny_staged_row_groups_bit_equal(dev):
    """The skinny kernel stages ceil(M/8) groups of 8 activation rows per
    K-block (1..6 for M up to 48); the lanes past them read a staged row and
    their outputs are not stored. Its K ranges, fold and wave-order sum do
    not depend on M, so every row of the 48-row call must equal, bit for
    bit, the same row computed by calls on 1, 8, 9, 16, 17, 24, 25, 32, 33,
    40 and 41 rows (each staged row-group count, at its edges), and the
    48-row call matches the oracle on sampled rows."""
    from hf_kernels_helion_amd import _native
    N, K = 2048, 8192
    print(f"gemm skinny row groups N={N} K={K}", flush=True)
    x = synthetic.activations(48, K, seed=48, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + K)
    W, Bs = W.to(dev), Bs.to(dev)
    full = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    for M in (1, 8, 9, 16, 17, 24, 25, 32, 33, 40, 41, 48):
        assert _native.gemm_plan(M, N, K)["kernel"] == "gemm_skinny_kernel", M
        r0 = 48 - M  # the last M rows, so each call's rows start at a different row
        part = fp8.w8a8_block_fp8_matmul(q[r0:], W, s[r0:], Bs, [128, 128], torch.bfloat16)
        torch.testing.assert_close(part, full[r0:], rtol=0, atol=0)
    rows = torch.tensor([0, 7, 8, 23, 40, 47])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(full[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K,block_n", [(3001, 28672, 4096, 128), (4224, 4096, 1024, 128),
                                           (4096, 4224, 1024, 128), (4100, 4096, 2048, 128),
                                           (4224, 4096, 1024, 1)])
def test_gemm_partial_last_wave_on_128_tiles(M, N, K, block_n, dev):
    """Grids of 256x256 tiles that leave a last partial wave of at most a
    quarter of the CUs run it as 128x128 quarters on the 128x128 kernel. The
    per-output arithmetic of every unsplit MFMA plan is the same (one MFMA per
    K-block, folded as acc + dot * (As * Bs) in K order), so the result must
    equal, bit for bit, the same rows computed by separate calls on row
    slices (the last one ending at row M) whose grids have no split-K and
    no tail run on other kernels. Covers the MLP gate/up shape (1344
    tiles), quarters past the M or N edge (4224 = 16.5 tiles), a ragged last
    row of tiles, and per-row weight scales."""
    from hf_kernels_helion_amd import _native
    print(f"gemm 128x128 tail M={M} N={N} K={K} block_n={block_n}", flush=True)
    x = synthetic.activations(M, K, seed=M + N)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], torch.bfloat16)
    lib = _native.load()
    # slices whose 128x128 grids end in whole waves or in a last wave too
    # large for 64x64 quarters (4224 columns: 1280 rows, 330 tiles)
    h = 1280 if N == 4224 else 1024
    slices = [(r0, r0 + h) for r0 in range(0, M - h, h)] + [(M - h, M)]
    for r0, r1 in slices:
        assert lib.fp8b_gemm_workspace_size(r1 - r0, N, K, block_n, 128) == 0
        part = fp8.w8a8_block_fp8_matmul(q[r0:r1], W, s[r0:r1], Bs, [block_n, 128],
                                         torch.bfloat16)
        torch.testing.assert_close(out[r0:r1], part, rtol=0, atol=0)
    rows = torch.tensor([0, M // 2, M - 1])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy(), (block_n, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(64, 4096, 14336), (64, 57344, 2048), (56, 14336, 14336),
                                   (64, 28672, 4096), (50, 2048, 14336), (64, 8192, 8192),
                                   (50, 6144, 8192)])
def test_gemm_49_to_64_rows_past_small_grids(M, N, K, dev):
    """49..64 rows beyond the small-grid rules: the decode kernel with 64
    activation rows, split along K over the CUs (16, 32, 48, 64 or 112
    column tiles), unsplit (224 column tiles), or two workgroups per CU (448);
    64 x 8192 x 8192 and 50 x 6144 x 8192 would fit the small-grid kernel but
    stream faster here. Every element against torch's
    fp32 dequant-matmul, sampled rows against the oracle; unit-scale small
    integers give the exact product."""
    print(f"gemm 49..64 rows M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 5)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (
        W.float() * Bs.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor([0, M // 2, M - 1])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    g = torch.Generator().manual_seed(M * N)
    Ai = torch.randint(-3, 4, (M, K), generator=g).float().to(torch.float8_e4m3fn)
    Bi = torch.randint(-3, 4, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    outi = fp8.w8a8_block_fp8_matmul(Ai.to(dev), Bi.to(dev),
                                     torch.ones(M, K // 128, device=dev),
                                     torch.ones((N + 127) // 128, K // 128, device=dev),
                                     [128, 128])
    assert torch.equal(outi.cpu().double(), Ai.double() @ Bi.double().T)


@pytest.mark.parametrize("M,N,K,block_n", [(2048, 2560, 4096, 128), (1950, 2560, 2048, 128),
                                           (1024, 5120, 1024, 128), (2048, 2560, 2048, 1)])
def test_gemm_128_tiles_last_wave_as_64_quarters(M, N, K, block_n, dev):
    """Grids of 128x128 tiles (one per CU per wave) that leave at most a
    quarter of the CUs for a last wave run that wave's tiles as 64x64
    quarters on the small-grid kernel (320 tiles: 256 + 64 as 256 quarters):
    every element against torch's fp32 dequant-matmul, sampled rows against
    the oracle; 1950 rows leaves quarters wholly past the M edge (skipped by
    their workgroups); per-row weight scales too. Exact small-integer
    operands give the exact product."""
    from hf_kernels_helion_amd import _native
    print(f"gemm 128x128 tiles, 64x64 last wave M={M} N={N} K={K} block_n={block_n}",
          flush=True)
    assert _native.load().fp8b_gemm_workspace_size(M, N, K, block_n, 128) == 0
    x = synthetic.activations(M, K, seed=M + 3 * N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 11, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], torch.bfloat16)
    full = (q.float() * s.repeat_interleave(128, 1)) @ (
        W.float() * Bs.repeat_interleave(block_n, 0)[:N].repeat_interleave(128, 1)[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    rows = torch.tensor([0, 1023, M // 2, M - 1])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy(), (block_n, 128))
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    g = torch.Generator().manual_seed(M + N)
    Ai = torch.randint(-3, 4, (M, K), generator=g).float().to(torch.float8_e4m3fn)
    Bi = torch.randint(-3, 4, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    Asi = torch.exp2(torch.randint(-2, 3, (M, K // 128), generator=g).float())
    Bsi = torch.exp2(torch.randint(-2, 3, ((N + block_n - 1) // block_n, K // 128),
                                   generator=g).float())
    outi = fp8.w8a8_block_fp8_matmul(Ai.to(dev), Bi.to(dev), Asi.to(dev), Bsi.to(dev),
                                     [block_n, 128])
    exact = (Ai.double() * Asi.double().repeat_interleave(128, 1)) @ (
        Bi.double() * Bsi.double().repeat_interleave(block_n, 0)[:N].repeat_interleave(
            128, 1)).T
    assert torch.equal(outi.cpu().double(), exact)


@pytest.mark.parametrize("M,N,K", [(3001, 4096, 14336), (1500, 8192, 4096), (3001, 8192, 1024),
                                   (1500, 8064, 1024), (1536, 6144, 2048), (1536, 7168, 1024)])
def test_gemm_192_row_tiles_equal_other_plans(M, N, K, dev):
    """Grids whose 256x256 tiles leave a partial last wave too large for
    128x128 quarters while 192x256 tiles fill whole waves (3001 x 4096: 256
    tiles against 192; 1500 x 8192: 256 against 192; 3001 x 8192: 512
    against 384; 1500 x 8064: half a tile column past N), or one partial
    wave of 256x256 tiles that 192x256 tiles still hold in one wave (1536 x
    6144: 192 against 144; 1536 x 7168: 224 against 168) run
    gemm_pipe192_kernel, ragged last tile row included. Per output its
    arithmetic is that of every unsplit MFMA plan, so row slices of 1024 or
    1280 (which run the 128x128 or 256x128 kernels unsplit) give the same
    bits; sampled rows against the oracle. (The gate/up GEMM with the SiLU epilogue on 192-row
    tiles is checked against the plain GEMM in test_gpu_mlp.py.)"""
    from hf_kernels_helion_amd import _native
    print(f"gemm 192-row tiles M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 2 * N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 3)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    lib = _native.load()
    # row slices of a height whose plan is unsplit (1024 rows of a long-K
    # grid split along K on 256x128 tiles)
    h = next(h for h in (1024, 1280, 1536) if lib.fp8b_gemm_workspace_size(h, N, K, 128, 128) == 0)
    slices = [(r0, r0 + h) for r0 in range(0, M - h, h)] + [(M - h, M)]
    for r0, r1 in slices:
        part = fp8.w8a8_block_fp8_matmul(q[r0:r1], W, s[r0:r1], Bs, [128, 128], torch.bfloat16)
        torch.testing.assert_close(out[r0:r1], part, rtol=0, atol=0)
    rows = torch.tensor([0, 191, 192, M // 2, M - 1])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    # fp32 output through the same kernel's fp32 epilogue
    out32 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.float32)
    assert torch.equal(out32.to(torch.bfloat16), out)


def _tiles(M, N, bm, bn):
    return -(-M // bm) * -(-N // bn)


def _is_256x128_grid(M, N, cus):
    """The planner's rule for 256x128 tiles: they fit one wave of workgroups
    while 128x128 tiles would need more than one."""
    return _tiles(M, N, 128, 128) > cus >= _tiles(M, N, 256, 128)


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (1000, 6144, 2048), (768, 7000, 1024),
                                   (256, 28672, 1024), (1537, 4096, 1024), (4096, 2048, 7168)])
def test_gemm_256x128_tiles(M, N, K, dev):
    """Grids whose 256x128 tiles fit one wave of workgroups while 128x128
    tiles need two or more run gemm_pipe256x128_kernel (ragged last tile row
    and column, a last tile row of one row): sampled rows against the oracle,
    and bit for bit against row slices that run the unsplit 128x128 plan
    (every unsplit MFMA plan folds the same products in the same K order);
    fp32 and fp16 outputs through the kernel's other epilogues."""
    from hf_kernels_helion_amd import _native
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if not _is_256x128_grid(M, N, cus):
        pytest.skip(f"{M}x{N} is not a 256x128 grid on {cus} CUs")
    print(f"gemm 256x128 tiles M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 5 * N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 7)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    lib = _native.load()
    # slices of whole 128-row tiles filling between half a wave and one wave
    # of 128x128 tiles: neither split nor another tiling
    h = 128 * (cus // -(-N // 128))
    assert h < M and _tiles(h, N, 128, 128) * 2 > cus
    slices = [(r0, r0 + h) for r0 in range(0, M - h, h)] + [(M - h, M)]
    for r0, r1 in slices:
        assert lib.fp8b_gemm_workspace_size(r1 - r0, N, K, 128, 128) == 0
        part = fp8.w8a8_block_fp8_matmul(q[r0:r1], W, s[r0:r1], Bs, [128, 128], torch.bfloat16)
        torch.testing.assert_close(out[r0:r1], part, rtol=0, atol=0)
    rows = torch.tensor(sorted({r for r in (0, 255, 256, M // 2, M - 1) if r < M}))
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    out32 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.float32)
    assert torch.equal(out32.to(torch.bfloat16), out)
    out16 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.float16)
    assert torch.equal(out32.to(torch.float16), out16)


@pytest.mark.parametrize("M,N,K", [(4096, 6144, 1024), (1500, 13900, 512), (768, 28672, 512)])
def test_gemm_256_tiles_last_wave_as_halves(M, N, K, dev):
    """Unsplit 256x256 grids whose last partial wave holds more than a
    quarter and at most half of the CUs (4096 x 6144: 384 tiles, 128 left;
    1500 x 13900: 330, 74 left, the last tile column 76 wide so its second
    half lies past N; 768 x 28672: 336, 80 left) run that wave as 256x128
    halves on gemm_pipe256x128_kernel: every element against torch's fp32
    dequant-matmul, and bit for bit against row slices of 512 (other unsplit
    plans)."""
    from hf_kernels_helion_amd import _native
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    t, rest = _tiles(M, N, 256, 256), _tiles(M, N, 256, 256) % cus
    if not (t >= cus and 4 * rest > cus and 2 * rest <= cus):
        pytest.skip(f"{M}x{N} leaves no half-sized last wave on {cus} CUs")
    print(f"gemm 256 tiles, last wave as halves M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 3 * N)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 9)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    saf = s.repeat_interleave(128, 1)
    sbf = Bs.repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)
    lib = _native.load()
    for r0 in range(0, M, 512):
        r1 = min(r0 + 512, M)
        assert lib.fp8b_gemm_workspace_size(r1 - r0, N, K, 128, 128) == 0
        part = fp8.w8a8_block_fp8_matmul(q[r0:r1], W, s[r0:r1], Bs, [128, 128], torch.bfloat16)
        assert torch.equal(out[r0:r1], part)


@pytest.mark.parametrize("M,N,K,block_n,splits", [(512, 4096, 14336, 128, 4),
                                                  (768, 2000, 14336, 128, 4),
                                                  (1024, 1536, 28672, 128, 4),
                                                  (512, 4096, 14336, 1, 4),
                                                  (1024, 3072, 14336, 128, 2),
                                                  (2048, 2048, 14336, 1, 2)])
def test_gemm_256x128_split_k(M, N, K, block_n, splits, dev):
    """Long-K grids the planner gives 256x128 tiles split along K (a ragged
    last tile column; per-row weight scales): every element against torch's
    fp32 dequant-matmul. The plan is asserted through the plan query on a
    256-CU device."""
    from hf_kernels_helion_amd import _native
    print(f"gemm 256x128 split-K M={M} N={N} K={K} block_n={block_n}", flush=True)
    plan = _native.gemm_plan(M, N, K, block_n)
    if plan["cu_count"] == 256:
        assert (plan["kernel"], plan["splits"]) == ("gemm_pipe256x128_kernel", splits), plan
    assert _native.load().fp8b_gemm_workspace_size(M, N, K, block_n, 128) > 0
    x = synthetic.activations(M, K, seed=M + N)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 5, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], torch.bfloat16)
    saf = s.repeat_interleave(128, 1)
    sbf = (Bs if block_n == 1 else Bs.repeat_interleave(128, 0)[:N]).repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf).T
    torch.testing.assert_close(out.float(), full.to(torch.bfloat16).float(), rtol=RTOL,
                               atol=ATOL)


def test_gemm_256x128_tiles_exact_integers(dev):
    """gemm_pipe256x128_kernel on small-integer operands with power-of-two
    scales per activation row and weight block (every product and partial
    sum exact in fp32): the whole fp32 output equals the float64 product,
    ragged last tile row and column included."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    M, N, K = 1800, 4000, 1024
    if not _is_256x128_grid(M, N, cus):
        pytest.skip(f"{M}x{N} is not a 256x128 grid on {cus} CUs")
    print(f"gemm 256x128 exact M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(17)
    A = torch.randint(-4, 5, (M, K), generator=g).float().to(torch.float8_e4m3fn)
    B = torch.randint(-4, 5, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    As = torch.exp2(torch.randint(-2, 3, (M, K // 128), generator=g).float())
    Bs = torch.exp2(torch.randint(-2, 3, ((N + 127) // 128, K // 128), generator=g).float())
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128],
                                    torch.float32)
    exact = (A.double() * As.double().repeat_interleave(128, 1)) @ (
        B.double() * Bs.double().repeat_interleave(128, 0)[:N].repeat_interleave(128, 1)).T
    assert torch.equal(out.cpu().double(), exact)


# Small-grid shapes and the waves per 32x32 tile gemm_tiny_kernel runs them
# with on a 256-CU MI355X (8: at most one tile per CU; 4: 2.5; 2: four; 1:
# up to eight), ragged edges, one K-block (seven of eight waves idle), a
# long K, 49..64 rows, decode-sized M (1, 17, 24, 32), the 64x64-tile band
# (two waves per tile for 1024 x 2048, four for 960 x 1024) and 32x16 tiles
# (decode shapes with N = 4096). Up to 16 rows with block scales the kernel
# computes only the first 16 rows of each 32-row tile (1, 3, 5, 8, 12, 13,
# 16 rows here, with 8, 4 and 2 waves per tile and 32x16 tiles).
SMALL_GRIDS = [(512, 512, 2048), (500, 300, 1024), (65, 96, 4096), (100, 2000, 7168),
               (256, 1024, 128), (512, 1024, 2048), (1024, 512, 7168), (768, 768, 4096),
               (2048, 1024, 2048), (1000, 2000, 1024), (64, 4096, 4096), (49, 500, 2048),
               (56, 14336, 4096), (32, 14336, 4096), (1, 8192, 4096), (24, 4096, 4096),
               (17, 8192, 1024), (1024, 2048, 4096), (960, 1024, 4096), (1000, 1800, 2048),
               (32, 4096, 7168), (12, 4096, 4096), (16, 4096, 7168), (1, 28672, 4096),
               (8, 14336, 4096), (5, 8200, 512), (3, 8704, 1024), (13, 8192, 2048)]


def _one_wave_per_tile(M, N, K):
    """Whether the planner (256 CUs) runs this small grid with one wave per
    tile: 32x32 tiles, more than four per CU, and not the 64x64 band."""
    t64 = -(-M // 64) * -(-N // 64)
    kb = K // 128
    band64 = M > 64 and 16 <= kb <= 64 and (
        (t64 == 512 and kb <= 32) or (256 < t64 < 512 and 24 <= kb <= 48 and N <= 16 * M) or (224 <= t64 <= 256 and (kb <= 32 or N <= 16 * M)))
    return not band64 and -(-M // 32) * -(-N // 32) > 4 * 256


@pytest.mark.parametrize("M,N,K", SMALL_GRIDS)
def test_gemm_small_grid_tiles(M, N, K, dev):
    """Grids of at most eight 32x32 tiles per CU (512 x 512 and the like) run
    gemm_tiny_kernel: one workgroup per 32x32 tile whose waves split K and
    sum their partial tiles in wave order, no workspace. Sampled rows
    against the oracle; the same bits on a second call, with column-major
    activation scales and through the fp32 epilogue. With one wave per tile
    (eight tiles per CU) the arithmetic is that of every unsplit plan, so
    the same rows inside a 32768-row grid give the same bits."""
    from hf_kernels_helion_amd import _native
    print(f"gemm small-grid tiles M={M} N={N} K={K}", flush=True)
    lib = _native.load()
    assert lib.fp8b_gemm_workspace_size(M, N, K, 128, 128) == 0
    x = synthetic.activations(M, K, seed=M + 5 * N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 7)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    rows = torch.tensor(sorted({r for r in (0, 31, 32, M // 2, M - 1) if r < M}))
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(out[rows.to(dev)].float().cpu(),
                               torch.from_numpy(orc).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)
    again = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    assert torch.equal(again, out)
    s_cm = torch.empty_strided(s.shape, (1, M), dtype=s.dtype, device=dev).copy_(s)
    out_cm = fp8.w8a8_block_fp8_matmul(q, W, s_cm, Bs, [128, 128], torch.bfloat16)
    assert torch.equal(out_cm, out)
    out32 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.float32)
    assert torch.equal(out32.to(torch.bfloat16), out)
    if _one_wave_per_tile(M, N, K):
        big = 32768
        reps = (big + M - 1) // M
        qb = q.repeat(reps, 1)[:big].contiguous()
        sb = s.repeat(reps, 1)[:big].contiguous()
        assert lib.fp8b_gemm_workspace_size(big, N, K, 128, 128) == 0
        ref = fp8.w8a8_block_fp8_matmul(qb, W, sb, Bs, [128, 128], torch.bfloat16)
        assert torch.equal(out, ref[:M])


@pytest.mark.parametrize("M,N,K", [(1024, 512, 7168), (512, 512, 2048), (768, 768, 4096),
                                   (1024, 2048, 4096), (960, 1024, 4096), (32, 14336, 4096)])
def test_gemm_small_grid_repeatable(M, N, K, dev):
    """The small-grid kernel refills each wave's LDS slots without a barrier,
    so a refill issued before that wave's reads of the slot complete would
    race them. Sixteen calls, alternating row- and column-major activation
    scales (different DMA timing), must give the same bits."""
    print(f"gemm small-grid repeatable M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 5 * N, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 7)
    W, Bs = W.to(dev), Bs.to(dev)
    s_cm = torch.empty_strided(s.shape, (1, M), dtype=s.dtype, device=dev).copy_(s)
    first = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    for i in range(16):
        out = fp8.w8a8_block_fp8_matmul(q, W, s_cm if i % 2 == 0 else s, Bs, [128, 128],
                                        torch.bfloat16)
        assert torch.equal(out, first), f"call {i}"


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (256, 1024, 128), (512, 1024, 2048),
                                   (768, 768, 4096), (2048, 1024, 1024), (1024, 2048, 2048),
                                   (1024, 1024, 4096), (32, 4096, 4096), (16, 4096, 7168),
                                   (1, 28672, 4096), (8, 14336, 512), (13, 8192, 2048)])
def test_gemm_small_grid_exact_integers(M, N, K, dev):
    """Small-integer fp8 operands and power-of-two scales: every MFMA dot,
    fold and sum of partial tiles is exact, so each small-grid configuration
    (8, 4, 2 and 1 waves per 32x32 tile; 2 and 4 per 64x64 tile; 8 per
    32x16 tile; the 16-row form of a 32-row tile) must give the exact
    product bit for bit."""
    print(f"gemm small-grid exact M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randint(-3, 4, (M, K), generator=g).float().to(torch.float8_e4m3fn)
    B = torch.randint(-3, 4, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    As = torch.exp2(torch.randint(-2, 3, (M, K // 128), generator=g).float())
    Bs = torch.exp2(torch.randint(-2, 3, (N // 128, K // 128), generator=g).float())
    out = fp8.w8a8_block_fp8_matmul(A.to(dev), B.to(dev), As.to(dev), Bs.to(dev), [128, 128])
    Ad = A.double() * As.double().repeat_interleave(128, 1)
    Bd = B.double() * Bs.double().repeat_interleave(128, 0).repeat_interleave(128, 1)
    exact = Ad @ Bd.T
    assert exact.abs().max() < 2 ** 20
    assert torch.equal(out.cpu().double(), exact)


def _one_hot_rows(N, K, dev):
    """B [N,K] e4m3fn with row n = 1.0 at k < 8(n+1) and 0 elsewhere, so that
    with A = 1.0 and unit scales C[m,n] = 8(n+1) exactly."""
    k = torch.arange(K, device=dev)
    n = torch.arange(N, device=dev)
    return (k[None, :] < 8 * (n[:, None] + 1)).to(torch.float8_e4m3fn)


@pytest.mark.parametrize("block_n", [128, 1])
def test_gemm_decode_leading_dim_past_32bit_offsets(block_n, dev):
    """Decode-sized M (16 rows) against weight rows 34e6 bytes apart: the
    decode kernel's 32-bit DMA offsets (row * ldb, rows up to 127) would wrap
    past 2^32, so the plan falls back to kernels with 64-bit addressing
    (skinny for 128x128 blocks, generic for per-row scales). Closed-form
    result: A = 1.0, unit scales and one-hot-prefix weight rows give
    C[m,n] = 8(n+1). block_n = 128 needs K = 139264 (1088 K-blocks) for the
    decode plan's split size to exceed four K-blocks at N = 128."""
    M, N = 16, 128
    K = 139264 if block_n == 128 else 1024
    ldb = 34_000_000
    assert 127 * ldb + K > 2 ** 32 and ldb % 16 == 0
    print(f"gemm decode ldb={ldb} K={K} block_n={block_n}", flush=True)
    buf = torch.zeros((N - 1) * ldb + K, dtype=torch.uint8, device=dev)
    B = buf.view(torch.float8_e4m3fn).as_strided((N, K), (ldb, 1))
    B.copy_(_one_hot_rows(N, K, dev))
    A = torch.ones(M, K, device=dev).to(torch.float8_e4m3fn)
    KB = K // 128
    As = torch.ones(M, KB, device=dev)
    Bs = torch.ones(N if block_n == 1 else 1, KB, device=dev)
    out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [block_n, 128], torch.float32)
    expect = (8.0 * (torch.arange(N, device=dev) + 1)).expand(M, N)
    assert torch.equal(out, expect), (out[0, :8], expect[0, :8])
    del buf


def test_gemm_expanded_and_transposed_operands(dev):
    """Operands whose rows overlap (an expanded row, stride 0) or whose K
    stride is not 1 are copied to rows before the launch: the result equals
    the contiguous operands' bit for bit."""
    M, N, K = 96, 384, 1024
    A, B, As, Bs = [t.to(dev) for t in _operands(M, N, K, seed=12)]
    Ae = A[:1].expand(M, K)
    ref = fp8.w8a8_block_fp8_matmul(Ae.contiguous(), B, As, Bs, [128, 128], torch.bfloat16)
    out = fp8.w8a8_block_fp8_matmul(Ae, B, As, Bs, [128, 128], torch.bfloat16)
    torch.testing.assert_close(out, ref, rtol=0, atol=0)
    Bt = B.t().contiguous().t()                     # [N,K] with strides (1, N)
    assert Bt.stride(1) != 1
    ref = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
    torch.testing.assert_close(fp8.w8a8_block_fp8_matmul(A, Bt, As, Bs, [128, 128],
                                                         torch.bfloat16), ref, rtol=0, atol=0)
    x1 = synthetic.activations(1, 2 * K, seed=3).to(dev)[:, ::2]   # one row, K stride 2
    q1, s1 = fp8.act_quant(x1, 128)
    q2, s2 = fp8.act_quant(x1.contiguous(), 128)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)


def _random_shapes(n, seed):
    g = torch.Generator().manual_seed(seed)
    shapes = []
    for _ in range(n):
        M = int(torch.randint(1, 700, (1,), generator=g))
        N = int(torch.randint(1, 2000, (1,), generator=g))
        KB = int(torch.randint(1, 33, (1,), generator=g))
        block_n = 1 if int(torch.randint(0, 4, (1,), generator=g)) == 0 else 128
        dtype = [torch.bfloat16, torch.float32, torch.float16][int(torch.randint(0, 3, (1,),
                                                                                  generator=g))]
        shapes.append((M, N, 128 * KB, block_n, dtype))
    return shapes


@pytest.mark.parametrize("M,N,K,block_n,dtype", _random_shapes(48, 2024))
def test_gemm_random_shapes(M, N, K, block_n, dtype, dev):
    """A seeded sweep over shapes (M 1-699, N 1-1999, K 128-4096), weight
    block sizes 128 and 1 (per-row) and output dtypes: the small-grid,
    skinny, split-K decode and 128x128 plans against torch's fp32
    dequant-matmul of the same operands, within the north-star tolerance."""
    print(f"gemm random M={M} N={N} K={K} block_n={block_n} {dtype}", flush=True)
    x = synthetic.activations(M, K, seed=M * 31 + N)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N * 17 + K, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], dtype)
    assert out.dtype == dtype and out.shape == (M, N)
    saf = s.repeat_interleave(128, 1)[:, :K]
    sbf = (Bs if block_n == 1 else Bs.repeat_interleave(128, 0)[:N]).repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(dtype).float(), rtol=RTOL, atol=ATOL)


def _random_shapes_large(n, seed):
    g = torch.Generator().manual_seed(seed)
    shapes = []
    for _ in range(n):
        M = int(torch.randint(1, 4097, (1,), generator=g))
        N = int(torch.randint(1, 6145, (1,), generator=g))
        KB = int(torch.randint(1, 65, (1,), generator=g))
        block_n = 1 if int(torch.randint(0, 4, (1,), generator=g)) == 0 else 128
        dtype = [torch.bfloat16, torch.float32, torch.float16][int(torch.randint(0, 3, (1,),
                                                                                  generator=g))]
        shapes.append((M, N, 128 * KB, block_n, dtype))
    return shapes


def _random_256x128_shapes(n, seed, cus=256):
    """Random grids that the planner gives 256x128 tiles on a 256-CU device
    (K a multiple of 512 for three in four: 16-byte scale windows; the rest
    take the 4-byte window lanes)."""
    g = torch.Generator().manual_seed(seed)
    shapes = []
    while len(shapes) < n:
        M = int(torch.randint(129, 4097, (1,), generator=g))
        N = int(torch.randint(129, 16385, (1,), generator=g))
        KB = int(torch.randint(1, 13, (1,), generator=g)) * (4 if len(shapes) % 4 else 1)
        dtype = [torch.bfloat16, torch.float32][len(shapes) % 2]
        if _is_256x128_grid(M, N, cus):
            shapes.append((M, N, 128 * KB, 128, dtype))
    return shapes


@pytest.mark.parametrize("M,N,K,block_n,dtype",
                         _random_shapes_large(24, 2025) + _random_256x128_shapes(8, 7))
def test_gemm_random_shapes_large(M, N, K, block_n, dtype, dev):
    """A seeded sweep over larger shapes (M up to 4096, N up to 6144, K up
    to 8192) and output dtypes: the small-grid tilings (32x16, 32x32,
    64x64), 128x128 grids with split-K or with their last wave as 64x64
    quarters, 256x128 tiles (with 16- and 4-byte scale window lanes),
    192- and 256-row tiles and their quarters, against torch's fp32 dequant-matmul of the same operands,
    within the north-star tolerance."""
    print(f"gemm random large M={M} N={N} K={K} block_n={block_n} {dtype}", flush=True)
    x = synthetic.activations(M, K, seed=M * 7 + N)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N * 13 + K, block_n=block_n)
    W, Bs = W.to(dev), Bs.to(dev)
    out = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [block_n, 128], dtype)
    assert out.dtype == dtype and out.shape == (M, N)
    saf = s.repeat_interleave(128, 1)[:, :K]
    sbf = (Bs if block_n == 1 else Bs.repeat_interleave(128, 0)[:N]).repeat_interleave(128, 1)
    full = (q.float() * saf) @ (W.float() * sbf[:, :K]).T
    torch.testing.assert_close(out.float(), full.to(dtype).float(), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (300, 1024, 16384), (2048, 2560, 4096),
                                   (32, 4096, 14336), (4096, 4096, 1024), (64, 4096, 14336),
                                   (2048, 4096, 2048), (1024, 2048, 14336), (4096, 6144, 1024)])
def test_gemm_graph_replays(M, N, K, dev):
    """The GEMM captured in a HIP graph on each plan family (small-grid
    tiles; split-K 128x128 with its sum; a 128x128 grid whose last wave runs
    as 64x64 quarters; the split-K decode kernel; 256x256 tiles; the decode
    kernel with 64 rows; 256x128 tiles, unsplit and split-K; a 256x256 grid
    whose last wave runs as 256x128 halves): every replay, with eager work
    in between, equals the eager result."""
    print(f"gemm graph M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + N + K)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 1)
    W, Bs = W.to(dev), Bs.to(dev)
    f = lambda: fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    eager = f()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        f()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K,kernel", [
    (4096, 4096, 1024, "gemm_pipe256_kernel"), (4224, 4096, 1024, "gemm_pipe256_kernel"),
    (2048, 2048, 4096, "gemm_pipe128_kernel"), (128, 4096, 11008, "gemm_pipe128_kernel"),
    (512, 4096, 14336, "gemm_pipe256x128_kernel"), (32, 4096, 14336, "gemm_decode_kernel"),
    (1000, 4100, 2048, None)])
def test_gemm_fp32_output_rounds_to_the_bf16_output(M, N, K, kernel, dev):
    """fp32 C (the public op's default dtype) leaves the tiled and decode
    kernels through the LDS-staged fp32 tile write, bf16 C through the 16-bit
    epilogue; split-K plans reduce staged fp32 partials. Both round the same
    fp32 results, so the fp32 output rounded to bf16 must equal the bf16
    output bit for bit, on each kernel (4224 rows: 128x128 quarters after the
    256x256 tiles; 4100 columns: a ragged last column tile on per-lane
    stores), and it matches the oracle on sampled rows."""
    from hf_kernels_helion_amd import _native
    if kernel is not None:
        assert _native.gemm_plan(M, N, K)["kernel"] == kernel
    print(f"gemm fp32 vs bf16 output M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + K, outlier_frac=0.01)
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=N + 2 * K)
    W, Bs = W.to(dev), Bs.to(dev)
    o32 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128])
    o16 = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
    assert o32.dtype == torch.float32
    assert torch.equal(o32.to(torch.bfloat16).view(torch.int16), o16.view(torch.int16))
    rows = torch.tensor([0, M // 2, M - 1])
    orc = oracle.block_gemm(_u8(q.cpu()[rows]), _u8(W.cpu()), s.cpu()[rows].numpy(),
                            Bs.cpu().numpy())
    torch.testing.assert_close(o32[rows.to(dev)].cpu(), torch.from_numpy(orc),
                               rtol=RTOL, atol=ATOL)
