"""GPU parity of the act-quant + GEMM op (act_quant_w8a8_block_fp8_matmul),
on each of its paths (one kernel that quantises inside the decode or the
skinny GEMM, or act-quant then the GEMM): bit for bit against the two public ops it composes
(act_quant, then w8a8_block_fp8_matmul), and against the CPU oracle chain
oracle.block_gemm(oracle.act_quant(x)) within the north-star tolerance
(1e-2 relative, 1e-3 absolute of the oracle's result rounded to the output
dtype)."""
import numpy as np
import pytest
import torch

import oracle
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _weights(N, K, seed, dev):
    W, Bs = synthetic.weights(N, K, seed=seed)
    return W.to(dev), Bs.to(dev)


def _two_op(x, W, Bs, dtype):
    q, s = fp8.act_quant(x, 128)
    return fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], dtype)


def _same(a, b):
    torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True)


def _bits(x):
    return x.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _oracle_chain(x, W, Bs, rows):
    """oracle.act_quant then oracle.block_gemm on the given rows of x."""
    q, s = oracle.act_quant(_bits(x[rows]), 128)
    return oracle.block_gemm(q, W.cpu().view(torch.uint8).numpy(), s, Bs.cpu().numpy())


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (16, 4096, 14336), (17, 1000, 1024),
                                   (32, 4096, 14336), (33, 512, 2048), (48, 640, 3072),
                                   (32, 28672, 4096), (64, 512, 1024), (100, 384, 512)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_equals_two_ops_and_oracle(M, N, K, dtype, dev):
    print(f"act-quant matmul M={M} N={N} K={K} {dtype}", flush=True)
    x = synthetic.activations(M, K, seed=M + K, outlier_frac=0.01).to(dev)
    W, Bs = _weights(N, K, N, dev)
    out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], dtype)
    assert out.dtype == dtype and out.shape == (M, N)
    _same(out, _two_op(x, W, Bs, dtype))
    rows = torch.unique(torch.tensor([0, M // 3, M // 2, M - 1]))
    cols = slice(0, min(N, 1024))
    ref = _oracle_chain(x, W[cols], Bs, rows)
    ref_t = torch.from_numpy(ref).to(dtype).float()
    torch.testing.assert_close(out[rows.to(dev), cols].float().cpu(), ref_t, rtol=RTOL,
                               atol=ATOL)


# Shapes whose plan is the one-kernel path (gemm_decode_quant_kernel) on a
# 256-CU MI355X, with the split layouts it must handle: K splits whose last
# split has one or two K-blocks (fewer than the ring's prologue stages), a
# ragged last column tile, 29 K-blocks per split (four scale windows), and
# one unsplit K range; 9..32 rows (16-row and 32-row kernels).
ONE_KERNEL = [(9, 2048, 8448), (32, 2048, 8576), (17, 4160, 7296), (9, 8192, 14464),
              (32, 4160, 5248), (24, 4096, 14336), (31, 28672, 4096), (16, 13824, 5120)]


# Shapes whose plan is the skinny one-kernel path (gemm_skinny_quant_kernel,
# M <= 8): 4- and 8-row forms, one K-block (seven of the eight waves have an
# empty K range), K-block counts the eight waves split unevenly, ragged
# 16-column tiles.
SKINNY_ONE_KERNEL = [(1, 4096, 14336), (3, 1000, 1024), (4, 4096, 4096), (5, 2048, 8192),
                     (8, 4096, 14336), (2, 520, 128), (7, 4096, 1920), (6, 3000, 640)]


# Shapes whose plan is the small-grid one-kernel path (gemm_tiny_quant_kernel,
# M <= 8, or up to 16 rows with at most 4 K-blocks per wave; 32-row tiles):
# 8, 4 and 2 waves per tile, one K-block, ragged last 32-column tiles,
# 32x16 tiles, 4-, 8- and 16-row forms.
TINY_ONE_KERNEL = [(1, 8192, 128), (3, 8704, 1024), (1, 20992, 4096), (6, 28672, 4096),
                   (8, 14336, 2048), (5, 8200, 512), (7, 9000, 640), (12, 8192, 2048),
                   (16, 4096, 4096), (13, 8200, 1024)]


def _one_kernel(M, N, K, kernel="gemm_decode_quant_kernel"):
    from hf_kernels_helion_amd import _native
    return _native.act_quant_matmul_plan(M, N, K)["kernel"] == kernel


@pytest.mark.parametrize("M,N,K,kernel",
                         [s + ("gemm_skinny_quant_kernel",) for s in SKINNY_ONE_KERNEL] +
                         [s + ("gemm_tiny_quant_kernel",) for s in TINY_ONE_KERNEL])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_m_one_kernel_paths_equal_two_ops(M, N, K, kernel, dtype, dev):
    """act-quant inside the skinny or the small-grid GEMM: the same bits as
    act_quant then the GEMM, and the oracle chain within the north-star
    tolerance."""
    print(f"{kernel} act-quant matmul M={M} N={N} K={K} {dtype}", flush=True)
    assert _one_kernel(M, N, K, kernel)
    x = synthetic.activations(M, K, seed=M * 5 + K, outlier_frac=0.01).to(dev)
    W, Bs = _weights(N, K, N + 2, dev)
    out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], dtype)
    _same(out, _two_op(x, W, Bs, dtype))
    lb = (N - 1) // 128
    cols = torch.cat([torch.arange(0, 128), torch.arange(lb * 128, N)])
    ref = _oracle_chain(x, W[cols.to(dev)], Bs[torch.tensor([0, lb]).to(dev)],
                        torch.arange(M))
    torch.testing.assert_close(out[:, cols.to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(dtype).float(), rtol=RTOL, atol=ATOL)


def test_skinny_one_kernel_path_nonfinite_and_strided_rows(dev):
    """NaN, +-inf and all-zero groups, a row stride past K, a 16-byte offset
    base, and a 2-byte offset base (two-launch path) on a skinny plan."""
    M, N, K = 6, 3000, 2048
    assert _one_kernel(M, N, K, "gemm_skinny_quant_kernel")
    big = synthetic.activations(M, K + 64, seed=17).to(dev)
    big[1, 8 + 5] = float("nan")
    big[2, 8 + 1000] = float("inf")
    big[3, 8 + 2000] = -float("inf")
    big[4, :] = 0
    W, Bs = _weights(N, K, 18, dev)
    for xv in (big[:, 8:K + 8], big[:, :K], big[:, 1:K + 1]):
        out = fp8.act_quant_w8a8_block_fp8_matmul(xv, W, Bs, [128, 128], torch.float32)
        _same(out, _two_op(xv.contiguous(), W, Bs, torch.float32))
    out = fp8.act_quant_w8a8_block_fp8_matmul(big[:, 8:K + 8], W, Bs, [128, 128], torch.float32)
    assert torch.equal(out[4], torch.zeros_like(out[4]))
    assert torch.isnan(out[1]).all() and torch.isnan(out[2]).all() and torch.isnan(out[3]).all()


@pytest.mark.parametrize("M,N,K", ONE_KERNEL)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_one_kernel_path_equals_two_ops(M, N, K, dtype, dev):
    """act-quant inside the decode GEMM: the same bits as act_quant then the
    GEMM, and the oracle chain within the north-star tolerance."""
    print(f"one-kernel act-quant matmul M={M} N={N} K={K} {dtype}", flush=True)
    assert _one_kernel(M, N, K)
    x = synthetic.activations(M, K, seed=M * 7 + K, outlier_frac=0.01).to(dev)
    W, Bs = _weights(N, K, N + 1, dev)
    out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], dtype)
    _same(out, _two_op(x, W, Bs, dtype))
    # rows of x; output columns of the first two and the last (ragged) weight
    # blocks, with their block scales
    rows = torch.unique(torch.tensor([0, M // 2, M - 1]))
    lb = (N - 1) // 128
    cols = torch.cat([torch.arange(0, 256), torch.arange(lb * 128, N)])
    ref = _oracle_chain(x, W[cols.to(dev)], Bs[torch.tensor([0, 1, lb]).to(dev)], rows)
    ref_t = torch.from_numpy(ref).to(dtype).float()
    torch.testing.assert_close(out[rows.to(dev)][:, cols.to(dev)].float().cpu(), ref_t,
                               rtol=RTOL, atol=ATOL)


def test_one_kernel_path_nonfinite_zero_and_strided_rows(dev):
    """NaN, +-inf and all-zero groups, a row stride past K and a 16-byte
    offset base through the one-kernel path; a 2-byte offset base takes the
    two-launch path (the kernel's DMA needs 16-byte aligned rows)."""
    M, N, K = 17, 4160, 7296
    assert _one_kernel(M, N, K)
    big = synthetic.activations(M, K + 64, seed=11).to(dev)
    big[2, 8 + 5] = float("nan")
    big[7, 8 + 3000] = float("inf")
    big[11, 8 + 6000] = -float("inf")
    big[13, :] = 0
    W, Bs = _weights(N, K, 12, dev)
    for xv in (big[:, 8:K + 8], big[:, :K], big[:, 1:K + 1]):
        out = fp8.act_quant_w8a8_block_fp8_matmul(xv, W, Bs, [128, 128], torch.float32)
        _same(out, _two_op(xv.contiguous(), W, Bs, torch.float32))
    out = fp8.act_quant_w8a8_block_fp8_matmul(big[:, 8:K + 8], W, Bs, [128, 128], torch.float32)
    assert torch.equal(out[13], torch.zeros_like(out[13]))
    assert torch.isnan(out[2]).all() and torch.isnan(out[7]).all() and torch.isnan(out[11]).all()


def test_one_kernel_path_graph_replays(dev):
    """Captured in a HIP graph, every replay of the one-kernel path (with
    eager work between) equals the eager result."""
    M, N, K = 32, 2048, 8576
    assert _one_kernel(M, N, K)
    x = synthetic.activations(M, K, seed=13).to(dev)
    W, Bs = _weights(N, K, 14, dev)
    f = lambda: fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], torch.bfloat16)
    eager = f()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        _same(out, eager)
        _same(out, _two_op(x, W, Bs, torch.bfloat16))
        torch.cuda.synchronize()


def test_fused_nonfinite_and_zero_groups(dev):
    M, N, K = 24, 512, 1024
    x = synthetic.activations(M, K, seed=3).to(dev)
    x[2, 5] = float("nan")
    x[7, 300] = float("inf")
    x[11, 600] = -float("inf")
    x[13, :] = 0
    W, Bs = _weights(N, K, 4, dev)
    out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], torch.float32)
    _same(out, _two_op(x, W, Bs, torch.float32))
    # the all-zero row is exactly zero; rows with a NaN or inf group are NaN
    assert torch.equal(out[13], torch.zeros_like(out[13]))
    assert torch.isnan(out[2]).all() and torch.isnan(out[7]).all() and torch.isnan(out[11]).all()
    finite = [r for r in range(M) if r not in (2, 7, 11)]
    rows = torch.tensor(finite)
    ref = _oracle_chain(x, W, Bs, rows)
    torch.testing.assert_close(out[rows.to(dev)].cpu(), torch.from_numpy(ref), rtol=RTOL,
                               atol=ATOL)


def test_fused_strided_and_unaligned_rows(dev):
    M, N, K = 20, 384, 1024
    big = synthetic.activations(M, K + 64, seed=5).to(dev)
    W, Bs = _weights(N, K, 6, dev)
    xs = big[:, :K]                        # row stride K + 64
    _same(fp8.act_quant_w8a8_block_fp8_matmul(xs, W, Bs, [128, 128], torch.bfloat16),
          _two_op(xs, W, Bs, torch.bfloat16))
    xu = big[:, 1:K + 1]                   # 2-byte offset rows: the generic quantiser
    _same(fp8.act_quant_w8a8_block_fp8_matmul(xu, W, Bs, [128, 128], torch.bfloat16),
          _two_op(xu.contiguous(), W, Bs, torch.bfloat16))
    xe = big[:1, :K].expand(M, K)          # row stride 0: copied to rows before the launch
    _same(fp8.act_quant_w8a8_block_fp8_matmul(xe, W, Bs, [128, 128], torch.bfloat16),
          _two_op(xe.contiguous(), W, Bs, torch.bfloat16))


def test_fused_graph_replays(dev):
    """Captured in a HIP graph, every replay (with eager work between) equals
    the eager result."""
    M, N, K = 32, 2048, 4096
    x = synthetic.activations(M, K, seed=7).to(dev)
    W, Bs = _weights(N, K, 8, dev)
    f = lambda: fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], torch.bfloat16)
    eager = f()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = f()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        _same(out, eager)
        _two_op(x, W, Bs, torch.bfloat16)  # eager work between replays
        torch.cuda.synchronize()


def test_fused_rejects_bad_inputs(dev):
    x = torch.zeros(4, 200, dtype=torch.bfloat16, device=dev)
    W = torch.zeros(128, 200, dtype=torch.float8_e4m3fn, device=dev)
    Bs = torch.ones(1, 2, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs)
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=dev)
    W = torch.zeros(128, 256, dtype=torch.float8_e4m3fn, device=dev)
    with pytest.raises(RuntimeError, match="128, 128"):
        fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [64, 128])


def _random_small_m(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        M = int(torch.randint(1, 65, (1,), generator=g))
        N = int(torch.randint(1, 12289, (1,), generator=g))
        K = 128 * int(torch.randint(1, 113, (1,), generator=g))
        out.append((M, N, K))
    return out


@pytest.mark.parametrize("M,N,K", _random_small_m(24, 2026))
def test_fused_random_small_m_both_dtypes(M, N, K, dev):
    """A seeded sweep of decode-sized shapes (M 1-64, N up to 12288, K up to
    14336) over every act-quant + GEMM path the planner picks (one kernel on
    decode, skinny and small-grid plans, or two launches): bf16 and fp32
    outputs each equal the two public ops bit for bit, and the fp32 output
    rounded to bf16 equals the bf16 output."""
    print(f"fused random M={M} N={N} K={K}", flush=True)
    gx = torch.Generator(device=dev).manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=gx, device=dev).to(torch.bfloat16)
    W, Bs = _weights(N, K, seed=N + K, dev=dev)
    outs = {}
    for dtype in (torch.bfloat16, torch.float32):
        out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], dtype)
        _same(out, _two_op(x, W, Bs, dtype))
        outs[dtype] = out
    _same(outs[torch.float32].to(torch.bfloat16), outs[torch.bfloat16])
