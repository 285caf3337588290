"""GPU parity of the fused act-quant + GEMM op against the two-op composition
act_quant -> w8a8_block_fp8_matmul, bit for bit, on both of its paths: the
decode kernel that quantises bf16 x itself (M <= 48, FP8B_FUSED_QUANT=1)
quantises with the same arithmetic and sums in the same order; the default
path quantises into the workspace and runs the GEMM. The composition itself
is checked against the oracle in test_gpu_act_quant.py and test_gpu_gemm.py."""
import os

import pytest
import torch

from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["fused", "two_kernel"], autouse=True)
def quant_path(request):
    old = os.environ.get("FP8B_FUSED_QUANT")
    os.environ["FP8B_FUSED_QUANT"] = "1" if request.param == "fused" else "0"
    yield request.param
    if old is None:
        del os.environ["FP8B_FUSED_QUANT"]
    else:
        os.environ["FP8B_FUSED_QUANT"] = old


def _weights(N, K, seed, dev):
    W, Bs = synthetic.weights(N, K, seed=seed)
    return W.to(dev), Bs.to(dev)


def _two_op(x, W, Bs, dtype):
    q, s = fp8.act_quant(x, 128)
    return fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], dtype)


def _same(a, b):
    torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (16, 4096, 14336), (17, 1000, 1024),
                                   (32, 4096, 14336), (33, 512, 2048), (48, 640, 3072),
                                   (32, 28672, 4096), (64, 512, 1024), (100, 384, 512)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_equals_two_ops(M, N, K, dtype, dev):
    print(f"fused act-quant matmul M={M} N={N} K={K} {dtype}", flush=True)
    x = synthetic.activations(M, K, seed=M + K, outlier_frac=0.01).to(dev)
    W, Bs = _weights(N, K, N, dev)
    out = fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], dtype)
    assert out.dtype == dtype and out.shape == (M, N)
    _same(out, _two_op(x, W, Bs, dtype))


def test_fused_nonfinite_and_zero_groups(dev):
    M, N, K = 24, 512, 1024
    x = synthetic.activations(M, K, seed=3).to(dev)
    x[2, 5] = float("nan")
    x[7, 300] = float("inf")
    x[11, 600] = -float("inf")
    x[13, :] = 0
    W, Bs = _weights(N, K, 4, dev)
    _same(fp8.act_quant_w8a8_block_fp8_matmul(x, W, Bs, [128, 128], torch.float32),
          _two_op(x, W, Bs, torch.float32))


def test_fused_strided_and_unaligned_rows(dev):
    M, N, K = 20, 384, 1024
    big = synthetic.activations(M, K + 64, seed=5).to(dev)
    W, Bs = _weights(N, K, 6, dev)
    xs = big[:, :K]                        # row stride K + 64, aligned: fused kernel
    _same(fp8.act_quant_w8a8_block_fp8_matmul(xs, W, Bs, [128, 128], torch.bfloat16),
          _two_op(xs, W, Bs, torch.bfloat16))
    xu = big[:, 1:K + 1]                   # 2-byte offset rows: quantise-then-GEMM path
    _same(fp8.act_quant_w8a8_block_fp8_matmul(xu, W, Bs, [128, 128], torch.bfloat16),
          _two_op(xu.contiguous(), W, Bs, torch.bfloat16))


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
