"""GPU parity of the 128x128 weight-block quantiser (quantize_weight) with
the torch quantiser the tests build operands with (synthetic.
quantize_weight_blockwise), which the oracle pins
(test_host_api.test_synthetic_weight_quantiser_matches_oracle): bit for bit
on Wq and Bs, fp32 and bf16 inputs, ragged edges."""
import pytest
import torch

from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import checkpoint, synthetic

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.cpu().contiguous().view(torch.uint8)


@pytest.mark.parametrize("N,K", [(256, 384), (130, 260), (1, 129), (127, 1), (1024, 4096),
                                 (300, 4097)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weight_quant_matches_torch_quantiser(N, K, dtype, dev):
    print(f"weight quant N={N} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(N + K)
    W = (torch.randn(N, K, generator=g) * 0.02).to(dtype)
    W[0, 0] = 0.5  # one large element in the first block
    if N > 128 and K > 128:
        W[128:256, 128:256] = 0  # an all-zero block: scale 1e-10/448, zeros
    q, s = fp8.quantize_weight(W.to(dev))
    rq, rs = synthetic.quantize_weight_blockwise(W.float())
    assert q.dtype == torch.float8_e4m3fn and q.shape == (N, K)
    assert torch.equal(_u8(q), _u8(rq))
    assert torch.equal(s.cpu(), rs)


def test_weight_quant_feeds_the_gemm(dev):
    """Quantise on the GPU, multiply, compare with the fp32 dequant product."""
    N, K, M = 512, 1024, 64
    g = torch.Generator().manual_seed(9)
    W = (torch.randn(N, K, generator=g) * 0.02).to(dev)
    Wq, Bs = fp8.quantize_weight(W)
    x = synthetic.activations(M, K, seed=10).to(dev)
    q, s = fp8.act_quant(x, 128)
    out = fp8.w8a8_block_fp8_matmul(q, Wq, s, Bs, [128, 128], torch.float32)
    ref = (q.float() * s.repeat_interleave(128, 1)) @ (Wq.float() * Bs.repeat_interleave(
        128, 0).repeat_interleave(128, 1)).T
    torch.testing.assert_close(out, ref, rtol=1e-2, atol=1e-3)


def test_quantize_state_dict_on_gpu(dev):
    g = torch.Generator().manual_seed(2)
    sd = {"a.weight": torch.randn(256, 512, generator=g) * 0.02,
          "a.bias": torch.randn(256, generator=g),
          "b.weight": (torch.randn(384, 256, generator=g) * 0.02).to(torch.bfloat16)}
    out = checkpoint.quantize_state_dict(sd, device=dev)
    assert set(out) == {"a.weight", "a.weight_scale_inv", "a.bias", "b.weight",
                        "b.weight_scale_inv"}
    for name in ("a.weight", "b.weight"):
        rq, rs = synthetic.quantize_weight_blockwise(sd[name].float())
        assert torch.equal(_u8(out[name]), _u8(rq))
        assert torch.equal(out[checkpoint._scale_name(name)], rs)
    assert set(checkpoint.fp8_linear_weights(out)) == {"a.weight", "b.weight"}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weight_quant_vector_path_equals_scalar_path(dtype, dev):
    """W with 16-byte rows takes the 16-byte-load kernel (edge blocks inside
    it take the per-element path); a row-strided view of the same values
    (row stride not a multiple of 16 bytes) takes the per-element kernel.
    Same codes and scales, bit for bit, with NaN, +-inf, subnormal and zero
    blocks."""
    print(f"weight quant vector vs scalar path {dtype}", flush=True)
    N, K = 384, 640 + 72   # ragged last block column (K % 128 = 72)
    g = torch.Generator().manual_seed(77)
    buf = (torch.randn(N, K + 2, generator=g) * 0.02)
    buf[5, 300] = float("nan")
    buf[200, 10] = float("inf")
    buf[300, 600] = -float("inf")
    buf[130:140, 0:128] = 1e-40
    buf[256:384, 256:384] = 0.0
    buf = buf.to(dtype).to(dev)
    Wc = buf[:, :K].contiguous()
    Ws = buf[:, :K]
    assert (Ws.stride(0) * Ws.element_size()) % 16 != 0
    q1, s1 = fp8.quantize_weight(Wc)
    q2, s2 = fp8.quantize_weight(Ws)
    assert torch.equal(_u8(q1), _u8(q2))
    assert torch.equal(s1.cpu().view(torch.int32), s2.cpu().view(torch.int32))
    assert torch.isnan(s1[0, 2]) and torch.isinf(s1[1, 0]) and s1[2, 2] > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("strided", [False, True])
def test_weight_quant_nonfinite_blocks_match_oracle(dtype, strided, dev):
    """Codes and scales bit for bit against oracle.quant_weight_block, with a
    NaN block (NaN and +inf together), a +-inf block, a subnormal block, an
    all-zero block and a ragged edge; contiguous rows take the 16-byte-load
    kernel, a row stride of K + 2 the per-element kernel."""
    import numpy as np
    import oracle
    print(f"weight quant nonfinite vs oracle {dtype} strided={strided}", flush=True)
    N, K = 300, 640 + 72
    g = torch.Generator().manual_seed(78)
    buf = torch.randn(N, K + 2, generator=g) * 0.02
    buf[5, 30] = float("nan")
    buf[6, 31] = float("inf")
    buf[140, 200] = float("inf")
    buf[141, 201] = -float("inf")
    buf[142, 202] = -0.0
    buf[256:300, 384:512] = 1e-40
    buf[0:128, 512:640] = 0.0
    buf = buf.to(dtype)
    W = buf[:, :K] if strided else buf[:, :K].contiguous()
    q, s = fp8.quantize_weight(W.to(dev) if not strided else buf.to(dev)[:, :K])
    qo, so = oracle.quant_weight_block(W.float().contiguous().numpy(), (128, 128))
    np.testing.assert_array_equal(_u8(q).numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.isnan(so[0, 0]) and so[1, 1] == np.inf and so[2, 3] > 0


@pytest.mark.parametrize("N,K", [(256, 384), (130, 260), (1024, 4096), (300, 4097)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_weight_quant_matches_oracle(N, K, dtype, dev):
    import numpy as np
    import oracle
    print(f"weight quant vs oracle N={N} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(N * K)
    W = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    q, s = fp8.quantize_weight(W.to(dev))
    qo, so = oracle.quant_weight_block(W.float().numpy(), (128, 128))
    np.testing.assert_array_equal(_u8(q).numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
