"""The custom ops as torch sees them, on the GPU: torch.library.opcheck over
every op of both namespaces (fake-tensor kernels against the real outputs,
AOT dispatch with static and dynamic shapes, autograd registration, and the
schema's mutation annotations for the ops without fp8 inputs),
and a compiled decode chain (act_quant -> w8a8_block_fp8_matmul, the
mutating silu_and_mul) under torch.compile(fullgraph=True) equal to eager.
This is how a model compiled around the reference's ops
(finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-16,
activation-helion/.../op.py:15-23, deep-gemm-helion/.../op.py:8-16)
reaches these kernels."""
import pytest
import torch

from hf_kernels_helion_amd import deep_gemm_helion as dg
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.deep_gemm_helion import _ops as dg_ops
from hf_kernels_helion_amd.finegrained_fp8_helion import _ops
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

OPS = _ops.ops


def _operands(M, N, K, dev, block_n=128):
    x = synthetic.activations(M, K, seed=M + K).to(dev)
    W, Bs = synthetic.weights(N, K, seed=N, block_n=block_n)
    q, s = fp8.act_quant(x, 128)
    return x, q, s, W.to(dev), Bs.to(dev)


# test_schema runs the op under torch's SchemaCheckMode, which multiplies the
# inputs to detect mutation and has no float8_e4m3fn kernel for that: ops
# with fp8 inputs run the other three checks (their schemas are pinned in
# test_host_api.py).
ALL = ("test_schema", "test_autograd_registration", "test_faketensor",
       "test_aot_dispatch_dynamic")
NO_FP8_SCHEMA = ALL[1:]


def _check(op, args):
    fp8_in = any(isinstance(a, torch.Tensor) and a.dtype == torch.float8_e4m3fn for a in args)
    torch.library.opcheck(op, args, test_utils=NO_FP8_SCHEMA if fp8_in else ALL)


@pytest.mark.parametrize("M,N,K", [(32, 4096, 14336), (300, 700, 1536)])
def test_opcheck_matmul_ops(M, N, K, dev):
    print(f"opcheck matmul ops M={M} N={N} K={K}", flush=True)
    x, q, s, W, Bs = _operands(M, N, K, dev)
    _check(OPS.w8a8_block_fp8_matmul.default, (q, W, s, Bs, 128, 128))
    _check(OPS.w8a8_block_fp8_matmul_dtype.default, (q, W, s, Bs, 128, 128, torch.bfloat16))
    _check(OPS.act_quant_matmul.default, (x, W, Bs, 128, 128, torch.bfloat16))
    _, _, _, Wr, Bsr = _operands(M, N, K, dev, block_n=1)
    _check(dg_ops.ops.gemm_fp8_fp8_bf16_nt.default, (q, Wr, s, Bsr, 128))


def test_opcheck_elementwise_ops(dev):
    x = synthetic.activations(64, 1024, seed=3).to(dev)
    _check(OPS.act_quant.default, (x, 128))
    h = synthetic.activations(64, 2048, seed=4).to(dev)
    _check(OPS.silu_and_mul_quant.default, (h, 128))
    out = torch.empty(64, 1024, dtype=torch.bfloat16, device=dev)
    _check(OPS.silu_and_mul.default, (out, h))
    W = torch.randn(300, 260, device=dev) * 0.02
    _check(OPS.weight_quant.default, (W, 128, 128))


def test_opcheck_gate_up_silu_quant(dev):
    M, I, H = 96, 256, 512
    x, q, s, W, Bs = _operands(M, 2 * I, H, dev)
    wi, si = fp8.interleave_gate_up(W, Bs)
    _check(OPS.gate_up_silu_quant.default, (q, wi, s, si))


def test_compiled_decode_chain_equals_eager(dev):
    """act_quant -> GEMM -> silu_and_mul(out=...) traced in one graph."""
    M, N, K = 32, 4096, 14336
    x, _, _, W, Bs = _operands(M, N, K, dev)

    def chain(x):
        q, s = fp8.act_quant(x, 128)
        y = fp8.w8a8_block_fp8_matmul(q, W, s, Bs, [128, 128], torch.bfloat16)
        out = torch.empty(M, N // 2, dtype=torch.bfloat16, device=x.device)
        fp8.silu_and_mul(out, y)
        return y, out

    eager = chain(x)
    torch._dynamo.reset()
    compiled = torch.compile(chain, fullgraph=True, backend="aot_eager")
    got = compiled(x)
    for a, b in zip(got, eager):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
    # a second input of another row count goes through the same compiled code
    x2 = synthetic.activations(M, K, seed=99).to(dev)
    for a, b in zip(compiled(x2), chain(x2)):
        torch.testing.assert_close(a, b, rtol=0, atol=0)


def test_compiled_deep_gemm_equals_eager(dev):
    M, N, K = 64, 512, 1024
    _, q, s, Wr, Bsr = _operands(M, N, K, dev, block_n=1)
    f = lambda a, b, sa, sb: dg.gemm_fp8_fp8_bf16_nt(a, b, sa, sb, 128)
    torch._dynamo.reset()
    got = torch.compile(f, fullgraph=True, backend="aot_eager")(q, Wr, s, Bsr)
    torch.testing.assert_close(got, f(q, Wr, s, Bsr), rtol=0, atol=0)
