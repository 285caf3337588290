"""The public functions' direct bindings (module _fp8_fast) against the
registered torch ops they stand in for on plain eager calls: the same
result bits for every bound op, and the torch.ops route whenever a
dispatch mode, tensor subclass or torch.compile is involved."""
import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from hf_kernels_helion_amd import deep_gemm_helion as dg
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import _ops, op, synthetic
from hf_kernels_helion_amd.deep_gemm_helion import _ops as dg_ops

pytestmark = pytest.mark.gpu
ops = _ops.ops


def _operands(M, N, K, dev, seed=0):
    return [t.to(dev) for t in synthetic.harness_operands(M, N, K, seed=seed)]


def _same(a, b):
    """Same dtype, shape and bits."""
    return (a.dtype == b.dtype and a.shape == b.shape and
            torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8)))


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (32, 4096, 14336), (300, 700, 1536)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32, torch.float16])
def test_matmul_binding_equals_op(M, N, K, dt, dev):
    print(f"fast matmul {M}x{N}x{K} {dt}", flush=True)
    A, B, As, Bs = _operands(M, N, K, dev)
    fast = op.fast.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, 128, 128, dt)
    ref = ops.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, 128, 128, dt)
    assert fast is not None and _same(fast, ref)
    assert _same(fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], dt), ref)


def test_other_bindings_equal_ops(dev):
    print("fast act_quant / silu / fused / deep-gemm", flush=True)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        x = torch.randn(37, 4096, device=dev).to(dt)
        qf, sf = op.fast.act_quant(x, 128)
        qo, so = ops.act_quant(x, 128)
        assert _same(qf, qo) and _same(sf, so)
    h = torch.randn(9, 2, 1024, device=dev).to(torch.bfloat16)
    out_f = torch.empty(9, 2, 512, dtype=torch.bfloat16, device=dev)
    out_o = torch.empty_like(out_f)
    assert op.fast.silu_and_mul(out_f, h) is out_f
    ops.silu_and_mul(out_o, h)
    assert _same(out_f, out_o)
    qf, sf = op.fast.silu_and_mul_quant(h, 128)
    qo, so = ops.silu_and_mul_quant(h, 128)
    assert _same(qf, qo) and _same(sf, so)
    x = synthetic.activations(32, 14336, seed=2).to(dev)
    W, Bs = synthetic.quantize_weight_blockwise(torch.randn(4096, 14336) * 0.02, 128, 128)
    W, Bs = W.to(dev), Bs.to(dev)
    f = op.fast.act_quant_matmul(x, W, Bs, 128, 128, torch.bfloat16)
    assert _same(f, ops.act_quant_matmul(x, W, Bs, 128, 128, torch.bfloat16))
    A, B, As, _ = _operands(64, 1024, 2048, dev)
    Bs_row = torch.rand(1024, 16, device=dev) + 0.5
    f = op.fast.gemm_fp8_fp8_bf16_nt(A, B, As, Bs_row, 128)
    assert _same(f, dg_ops.ops.gemm_fp8_fp8_bf16_nt(A, B, As, Bs_row, 128))
    assert _same(dg.gemm_fp8_fp8_bf16_nt(A, B, As, Bs_row), f)


class _Log(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.names = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.names.append(str(func))
        return func(*args, **(kwargs or {}))


def test_dispatch_mode_sees_the_ops(dev):
    """With a TorchDispatchMode active the bindings decline and the calls go
    through the dispatcher, where the mode sees them."""
    A, B, As, Bs = _operands(128, 256, 512, dev)
    x = torch.randn(4, 512, device=dev).to(torch.bfloat16)
    ref = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
    with _Log() as log:
        out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
        fp8.act_quant(x, 128)
    assert any("w8a8_block_fp8_matmul_dtype" in n for n in log.names), log.names
    assert any("act_quant" in n for n in log.names), log.names
    assert _same(out, ref)


def test_compiled_call_equals_eager(dev):
    A, B, As, Bs = _operands(256, 512, 1024, dev)

    def f(A, B, As, Bs):
        return fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)

    torch._dynamo.reset()
    g = torch.compile(f, backend="eager", fullgraph=True)
    assert _same(g(A, B, As, Bs), f(A, B, As, Bs))
    torch._dynamo.reset()


def test_requires_grad_input_takes_the_op_route(dev):
    A, B, As, Bs = _operands(64, 256, 512, dev)
    As_g = As.clone().requires_grad_(True)
    assert op.fast.w8a8_block_fp8_matmul_dtype(A, B, As_g, Bs, 128, 128, torch.bfloat16) is None
    out = fp8.w8a8_block_fp8_matmul(A, B, As_g, Bs, [128, 128], torch.bfloat16)
    assert _same(out.detach(), fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128],
                                                          torch.bfloat16))


def test_binding_errors_match_op_errors(dev):
    A, B, As, Bs = _operands(64, 256, 512, dev)
    with pytest.raises(RuntimeError, match="must be float8_e4m3fn|float8"):
        fp8.w8a8_block_fp8_matmul(A.float(), B, As, Bs, [128, 128], torch.bfloat16)
    with pytest.raises(RuntimeError, match="group size"):
        fp8.act_quant(torch.zeros(4, 256, dtype=torch.bfloat16, device=dev), 100)
