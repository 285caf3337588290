"""CPU checks of the Python op surface: signature parity with the reference
package, op registration, fake (meta) shapes, and loud failure instead of a
CPU fallback."""
import inspect

import pytest
import torch

from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import _ops


def test_public_signature_matches_reference():
    # finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/__init__.py:7-8
    sig = inspect.signature(fp8.w8a8_block_fp8_matmul)
    assert list(sig.parameters) == ["A", "B", "As", "Bs", "block_size", "output_dtype"]
    assert sig.parameters["output_dtype"].default is torch.float32
    assert "w8a8_block_fp8_matmul" in fp8.__all__


def test_namespace_follows_kernel_builder_scheme():
    assert _ops._OPS_NAME == "_finegrained_fp8_helion_rocm_mi355x"
    assert _ops.add_op_namespace_prefix("x") == "_finegrained_fp8_helion_rocm_mi355x::x"
    for name in ("w8a8_block_fp8_matmul", "w8a8_block_fp8_matmul_dtype", "act_quant",
                 "silu_and_mul", "silu_and_mul_quant", "act_quant_matmul", "weight_quant",
                 "gate_up_silu_quant"):
        assert hasattr(_ops.ops, name)


def _fp8(*shape, device="cpu"):
    return torch.zeros(*shape, dtype=torch.float8_e4m3fn, device=device)


def test_cpu_tensors_raise_not_fallback():
    A, B = _fp8(4, 256), _fp8(128, 256)
    As, Bs = torch.ones(4, 2), torch.ones(1, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fp8.act_quant(torch.zeros(4, 256, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fp8.act_quant_w8a8_block_fp8_matmul(torch.zeros(4, 256, dtype=torch.bfloat16), B, Bs)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fp8.silu_and_mul(torch.empty(2, 8, dtype=torch.bfloat16),
                         torch.zeros(2, 16, dtype=torch.bfloat16))


def test_fake_impls_give_reference_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        A, B = _fp8(7, 384), _fp8(200, 384)
        As, Bs = torch.ones(7, 3), torch.ones(2, 3)
        out = _ops.ops.w8a8_block_fp8_matmul(A, B, As, Bs, 128, 128)
        assert out.shape == (7, 200) and out.dtype == torch.float32  # reference op.py:14-16
        out = _ops.ops.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, 128, 128, torch.bfloat16)
        assert out.dtype == torch.bfloat16
        q, s = _ops.ops.act_quant(torch.zeros(3, 5, 300, dtype=torch.bfloat16), 128)
        assert q.shape == (3, 5, 300) and q.dtype == torch.float8_e4m3fn
        assert s.shape == (3, 5, 3) and s.dtype == torch.float32
        q, s = _ops.ops.silu_and_mul_quant(torch.zeros(4, 512, dtype=torch.bfloat16), 128)
        assert q.shape == (4, 256) and s.shape == (4, 2)
        q, s = _ops.ops.gate_up_silu_quant(_fp8(7, 512), _fp8(512, 512), torch.ones(7, 4),
                                           torch.ones(4, 4))
        assert q.shape == (7, 256) and q.dtype == torch.float8_e4m3fn and s.shape == (7, 2)
        out = _ops.ops.act_quant_matmul(torch.zeros(7, 384, dtype=torch.bfloat16), B, Bs, 128,
                                        128, torch.bfloat16)
        assert out.shape == (7, 200) and out.dtype == torch.bfloat16
        q, s = _ops.ops.weight_quant(torch.zeros(300, 260), 128, 128)
        assert q.shape == (300, 260) and s.shape == (3, 3) and s.dtype == torch.float32


def test_public_api_under_fake_tensors_takes_the_op_route():
    """The direct bindings decline tensor subclasses (FakeTensor here), so the
    public functions reach the registered ops and their fake kernels."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from hf_kernels_helion_amd import deep_gemm_helion as dg
    from hf_kernels_helion_amd.finegrained_fp8_helion import op
    with FakeTensorMode():
        A, B = _fp8(7, 384), _fp8(200, 384)
        As, Bs = torch.ones(7, 3), torch.ones(2, 3)
        assert op.fast.w8a8_block_fp8_matmul_dtype(A, B, As, Bs, 128, 128,
                                                   torch.bfloat16) is None
        out = fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16)
        assert out.shape == (7, 200) and out.dtype == torch.bfloat16
        q, s = fp8.act_quant(torch.zeros(3, 300, dtype=torch.float16), 128)
        assert q.shape == (3, 300) and s.shape == (3, 3)
        q, s = fp8.silu_and_mul_quant(torch.zeros(4, 512, dtype=torch.bfloat16))
        assert q.shape == (4, 256)
        out = fp8.act_quant_w8a8_block_fp8_matmul(torch.zeros(7, 384, dtype=torch.bfloat16),
                                                  B, Bs, [128, 128], torch.bfloat16)
        assert out.shape == (7, 200)
        out = dg.gemm_fp8_fp8_bf16_nt(A, B, As, torch.ones(200, 3))
        assert out.shape == (7, 200) and out.dtype == torch.bfloat16


def test_public_api_compiles_to_the_registered_op():
    """Under torch.compile the wrappers call torch.ops (no graph break with
    fullgraph=True): the traced graph holds the custom op."""
    import torch._dynamo
    seen = []

    class Traced(Exception):
        pass

    def backend(gm, example_inputs):
        seen.extend(str(n.target) for n in gm.graph.nodes if n.op == "call_function")

        def run(*args):
            raise Traced()
        return run

    def f(A, B, As, Bs, x):
        q, s = fp8.act_quant(x, 128)
        return fp8.w8a8_block_fp8_matmul(A, B, As, Bs, [128, 128], torch.bfloat16), q, s

    torch._dynamo.reset()
    g = torch.compile(f, backend=backend, fullgraph=True)
    with pytest.raises(Traced):
        g(_fp8(7, 384), _fp8(200, 384), torch.ones(7, 3), torch.ones(2, 3),
          torch.zeros(7, 384, dtype=torch.bfloat16))
    torch._dynamo.reset()
    assert any("w8a8_block_fp8_matmul_dtype" in t for t in seen), seen
    assert any("act_quant" in t for t in seen), seen


def test_op_schemas_match_reference():
    # finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-11 and
    # activation-helion/.../op.py:15-16
    ops = _ops.ops
    sch = str(ops.w8a8_block_fp8_matmul.default._schema)
    assert "(Tensor A, Tensor B, Tensor As, Tensor Bs, int block_n, int block_k) -> Tensor" in sch
    sch = str(ops.silu_and_mul.default._schema)
    assert "Tensor(a!) out, Tensor x) -> ()" in sch


def test_synthetic_weight_quantiser_matches_oracle():
    """The torch weight-block quantiser used for test/bench inputs is the
    oracle's, bit for bit."""
    import numpy as np
    import oracle
    from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic
    g = torch.Generator().manual_seed(3)
    W = torch.randn(300, 260, generator=g) * 0.02
    Wq, Bs = synthetic.quantize_weight_blockwise(W, 128, 128)
    oq, obs = oracle.quant_weight_block(W.numpy(), (128, 128))
    np.testing.assert_array_equal(Wq.view(torch.uint8).numpy(), oq)
    np.testing.assert_array_equal(Bs.numpy(), obs)


def test_bench_rejects_multi_gpu():
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr


def test_deep_gemm_surface_matches_reference():
    # deep-gemm-helion/torch-ext/deep_gemm_helion/__init__.py:6-8 and op.py:8-16
    from hf_kernels_helion_amd import deep_gemm_helion as dg
    from hf_kernels_helion_amd.deep_gemm_helion import _ops as dg_ops
    from torch._subclasses.fake_tensor import FakeTensorMode
    sig = inspect.signature(dg.gemm_fp8_fp8_bf16_nt)
    assert list(sig.parameters) == ["A", "B", "As", "Bs", "block_size"]
    assert sig.parameters["block_size"].default == 128
    assert dg_ops._OPS_NAME == "_deep_gemm_helion_rocm_mi355x"
    sch = str(dg_ops.ops.gemm_fp8_fp8_bf16_nt.default._schema)
    assert "(Tensor A, Tensor B, Tensor As, Tensor Bs, int block_k) -> Tensor" in sch
    with FakeTensorMode():
        out = dg.gemm_fp8_fp8_bf16_nt(_fp8(5, 256), _fp8(7, 256), torch.ones(5, 2),
                                      torch.ones(7, 2))
        assert out.shape == (5, 7) and out.dtype == torch.bfloat16
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        dg.gemm_fp8_fp8_bf16_nt(_fp8(5, 256), _fp8(7, 256), torch.ones(5, 2), torch.ones(7, 2))


def test_interleave_gate_up_layout():
    """128-row blocks [gate t, up t]; scale block rows 2t = gate t, 2t+1 = up t."""
    I, H = 384, 256
    w = torch.arange(2 * I, dtype=torch.float32)[:, None].expand(2 * I, H).contiguous()
    s = torch.arange(2 * I // 128, dtype=torch.float32)[:, None].expand(-1, 2).contiguous()
    wi, si = fp8.interleave_gate_up(w, s)
    for t in range(I // 128):
        assert torch.equal(wi[256 * t: 256 * t + 128, 0], torch.arange(128 * t, 128 * t + 128.))
        assert torch.equal(wi[256 * t + 128: 256 * t + 256, 0],
                           torch.arange(I + 128 * t, I + 128 * t + 128.))
        assert si[2 * t, 0] == t and si[2 * t + 1, 0] == I // 128 + t
    with pytest.raises(ValueError):
        fp8.interleave_gate_up(torch.zeros(200, 256), torch.zeros(2, 2))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fp8.gate_up_silu_quant(_fp8(4, 512), torch.ones(4, 4), _fp8(256, 512), torch.ones(2, 4))
    # below FUSED_GATE_UP_MIN_ROWS rows the two-op route keeps the fused
    # kernel's shape contract
    with pytest.raises(RuntimeError, match="multiple of 128"):
        fp8.gate_up_silu_quant(_fp8(4, 200), torch.ones(4, 2), _fp8(256, 200), torch.ones(2, 2))
    with pytest.raises(RuntimeError, match="multiple of 128"):
        fp8.gate_up_silu_quant(_fp8(4, 512), torch.ones(4, 4), _fp8(200, 512), torch.ones(2, 4))
