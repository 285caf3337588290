"""GPU parity of the act-quant kernels against the CPU oracle: bit-exact fp8
codes and fp32 scales (bits compared, NaN included)."""
import numpy as np
import pytest
import torch

import oracle
from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu


def _bits(x_bf16: torch.Tensor) -> np.ndarray:
    return x_bf16.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _run(x_cpu: torch.Tensor, group: int, dev):
    q, s = fp8.act_quant(x_cpu.to(dev), group)
    torch.cuda.synchronize()
    return q.cpu().view(torch.uint8).numpy(), s.cpu().numpy()


def _assert_exact(x_cpu, group, dev):
    q, s = _run(x_cpu, group, dev)
    x2 = _bits(x_cpu).reshape(-1, x_cpu.shape[-1])
    qo, so = oracle.act_quant(x2, group)
    np.testing.assert_array_equal(q.reshape(qo.shape), qo)
    np.testing.assert_array_equal(s.reshape(so.shape).view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("M,K", [(1, 128), (4, 512), (32, 14336), (57, 4096), (3001, 1024),
                                 (512, 2048)])
def test_act_quant_g128_exact(M, K, dev):
    print(f"act_quant g128 M={M} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M * 7 + K)
    _assert_exact(x, 128, dev)


@pytest.mark.parametrize("M,K", [(70000, 256), (66000, 1024)])
def test_act_quant_more_rows_than_grid_y(M, K, dev):
    """Many rows of few groups (the flat-mapped kernel, one (row, group)
    slot per 16-lane row) past the 65535 grid rows."""
    print(f"act_quant rows M={M} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + K)
    _assert_exact(x, 128, dev)


@pytest.mark.parametrize("silu,K", [(False, 4096), (False, 8192), (False, 7168),
                                    (True, 14336), (True, 7168), (True, 4096)])
def test_quant_row_walk_past_grid_y_equals_slices(silu, K, dev):
    """Past 65535 rows the row-mapped kernels cap the grid and each block
    walks rows m, m + 65535, ..., alternating its two LDS scale slots from
    row to row. The result must equal, bit for bit, calls on row slices that
    fit the grid (one row per block): act-quant at U = 2, 4 and 4 with idle
    16-lane rows, SiLU-quant in blocks of 8, 4 and 16 rows."""
    M = 66000
    print(f"quant row walk silu={silu} M={M} K={K}", flush=True)
    width = 2 * K if silu else K
    g = torch.Generator(device=dev).manual_seed(K + silu)
    x = (torch.randn(M, width, generator=g, device=dev) * 2).to(torch.bfloat16)
    fn = fp8.silu_and_mul_quant if silu else fp8.act_quant
    q, s = fn(x, 128)
    for r0, r1 in ((0, 33000), (33000, M)):
        qp, sp = fn(x[r0:r1], 128)
        assert torch.equal(q[r0:r1].view(torch.uint8), qp.view(torch.uint8)), (r0, r1)
        assert torch.equal(s[r0:r1].view(torch.int32), sp.view(torch.int32)), (r0, r1)
    del x, q, s


def _g128_unroll(M, K):
    """Groups per block column / 16 that fp8b_act_quant picks for group 128
    (g128_unroll in act_quant.hip)."""
    gpr = K // 128
    if M * gpr < 16 * 1024:
        return 1
    if gpr % 64 == 0:
        return 4
    if gpr % 32 == 0:
        return 2
    return 4 if 32 < gpr < 64 else 2


def _silu_quant_shape(M, d):
    """(16-lane rows per block, groups per lane) that fp8b_silu_and_mul_quant
    picks for group 128 (silu_quant_shape in act_quant.hip)."""
    gpr = d // 128
    if M * gpr < 16 * 1024 or gpr % 64 == 0 or gpr % 8 != 0:
        return 16, _g128_unroll(M, d)
    h = gpr // 2
    return (16 if h % 16 == 0 else 8 if h % 8 == 0 else 4), 2


@pytest.mark.parametrize("M,K,unroll", [(2048, 4096, 2), (3001, 4096, 2), (512, 4096, 2),
                                        (256, 8192, 4), (300, 14336, 2), (600, 7168, 4),
                                        (1000, 2560, 2), (100, 7168, 1)])
def test_act_quant_every_unroll_on_config_inputs(M, K, unroll, dev):
    """The BASELINE config inputs (~N(0,1) with 1% outliers x20 per row) on
    each unrolled kernel variant: [2048,4096] (C2) and [3001,4096] (C5) run
    act_quant_g128_kernel<2>, [256,8192] <4>; rows whose groups 16*U does
    not divide leave idle 16-lane rows in their last block column:
    [300,14336] (112 groups) and [1000,2560] (20) at <2>, [600,7168] (56) at
    <4>; [100,7168] has too few groups in all and runs <1>."""
    assert _g128_unroll(M, K) == unroll
    print(f"act_quant U={unroll} M={M} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 3 * K, outlier_frac=0.01)
    _assert_exact(x, 128, dev)


def test_act_quant_outliers_exact(dev):
    print("act_quant outliers", flush=True)
    x = synthetic.activations(256, 4096, seed=99, outlier_frac=0.01)
    _assert_exact(x, 128, dev)


@pytest.mark.parametrize("group", [32, 64, 128, 256])
@pytest.mark.parametrize("K", [100, 300, 1000])
def test_act_quant_generic_exact(group, K, dev):
    print(f"act_quant generic group={group} K={K}", flush=True)
    x = synthetic.activations(9, K, seed=group + K)
    _assert_exact(x, group, dev)


def test_act_quant_every_bf16_through_cvt(dev):
    """Groups whose amax is exactly 448 have scale 1.0, so q = e4m3fn(x) for
    every bf16 x with |x| <= 448: the hardware convert is checked on all of
    them. Each 128-group holds one 448 and 127 test values."""
    print("act_quant exhaustive bf16 cvt", flush=True)
    bits = np.arange(65536, dtype=np.uint32)
    f = (bits << 16).view(np.float32)
    vals = f[np.isfinite(f) & (np.abs(f) <= 448.0)]
    per = 127
    G = -(-vals.size // per)
    padded = np.zeros(G * per, dtype=np.float32)
    padded[: vals.size] = vals
    grid = np.full((G, 128), 448.0, dtype=np.float32)
    grid[:, 1:] = padded.reshape(G, per)
    x = torch.from_numpy(grid.reshape(-1, 1024 if G % 8 == 0 else 128)).to(torch.bfloat16)
    _assert_exact(x, 128, dev)
    q, s = _run(x, 128, dev)
    assert np.all(s == 1.0)


def test_act_quant_scales_sweep_exact(dev):
    """Same values under many amax values: exercises the IEEE division."""
    print("act_quant scale sweep", flush=True)
    g = torch.Generator().manual_seed(7)
    rows = []
    for e in range(-30, 30, 3):
        r = torch.randn(1, 4096, generator=g) * (2.0 ** e)
        rows.append(r)
    x = torch.cat(rows).to(torch.bfloat16)
    _assert_exact(x, 128, dev)


def test_act_quant_every_amax_exact(dev):
    """One group per finite bf16 magnitude as its amax (0 included): the
    scale and its reciprocal, formed without a division, take every value
    the kernels can produce; the group's other 127 values are random bf16
    no larger in magnitude, with random signs."""
    print("act_quant every amax", flush=True)
    g = torch.Generator().manual_seed(11)
    amax = torch.arange(0, 0x7F80, dtype=torch.int32)                     # 32640 patterns
    frac = torch.rand(amax.numel(), 127, generator=g)
    others = (frac * (amax[:, None].float() + 1)).floor().clamp(max=amax[:, None].float())
    pats = torch.cat([amax[:, None], others.to(torch.int32)], 1)
    signs = torch.randint(0, 2, pats.shape, generator=g, dtype=torch.int32) << 15
    perm = torch.argsort(torch.rand(pats.shape, generator=g), 1)            # amax anywhere
    pats = torch.gather(pats | signs, 1, perm)
    x = pats.to(torch.int16).view(torch.bfloat16).reshape(-1, 64 * 128)     # 510 x 8192
    _assert_exact(x, 128, dev)


def test_act_quant_nonfinite_and_zero_groups(dev):
    print("act_quant nonfinite", flush=True)
    x = torch.randn(4, 512).to(torch.bfloat16)
    x[0, 0:128] = 0.0
    x[0, 5] = -0.0
    x[1, 130] = float("nan")
    x[2, 300] = float("inf")
    x[2, 301] = -float("inf")
    x[3, 400] = 1e-39  # bf16 subnormal
    x[3, 384:512] = 1e-30
    _assert_exact(x, 128, dev)
    _assert_exact(x, 64, dev)


def test_act_quant_strided_and_3d(dev):
    print("act_quant strided/3d", flush=True)
    x = synthetic.activations(64, 1024, seed=3)
    xs = x[:, :512]  # row stride 1024
    q, s = fp8.act_quant(xs.to(dev), 128)
    qo, so = oracle.act_quant(_bits(xs.contiguous()), 128)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    x3 = x.view(4, 16, 1024)
    q3, s3 = fp8.act_quant(x3.to(dev), 128)
    assert q3.shape == (4, 16, 1024) and s3.shape == (4, 16, 8)
    qo, so = oracle.act_quant(_bits(x), 128)
    np.testing.assert_array_equal(q3.cpu().view(torch.uint8).numpy().reshape(64, 1024), qo)


def test_act_quant_empty(dev):
    q, s = fp8.act_quant(torch.empty(0, 256, dtype=torch.bfloat16, device=dev), 128)
    assert q.shape == (0, 256) and s.shape == (0, 2)


def test_act_quant_full_size_properties(dev):
    """At the 4096x8192 benchmark size: check a sample of rows bit-exactly and
    the size-independent properties on all rows (amax element -> +-448,
    s == amax/448 exactly, |dequant - x| within half an fp8 step)."""
    print("act_quant 4096x8192 properties", flush=True)
    M, K = 4096, 8192
    x = synthetic.activations(M, K, seed=11)
    xd = x.to(dev)
    q, s = fp8.act_quant(xd, 128)
    xf = xd.float().view(M, K // 128, 128)
    amax = xf.abs().amax(-1)
    # IEEE fp32 division on the host (torch's GPU scalar division multiplies
    # by the reciprocal, which is not the contract)
    s_expect = np.maximum(amax.cpu().numpy(), np.float32(1e-10)) / np.float32(448.0)
    np.testing.assert_array_equal(s.cpu().numpy(), s_expect)
    qf = q.float().view(M, K // 128, 128)
    assert torch.all(qf.abs().amax(-1) == 448.0)
    # |q*s - x| <= half an e4m3 step at x/s, in float64 on the host.
    # e4m3 spacing at |v| in [2^e, 2^(e+1)) is 2^(e-3) (2^-9 below 2^-6).
    q64 = qf.cpu().double()
    s64 = torch.from_numpy(s_expect).double().unsqueeze(-1)
    x64 = xf.cpu().double()
    y = (x64 / s64).abs().clamp_min(2.0 ** -6)
    half_step = torch.exp2(torch.floor(torch.log2(y)) - 4)
    assert torch.all((q64 - x64 / s64).abs() <= half_step * (1 + 1e-6))
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(5))[:64]
    qo, so = oracle.act_quant(_bits(x[rows]), 128)
    np.testing.assert_array_equal(q[rows.to(dev)].cpu().view(torch.uint8).numpy(), qo)
    np.testing.assert_array_equal(s[rows.to(dev)].cpu().numpy(), so)


# ------------------------------------------------ float32 / float16 inputs

def _wide(M, K, dtype, seed):
    """Random values over many binades (each row its own magnitude); fp16
    rows stay inside the fp16 range, subnormals included."""
    g = torch.Generator().manual_seed(seed)
    e = torch.randint(-24, 14, (M, 1), generator=g).float() if dtype == torch.float16 else \
        torch.randint(-40, 40, (M, 1), generator=g).float()
    return (torch.randn(M, K, generator=g) * torch.exp2(e)).to(dtype)


def _assert_exact_typed(x_cpu, group, dev):
    q, s = fp8.act_quant(x_cpu.to(dev), group)
    torch.cuda.synchronize()
    K = x_cpu.shape[-1]
    qo, so = oracle.act_quant_f32(x_cpu.float().reshape(-1, K).numpy(), group)
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy().reshape(qo.shape), qo)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(so.shape).view(np.uint32),
                                  so.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("M,K,group", [(1, 128, 128), (37, 4096, 128), (3001, 1024, 128),
                                       (9, 14336, 128), (5, 300, 128), (7, 1000, 64),
                                       (4, 512, 32), (3, 768, 256)])
def test_act_quant_typed_exact(dtype, M, K, group, dev):
    """fp32 and fp16 activations: the group-128 vector kernel (K % 128 == 0)
    and the scalar kernel (other groups, ragged K), bit-exact against the
    oracle's fp32-value quantiser."""
    print(f"act_quant typed {dtype} M={M} K={K} group={group}", flush=True)
    _assert_exact_typed(_wide(M, K, dtype, M * 3 + K + group), group, dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_act_quant_typed_nonfinite_and_extremes(dtype, dev):
    print(f"act_quant typed nonfinite {dtype}", flush=True)
    big = torch.finfo(dtype).max
    tiny = 1e-40 if dtype == torch.float32 else 6e-8
    x = torch.randn(6, 512).to(dtype)
    x[0, 0:128] = 0.0
    x[0, 5] = -0.0
    x[0, 6] = tiny
    x[1, 130] = float("nan")
    x[2, 300] = float("inf")
    x[2, 301] = -float("inf")
    x[3, 384:512] = tiny
    x[4, 0:128] = big
    x[4, 1] = -1.0
    x[5, 128:256] = x[5, 128:256].float().mul(1e-12).to(dtype)  # amax under the 1e-10 floor (fp32)
    _assert_exact_typed(x, 128, dev)
    _assert_exact_typed(x, 64, dev)


def test_act_quant_typed_scale_with_all_ones_mantissa(dev):
    """fp32 groups whose scale has an all-ones mantissa (no bf16 amax gives
    one): the reciprocal and the quotients still match IEEE division."""
    print("act_quant typed all-ones scale", flush=True)
    g = np.random.default_rng(21)
    rows = []
    for e in range(-20, 20):
        s_t = np.float32(np.ldexp(np.float32(2.0 - 2.0 ** -23), e))
        center = int(np.float32(s_t * np.float32(448)).view(np.uint32))
        for u in range(center - 3, center + 4):
            a = np.uint32(u).view(np.float32)
            if ((a / np.float32(448)).view(np.uint32) & 0x7FFFFF) == 0x7FFFFF:
                r = (g.standard_normal(128) * float(a) / 4).astype(np.float32)
                r = np.clip(r, -a, a)
                r[g.integers(128)] = a
                rows.append(r)
    assert len(rows) >= 40
    x = torch.from_numpy(np.stack(rows))
    _assert_exact_typed(x, 128, dev)


def test_act_quant_every_fp16_through_cvt(dev):
    """Groups whose amax is exactly 448 have scale 1.0: every finite fp16
    value with |x| <= 448 goes through the convert (127 per group)."""
    print("act_quant exhaustive fp16 cvt", flush=True)
    f = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    vals = f[np.isfinite(f) & (np.abs(f) <= 448.0)]
    per = 127
    G = -(-vals.size // per)
    padded = np.zeros(G * per, dtype=np.float32)
    padded[: vals.size] = vals
    grid = np.full((G, 128), 448.0, dtype=np.float32)
    grid[:, 1:] = padded.reshape(G, per)
    x = torch.from_numpy(grid).to(torch.float16)
    _assert_exact_typed(x, 128, dev)


def test_act_quant_typed_strided_and_3d(dev):
    print("act_quant typed strided/3d", flush=True)
    x = _wide(64, 1024, torch.float32, 5)
    for xs in (x[:, :512], x[:, 3:515]):  # row stride 1024; the second unaligned (scalar kernel)
        q, s = fp8.act_quant(xs.to(dev), 128)
        qo, so = oracle.act_quant_f32(xs.contiguous().numpy(), 128)
        np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), qo)
        np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    x3 = _wide(64, 1024, torch.float16, 6).view(4, 16, 1024)
    q3, s3 = fp8.act_quant(x3.to(dev), 128)
    assert q3.shape == (4, 16, 1024) and s3.shape == (4, 16, 8) and q3.dtype == torch.float8_e4m3fn
    qo, so = oracle.act_quant_f32(x3.float().reshape(64, 1024).numpy(), 128)
    np.testing.assert_array_equal(q3.cpu().view(torch.uint8).numpy().reshape(64, 1024), qo)


def test_act_quant_typed_entry_point_bf16_is_act_quant(dev):
    """Through the C ABI: x_dtype = BF16 gives fp8b_act_quant's bits."""
    from hf_kernels_helion_amd import _native
    lib = _native.load()
    x = synthetic.activations(33, 2048, seed=9).to(dev)
    q1 = torch.empty(33, 2048, dtype=torch.uint8, device=dev)
    q2 = torch.empty_like(q1)
    s1 = torch.empty(33, 16, device=dev)
    s2 = torch.empty_like(s1)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fp8b_act_quant(x.data_ptr(), 2048, q1.data_ptr(), 2048, s1.data_ptr(), 16, 1,
                              33, 2048, 128, st) == 0
    assert lib.fp8b_act_quant_typed(x.data_ptr(), 2048, _native.BF16, q2.data_ptr(), 2048,
                                    s2.data_ptr(), 16, 1, 33, 2048, 128, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1.view(torch.int32), s2.view(torch.int32))
