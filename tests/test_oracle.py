"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

The reference ships no golden vectors or known-answer tests for this path
(its fp8 test is an unedited scaffold), and its Helion kernel cannot run
here. Each oracle function is therefore pinned by something independent of
its own code:
  * library routines: torch's float8_e4m3fn cast and fp32/fp64 CPU math;
  * closed forms the contract fixes (s == amax/448, the amax element maps to
    +-448, power-of-two scale invariance, exact small-integer products);
  * brute force: nearest-grid search over all e4m3 codes, float64 matmul of
    the dequantised operands on tiny shapes.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def _bf16_bits_all():
    return np.arange(65536, dtype=np.uint32)


def _f32_of_bf16(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def _torch_e4m3(x_f32):
    return torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


# ---------------------------------------------------------------- e4m3 codec

def test_e4m3_encode_matches_torch_for_every_bf16():
    f = _f32_of_bf16(_bf16_bits_all())
    np.testing.assert_array_equal(oracle.e4m3fn_from_f32(f), _torch_e4m3(f))


def test_e4m3_encode_matches_golden_table():
    z = np.load(GOLDEN / "e4m3fn_cast_table.npz")
    f = _f32_of_bf16(_bf16_bits_all())
    np.testing.assert_array_equal(oracle.e4m3fn_from_f32(f), z["enc"])


def test_e4m3_encode_dense_fp32_sweep_and_ties():
    # every 97th fp32 pattern in [2^-12, 512) plus exact midpoints and their
    # one-ulp neighbours around every representable magnitude
    lo, hi = np.float32(2.0 ** -12).view(np.uint32), np.float32(512.0).view(np.uint32)
    pats = np.arange(lo, hi, 97, dtype=np.uint32)
    vals = pats.view(np.float32)
    dec = oracle.e4m3fn_to_f32(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((dec[:-1] + dec[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)),
                           np.nextafter(mids, np.float32(1e9)), np.float32([464, 480, 479.99997])])
    x = np.concatenate([vals, near, -vals[::7], -near])
    np.testing.assert_array_equal(oracle.e4m3fn_from_f32(x), _torch_e4m3(x))


def test_e4m3_decode_matches_torch_and_golden():
    codes = np.arange(256, dtype=np.uint8)
    mine = oracle.e4m3fn_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    z = np.load(GOLDEN / "e4m3fn_cast_table.npz")
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(mine), nan) and np.array_equal(np.isnan(z["dec"]), nan)
    np.testing.assert_array_equal(mine[~nan], ref[~nan])
    np.testing.assert_array_equal(mine[~nan], z["dec"][~nan])


# ---------------------------------------------------------------- act_quant

def _rand_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)
    return x, x.view(torch.int16).numpy().view(np.uint16)


def _nearest_e4m3_bruteforce(y):
    """RNE to e4m3fn by exhaustive search over the finite codes (ties to the
    even code), for finite |y| <= 464."""
    codes = np.arange(0, 0x7F, dtype=np.uint8)  # non-negative finite codes
    vals = oracle.e4m3fn_to_f32(codes).astype(np.float64)
    a = np.abs(y.astype(np.float64))[:, None]
    d = np.abs(vals[None, :] - a)
    best = d.min(axis=1, keepdims=True)
    cand = np.where(d == best, codes[None, :].astype(np.int32), 10 ** 6)
    even = np.where((cand % 2 == 0) & (cand < 10 ** 6), cand, 10 ** 6).min(axis=1)
    anyc = cand.min(axis=1)
    pick = np.where(even < 10 ** 6, even, anyc).astype(np.uint8)
    return pick | np.where(np.signbit(y), 0x80, 0).astype(np.uint8)


def test_act_quant_closed_forms():
    x, bits = _rand_bf16((37, 640), 1)
    q, s = oracle.act_quant(bits, 128)
    xf = x.float().numpy().reshape(37, 5, 128)
    amax = np.abs(xf).max(axis=-1)
    # scale = amax / 448 as one IEEE fp32 division
    np.testing.assert_array_equal(s, np.maximum(amax, np.float32(1e-10)) / np.float32(448.0))
    # the element holding the group's amax quantises to +-448
    qg = oracle.e4m3fn_to_f32(q).reshape(37, 5, 128)
    np.testing.assert_array_equal(np.abs(qg).max(axis=-1), np.float32(448.0))


def test_act_quant_rounding_is_nearest_even_bruteforce():
    x, bits = _rand_bf16((8, 256), 2, scale=3.0)
    q, s = oracle.act_quant(bits, 128)
    xf = x.float().numpy().reshape(8, 2, 128)
    y = (xf / s[:, :, None]).astype(np.float32).ravel()  # IEEE fp32 division
    np.testing.assert_array_equal(q.ravel(), _nearest_e4m3_bruteforce(y))


def test_act_quant_power_of_two_scale_invariance():
    x, bits = _rand_bf16((16, 512), 3)
    q, s = oracle.act_quant(bits, 128)
    for k in (-8, -1, 3, 10):
        xk = (x.float() * (2.0 ** k)).to(torch.bfloat16)  # exact in bf16
        qk, sk = oracle.act_quant(xk.view(torch.int16).numpy().view(np.uint16), 128)
        np.testing.assert_array_equal(qk, q)
        np.testing.assert_array_equal(sk, s * np.float32(2.0 ** k))


def test_act_quant_matches_torch_formulation():
    x, bits = _rand_bf16((64, 1024), 4, scale=0.7)
    q, s = oracle.act_quant(bits, 128)
    tq, ts = torch_ref.act_quant(x, 128)
    np.testing.assert_array_equal(q, tq.view(torch.uint8).numpy())
    np.testing.assert_array_equal(s, ts.numpy())


def test_act_quant_ragged_group_and_sizes():
    x, bits = _rand_bf16((3, 300), 5)
    for g in (32, 64, 128, 256):
        q, s = oracle.act_quant(bits, g)
        assert q.shape == (3, 300) and s.shape == (3, -(-300 // g))
        xf = x.float().numpy()
        last = np.abs(xf[:, (s.shape[1] - 1) * g:]).max(axis=1)
        np.testing.assert_array_equal(s[:, -1], np.maximum(last, np.float32(1e-10)) / np.float32(448))


def test_act_quant_nonfinite_and_zero_policy():
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    x[0, :] = 0.0
    x[0, 3] = -0.0
    x[1, 7] = float("nan")
    x[1, 8] = 2.0
    x[2, 9] = float("inf")
    x[2, 10] = -3.0
    x[2, 11] = -float("inf")
    x[3, :] = 1.0
    bits = x.view(torch.int16).numpy().view(np.uint16)
    q, s = oracle.act_quant(bits, 128)
    assert s[0, 0] == np.float32(1e-10) / np.float32(448) and q[0, 3] == 0x80 and q[0, 0] == 0
    assert np.isnan(s[1, 0]) and np.all(q[1] == 0x7F)
    assert np.isinf(s[2, 0]) and q[2, 9] == 0x7F and q[2, 11] == 0x7F and q[2, 10] == 0x80
    assert q[2, 0] == 0x00
    assert s[3, 0] == np.float32(1.0) / np.float32(448) and np.all(q[3] == 0x7E)


def _wide_f32(shape, seed):
    """fp32 values over many binades (each group gets its own magnitude)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    e = torch.randint(-30, 30, (shape[0], 1), generator=g).float()
    return (x * torch.exp2(e)).numpy()


def test_act_quant_f32_equals_bf16_oracle_on_bf16_values():
    x, bits = _rand_bf16((24, 640), 11, scale=2.0)
    q, s = oracle.act_quant(bits, 128)
    qf, sf = oracle.act_quant_f32(x.float().numpy(), 128)
    np.testing.assert_array_equal(qf, q)
    np.testing.assert_array_equal(sf.view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_act_quant_f32_matches_torch_formulation(dtype):
    xw = torch.from_numpy(_wide_f32((48, 1024), 12))
    if dtype == torch.float16:
        xw = (xw * 1e-4).clamp(-6e4, 6e4).to(torch.float16)
    q, s = oracle.act_quant_f32(xw.float().numpy(), 128)
    tq, ts = torch_ref.act_quant(xw, 128)
    np.testing.assert_array_equal(q, tq.view(torch.uint8).numpy())
    np.testing.assert_array_equal(s.view(np.uint32), ts.numpy().view(np.uint32))


def test_act_quant_f32_rounding_bruteforce_and_closed_form():
    x = _wide_f32((8, 256), 13)
    q, s = oracle.act_quant_f32(x, 128)
    xg = x.reshape(8, 2, 128)
    amax = np.abs(xg).max(axis=-1)
    np.testing.assert_array_equal(s, np.maximum(amax, np.float32(1e-10)) / np.float32(448.0))
    y = (xg / s[:, :, None]).astype(np.float32).ravel()
    np.testing.assert_array_equal(q.ravel(), _nearest_e4m3_bruteforce(y))


def test_act_quant_f32_scale_with_all_ones_mantissa():
    """A group whose scale has an all-ones mantissa (possible for fp32 and
    fp16 amax, never for bf16): the quotients still follow the IEEE
    division."""
    amax = np.float32(117440504.0)  # / 448 rounds to 262143.98... = (2 - 2^-23) * 2^17
    s_want = amax / np.float32(448)
    assert (s_want.view(np.uint32) & 0x7FFFFF) == 0x7FFFFF
    g = np.random.default_rng(14)
    x = (g.standard_normal((2, 128)) * 3e7).astype(np.float32)
    x[:, 5] = amax
    q, s = oracle.act_quant_f32(x, 128)
    assert np.all(s[:, 0] == s_want)
    np.testing.assert_array_equal(q.ravel(), _nearest_e4m3_bruteforce((x / s_want).ravel()))


def test_act_quant_f32_nonfinite_subnormal_and_extremes():
    x = np.zeros((5, 128), dtype=np.float32)
    x[0, 3] = -0.0
    x[0, 4] = np.float32(1e-40)            # subnormal, below the 1e-10 floor
    x[1, 7] = np.nan
    x[1, 8] = 2.0
    x[2, 9] = np.inf
    x[2, 10] = -3.0
    x[2, 11] = -np.inf
    x[3, :] = np.float32(3.4028235e38)     # FLT_MAX
    x[3, 1] = -np.float32(1.0)
    x[4, :] = np.float32(5e-11)            # amax below the floor
    q, s = oracle.act_quant_f32(x, 128)
    assert s[0, 0] == np.float32(1e-10) / np.float32(448) and q[0, 3] == 0x80 and q[0, 4] == 0
    assert np.isnan(s[1, 0]) and np.all(q[1] == 0x7F)
    assert np.isinf(s[2, 0]) and q[2, 9] == 0x7F and q[2, 11] == 0x7F and q[2, 10] == 0x80
    assert s[3, 0] == np.float32(3.4028235e38) / np.float32(448) and q[3, 0] == 0x7E
    assert q[3, 1] == 0x80  # -1 / 7.6e35 underflows to a signed fp8 zero
    assert s[4, 0] == np.float32(1e-10) / np.float32(448)
    np.testing.assert_array_equal(q[4], _torch_e4m3(x[4] / s[4, 0]))


# ---------------------------------------------------------------- block GEMM

def _dequant64(A, B, As, Bs, bn, bk):
    M, K = A.shape
    N = B.shape[0]
    a = oracle.e4m3fn_to_f32(A).astype(np.float64) * np.repeat(As.astype(np.float64), bk, 1)[:, :K]
    sb = np.repeat(np.repeat(Bs.astype(np.float64), bn, 0)[:N], bk, 1)[:, :K]
    b = oracle.e4m3fn_to_f32(B).astype(np.float64) * sb
    return a, b


def _operands(M, N, K, bn, bk, seed):
    g = torch.Generator().manual_seed(seed)
    A = (torch.randn(M, K, generator=g) * 0.3).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    B = (torch.randn(N, K, generator=g) * 0.3).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    As = (torch.rand(M, -(-K // bk), generator=g) * 0.5 + 0.5).numpy()
    Bs = (torch.rand(-(-N // bn), -(-K // bk), generator=g) * 0.5 + 0.5).numpy()
    return A, B, As, Bs


@pytest.mark.parametrize("M,N,K,bn,bk", [(5, 131, 256, 128, 128), (7, 33, 200, 16, 64),
                                         (3, 9, 130, 4, 32), (1, 300, 512, 128, 128)])
def test_block_gemm_vs_float64_bruteforce(M, N, K, bn, bk):
    A, B, As, Bs = _operands(M, N, K, bn, bk, seed=M * N + K)
    got = oracle.block_gemm(A, B, As, Bs, (bn, bk))
    a, b = _dequant64(A, B, As, Bs, bn, bk)
    np.testing.assert_allclose(got, a @ b.T, rtol=1e-5, atol=1e-5)


def test_block_gemm_golden_fixture():
    z = np.load(GOLDEN / "gemm_fp64_small.npz")
    got = oracle.block_gemm(z["A"], z["B"], z["As"], z["Bs"], z["block"].tolist())
    np.testing.assert_allclose(got, z["C"], rtol=1e-6, atol=1e-6)


def test_block_gemm_exact_small_integers():
    g = torch.Generator().manual_seed(9)
    A = torch.randint(-6, 7, (12, 384), generator=g).float().to(torch.float8_e4m3fn)
    B = torch.randint(-6, 7, (20, 384), generator=g).float().to(torch.float8_e4m3fn)
    got = oracle.block_gemm(A.view(torch.uint8).numpy(), B.view(torch.uint8).numpy(),
                            np.ones((12, 3), np.float32), np.ones((1, 3), np.float32))
    np.testing.assert_array_equal(got, (A.double() @ B.double().T).numpy().astype(np.float32))


def test_block_gemm_row_scale_power_of_two_is_exact():
    A, B, As, Bs = _operands(6, 256, 512, 128, 128, seed=11)
    base = oracle.block_gemm(A, B, As, Bs)
    As2 = As.copy()
    As2[2] *= 8.0
    got = oracle.block_gemm(A, B, As2, Bs)
    np.testing.assert_array_equal(got[2], base[2] * 8.0)
    np.testing.assert_array_equal(np.delete(got, 2, 0), np.delete(base, 2, 0))


def test_block_gemm_weight_block_scale_selects_column_block():
    # Bs row nb scales exactly the output columns nb*128 .. nb*128+127
    A, B, As, Bs = _operands(4, 384, 256, 128, 128, seed=12)
    base = oracle.block_gemm(A, B, As, Bs)
    Bs2 = Bs.copy()
    Bs2[1] *= 4.0
    got = oracle.block_gemm(A, B, As, Bs2)
    np.testing.assert_array_equal(got[:, 128:256], base[:, 128:256] * 4.0)
    np.testing.assert_array_equal(got[:, :128], base[:, :128])
    np.testing.assert_array_equal(got[:, 256:], base[:, 256:])


def test_block_gemm_kblock_permutation_invariance():
    A, B, As, Bs = _operands(8, 128, 512, 128, 128, seed=13)
    perm = [2, 0, 3, 1]
    Ap = A.reshape(8, 4, 128)[:, perm].reshape(8, 512)
    Bp = B.reshape(128, 4, 128)[:, perm].reshape(128, 512)
    got = oracle.block_gemm(Ap, Bp, As[:, perm], Bs[:, perm])
    np.testing.assert_allclose(got, oracle.block_gemm(A, B, As, Bs), rtol=1e-6, atol=1e-6)


def test_dequant_matmul_vs_torch_float64():
    A, B, As, Bs = _operands(9, 200, 384, 128, 128, seed=14)
    got = oracle.dequant_matmul(A, B, As, Bs)
    a, b = _dequant64(A, B, As, Bs, 128, 128)
    np.testing.assert_allclose(got, (torch.from_numpy(a) @ torch.from_numpy(b).T).numpy(),
                               rtol=1e-6, atol=1e-6)
    # and the reference's torch CPU restatement agrees in bf16
    t = torch_ref.dequant_matmul(torch.from_numpy(A).view(torch.float8_e4m3fn),
                                 torch.from_numpy(B).view(torch.float8_e4m3fn),
                                 torch.from_numpy(As), torch.from_numpy(Bs))
    np.testing.assert_allclose(t.float().numpy(), got, rtol=1e-2, atol=1e-3)


# ---------------------------------------------------------------- silu_and_mul

def test_silu_and_mul_vs_torch_silu():
    g = torch.Generator().manual_seed(15)
    x = (torch.randn(33, 2 * 300, generator=g) * 4).to(torch.bfloat16)
    got = oracle.silu_and_mul(x.view(torch.int16).numpy().view(np.uint16))
    ref = torch_ref.silu_and_mul(x).view(torch.int16).numpy().view(np.uint16)
    gf = _f32_of_bf16(got)
    rf = _f32_of_bf16(ref)
    # silu goes through two different expf implementations: 1 bf16 ulp
    np.testing.assert_allclose(gf, rf, rtol=2 ** -7, atol=1e-30)
    assert np.mean(got == ref) > 0.99


def test_silu_and_mul_special_values():
    x = torch.tensor([[0.0, -0.0, 100.0, -100.0, 2.0, 2.0, 2.0, 2.0]], dtype=torch.bfloat16)
    got = _f32_of_bf16(oracle.silu_and_mul(x.view(torch.int16).numpy().view(np.uint16)))
    # silu(0)=0, silu(100)=100, silu(-100) ~ -3.7e-42 -> times 2
    assert got[0, 0] == 0.0 and got[0, 2] == 200.0 and abs(got[0, 3]) < 1e-30


# ---------------------------------------------------------------- weight quantiser

def test_quant_weight_block_closed_forms():
    g = torch.Generator().manual_seed(16)
    W = (torch.randn(300, 260, generator=g) * 0.02).numpy()
    Wq, Bs = oracle.quant_weight_block(W, (128, 128))
    assert Bs.shape == (3, 3)
    for nb in range(3):
        for kb in range(3):
            blk = W[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            assert Bs[nb, kb] == np.maximum(np.abs(blk).max(), np.float32(1e-10)) / np.float32(448)
            qb = oracle.e4m3fn_to_f32(Wq[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128])
            assert np.abs(qb).max() == 448.0
    np.testing.assert_array_equal(
        Wq, _torch_e4m3((W.reshape(300, 260) /
                         np.repeat(np.repeat(Bs, 128, 0)[:300], 128, 1)[:, :260]).astype(np.float32)))


def test_quant_weight_block_nonfinite_policy():
    """NaN block -> scale NaN and every code 0x7F; +-inf block (no NaN) ->
    scale +inf, 0x7F for the infinities and a signed zero for every finite
    element; the other blocks are untouched by their neighbours."""
    g = torch.Generator().manual_seed(17)
    W = (torch.randn(256, 384, generator=g) * 0.02).numpy()
    W[3, 5] = np.nan                      # block (0, 0)
    W[4, 6] = np.inf                      # NaN wins in the same block
    W[130, 140] = -np.inf                 # block (1, 1)
    W[131, 141] = -0.0
    W[200, 300] = np.inf                  # block (1, 2)
    Wq, Bs = oracle.quant_weight_block(W, (128, 128))
    assert np.isnan(Bs[0, 0]) and np.all(Wq[:128, :128] == 0x7F)
    assert Bs[1, 1] == np.inf and Bs[1, 2] == np.inf
    blk = W[128:256, 128:256]
    expect = np.where(np.isinf(blk), 0x7F, np.where(np.signbit(blk), 0x80, 0x00)).astype(np.uint8)
    np.testing.assert_array_equal(Wq[128:256, 128:256], expect)
    assert Wq[130, 140] == 0x7F and Wq[131, 141] == 0x80
    assert Wq[200, 300] == 0x7F
    # finite blocks: max(amax, 1e-10) / 448 and torch's cast of W / Bs
    for nb, kb in ((0, 1), (0, 2), (1, 0)):
        b = W[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
        s = np.maximum(np.abs(b).max(), np.float32(1e-10)) / np.float32(448)
        assert Bs[nb, kb] == s
        np.testing.assert_array_equal(Wq[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128],
                                      _torch_e4m3((b / s).astype(np.float32)))


def test_quant_weight_block_subnormal_and_zero_blocks():
    """amax below 1e-10 (fp32 subnormals, zeros): the floor sets the scale to
    1e-10/448 and the codes are torch's cast of W / scale (all signed zeros
    here, since |W| / scale < 2^-10)."""
    W = np.zeros((128, 256), np.float32)
    W[:, :128] = np.float32(1e-40) * np.where(np.arange(128) % 2, 1, -1)[:, None]
    W[5, 200] = -0.0
    Wq, Bs = oracle.quant_weight_block(W, (128, 128))
    floor = np.float32(1e-10) / np.float32(448)
    assert Bs[0, 0] == floor and Bs[0, 1] == floor
    np.testing.assert_array_equal(Wq, _torch_e4m3(W / floor))
    assert Wq[0, 0] == 0x80 and Wq[1, 0] == 0x00 and Wq[5, 200] == 0x80


@pytest.mark.parametrize("xt", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("ot", ["float32", "float16", "bfloat16"])
def test_silu_and_mul_typed_vs_torch(xt, ot):
    """The typed silu oracle against torch's CPU evaluation of act.py:25-28
    ((a * sigmoid(a)).to(b.dtype) * b, then .to(out.dtype)): bit-equal for
    fp16 and bf16 inputs; for fp32 inputs torch's vectorised sigmoid and
    numpy's exp differ by an fp32 ulp or two, which can move the output by
    one ulp of its type (rarely, where the product sits on a rounding
    boundary)."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(64, 512, generator=g) * 4).to(getattr(torch, xt))
    a, b = x[:, :256], x[:, 256:]
    ref = ((a.float() * torch.sigmoid(a.float())).to(x.dtype) * b).to(getattr(torch, ot))
    got = oracle.silu_and_mul_typed(x.float().numpy(), xt, ot)
    if xt == "float32":
        ulp = {"float32": 1e-6, "float16": 2 ** -10, "bfloat16": 2 ** -7}[ot]
        torch.testing.assert_close(torch.from_numpy(got), ref.float(), rtol=ulp, atol=1e-30)
        assert (got == ref.float().numpy()).mean() > 0.8
    else:
        assert np.array_equal(got, ref.float().numpy())


def test_silu_and_mul_typed_equals_bf16_oracle():
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(16, 512, generator=g) * 3).to(torch.bfloat16)
    c = oracle.silu_and_mul(x.view(torch.int16).numpy().view(np.uint16))
    cf = (c.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(cf, oracle.silu_and_mul_typed(x.float().numpy(), "bfloat16",
                                                        "bfloat16"))
