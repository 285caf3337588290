"""The C ABI driven the way the reference's Python side would bind it: a
plain ctypes binding of include/fp8_blockwise.h (it replaces the custom op of
finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/op.py:8-11 and its
call in __init__.py:12-14), loaded straight from the built
libfp8_blockwise.so with no torch op in between, on real operands, against
the CPU oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from hf_kernels_helion_amd import _native
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3

# ---- the ctypes binding a maintainer of the reference would add -----------
lib = ctypes.CDLL(str(_native.LIB_PATH))
P, I = ctypes.c_void_p, ctypes.c_int64
lib.fp8b_w8a8_block_matmul.argtypes = [P, I, P, I, P, I, I, P, I, I, P, I, ctypes.c_int,
                                       I, I, I, I, I, P, ctypes.c_size_t, P]
lib.fp8b_gemm_workspace_size.restype = ctypes.c_size_t
lib.fp8b_gemm_workspace_size.argtypes = [I, I, I, I, I]
lib.fp8b_act_quant.argtypes = [P, I, P, I, P, I, I, I, I, I, P]
lib.fp8b_silu_and_mul_quant.argtypes = [P, I, P, I, P, I, I, I, I, I, P]
lib.fp8b_last_error.restype = ctypes.c_char_p


def w8a8_block_fp8_matmul_bf16(A, B, As, Bs):
    M, K = A.shape; N = B.shape[0]
    C = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    ws_n = lib.fp8b_gemm_workspace_size(M, N, K, 128, 128)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=A.device)
    st = lib.fp8b_w8a8_block_matmul(
        A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0),
        As.data_ptr(), As.stride(0), As.stride(1), Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
        C.data_ptr(), C.stride(0), 1,            # 1 = FP8B_BF16
        M, N, K, 128, 128, ws.data_ptr() if ws_n else None, ws_n,
        torch.cuda.current_stream().cuda_stream)
    if st:
        raise RuntimeError(lib.fp8b_last_error().decode())
    return C


def act_quant(x):
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(M, (K + 127) // 128, dtype=torch.float32, device=x.device)
    st = lib.fp8b_act_quant(x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0),
                            s.data_ptr(), s.stride(0), s.stride(1), M, K, 128,
                            torch.cuda.current_stream().cuda_stream)
    if st:
        raise RuntimeError(lib.fp8b_last_error().decode())
    return q, s
# ------------------------------------------------------------------------------


def _u8(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


@pytest.mark.parametrize("M,N,K", [(512, 512, 2048), (32, 4096, 14336), (300, 640, 1024),
                                   (4096, 4096, 1024)])
def test_ctypes_binding_act_quant_then_gemm_vs_oracle(M, N, K, dev):
    """act_quant and the GEMM through the raw C ABI: codes and scales
    bit-exact, the bf16 output within the north-star tolerance of
    oracle.block_gemm (sampled rows for the large shape)."""
    print(f"ctypes C ABI M={M} N={N} K={K}", flush=True)
    x = synthetic.activations(M, K, seed=M + 5 * N, outlier_frac=0.01)
    W, Bs = synthetic.weights(N, K, seed=K + N)
    q, s = act_quant(x.to(dev))
    torch.cuda.synchronize()
    qo, so = oracle.act_quant(x.view(torch.int16).numpy().view(np.uint16), 128)
    np.testing.assert_array_equal(_u8(q), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    C = w8a8_block_fp8_matmul_bf16(q, W.to(dev), s, Bs.to(dev))
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 512 else np.array([0, 1, M // 2, M - 2, M - 1])
    ref = oracle.block_gemm(qo[rows], _u8(W), so[rows], Bs.numpy())
    torch.testing.assert_close(C[torch.from_numpy(rows).to(dev)].float().cpu(),
                               torch.from_numpy(ref).to(torch.bfloat16).float(),
                               rtol=RTOL, atol=ATOL)


def test_ctypes_binding_reports_errors(dev):
    """A row stride below K is rejected on the host (FP8B_ERR_DIMS) before
    any launch, and the binding raises with the library's text; K = 0 gives
    zeros."""
    A = torch.zeros(4, 512, dtype=torch.float8_e4m3fn, device=dev)
    B = torch.zeros(128, 256, dtype=torch.float8_e4m3fn, device=dev)
    Bs = torch.ones(1, 2, device=dev)
    overlapping = A.as_strided((4, 256), (128, 1))     # lda = 128 < K = 256
    with pytest.raises(RuntimeError, match="bad dims"):
        w8a8_block_fp8_matmul_bf16(overlapping, B, torch.ones(4, 2, device=dev), Bs)
    C = w8a8_block_fp8_matmul_bf16(A[:, :256], B, torch.ones(4, 2, device=dev), Bs)
    assert torch.equal(C.float(), torch.zeros(4, 128, device=dev))


def _quant_call(fn, x, ldx, q, ldq, s, s_sm, s_sg, M, K):
    st = fn(x.data_ptr(), ldx, q.data_ptr(), ldq, s.data_ptr(), s_sm, s_sg, M, K, 128,
            torch.cuda.current_stream().cuda_stream)
    if st:
        raise RuntimeError(lib.fp8b_last_error().decode())


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("K", [7168, 8192, 14336, 4096])
def test_ctypes_quant_block_shapes_strided(silu, K, dev):
    """fp8b_act_quant and fp8b_silu_and_mul_quant on padded rows (ldx, ldq
    past the row), column-major scales and a guard band after every row:
    the same codes and scales as the packed call, and nothing written past
    a row's end. K covers each block shape of the group-128 kernels at 600
    rows: act-quant 16 x 4 with 8 idle 16-lane rows (K = 7168), 16 x 4
    (8192), 16 x 2 with 16 idle rows (14336), 16 x 2 (4096); SiLU-quant
    (K = d) 4 x 2, 16 x 4, 8 x 2, 16 x 2."""
    M = 600
    fn = lib.fp8b_silu_and_mul_quant if silu else lib.fp8b_act_quant
    width = 2 * K if silu else K
    print(f"ctypes quant strided silu={silu} M={M} K={K}", flush=True)
    x = (synthetic.activations(M, width, seed=K + silu, outlier_frac=0.01) * 2).to(dev)
    G = K // 128
    q0 = torch.empty(M, K, dtype=torch.uint8, device=dev)
    s0 = torch.empty(M, G, dtype=torch.float32, device=dev)
    _quant_call(fn, x, width, q0, K, s0, G, 1, M, K)
    xp = torch.zeros(M, width + 256, dtype=torch.bfloat16, device=dev)
    xp[:, :width] = x
    qp = torch.full((M, K + 128), 0xA5, dtype=torch.uint8, device=dev)
    sp = torch.full((G + 1, M), -7.0, dtype=torch.float32, device=dev)  # column-major + a guard row
    _quant_call(fn, xp, width + 256, qp, K + 128, sp, 1, M, M, K)
    torch.cuda.synchronize()
    assert torch.equal(qp[:, :K], q0)
    assert torch.all(qp[:, K:] == 0xA5)
    assert torch.equal(sp[:G].t().contiguous().view(torch.int32), s0.view(torch.int32))
    assert torch.all(sp[G] == -7.0)
