"""CPU checks of the C ABI: the library loads, exports every symbol that
include/fp8_blockwise.h declares, and rejects bad arguments before touching
the GPU."""
import ctypes
import re
from pathlib import Path

import pytest

from hf_kernels_helion_amd import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "fp8_blockwise.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fp8b_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ("fp8b_act_quant", "fp8b_w8a8_block_matmul", "fp8b_gemm_workspace_size",
              "fp8b_silu_and_mul", "fp8b_silu_and_mul_quant", "fp8b_version", "fp8b_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for n in declared_functions():
        assert hasattr(lib, n), n
        assert n in _native.SIGNATURES, f"{n} missing from the ctypes signature table"


def test_version_and_error_text():
    lib = _native.load()
    assert lib.fp8b_version() == 0x000100
    assert isinstance(lib.fp8b_last_error(), bytes)


def test_gemm_rejects_bad_args_without_gpu():
    lib = _native.load()
    # negative M
    st = lib.fp8b_w8a8_block_matmul(None, 128, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    _native.BF16, -1, 128, 128, 128, 128, None, 0, None)
    assert st == 2 and b"bad dims" in lib.fp8b_last_error()
    # lda < K
    st = lib.fp8b_w8a8_block_matmul(None, 64, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    _native.BF16, 4, 128, 128, 128, 128, None, 0, None)
    assert st == 2
    # bad block size
    st = lib.fp8b_w8a8_block_matmul(None, 128, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    _native.BF16, 4, 128, 128, 0, 128, None, 0, None)
    assert st == 4
    # bad out dtype
    st = lib.fp8b_w8a8_block_matmul(None, 128, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    9, 4, 128, 128, 128, 128, None, 0, None)
    assert st == 5
    # null pointers with non-empty sizes
    st = lib.fp8b_w8a8_block_matmul(None, 128, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    _native.BF16, 4, 128, 128, 128, 128, None, 0, None)
    assert st == 1
    # empty problem is a no-op success
    st = lib.fp8b_w8a8_block_matmul(None, 128, None, 128, None, 1, 1, None, 1, 1, None, 128,
                                    _native.BF16, 0, 128, 128, 128, 128, None, 0, None)
    assert st == 0


def test_act_quant_rejects_bad_args_without_gpu():
    lib = _native.load()
    assert lib.fp8b_act_quant(None, 128, None, 128, None, 1, 1, 4, 128, 100, None) == 4
    assert lib.fp8b_act_quant(None, 64, None, 128, None, 1, 1, 4, 128, 128, None) == 2
    assert lib.fp8b_act_quant(None, 128, None, 128, None, 1, 1, 4, 128, 128, None) == 1
    assert lib.fp8b_act_quant(None, 128, None, 128, None, 1, 1, 0, 128, 128, None) == 0
    # typed: bad dtype, then the same checks per input type (bf16 delegates)
    aq = lib.fp8b_act_quant_typed
    assert aq(None, 128, 7, None, 128, None, 1, 1, 4, 128, 128, None) == 5
    for t in (_native.F32, _native.BF16, _native.F16):
        assert aq(None, 128, t, None, 128, None, 1, 1, 4, 128, 100, None) == 4
        assert aq(None, 64, t, None, 128, None, 1, 1, 4, 128, 128, None) == 2
        assert aq(None, 128, t, None, 128, None, 1, 1, 4, 128, 128, None) == 1
        assert aq(None, 128, t, None, 128, None, 1, 1, 0, 128, 128, None) == 0
    assert lib.fp8b_silu_and_mul(None, 10, None, 8, 2, 8, None) == 2
    assert lib.fp8b_silu_and_mul_quant(None, 256, None, 128, None, 1, 1, 2, 128, 48, None) == 4


def test_gate_up_silu_quant_rejects_bad_args_without_gpu():
    lib = _native.load()
    f = lib.fp8b_gate_up_silu_quant
    # (A, lda, B, ldb, As, as_sm, as_sk, Bs, bs_sn, bs_sk, q, ldq, s, s_sm, s_sg, M, I, K, stream)
    assert f(None, 512, None, 512, None, 4, 1, None, 4, 1, None, 128, None, 1, 1,
             -1, 128, 512, None) == 2
    assert f(None, 512, None, 512, None, 4, 1, None, 4, 1, None, 64, None, 1, 1,
             4, 128, 512, None) == 2                                     # ldq < I
    assert f(None, 512, None, 512, None, 4, 1, None, 4, 1, None, 192, None, 1, 1,
             4, 192, 512, None) == 2                                     # I % 128
    assert f(None, 208, None, 208, None, 4, 1, None, 4, 1, None, 128, None, 1, 1,
             4, 128, 200, None) == 2                                     # K % 128
    assert b"multiple of 128" in lib.fp8b_last_error()
    assert f(None, 512, None, 512, None, 4, 1, None, 4, 1, None, 128, None, 1, 1,
             4, 128, 512, None) == 1                                     # null pointers
    assert f(None, 512, None, 512, None, 4, 1, None, 4, 1, None, 128, None, 1, 1,
             0, 128, 512, None) == 0                                     # empty
    # rejected before any launch (fake, non-null, 256-byte aligned pointers:
    # nothing is dereferenced or launched on these paths; scale layouts are
    # free, so only operand and output alignment can be refused here)
    P = 1 << 20
    assert f(P + 8, 512, P, 512, P, 4, 1, P, 4, 1, P, 128, P, 1, 1,
             4, 128, 512, None) == 3                                     # A not 16-byte aligned
    assert f(P, 512, P, 512, P, 4, 1, P, 4, 1, P + 4, 128, P, 1, 1,
             4, 128, 512, None) == 3                                     # q not 8-byte aligned
    assert f(P, 512, P, 512, P, 4, 1, P, 4, 1, P, 132, P, 1, 1,
             4, 128, 512, None) == 3                                     # ldq % 8


def test_noalloc_reports_argument_errors_before_scratch():
    """fp8b_w8a8_block_matmul_noalloc checks dims and null pointers before it
    looks at the plan's partials or the scratch array (which needs a device):
    the same codes as fp8b_w8a8_block_matmul, here without a GPU."""
    lib = _native.load()
    f = lib.fp8b_w8a8_block_matmul_noalloc
    P = 1 << 20
    # a decode shape whose plan splits K (partials in the scratch array)
    st = f(None, 14336, P, 14336, P, 112, 1, P, 112, 1, P, 4096, _native.BF16,
           32, 4096, 14336, 128, 128, None)
    assert st == 1 and b"null pointer" in lib.fp8b_last_error()
    st = f(P, 14336, P, 14336, P, 112, 1, P, 112, 1, None, 4096, _native.BF16,
           32, 4096, 14336, 128, 128, None)
    assert st == 1
    st = f(P, 100, P, 14336, P, 112, 1, P, 112, 1, P, 4096, _native.BF16,
           32, 4096, 14336, 128, 128, None)
    assert st == 2 and b"bad dims" in lib.fp8b_last_error()


def test_workspace_size_zero_for_unsupported_blocks():
    lib = _native.load()
    assert lib.fp8b_gemm_workspace_size(32, 4096, 14336, 64, 128) == 0
    assert lib.fp8b_gemm_workspace_size(0, 4096, 14336, 128, 128) == 0


def test_plans_split_k_only_within_one_wave():
    """The tile planner through the split-K workspace it asks for, on 256 CUs
    (MI355X, and the count assumed without a device): small grids run one
    workgroup per 32x32 tile and need no partials, for block and per-row
    weight scales; 128x128 grids split K only while the split grid still
    fits one workgroup per CU; long-K grids of 256x128 tiles split twice as
    often, keeping 28 K-blocks per split; the decode plan splits K as often
    as the grid still fits one workgroup per CU, once more where block
    scales would otherwise get exactly 32 K-blocks per split."""
    lib = _native.load()

    def ws(M, N, K, block_n=128):
        return lib.fp8b_gemm_workspace_size(M, N, K, block_n, 128)

    for shape in [(512, 512, 2048), (64, 4096, 4096), (32, 14336, 4096), (1, 8192, 4096),
                  (2048, 1024, 2048), (768, 768, 4096), (65, 96, 4096), (32, 4096, 4096)]:
        assert ws(*shape) == 0 and ws(*shape, block_n=1) == 0, shape
    assert ws(1536, 1536, 4096) == 0                      # 144 tiles: two ways would need two waves
    assert ws(1024, 2048, 14336) == 4 * 1024 * 2048 * 4   # 64 tiles of 256x128, four ways
    assert ws(512, 2048, 14336) == 4 * 512 * 2048 * 4     # 64 tiles of 128x128, four ways
    #                                                       (eight 256x128 ways: 14 K-blocks)
    assert ws(2048, 1024, 14336) == 2 * 2048 * 1024 * 4   # N = 1024: 128x128, two ways
    assert ws(1024, 1024, 16384) == 4 * 1024 * 1024 * 4   # 64 tiles, four ways
    assert ws(1024, 2048, 4096) == 0 and ws(960, 1024, 4096) == 0   # 64x64 tiles
    assert ws(256, 8192, 2048) == 0                       # 512 64x64 tiles, 16 K-blocks
    assert ws(768, 2048, 4096) == 0                       # 384 64x64 tiles, N <= 16 M
    assert ws(128, 11008, 4096) > 0                       # 344 64x64 tiles, N > 16 M: split
    assert ws(128, 8192, 8192) > 0                        # 256 64x64 tiles of 64 K-blocks,
    #                                                       N > 16 M: split 128x128 tiles
    assert ws(128, 4096, 4096) == 0 and ws(256, 4096, 8192) == 0    # 64x64 tiles
    assert ws(256, 8192, 8192) == 2 * 256 * 8192 * 4      # 512 64x64 tiles of 64 K-blocks:
    #                                                       128x128 tiles split two ways
    assert ws(32, 2048, 14336) == 16 * 32 * 2048 * 4      # decode: 16 column tiles x 16
    assert ws(32, 4096, 14336) == 8 * 32 * 4096 * 4       # decode: 32 column tiles x 8
    assert ws(64, 4096, 14336) == 8 * 64 * 4096 * 4       # decode with 64 rows
    assert ws(32, 7168, 8192) == 4 * 32 * 7168 * 4        # 56 column tiles x 4, not 5
    assert ws(32, 7168, 8192, block_n=1) == 4 * 32 * 7168 * 4
    assert ws(16, 12800, 8192) == 3 * 16 * 12800 * 4      # 100 tiles: 2 splits of 32 -> 3
    assert ws(16, 12800, 8192, block_n=1) == 2 * 16 * 12800 * 4   # per-row: 2
    assert ws(64, 8192, 8192, block_n=1) == 4 * 64 * 8192 * 4     # per-row decode, 64 rows
    assert ws(8, 18432, 8192) == 0                        # 144 tiles, unsplit
    assert ws(32, 28672, 4096) == 0                       # 224 tiles, unsplit
    assert ws(48, 16384, 4096) == 2 * 48 * 16384 * 4      # decode over 32x32 tiles: 128 x 2
    assert ws(48, 16384, 4096, block_n=1) == 2 * 48 * 16384 * 4
    assert ws(8, 16384, 2048) == 0 and ws(16, 28672, 2048) == 0   # small-grid or unsplit
    assert ws(96, 4096, 7168) > 0                         # 384 32x32 tiles of 56 K-blocks: split
    assert ws(72, 5120, 7168) == 0 and ws(96, 4096, 4096) == 0     # 32x32 tiles
    assert ws(32, 14336, 4096) == 0                       # 448 32x32 tiles (112 columns)
    assert ws(56, 14336, 14336) == 2 * 56 * 14336 * 4     # decode: 112 column tiles x 2
    assert ws(64, 28672, 4096) == 0                       # decode: 224 column tiles, unsplit
    assert ws(64, 8192, 8192) == 4 * 64 * 8192 * 4        # decode, not 512 32x32 tiles
    assert ws(64, 4096, 8192) == 0                        # 256 32x32 tiles (one per CU)
    assert ws(64, 12288, 4096) == 0                       # 768 32x32 tiles of 32 K-blocks
    assert ws(4096, 4096, 8192) == 0


def test_status_to_runtime_error():
    with pytest.raises(RuntimeError, match="FP8B_ERR_DIMS"):
        _native.check(2, "probe")
