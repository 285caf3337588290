"""CPU checks of the GEMM planner through the C ABI's plan query
(fp8b_gemm_plan, fp8b_gate_up_plan, fp8b_act_quant_matmul_plan): the kernel, tile, K splits and grid that
one call launches, pinned for the five BASELINE configurations, the
reference's fp8 tuning shapes (scripts/aot_tune.py:134-136) and the MLP
chain, on a 256-CU MI355X. The plan query makes no GPU call for a given CU
count, so these run without a device; the GPU tests check that every plan
computes the right result."""
import pytest

from hf_kernels_helion_amd import _native

CUS = 256


def plan(M, N, K, block_n=128):
    return _native.gemm_plan(M, N, K, block_n, 128, cu_count=CUS)


def brief(p):
    t = (p["kernel"], p["tile_m"], p["tile_n"], p["splits"], p["workgroups"])
    if p["tail_kernel"] != "none":
        t += (p["tail_kernel"], p["tail_tile_m"], p["tail_tile_n"], p["tail_workgroups"])
    return t


# (M, N, K) -> (kernel, tile_m, tile_n, splits, workgroups[, tail kernel, tile, workgroups])
PINNED = {
    # BASELINE configs
    (512, 512, 2048): ("gemm_tiny_kernel", 32, 32, 1, 256),
    (2048, 2048, 4096): ("gemm_pipe128_kernel", 128, 128, 1, 256),
    (4096, 4096, 8192): ("gemm_pipe256_kernel", 256, 256, 1, 256),
    (32, 4096, 14336): ("gemm_decode_kernel", 32, 128, 8, 256),
    (3001, 28672, 4096): ("gemm_pipe256_kernel", 256, 256, 1, 1280,
                          "gemm_pipe128_kernel", 128, 128, 256),
    (3001, 4096, 14336): ("gemm_pipe192_kernel", 192, 256, 1, 256),
    # the reference's tuning shapes not listed above
    (1024, 1024, 2048): ("gemm_tiny_kernel", 64, 64, 1, 256),
    (4096, 2048, 4096): ("gemm_pipe256x128_kernel", 256, 128, 1, 256),
    (8192, 4096, 8192): ("gemm_pipe256_kernel", 256, 256, 1, 512),
    (8192, 8192, 8192): ("gemm_pipe256_kernel", 256, 256, 1, 1024),
}


@pytest.mark.parametrize("shape", sorted(PINNED))
def test_plan_pinned(shape):
    p = plan(*shape)
    assert brief(p) == PINNED[shape], (shape, p)
    assert p["cu_count"] == CUS
    KB = shape[2] // 128
    assert p["splits"] * p["kb_per_split"] >= KB > (p["splits"] - 1) * p["kb_per_split"]


def test_decode_plan_details():
    """C4: 32 column tiles of 128 x 8 K-splits of 14 K-blocks, the four-stage
    ring, fp32 partials [8, 32, 4096] and the split-K sum."""
    p = plan(32, 4096, 14336)
    assert (p["kb_per_split"], p["ring"], p["reduce"]) == (14, 4, 1)
    assert p["workspace_bytes"] == 8 * 32 * 4096 * 4
    assert p["workspace_bytes"] == _native.load().fp8b_gemm_workspace_size(32, 4096, 14336, 128, 128)


def test_small_grid_waves():
    # C1: one 32x32 tile per CU, eight waves splitting its 16 K-blocks
    assert plan(512, 512, 2048)["waves"] == 8
    # 64x64 tiles, one per CU: four waves
    assert plan(1024, 1024, 2048)["waves"] == 4


@pytest.mark.parametrize("shape,expect", [
    ((4096, 4096, 8192), ("gemm_pipe256_kernel", 256, 256, 1, 256)),
    ((32, 4096, 14336), ("gemm_decode_kernel", 32, 128, 8, 256)),
    ((512, 512, 2048), ("gemm_tiny_kernel", 32, 32, 1, 256)),
])
def test_per_row_plans(shape, expect):
    """deep-gemm's per-row weight scales (block_n = 1) take the same tiles."""
    assert brief(plan(*shape, block_n=1)) == expect


def test_plans_follow_the_cu_count():
    """The CU count is an input: on 128 CUs the decode grid splits four ways
    and C3's 256 tiles of 256x256 are two full waves."""
    p = _native.gemm_plan(32, 4096, 14336, cu_count=128)
    assert (p["kernel"], p["splits"], p["workgroups"]) == ("gemm_decode_kernel", 4, 128)
    p = _native.gemm_plan(4096, 4096, 8192, cu_count=128)
    assert (p["kernel"], p["workgroups"], p["tail_kernel"]) == ("gemm_pipe256_kernel", 256, "none")


def test_generic_plan_for_other_block_sizes():
    p = plan(256, 256, 1000, block_n=64)
    assert p["kernel"] == "gemm_generic_kernel" and p["splits"] == 1


@pytest.mark.parametrize("M,I,K,kernel,tile_m", [
    (3001, 14336, 4096, "gemm_pipe192_kernel", 192),   # C5: 7 full waves of 192x256 tiles
    (1024, 8192, 512, "gemm_pipe256_kernel", 256),     # 256 tiles of 256x256: one wave
    (2048, 14336, 512, "gemm_pipe256_kernel", 256),    # 896 tiles (0.875 fill) vs 1232 (0.96)
    (600, 1024, 512, "gemm_pipe192_kernel", 192),      # one partial wave either way
])
def test_gate_up_plans(M, I, K, kernel, tile_m):
    p = _native.gate_up_plan(M, I, K, cu_count=CUS)
    assert (p["kernel"], p["tile_m"], p["tile_n"], p["splits"]) == (kernel, tile_m, 256, 1)
    assert p["workgroups"] == -(-M // tile_m) * (2 * I // 256)


@pytest.mark.parametrize("M,N,K,kernel,splits,ring", [
    (32, 4096, 14336, "gemm_decode_quant_kernel", 8, 3),   # C4: one kernel, same split
    (16, 4096, 14336, "gemm_decode_quant_kernel", 8, 4),
    (8, 13824, 5120, "gemm_decode_quant_kernel", 2, 4),
    (32, 28672, 4096, "gemm_decode_quant_kernel", 1, 3),
    (1, 4096, 14336, "gemm_skinny_quant_kernel", 1, 0),    # skinny plans, M <= 8
    (8, 4096, 4096, "gemm_skinny_quant_kernel", 1, 0),
    (9, 2048, 8192, "gemm_skinny_kernel", 1, 0),           # 9+ rows: two launches
    (1, 28672, 4096, "gemm_tiny_quant_kernel", 1, 0),      # small-grid plans, M <= 8
    (9, 28672, 4096, "gemm_tiny_kernel", 1, 0),            # 9+ rows, 16 K-blocks per wave
    (12, 8192, 2048, "gemm_tiny_quant_kernel", 1, 0),      # 9..16 rows, 2 K-blocks per wave
    (24, 7168, 8192, "gemm_decode_quant_kernel", 4, 3),
    (33, 4096, 14336, "gemm_decode_kernel", 8, 4),         # 17+ rows of fragments: two launches
    (64, 4096, 14336, "gemm_decode_kernel", 8, 4),
    (3001, 4096, 14336, "gemm_pipe192_kernel", 1, 0),      # not a decode plan
])
def test_act_quant_matmul_plans(M, N, K, kernel, splits, ring):
    """act_quant_w8a8_block_fp8_matmul runs one kernel (act-quant inside the
    GEMM) exactly where the GEMM plan is the one-workgroup-per-CU decode grid
    and M <= 32, the skinny grid and M <= 8, or the small grid and M <= 8
    (M <= 16 with at most 4 K-blocks per wave), with that plan's K split, so
    its result bits equal act-quant + GEMM; elsewhere the GEMM of the
    two-launch path."""
    p = _native.act_quant_matmul_plan(M, N, K, cu_count=CUS)
    g = plan(M, N, K)
    assert (p["kernel"], p["splits"], p["ring"]) == (kernel, splits, ring), p
    assert (p["splits"], p["kb_per_split"], p["workgroups"]) == (
        g["splits"], g["kb_per_split"], g["workgroups"])
    assert p["workspace_bytes"] == _native.load().fp8b_act_quant_matmul_workspace_size(M, N, K)


def test_act_quant_matmul_plan_grids_past_the_cus():
    """A decode grid of more than one workgroup per CU (three-stage ring of
    the GEMM, two workgroups per CU) keeps the two-launch path."""
    g = plan(32, 28672, 8192)
    p = _native.act_quant_matmul_plan(32, 28672, 8192, cu_count=CUS)
    if g["kernel"] == "gemm_decode_kernel" and g["ring"] == 3:
        assert p["kernel"] == "gemm_decode_kernel"
    else:
        assert g["workgroups"] <= CUS and p["kernel"] == "gemm_decode_quant_kernel"


def test_plan_query_rejects_bad_args():
    import ctypes
    lib = _native.load()
    info = _native.PlanInfo()
    assert lib.fp8b_gemm_plan(0, 128, 128, 128, 128, CUS, ctypes.byref(info)) == 2
    assert lib.fp8b_gemm_plan(128, 128, 128, 128, 128, CUS, None) == 1
    assert lib.fp8b_gate_up_plan(128, 100, 512, CUS, ctypes.byref(info)) == 2
    assert lib.fp8b_act_quant_matmul_plan(32, 4096, 200, CUS, ctypes.byref(info)) == 2
    assert lib.fp8b_act_quant_matmul_plan(32, 4096, 256, CUS, None) == 1
