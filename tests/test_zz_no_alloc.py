"""fp8b_w8a8_block_matmul_noalloc (the entry point that allocates nothing)
against fp8b_w8a8_block_matmul with a caller workspace, through the C ABI:
bit for bit (same kernels, same summation order), on calls in a row that
reuse the library's scratch array with a smaller problem second, on the
split-K 256x128, 128x128 and decode plans and a plan without split-K, and
captured in a HIP graph as the process's first calls of the entry point (the
scratch address is resolved inside the capture); the scratch holds the
partials of every plan on this device, for block and per-row weight scales
(plans whose partials would exceed it are refused with FP8B_ERR_WORKSPACE)."""
import gc

import pytest
import torch

from hf_kernels_helion_amd import _native
from hf_kernels_helion_amd.finegrained_fp8_helion import synthetic

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # FP8B_NOALLOC_SCRATCH_BYTES


def _operands(M, N, K, seed, dev):
    x = synthetic.activations(M, K, seed=seed)
    from hf_kernels_helion_amd import finegrained_fp8_helion as fp8
    q, s = fp8.act_quant(x.to(dev), 128)
    W, Bs = synthetic.weights(N, K, seed=seed + 1)
    return q, W.to(dev), s, Bs.to(dev)


def _args(A, B, As, Bs, C, code):
    M, K = A.shape
    N = B.shape[0]
    return (A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0), As.data_ptr(), As.stride(0),
            As.stride(1), Bs.data_ptr(), Bs.stride(0), Bs.stride(1), C.data_ptr(), C.stride(0),
            code, M, N, K, 128, 128)


def _reference(A, B, As, Bs, out):
    """fp8b_w8a8_block_matmul with a caller workspace into out (bf16)."""
    lib = _native.load()
    M, K = A.shape
    N = B.shape[0]
    ws_n = lib.fp8b_gemm_workspace_size(M, N, K, 128, 128)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=A.device)
    st = lib.fp8b_w8a8_block_matmul(*_args(A, B, As, Bs, out, _native.BF16),
                                    ws.data_ptr() if ws_n else None, ws_n,
                                    torch.cuda.current_stream().cuda_stream)
    _native.check(st, "fp8b_w8a8_block_matmul")
    torch.cuda.synchronize()
    return ws_n


def test_noalloc_in_graph_capture(dev):
    """A decode call (split-K over 16 column tiles) and a 128x128 split-K call
    captured in one HIP graph. First in this file, so in a fresh process (or
    after the other test files, none of which calls this entry point) these
    are the process's first calls of it: the scratch address is resolved
    inside the capture. Nothing is allocated across the calls (torch's
    allocator unchanged, the device's free memory not lowered), and every
    replay, with eager work and synchronisation in between, equals the
    workspace entry point bit for bit."""
    lib = _native.load()
    cases = [_operands(32, 2048, 14336, seed=301, dev=dev),
             _operands(300, 1024, 16384, seed=303, dev=dev)]
    outs = [torch.empty(c[0].shape[0], c[1].shape[0], dtype=torch.bfloat16, device=dev)
            for c in cases]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        alloc0 = torch.cuda.memory_allocated()
        for c, o in zip(cases, outs):
            st = lib.fp8b_w8a8_block_matmul_noalloc(*_args(*c, o, _native.BF16),
                                                    side.cuda_stream)
            _native.check(st, "fp8b_w8a8_block_matmul_noalloc (captured)")
        assert torch.cuda.memory_allocated() == alloc0
    torch.cuda.synchronize()
    # eager calls take no device memory (torch's graph context itself
    # releases cached blocks, so this is checked outside it). The runtime may
    # hand back memory that earlier tests released (destroyed graphs, freed
    # pools) at any synchronisation, which only raises the free figure; an
    # allocation by the calls would lower it.
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free0 = torch.cuda.mem_get_info()[0]
    for c, o in zip(cases, outs):
        _native.check(lib.fp8b_w8a8_block_matmul_noalloc(
            *_args(*c, o, _native.BF16), torch.cuda.current_stream().cuda_stream), "noalloc")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] >= free0
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for c, o in zip(cases, outs):
            ref = torch.empty_like(o)
            assert _reference(*c, ref) > 0
            assert torch.equal(o, ref)


def _both(A, B, As, Bs, dtype):
    lib = _native.load()
    code = {torch.float32: _native.F32, torch.bfloat16: _native.BF16}[dtype]
    M, K = A.shape
    N = B.shape[0]
    stream = torch.cuda.current_stream().cuda_stream
    ws_n = lib.fp8b_gemm_workspace_size(M, N, K, 128, 128)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=A.device)
    ref = torch.empty(M, N, dtype=dtype, device=A.device)
    st = lib.fp8b_w8a8_block_matmul(*_args(A, B, As, Bs, ref, code),
                                    ws.data_ptr() if ws_n else None, ws_n, stream)
    _native.check(st, "fp8b_w8a8_block_matmul")
    out = torch.full((M, N), float("nan"), dtype=dtype, device=A.device)
    st = lib.fp8b_w8a8_block_matmul_noalloc(*_args(A, B, As, Bs, out, code), stream)
    _native.check(st, "fp8b_w8a8_block_matmul_noalloc")
    torch.cuda.synchronize()
    return out, ref, ws_n


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_point_twice(dtype, dev):
    """Two calls in a row through the scratch array, the second smaller (so
    the scratch still holds the first call's partials beyond the second's):
    256x128 tiles split four ways (32 MiB of partials, the whole array),
    then 128x128 tiles split eight ways; then a decode shape and an unsplit
    one."""
    shapes = [(1024, 2048, 14336), (300, 1024, 16384), (32, 2048, 14336), (1024, 4096, 1024)]
    used = []
    for i, (M, N, K) in enumerate(shapes):
        print(f"noalloc M={M} N={N} K={K} {dtype}", flush=True)
        A, B, As, Bs = _operands(M, N, K, seed=100 + i, dev=dev)
        out, ref, ws_n = _both(A, B, As, Bs, dtype)
        used.append(ws_n)
        assert torch.equal(out, ref)
    assert used[0] > used[1] > 0 and used[2] > 0 and used[3] == 0
    assert max(used) <= SCRATCH_BYTES


def test_noalloc_scratch_holds_every_split_plan(dev):
    """Split-K plans keep their grids within about one wave of workgroups:
    128x128 grids at most one per CU (16 MiB of fp32 partials on 256 CUs),
    256x128 grids one per CU (32 MiB), decode grids (at most 64 rows) under
    two per CU (under 16 MiB). Sweeps the worst cases of each over N at a
    long K: on this device every plan fits the scratch array, or (a device
    with more CUs) the largest is refused before any launch, with the limit
    named."""
    lib = _native.load()
    K = 131072
    worst, shape = 0, None
    for block_n in (128, 1):
        for M in (1, 16, 32, 48, 49, 64, 65, 128, 129, 256, 1000):
            for N in range(128, 40064, 128):
                need = lib.fp8b_gemm_workspace_size(M, N, K, block_n, 128)
                if need > worst:
                    worst, shape = need, (M, N, block_n)
    print(f"largest split-K partials: {worst} bytes at M, N = {shape}, K = {K}", flush=True)
    assert worst > 0
    if worst <= SCRATCH_BYTES:
        return
    M, N, block_n = shape
    A = torch.zeros(M, K, dtype=torch.float8_e4m3fn, device=dev)
    B = torch.zeros(N, K, dtype=torch.float8_e4m3fn, device=dev)
    As = torch.ones(M, K // 128, device=dev)
    Bs = torch.ones((N + block_n - 1) // block_n, K // 128, device=dev)
    C = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    args = list(_args(A, B, As, Bs, C, _native.BF16))
    args[-2] = block_n
    st = lib.fp8b_w8a8_block_matmul_noalloc(*args, torch.cuda.current_stream().cuda_stream)
    assert st == 6 and b"FP8B_NOALLOC_SCRATCH_BYTES" in lib.fp8b_last_error()


def test_noalloc_argument_errors_match(dev):
    lib = _native.load()
    st = lib.fp8b_w8a8_block_matmul_noalloc(None, 64, None, 128, None, 1, 1, None, 1, 1, None,
                                            128, _native.BF16, 4, 128, 128, 128, 128, None)
    assert st == 2 and b"bad dims" in lib.fp8b_last_error()
    st = lib.fp8b_w8a8_block_matmul_noalloc(None, 128, None, 128, None, 1, 1, None, 1, 1, None,
                                            128, _native.BF16, 0, 128, 128, 128, 128, None)
    assert st == 0
