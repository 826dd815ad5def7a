"""GPU tests of gemm_tn's decode plans (``dk_gemm_tn_ws`` and the torch op
``gemm_tn``, which passes it a workspace from the caching allocator).

Decode shapes run one workgroup per CU, with wide column tiles and, where
that leaves too few tiles, the K reduction split over workgroups writing fp32
partial tiles that a second kernel sums in a fixed order; from M = 32 (and
for N > 32768) the LDS-DMA kernel's 64-row tiles take over where they fill
the CUs. Checks: every (row tiles, workgroup shape, split or not) skinny plan
and every (tile columns, split or not) decode DMA plan against the fp32
oracle with a bias and a ragged N, in fp16 and bf16; every partial entry written
(workspace pre-filled with NaN); determinism (two calls equal bit for bit); a
missing or undersized workspace runs exactly ``dk_gemm_tn``; the torch op
equals the C-ABI call; graph replays equal the eager result.
"""

import ctypes

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from parity import assert_max_abs, gemm_f32
from test_gemm_plan import COVERAGE_SHAPES, DECODE_DMA_SHAPES

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# The Llama-3-8B decode projections that split K, and ragged splits.
SPLIT_SHAPES = [
    (64, 4096, 14336),  # MLP down projection: 64 x 128 tiles, 8 splits
    (32, 4096, 14336),  # the same
    (16, 4096, 14336),  # skinny, 2 splits
    (64, 4096, 4096),  # attention output projection: 64 x 64 tiles, 4 splits
    (48, 6144, 4096),  # fused qkv projection: 64 x 128 tiles, 4 splits
    (17, 1000, 8200),  # ragged N and K, the last split shorter
    (33, 4101, 4104),  # N not a multiple of 4 (scalar reduce)
    (64, 8, 1024),  # one N tile
    (1, 1536, 3072),  # 5 splits
    (16, 1280, 14336),  # 6 splits
    (1, 2304, 4096),  # 7 splits
]


def _operands(M, N, K, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype)
    return a, b, bias


def _call(fn, a, b, bias, c, *ws):
    M, K = a.shape
    N = b.shape[0]
    rc = fn(capi.dtype_code(a.dtype), a.data_ptr(), b.data_ptr(), None if bias is None else bias.data_ptr(),
            c.data_ptr(), M, N, K, a.stride(0), b.stride(0), c.stride(0), *ws, _stream())
    assert rc == 0, capi.last_error()


def _ws_call(a, b, bias, c, ws, nbytes):
    _call(capi.lib().dk_gemm_tn_ws, a, b, bias, c, None if ws is None else ws.data_ptr(), nbytes)


@pytest.mark.parametrize("M,N,K", COVERAGE_SHAPES + DECODE_DMA_SHAPES)
def test_every_plan_against_the_oracle(M, N, K):
    dtype = torch.bfloat16 if (M + N) % 2 else torch.float16
    a, b, bias = _operands(M, N, K, dtype, M * 131 + N)
    plan = capi.gemm_plan(M, N, K)
    print(f"gemm plan {M}x{N}x{K}: {plan}", flush=True)
    assert_max_abs(dk.gemm(a, b, bias), gemm_f32(a, b, bias), dtype, f"gemm {M}x{N}x{K} plan {plan}")
    if plan[2] > 1:  # the same shape unsplit (no workspace)
        c = torch.empty(M, N, device="cuda", dtype=dtype)
        _call(capi.lib().dk_gemm_tn, a, b, bias, c)
        assert_max_abs(c, gemm_f32(a, b, bias), dtype, f"gemm {M}x{N}x{K} unsplit")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_split_k_parity_and_determinism(dtype, M, N, K):
    L = capi.lib()
    splits = capi.gemm_plan(M, N, K)[2]
    assert splits > 1
    nbytes = L.dk_gemm_tn_workspace_bytes(M, N, K)
    assert nbytes == splits * M * N * 4
    a, b, bias = _operands(M, N, K, dtype, M * 31 + K)
    ws = torch.full((nbytes // 4,), float("nan"), device="cuda")
    c1 = torch.empty(M, N, device="cuda", dtype=dtype)
    c2 = torch.empty_like(c1)
    _ws_call(a, b, bias, c1, ws, nbytes)
    ws.fill_(float("nan"))
    _ws_call(a, b, bias, c2, ws, nbytes)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2), "split-K result is not deterministic"
    assert_max_abs(c1, gemm_f32(a, b, bias), dtype, f"gemm split-K {M}x{N}x{K}")
    # the torch op takes its workspace from the caching allocator: same kernels
    assert torch.equal(dk.gemm(a, b, bias), c1)
    _ws_call(a, b, None, c2, ws, nbytes)
    assert_max_abs(c2, gemm_f32(a, b), dtype, f"gemm split-K {M}x{N}x{K} no bias")


# Tiled (M > 64) shapes whose grid leaves CUs idle: K split over workgroup rows.
TILED_SPLIT_SHAPES = [
    (128, 4096, 14336),  # 128 x 128 tiles, 8 splits
    (256, 4096, 14336),  # 256 x 128, 8 splits
    (512, 4096, 14336),  # 256 x 128, 4 splits
    (128, 4096, 4096),  # 64 x 64, 2 splits
    (256, 6144, 4096),  # 128 x 128, 2 splits
    (300, 4101, 4104),  # ragged M and N, N not a multiple of 4 (scalar partial stores and reduce)
    (100, 1000, 8200),  # ragged K: the last split shorter
    (65, 4096, 14336),
    (961, 6113, 5704),  # 256 x 192 tiles, 2 splits, ragged M and N (scalar partial stores and reduce)
]


@pytest.mark.parametrize("M,N,K", TILED_SPLIT_SHAPES)
def test_tiled_split_k(M, N, K):
    L = capi.lib()
    plan = capi.gemm_plan(M, N, K)
    print(f"gemm tiled plan {M}x{N}x{K}: {plan}", flush=True)
    assert plan[2] > 1
    nbytes = L.dk_gemm_tn_workspace_bytes(M, N, K)
    dtype = torch.bfloat16 if M % 2 == 0 else torch.float16
    a, b, bias = _operands(M, N, K, dtype, M + 7 * N)
    ws = torch.full((nbytes // 4,), float("nan"), device="cuda")
    c1 = torch.empty(M, N, device="cuda", dtype=dtype)
    _ws_call(a, b, bias, c1, ws, nbytes)
    c2 = torch.empty_like(c1)
    ws.fill_(float("nan"))
    _ws_call(a, b, bias, c2, ws, nbytes)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2), "split-K result is not deterministic"
    ref = gemm_f32(a, b, bias)
    assert_max_abs(c1, ref, dtype, f"gemm tiled split-K {M}x{N}x{K} plan {plan}")
    assert torch.equal(dk.gemm(a, b, bias), c1)
    unsplit = torch.empty_like(c1)
    _call(L.dk_gemm_tn, a, b, bias, unsplit)
    assert_max_abs(unsplit, ref, dtype, f"gemm tiled unsplit {M}x{N}x{K}")
    small = torch.empty_like(c1)
    _ws_call(a, b, bias, small, ws, nbytes - 4)
    torch.cuda.synchronize()
    assert torch.equal(small, unsplit), "a workspace too small runs the unsplit kernel"


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES[:4])
def test_missing_or_small_workspace_runs_the_unsplit_kernel(M, N, K):
    L = capi.lib()
    dtype = torch.bfloat16
    nbytes = L.dk_gemm_tn_workspace_bytes(M, N, K)
    a, b, bias = _operands(M, N, K, dtype, 5)
    want = torch.empty(M, N, device="cuda", dtype=dtype)
    _call(L.dk_gemm_tn, a, b, bias, want)
    ws = torch.empty(nbytes // 4, device="cuda")
    for buf, size in [(None, 0), (None, nbytes), (ws, nbytes - 4)]:
        got = torch.empty_like(want)
        _ws_call(a, b, bias, got, buf, size)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (buf is None, size)


def test_unsplit_shapes_ignore_the_workspace():
    """Shapes planned unsplit (any workspace) run dk_gemm_tn's kernel."""
    L = capi.lib()
    ws = torch.empty(1 << 20, device="cuda")
    for M, N, K in [(8, 4096, 14336), (16, 6144, 4096), (64, 28672, 4096), (40, 33000, 1032), (34, 16507, 552),
                    (512, 6144, 4096), (4096, 4096, 1032)]:
        assert L.dk_gemm_tn_workspace_bytes(M, N, K) == 0
        a, b, bias = _operands(M, N, K, torch.bfloat16, M + N)
        want = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        got = torch.empty_like(want)
        _call(L.dk_gemm_tn, a, b, bias, want)
        _ws_call(a, b, bias, got, ws, ws.numel() * 4)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K)


def test_split_k_strided_rows_and_ldc():
    """Row strides past K for A and B, and an output of odd row stride."""
    M, N, K = 40, 1500, 8192
    g = torch.Generator(device="cuda").manual_seed(9)
    a_buf = torch.randn(M, K + 64, generator=g, device="cuda", dtype=torch.bfloat16)
    b_buf = torch.randn(N, K + 8, generator=g, device="cuda", dtype=torch.bfloat16) / K**0.5
    a, b = a_buf[:, :K], b_buf[:, :K]
    c_buf = torch.full((M, N + 3), 3.0, device="cuda", dtype=torch.bfloat16)
    assert capi.lib().dk_gemm_tn_workspace_bytes(M, N, K) > 0
    torch.ops.decode_kernels.gemm_tn(c_buf[:, :N], a, b, None)
    assert_max_abs(c_buf[:, :N], gemm_f32(a, b), torch.bfloat16, f"gemm split-K {M}x{N}x{K} strided")
    assert (c_buf[:, N:] == 3.0).all()


def test_split_k_graph_replay():
    """The torch op (workspace from the caching allocator) captured in a graph:
    every replay, with eager work between replays, equals the eager result."""
    M, N, K = 64, 4096, 14336
    a, b, bias = _operands(M, N, K, torch.bfloat16, 77)
    want = dk.gemm(a, b, bias)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dk.gemm(a, b, bias)  # warm the allocator on this stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = dk.gemm(a, b, bias)
    for i in range(3):
        out.fill_(float("nan"))
        noise = torch.randn(M, N, device="cuda", dtype=torch.bfloat16)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        del noise
