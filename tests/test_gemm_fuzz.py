"""Seeded random shapes through the tiled gemm_tn (M > 64, and M <= 64 where
the decode plan picks the same kernel's 64-row tiles): every tile shape and
split plan the launcher picks, ragged M / N / K, odd and 4-aligned N, with
and without a bias, fp16 and bf16, against an fp32 GEMM at the parity bar.
The torch op (workspace from the caching allocator, so split plans run) and
the workspace-free C entry point must also agree bit for bit whenever both run
the same unsplit plan."""

import ctypes
import random

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from parity import assert_max_abs, gemm_f32_gpu
from test_gemm_plan import replica_plan

pytestmark = pytest.mark.gpu


def _shapes(count=48, seed=2024):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        M = rng.choice([rng.randint(65, 700), rng.randint(700, 3000)])
        N = rng.choice([rng.randint(1, 6000), 4 * rng.randint(1, 2200), 64 * rng.randint(1, 140)])
        K = 8 * rng.randint(1, 400)
        out.append((M, N, K, rng.random() < 0.5, rng.random() < 0.5))
    # Decode sizes whose plan is the LDS-DMA kernel's 64-row tiles.
    while len(out) < count + 24:
        M = rng.randint(32, 64)
        N = rng.choice([rng.randint(1000, 20000), 4 * rng.randint(250, 5000), rng.randint(32769, 40000)])
        K = 8 * rng.randint(64, 1200)
        if replica_plan(M, N, K)[0] == 64:  # host arithmetic, checked against the library on the CPU
            out.append((M, N, K, rng.random() < 0.5, rng.random() < 0.5))
    return out


@pytest.mark.parametrize("M,N,K,with_bias,bf16", _shapes())
def test_tiled_gemm_random_shapes(M, N, K, with_bias, bf16):
    dtype = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator(device="cuda").manual_seed(M * 7919 + N * 31 + K)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype) if with_bias else None
    plan = capi.gemm_plan(M, N, K)
    print(f"gemm {M}x{N}x{K} bias={with_bias} {dtype} plan {plan}", flush=True)
    out = dk.gemm(a, b, bias)
    assert_max_abs(out, gemm_f32_gpu(a, b, bias), dtype, f"gemm {M}x{N}x{K} plan {plan}")
    if plan[2] == 1:  # unsplit: the C entry point without a workspace runs the same kernel
        c = torch.empty(M, N, device="cuda", dtype=dtype)
        rc = capi.lib().dk_gemm_tn(capi.dtype_code(dtype), a.data_ptr(), b.data_ptr(),
                                   None if bias is None else bias.data_ptr(), c.data_ptr(), M, N, K, K, K, N,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, capi.last_error()
        torch.cuda.synchronize()
        assert torch.equal(c, out)


# Shapes whose plan is the 256 x 224 or 192 x 224 tile, whose 28 B load groups
# do not divide among the 8 waves (the last 4 waves skip a load; 192 x 224 also
# fills its last epilogue pass half), or the 192 x 192 tile (3 stages): full
# tiles, ragged M, ragged N, both, and K in 4 or 8 splits.
TILE_SHAPES = [
    ((256, 224), (512, 28672, 4096)), ((256, 224), (1053, 11424, 88)), ((256, 224), (768, 18728, 120)),
    ((256, 224), (795, 13247, 64)), ((192, 224), (271, 6563, 5824)),
    ((192, 192), (1536, 6144, 4096)), ((192, 192), (1844, 4416, 72)), ((192, 192), (612, 11259, 64)),
    ((192, 192), (384, 6144, 4808)), ((192, 192), (1152, 1800, 3528)), ((192, 192), (131, 5464, 4512)),
    ((192, 224), (768, 28672, 4096)), ((192, 224), (1049, 8736, 144)), ((192, 224), (1728, 5472, 136)),
    ((192, 224), (263, 24976, 64)), ((192, 224), (132, 6168, 5440)),
]


@pytest.mark.parametrize("tile,shape", TILE_SHAPES, ids=[f"{t[0]}x{t[1]}-{m}x{n}x{k}" for t, (m, n, k) in TILE_SHAPES])
@pytest.mark.parametrize("bf16", [True, False])
def test_tile_shapes_against_fp32(tile, shape, bf16):
    M, N, K = shape
    dtype = torch.bfloat16 if bf16 else torch.float16
    plan = capi.gemm_plan(M, N, K)
    print(f"gemm {M}x{N}x{K} {dtype} plan {plan}", flush=True)
    assert plan[:2] == tile, plan
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype)
    out = dk.gemm(a, b, bias)
    assert_max_abs(out, gemm_f32_gpu(a, b, bias), dtype, f"gemm {M}x{N}x{K} plan {plan}")
    c = torch.full((M, N), float("nan"), device="cuda", dtype=dtype)
    rc = capi.lib().dk_gemm_tn(capi.dtype_code(dtype), a.data_ptr(), b.data_ptr(), None, c.data_ptr(), M, N, K, K, K, N,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    assert_max_abs(c, gemm_f32_gpu(a, b), dtype, f"gemm {M}x{N}x{K} unsplit, no bias")
