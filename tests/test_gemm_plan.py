"""CPU tests of gemm_tn's launch plans, through ``dk_gemm_tn_plan`` /
``dk_gemm_tn_workspace_bytes`` (host arithmetic, no kernel launch).

``skinny_plan`` (decodekernels_amd/csrc/gemm.hip) picks the workgroup shape
(waves along N, 16 columns each, x waves along K) and the number of K splits:
the widest unsplit grid of <= 256 workgroups when it fills >= 3/4 of the 256
CUs and each workgroup re-reads <= 256 KiB of activations; else, with a
workspace, the grid of 2..8 K splits (>= 512 columns each, <= 256
workgroups, within 10% of the fullest) with the fewest splits whose
workgroups re-read <= max(128 KiB, half their weight bytes) of activations
(else the fewest activation bytes); else the unsplit grid, or the wide plan
for N > 32768. This file restates that arithmetic and checks, over random
shapes, that the library plans exactly the same, plus the invariants the
kernels rely on: every split non-empty and a multiple of 64 columns, at most
256 workgroups whenever K is split, the workspace size, and a workgroup
shape the launcher instantiates. The Llama-3-8B decode projections map to
the shapes measured fastest.

At M <= 64 ``decode_dma_plan`` can replace the skinny plan with the LDS-DMA
kernel's 64-row tiles (reported as (64, tile columns, splits, k_split)): for
N > 32768 (no skinny grid of one workgroup per CU) 64 x 64 unsplit; else
from M = 32, among 64- and 128-column tiles with 1, 2, 4 or 8 K splits of
>= 768 columns and <= 256 workgroups, the one streaming the fewest weight
bytes per workgroup (128 columns on a tie), if it fills at least half the
CUs and, unsplit, the skinny kernel's own unsplit grid leaves over a quarter
of them idle. The M > 64 plan (``dma_plan``) is restated below it.
"""

import random

import pytest

from decodekernels_amd import capi

SHAPES = [(1, 8), (2, 4), (4, 2), (6, 2), (7, 2), (8, 1)]
KIB = 1024


def _wide(M, N, K):
    mt = 1 if M <= 16 else (2 if M <= 32 else 4)
    min_wgs = 384 if mt == 1 else 192
    wn = 8 if (M > 32 and N >= 24576) else (4 if N >= 64 * min_wgs else (2 if N >= 32 * min_wgs else 1))
    return (wn, 8 // wn, 1, K)


def _unsplit(N, K):
    for wn, wk in SHAPES:
        if -(-N // (16 * wn)) <= 256:
            return (wn, wk, 1, K)
    return None


def replica_decode_dma_plan(M, N, K, with_workspace=True, mistake=None):
    """(64, tile columns, splits, k_split) as decode_dma_plan computes it, or
    None (the skinny kernel). ``mistake``: "half" drops the half-fill
    condition, "full" lets an unsplit tile replace a full skinny grid."""
    if M > 64 or K <= 0:
        return None
    u = _unsplit(N, K)
    if u is None:
        return (64, 64, 1, K)
    if M < 32:
        return None
    best, best_bytes, best_wgs = None, -1, 0
    for bn in (128, 64):
        tiles = -(-N // bn)
        s = 1
        while s <= 8:
            ks, sp = K, 1
            if s > 1:
                if not with_workspace:
                    break
                ks = -(-(-(-K // s)) // 64) * 64
                sp = -(-K // ks)
                if ks < 768:
                    break
                if sp < 2:
                    s *= 2
                    continue
            if tiles * sp > 256:
                break
            if best_bytes < 0 or bn * ks < best_bytes:
                best, best_bytes, best_wgs = (64, bn, sp, ks), bn * ks, tiles * sp
            s *= 2
    if 2 * best_wgs < 256 and mistake != "half":
        return None
    if best is not None and best[2] == 1 and mistake != "full" and 4 * -(-N // (16 * u[0])) >= 3 * 256:
        return None
    return best


def replica_plan(M, N, K, with_workspace=True, mistake=None):
    """gemm_tn's plan at M <= 64: the decode DMA plan where it applies, else
    (wn, wk, splits, k_split) as skinny_plan computes it. ``mistake`` plants
    an error: "fill" drops the 3/4-fill condition of the unsplit grid,
    "limit" compares activation bytes with the weight bytes instead of half
    of them; "half" / "full" go to the decode DMA plan."""
    d = replica_decode_dma_plan(M, N, K, with_workspace, mistake)
    if d is not None:
        return d
    return replica_skinny_plan(M, N, K, with_workspace, mistake)


def replica_skinny_plan(M, N, K, with_workspace=True, mistake=None):
    u = _unsplit(N, K)
    if u is not None and M * K * 2 <= 256 * KIB and (mistake == "fill" or 4 * -(-N // (16 * u[0])) >= 3 * 256):
        return u
    cands = []
    if with_workspace and K > 0:
        for wn, wk in SHAPES:
            tiles = -(-N // (16 * wn))
            for s in range(2, 9):
                if K // s < 512:
                    break
                per = -(-K // s)
                ks = -(-per // 64) * 64
                if -(-K // ks) != s:
                    continue
                if tiles * s > 256:
                    break
                cands.append((wn, wk, s, ks, tiles * s))
    if cands:
        mx = max(c[4] for c in cands)
        near = [c for c in cands if 10 * c[4] >= 9 * mx]
        div = 1 if mistake == "limit" else 2
        ok = [c for c in near if M * c[3] * 2 <= max(128 * KIB, 16 * c[0] * c[3] * 2 // div)]
        best = min(ok, key=lambda c: (c[2], near.index(c))) if ok else min(near, key=lambda c: (M * c[3], c[2], near.index(c)))
        return best[:4]
    return u if u is not None else _wide(M, N, K)


DMA_SHAPES = [(256, 256, 5.355), (256, 224, 4.95), (256, 192, 5.15), (256, 128, 4.776), (192, 224, 4.55),
              (192, 192, 3.95), (128, 128, 3.48), (128, 64, 2.398), (64, 64, 2.007)]
DMA_MAX_WORKSPACE = 64 << 20


def replica_dma_plan(M, N, K, with_workspace=True):
    """(tile rows, tile columns, splits, k_split) as dma_plan computes it (M > 64):
    the shape and split count minimising rounds x tile flops per split / rate
    + (1.84 us + splits M N 8 B / 4.68 TB/s when split); splits only for grids
    of < 256 tiles, >= 512 columns each and <= 64 MiB of partials."""
    best, best_t = None, -1.0
    for bm, bn, rate in DMA_SHAPES:
        tiles = -(-M // bm) * -(-N // bn)
        s = 1
        while s <= 8:
            ks, sp = K, 1
            if s > 1:
                if not with_workspace or tiles >= 256 or K // s < 512:
                    break
                per = -(-K // s)
                ks = -(-per // 64) * 64
                sp = -(-K // ks)
                if sp < 2:
                    s *= 2
                    continue
                if sp * M * N * 4 > DMA_MAX_WORKSPACE:
                    break
            rounds = float(-(-(tiles * sp) // 256))
            t = rounds * bm * bn * 2.0 * ks / 1e6 / rate
            if sp > 1:
                t += 1.84 + float(sp) * M * N * 8 / 4.68e6
            if best_t < 0 or t < best_t:
                best, best_t = (bm, bn, sp, ks), t
            s *= 2
    return best


def _random_shapes(n, seed):
    rng = random.Random(seed)
    for _ in range(n):
        M = rng.randint(1, 64)
        N = rng.choice([rng.randint(1, 600), rng.randint(1, 8192), rng.randint(1, 40000)])
        K = 8 * rng.choice([rng.randint(0, 64), rng.randint(0, 3000)])
        yield M, N, K


def test_library_plans_like_the_replica():
    for M, N, K in _random_shapes(20000, 3):
        for ws in (True, False):
            assert capi.gemm_plan(M, N, K, ws) == replica_plan(M, N, K, ws), (M, N, K, ws)


def test_tiled_plans_like_the_replica():
    """M > 64: the tile shape and split of the LDS-DMA kernel, and the
    workspace it asks for."""
    L = capi.lib()
    rng = random.Random(8)
    for _ in range(20000):
        M = rng.choice([rng.randint(65, 600), rng.randint(65, 5000)])
        N = rng.choice([rng.randint(1, 2000), rng.randint(1, 30000)])
        K = 8 * rng.randint(1, 3000)
        for ws in (True, False):
            plan = capi.gemm_plan(M, N, K, ws)
            assert plan == replica_dma_plan(M, N, K, ws), (M, N, K, ws)
        bm, bn, sp, ks = capi.gemm_plan(M, N, K)
        assert L.dk_gemm_tn_workspace_bytes(M, N, K) == (sp * M * N * 4 if sp > 1 else 0)
        if sp > 1:
            assert (sp - 1) * ks < K <= sp * ks and ks % 64 == 0 and -(-M // bm) * -(-N // bn) < 256
            assert sp * M * N * 4 <= DMA_MAX_WORKSPACE


# (M, N, K) -> (tile rows, tile columns, splits) measured fastest at batched decode
# and, for the 256 x 192, 256 x 224, 192 x 224 and 192 x 192 tiles, at sizes where
# 256 x 256 leaves a round part-empty.
TILED_PICKS = {
    (128, 4096, 14336): (128, 128, 8), (256, 4096, 14336): (256, 128, 8), (512, 4096, 14336): (256, 128, 4),
    (256, 6144, 4096): (128, 128, 2), (256, 28672, 4096): (256, 128, 1), (512, 6144, 4096): (128, 128, 1),
    (4096, 4096, 4096): (256, 256, 1), (4096, 28672, 4096): (256, 256, 1),
    (4096, 6144, 4096): (256, 192, 1), (4096, 3072, 4096): (256, 192, 1),
    (512, 28672, 4096): (256, 224, 1), (2048, 28672, 4096): (256, 224, 1), (3072, 28672, 4096): (256, 224, 1),
    (768, 28672, 4096): (192, 224, 1), (384, 3584, 18944): (192, 224, 8), (768, 3584, 18944): (192, 224, 4),
    (3072, 3584, 18944): (192, 224, 1), (512, 37888, 3584): (192, 224, 1), (3072, 3584, 3584): (192, 224, 1),
    (2048, 4608, 3584): (192, 224, 1),
    (384, 6144, 4096): (192, 192, 4), (768, 6144, 4096): (192, 192, 2), (1536, 6144, 4096): (192, 192, 1),
    (3072, 6144, 4096): (192, 192, 1), (128, 37888, 3584): (192, 192, 1), (384, 37888, 3584): (192, 192, 1),
}


@pytest.mark.parametrize("shape", sorted(TILED_PICKS))
def test_batched_decode_projections_get_the_measured_tiles(shape):
    assert capi.gemm_plan(*shape)[:3] == TILED_PICKS[shape]


def test_plan_invariants_and_workspace_size():
    L = capi.lib()
    for M, N, K in _random_shapes(20000, 4):
        wn, wk, s, ks = capi.gemm_plan(M, N, K)
        tile = wn == 64
        assert (wn, wk) in SHAPES or (tile and wk in (64, 128)), (M, N, K)
        nbytes = L.dk_gemm_tn_workspace_bytes(M, N, K)
        if s == 1:
            assert ks == K and nbytes == 0
            continue
        assert 2 <= s <= 8 and ks % 64 == 0 and ks >= (768 if tile else 512), (M, N, K, s, ks)
        assert (s - 1) * ks < K <= s * ks, "a split is empty or K is not covered"
        assert -(-N // (wk if tile else 16 * wn)) * s <= 256, "a split plan over-fills the CUs"
        assert nbytes == s * M * N * 4
        # without a workspace the same shape is planned unsplit
        assert capi.gemm_plan(M, N, K, False)[2] == 1


# (M, N, K) -> (waves along N, waves along K, splits) of the skinny kernel, or
# (64, tile columns, splits) of the LDS-DMA kernel: the measured-fastest
# plans of the Llama-3-8B, Qwen2.5-7B and Qwen2.5-0.5B decode projections.
LLAMA_PICKS = {
    (1, 6144, 4096): (2, 4, 1), (16, 6144, 4096): (2, 4, 1), (32, 6144, 4096): (64, 128, 4),
    (48, 6144, 4096): (64, 128, 4), (64, 6144, 4096): (64, 128, 4),
    (1, 4096, 4096): (1, 8, 1), (16, 4096, 4096): (1, 8, 1), (32, 4096, 4096): (64, 64, 4),
    (48, 4096, 4096): (64, 64, 4), (64, 4096, 4096): (64, 64, 4),
    (8, 4096, 14336): (1, 8, 1), (16, 4096, 14336): (2, 4, 2), (32, 4096, 14336): (64, 128, 8),
    (48, 4096, 14336): (64, 128, 8), (64, 4096, 14336): (64, 128, 8),
    (1, 28672, 4096): (7, 2, 1), (32, 28672, 4096): (7, 2, 1), (64, 28672, 4096): (7, 2, 1),
    (64, 4608, 3584): (64, 128, 4), (64, 3584, 3584): (64, 64, 4), (64, 3584, 18944): (64, 128, 8),
    (1, 37888, 3584): (64, 64, 1), (64, 37888, 3584): (64, 64, 1),
    (64, 1152, 896): (1, 8, 1), (1, 9728, 896): (4, 2, 1), (64, 9728, 896): (64, 64, 1),
}


@pytest.mark.parametrize("shape", sorted(LLAMA_PICKS))
def test_llama_projections_get_the_measured_shapes(shape):
    assert capi.gemm_plan(*shape)[:3] == LLAMA_PICKS[shape]


@pytest.mark.parametrize("mistake", ["fill", "limit", "half", "full"])
def test_planted_mistake_is_caught(mistake):
    """A replica with one condition changed must disagree with the library on
    some shape: the comparison above can see both conditions."""
    diffs = sum(capi.gemm_plan(M, N, K) != replica_plan(M, N, K, mistake=mistake) for M, N, K in _random_shapes(5000, 5))
    assert diffs > 0


def test_plan_validation():
    L = capi.lib()
    assert L.dk_gemm_tn_plan(0, 8, 64, 1, None) == capi.HIP_ERROR_INVALID_VALUE
    with pytest.raises(ValueError, match="positive"):
        capi.gemm_plan(0, 8, 64)
    with pytest.raises(ValueError, match="positive"):
        capi.gemm_plan(4, 8, -8)


# One shape per (row tiles, workgroup shape, split or not) the skinny plan
# reaches, and per (tile columns, split or not) of the decode DMA plan (plus
# its N > 32768 case at M < 32), each with N not a multiple of the
# workgroup's columns; run on the GPU against the oracle by
# tests/test_gemm_splitk.py.
COVERAGE_SHAPES = [
    (1, 8, 520), (1, 8, 1032), (1, 4101, 520), (1, 2050, 1032), (1, 8200, 520), (1, 4101, 1032),
    (1, 20000, 520), (1, 8200, 1032), (1, 28600, 520), (1, 8200, 2056), (1, 28680, 520), (16, 6150, 8200),
    (17, 8, 520), (17, 8, 1032), (17, 4101, 520), (17, 2050, 1032), (17, 8200, 520), (17, 4101, 1032),
    (17, 20000, 520), (17, 8200, 1032), (17, 28600, 520), (17, 8200, 2056), (17, 28680, 520), (18, 9622, 1624),
    (33, 8, 520), (33, 8, 1032), (33, 4101, 520), (33, 2050, 1032), (35, 13089, 520), (33, 4101, 1032),
    (33, 20000, 520), (55, 12225, 2656), (33, 28600, 520), (42, 12474, 3128), (33, 28680, 520), (64, 8, 8200),
]
DECODE_DMA_SHAPES = [
    (33, 8296, 536), (32, 965, 5928), (34, 16507, 552), (32, 4162, 2952), (64, 4162, 2952), (7, 32780, 520),
]


def test_coverage_shapes_reach_every_plan():
    reached = set()
    for M, N, K in COVERAGE_SHAPES:
        wn, wk, s, _ = capi.gemm_plan(M, N, K)
        assert N % (16 * wn) != 0, (M, N, K)
        reached.add((1 if M <= 16 else (2 if M <= 32 else 4), wn, wk, s > 1))
    assert reached == {(mt, wn, wk, split) for mt in (1, 2, 4) for wn, wk in SHAPES for split in (False, True)}
    tiles = set()
    for M, N, K in DECODE_DMA_SHAPES:
        bm, bn, s, _ = capi.gemm_plan(M, N, K)
        assert bm == 64 and N % bn != 0, (M, N, K)
        tiles.add((bn, s > 1, M < 32))
    assert tiles == {(64, False, False), (64, True, False), (128, False, False), (128, True, False),
                     (64, False, True)}
