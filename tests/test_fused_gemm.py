"""GPU tests of the decode-layer fusions of a GEMM with its consumer.

* ``gemm_tn_add_rms_norm`` (o projection -> post-attention norm, down
  projection -> next layer's input norm) must equal ``gemm_tn`` followed by
  ``fused_add_rms_norm`` bit for bit: the output, the updated residual;
* ``gemm_tn_rotary_embedding_and_cache`` (qkv projection -> RoPE and the new
  token's cache write) must equal ``gemm_tn`` followed by
  ``rotary_embedding_and_cache`` bit for bit: the qkv rows (q and k rotated,
  v as projected) and both caches, 16-bit and fp8.

The unfused ops are each checked against the oracle by their own tests, so
bit equality pins the fused ones to the oracle too. The shapes cover the
plans that split K (skinny M <= 64 with 2 splits, the LDS-DMA kernel's
64-row tiles at M = 32 ... 64 with 4 and 8 splits, its split plans at M = 128 /
384 and, for qkv, 256), where the consumer sums the partial
tiles itself -- asserted from the plan -- and plans that do not, where the
fused call runs the two ops; plus rows the norm cannot vectorise (N not a
multiple of 8: the two ops run), strided rows, bias, and both dtypes.
"""

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from decodekernels_amd.testing import make_paged_kv
from oracle.rope_cache import rope_cos_sin_cache

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _splits(M, N, K):
    """K splits of gemm_tn's plan for this shape with a workspace."""
    return capi.gemm_plan(M, N, K)[2]


@pytest.mark.parametrize(
    "M,N,K,split",
    [
        (64, 4096, 4096, True),    # o projection at batch 64: 4 splits (64 x 64 tiles)
        (48, 4096, 4096, True),
        (64, 4096, 14336, True),   # down projection at batch 64: 8 splits (64 x 128 tiles)
        (32, 4096, 14336, True),   # 8 splits
        (16, 4096, 14336, True),   # 2 splits
        (8, 4096, 4096, False),
        (1, 4096, 14336, False),
        (128, 4096, 14336, True),  # LDS-DMA kernel, 8 splits
        (384, 4096, 4096, True),   # LDS-DMA kernel, 2 splits
        (256, 4096, 4096, False),
        (1000, 4096, 4096, False),
        (64, 4100, 4096, None),    # the norm has no vector path: the two ops
        (64, 2056, 1032, None),
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_add_rms_norm_equals_two_ops(M, N, K, split, dtype, with_bias):
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N + K)
    kw = dict(device="cuda", dtype=dtype)
    a = torch.randn(M, K, generator=g, **kw)
    w = torch.randn(N, K, generator=g, **kw) * 0.02
    bias = torch.randn(N, generator=g, **kw) * 0.5 if with_bias else None
    weight = (1 + 0.1 * torch.randn(N, generator=g, device="cuda")).to(dtype)
    # Residual and output rows padded past N (strided rows).
    resid0 = torch.randn(M, N + 24, generator=g, **kw)[:, :N]
    if split is not None:
        assert (_splits(M, N, K) > 1) == split
    ref_out = torch.empty(M, N + 8, **kw)[:, :N]
    ref_res = resid0.clone()
    torch.ops.decode_kernels.gemm_tn(ref_out, a, w, bias)
    torch.ops.decode_kernels.fused_add_rms_norm(ref_out, ref_res, weight, EPS)
    out = torch.full((M, N + 8), float("nan"), **kw)[:, :N]
    res = resid0.clone()
    dk.gemm_add_rms_norm(a, w, res, weight, EPS, bias=bias, out=out)
    torch.cuda.synchronize()
    assert torch.equal(res, ref_res), "residual differs from gemm_tn + fused_add_rms_norm"
    assert torch.equal(out, ref_out), "output differs from gemm_tn + fused_add_rms_norm"


def test_gemm_add_rms_norm_chained_layers():
    """The down projection of one layer into the next layer's input norm, then
    that layer's o projection into its post-attention norm, on the same
    residual stream: every intermediate equals the unfused chain's."""
    g = torch.Generator(device="cuda").manual_seed(3)
    kw = dict(device="cuda", dtype=torch.bfloat16)
    M, H, I = 64, 4096, 14336
    act = torch.randn(M, I, generator=g, **kw)
    w_down = torch.randn(H, I, generator=g, **kw) * 0.02
    w_o = torch.randn(H, H, generator=g, **kw) * 0.02
    ln = [(1 + 0.1 * torch.randn(H, generator=g, device="cuda")).to(torch.bfloat16) for _ in range(2)]
    resid = torch.randn(M, H, generator=g, **kw)
    r1, r2 = resid.clone(), resid.clone()
    x1, x2 = torch.empty(M, H, **kw), torch.empty(M, H, **kw)
    ops = torch.ops.decode_kernels
    ops.gemm_tn(x1, act, w_down, None)
    ops.fused_add_rms_norm(x1, r1, ln[0], EPS)
    y1 = torch.empty(M, H, **kw)
    ops.gemm_tn(y1, x1, w_o, None)
    ops.fused_add_rms_norm(y1, r1, ln[1], EPS)
    dk.gemm_add_rms_norm(act, w_down, r2, ln[0], EPS, out=x2)
    y2 = torch.empty(M, H, **kw)
    dk.gemm_add_rms_norm(x2, w_o, r2, ln[1], EPS, out=y2)
    torch.cuda.synchronize()
    assert torch.equal(x1, x2) and torch.equal(y1, y2) and torch.equal(r1, r2)


def _rope_case(M, hq, hkv, d, dtype, layout, fp8, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    kw = dict(device="cuda", dtype=dtype)
    lens = [int(x) for x in torch.randint(1, 3000, (M,), generator=g, device="cuda").tolist()]
    lens[0] = 0  # a padding row: position and slot -1
    cache_dtype = torch.float8_e4m3fn if fp8 else dtype
    kv = make_paged_kv([max(n, 1) for n in lens], hkv, d, 16, cache_dtype, "cuda", layout=layout, seed=seed + 1)
    bt = kv.block_tables.cpu()
    pos = [n - 1 for n in lens]
    pos[1 % M] = 1 << 20  # outside the table: that token is cached unrotated
    slots = [int(bt[s, p // 16]) * 16 + p % 16 if 0 <= p < (1 << 20) else -1 for s, p in enumerate(pos)]
    positions = torch.tensor(pos, device="cuda")
    slot_mapping = torch.tensor(slots, device="cuda")
    table = rope_cos_sin_cache(4096, d, base=5e5).cuda()
    return kv, positions, slot_mapping, table


@pytest.mark.parametrize("M", [8, 48, 64, 256])
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("fp8", [False, True])
def test_gemm_rotary_embedding_and_cache_equals_two_ops(M, is_neox, fp8):
    hq, hkv, d, hidden = 32, 8, 128, 4096
    dtype = torch.bfloat16
    N = (hq + 2 * hkv) * d
    g = torch.Generator(device="cuda").manual_seed(M + 100 * is_neox + 1000 * fp8)
    kw = dict(device="cuda", dtype=dtype)
    x = torch.randn(M, hidden, generator=g, **kw)
    w = torch.randn(N, hidden, generator=g, **kw) * 0.02
    bias = torch.randn(N, generator=g, **kw) * 0.1 if M == 48 else None
    kv, positions, slot_mapping, table = _rope_case(M, hq, hkv, d, dtype, "vllm", fp8, seed=M)
    scales = dict(k_scale=0.05, v_scale=0.04) if fp8 else {}
    kc2, vc2 = kv.k_cache.clone(), kv.v_cache.clone()
    qkv1 = torch.empty(M, N, **kw)
    torch.ops.decode_kernels.gemm_tn(qkv1, x, w, bias)
    dk.rotary_embedding_and_cache(positions, qkv1[:, : hq * d], qkv1[:, hq * d : (hq + hkv) * d],
                                  qkv1[:, (hq + hkv) * d :], d, table, is_neox, kv.k_cache, kv.v_cache, slot_mapping,
                                  **scales)
    qkv2 = torch.full((M, N), float("nan"), **kw)
    dk.gemm_rotary_embedding_and_cache(x, w, qkv2, hq, hkv, positions, d, table, is_neox, kc2, vc2, slot_mapping,
                                       bias=bias, **scales)
    torch.cuda.synchronize()
    assert (_splits(M, N, hidden) > 1) == (M in (48, 64, 256))
    assert torch.equal(qkv1, qkv2), "qkv rows differ from gemm_tn + rotary_embedding_and_cache"
    view = (lambda t: t.view(torch.uint8)) if fp8 else (lambda t: t)
    assert torch.equal(view(kv.k_cache), view(kc2)) and torch.equal(view(kv.v_cache), view(vc2)), "caches differ"


def test_gemm_rotary_embedding_and_cache_rejects_views_outside_the_output():
    hq, hkv, d = 4, 1, 128
    M, N, K = 64, (hq + 2 * hkv) * d, 256
    kw = dict(device="cuda", dtype=torch.bfloat16)
    x, w = torch.randn(M, K, **kw), torch.randn(N, K, **kw)
    kv, positions, slot_mapping, table = _rope_case(M, hq, hkv, d, torch.bfloat16, "nhd", False, seed=1)
    qkv, other = torch.zeros(M, N, **kw), torch.zeros(M, N, **kw)
    with pytest.raises(RuntimeError, match="views of the GEMM output"):
        torch.ops.decode_kernels.gemm_tn_rotary_embedding_and_cache(
            qkv, x, w, None, positions, other[:, : hq * d], qkv[:, hq * d : (hq + hkv) * d], qkv[:, (hq + hkv) * d :],
            d, table, True, kv.k_cache, kv.v_cache, slot_mapping)
    torch.cuda.synchronize()
    assert torch.count_nonzero(qkv) == 0, "a rejected call must not run the GEMM"
