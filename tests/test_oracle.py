"""CPU pins of the oracle (``oracle.reference``).

Every function is checked against an independent float64 brute force
(``oracle.brute``) and against a torch routine or closed form, plus the
reference's own CPU properties (``tests/test_reference.py:30-124`` of
DecodeKernels): split-K merge == dense at partition boundaries, paged gather ==
contiguous SDPA, strided layouts == contiguous copies, empty sequences ->
zeros, residual rounding. The last section plants plausible mistakes in copies
of the oracle and shows each is caught by one of these pins.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from decodekernels_amd.testing import make_paged_kv
from oracle import brute
from oracle.reference import (
    fused_add_rms_norm_reference,
    gather_kv,
    gemm_reference,
    paged_attention_reference,
    rms_norm_reference,
    silu_and_mul_reference,
    split_k_attention_reference,
)


def _queries(num_seqs, num_q_heads, head_dim, dtype=torch.float32, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(num_seqs, num_q_heads, head_dim, generator=g, dtype=dtype)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("partition_size", [64, 512])
@pytest.mark.parametrize("group", [1, 4, 8])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_split_k_merge_matches_dense(partition_size, group, head_dim):
    seq_lens = [1, 7, 63, 64, 65, 511, 512, 513, 1300]
    kv = make_paged_kv(seq_lens, 2, head_dim, block_size=16, dtype=torch.float32)
    q = _queries(len(seq_lens), 2 * group, head_dim)
    dense = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    split = split_k_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, partition_size=partition_size)
    torch.testing.assert_close(split, dense, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("block_size", [1, 16, 32])
def test_paged_gather_matches_sdpa(block_size):
    seq_lens = [5, 33, 100]
    kvh, group, d = 2, 4, 64
    kv = make_paged_kv(seq_lens, kvh, d, block_size=block_size, dtype=torch.float32)
    q = _queries(len(seq_lens), kvh * group, d)
    out = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    for s, L in enumerate(seq_lens):
        k = gather_kv(kv.k_cache, kv.block_tables[s], L).transpose(0, 1).repeat_interleave(group, dim=0)
        v = gather_kv(kv.v_cache, kv.block_tables[s], L).transpose(0, 1).repeat_interleave(group, dim=0)
        expected = F.scaled_dot_product_attention(q[s][:, None, :], k, v)[:, 0, :]
        torch.testing.assert_close(out[s], expected, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_dense_and_split_match_float64_brute_force(group, block_size):
    seq_lens = [1, 5, 37, 0]
    kv = make_paged_kv(seq_lens, 2, 64, block_size=block_size, dtype=torch.float32, seed=3)
    q = _queries(len(seq_lens), 2 * group, 64, seed=4)
    expected = brute.attention(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    dense = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    split = split_k_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, partition_size=8)
    np.testing.assert_allclose(dense.double().numpy(), expected, atol=2e-6, rtol=2e-6)
    np.testing.assert_allclose(split.double().numpy(), expected, atol=2e-6, rtol=2e-6)


def test_custom_scale_matches_brute_force():
    kv = make_paged_kv([9, 20], 1, 64, block_size=16, dtype=torch.float32, seed=5)
    q = _queries(2, 4, 64, seed=6)
    got = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, scale=0.05)
    np.testing.assert_allclose(
        got.double().numpy(), brute.attention(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, scale=0.05),
        atol=2e-6, rtol=2e-6,
    )


def test_lse_merge_of_two_halves_is_dense():
    """The merge rule itself, on one head in float64: splitting a softmax in two
    and merging (m, s, o) pairs gives the unsplit result."""
    rng = np.random.default_rng(0)
    logits = rng.normal(size=40) * 3
    v = rng.normal(size=(40, 8))
    parts = []
    for lo, hi in ((0, 13), (13, 40)):
        m = logits[lo:hi].max()
        e = np.exp(logits[lo:hi] - m)
        parts.append((m, e.sum(), (e[:, None] * v[lo:hi]).sum(0) / e.sum()))
    merged = brute.lse_merge(*zip(*parts))
    w = np.exp(logits - logits.max())
    np.testing.assert_allclose(merged, (w[:, None] * v).sum(0) / w.sum(), rtol=1e-12)


@pytest.mark.parametrize("layout", ["hnd", "vllm"])
def test_strided_layouts_match_nhd(layout):
    seq_lens = [3, 40, 129]
    kv = make_paged_kv(seq_lens, 2, 64, block_size=16, dtype=torch.float32, layout=layout)
    assert not kv.k_cache.is_contiguous() and kv.k_cache.stride(-1) == 1
    q = _queries(len(seq_lens), 8, 64)
    strided = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    contiguous = paged_attention_reference(q, kv.k_cache.contiguous(), kv.v_cache.contiguous(), kv.block_tables, kv.seq_lens)
    torch.testing.assert_close(strided, contiguous)


def test_layout_strides():
    d, bs, h = 64, 16, 2
    hnd = make_paged_kv([20], h, d, block_size=bs, layout="hnd")
    assert hnd.k_cache.stride() == (h * bs * d, d, bs * d, 1)
    vl = make_paged_kv([20], h, d, block_size=bs, layout="vllm")
    assert vl.k_cache.stride() == (h * bs * 2 * d, 2 * d, bs * 2 * d, 1)
    assert vl.k_cache.untyped_storage().data_ptr() == vl.v_cache.untyped_storage().data_ptr()
    assert vl.v_cache.data_ptr() - vl.k_cache.data_ptr() == d * vl.k_cache.element_size()


def test_block_tables_use_distinct_blocks():
    seq_lens = [1, 511, 512, 513]
    kv = make_paged_kv(seq_lens, 2, 128, block_size=16, dtype=torch.float32, extra_blocks=62)
    assert kv.k_cache.shape[0] == 160  # 1 + 32 + 32 + 33 blocks + 62 extra
    used = []
    for s, L in enumerate(seq_lens):
        n = math.ceil(L / 16)
        used += kv.block_tables[s, :n].tolist()
        assert (kv.block_tables[s, n:] == 0).all()
    assert len(set(used)) == len(used) and all(0 <= b < 160 for b in used)


def test_empty_sequence_gives_zeros():
    kv = make_paged_kv([0, 10], 1, 64, dtype=torch.float32)
    q = _queries(2, 1, 64)
    out = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    assert torch.count_nonzero(out[0]) == 0
    split = split_k_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, partition_size=4)
    torch.testing.assert_close(split, out)


def test_dense_rounds_once_to_input_dtype():
    kv = make_paged_kv([30], 1, 64, dtype=torch.float16, seed=2)
    q = _queries(1, 2, 64, dtype=torch.float16)
    out = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    assert out.dtype == torch.float16
    f32 = paged_attention_reference(q.float(), kv.k_cache.float(), kv.v_cache.float(), kv.block_tables, kv.seq_lens)
    torch.testing.assert_close(out, f32.half(), atol=0, rtol=0)


# ---------------------------------------------------------------------------
# GEMM / norms / activation
# ---------------------------------------------------------------------------
def test_gemm_reference_matches_linear_and_brute_force():
    g = torch.Generator().manual_seed(0)
    a, b, bias = torch.randn(7, 64, generator=g), torch.randn(48, 64, generator=g), torch.randn(48, generator=g)
    torch.testing.assert_close(gemm_reference(a, b, bias), F.linear(a, b, bias))
    np.testing.assert_allclose(gemm_reference(a, b, bias).double().numpy(), brute.gemm(a, b, bias), atol=1e-4, rtol=1e-5)
    np.testing.assert_allclose(gemm_reference(a, b).double().numpy(), brute.gemm(a, b), atol=1e-4, rtol=1e-5)


def test_gemm_reference_rounds_once():
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn(5, 32, generator=g).bfloat16(), torch.randn(9, 32, generator=g).bfloat16()
    bias = torch.randn(9, generator=g).bfloat16()
    expected = (a.float() @ b.float().t() + bias.float()).bfloat16()
    torch.testing.assert_close(gemm_reference(a, b, bias), expected, atol=0, rtol=0)


def test_rms_norm_reference_closed_form_and_brute_force():
    g = torch.Generator().manual_seed(0)
    x, w = torch.randn(4, 256, generator=g), torch.randn(256, generator=g)
    expected = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    torch.testing.assert_close(rms_norm_reference(x, w), expected)
    np.testing.assert_allclose(rms_norm_reference(x, w, 1e-5).double().numpy(), brute.rms_norm(x, w, 1e-5), rtol=1e-5, atol=1e-6)


def test_fused_add_rms_norm_reference_rounds_residual():
    g = torch.Generator().manual_seed(0)
    x, r, w = (torch.randn(4, 256, generator=g, dtype=torch.float16) for _ in range(3))
    normed, new_res = fused_add_rms_norm_reference(x, r, w)
    assert new_res.dtype == torch.float16
    torch.testing.assert_close(new_res, (x.float() + r.float()).half(), atol=0, rtol=0)
    torch.testing.assert_close(normed, rms_norm_reference(new_res, w), atol=0, rtol=0)


def test_silu_and_mul_reference():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 80, generator=g)
    torch.testing.assert_close(silu_and_mul_reference(x), F.silu(x[:, :40]) * x[:, 40:])
    torch.testing.assert_close(silu_and_mul_reference(x), x[:, :40] * torch.sigmoid(x[:, :40]) * x[:, 40:])
    np.testing.assert_allclose(silu_and_mul_reference(x).double().numpy(), brute.silu_and_mul(x), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# Planted mistakes: each mutated copy of an oracle function must fail a pin.
# ---------------------------------------------------------------------------
def _attn_pins_pass(fn) -> bool:
    kv = make_paged_kv([1, 5, 37], 2, 64, block_size=4, dtype=torch.float32, seed=3)
    q = _queries(3, 8, 64, seed=4)
    got = fn(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    return np.allclose(got.double().numpy(), brute.attention(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), atol=2e-6, rtol=2e-6)


def test_attention_pin_has_teeth():
    assert _attn_pins_pass(paged_attention_reference)

    def no_scale(q, k, v, bt, lens):
        return paged_attention_reference(q, k, v, bt, lens, scale=1.0)

    def tiled_gqa(q, k, v, bt, lens):  # query head h -> KV head h % Hkv instead of h // group
        perm = torch.arange(q.shape[1]).view(-1, k.shape[2]).t().reshape(-1)
        return paged_attention_reference(q[:, perm], k, v, bt, lens)

    def off_by_one_token(q, k, v, bt, lens):
        return paged_attention_reference(q, k, v, bt, torch.clamp(lens - 1, min=1))

    for mutant in (no_scale, tiled_gqa, off_by_one_token):
        assert not _attn_pins_pass(mutant), mutant.__name__


def test_split_merge_pin_has_teeth():
    seq_lens = [65, 513]
    kv = make_paged_kv(seq_lens, 2, 64, block_size=16, dtype=torch.float32)
    q = _queries(2, 8, 64)
    dense = paged_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)

    def unweighted_merge(q, k, v, bt, lens, partition_size):
        # Averages the normalised partials instead of weighting them by s_p e^(m_p - M).
        out = torch.zeros_like(dense)
        for s in range(q.shape[0]):
            L = int(lens[s])
            parts = []
            for lo in range(0, L, partition_size):
                sub_lens = torch.tensor([min(partition_size, L - lo)], dtype=torch.int32)
                kk = gather_kv(k, bt[s], L)[lo:]
                vv = gather_kv(v, bt[s], L)[lo:]
                tbl = torch.arange(kk.shape[0], dtype=torch.int32)[None]
                parts.append(paged_attention_reference(q[s : s + 1], kk[:, None], vv[:, None], tbl, sub_lens)[0])
            out[s] = torch.stack(parts).mean(0)
        return out

    assert torch.allclose(split_k_attention_reference(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, partition_size=64), dense, atol=1e-5)
    assert not torch.allclose(unweighted_merge(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, 64), dense, atol=1e-5)


def test_gemm_and_norm_pins_have_teeth():
    g = torch.Generator().manual_seed(0)
    a, b = torch.randn(8, 8, generator=g), torch.randn(8, 8, generator=g)
    assert not np.allclose((a.float() @ b.float()).numpy(), brute.gemm(a, b), atol=1e-4)  # transposed operand
    x, w = torch.randn(4, 64, generator=g), torch.randn(64, generator=g)
    assert not np.allclose((x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + 1e-6) * w).numpy(), brute.rms_norm(x, w, 1e-6))
    xh, rh, wh = (torch.randn(4, 64, generator=g, dtype=torch.float16) for _ in range(3))
    # Norm over the unrounded residual sum: the residual pin (exact equality
    # with the rounded sum) and the normed output both change.
    unrounded = rms_norm_reference(xh.float() + rh.float(), wh.float()).half()
    assert not torch.equal(unrounded, fused_add_rms_norm_reference(xh, rh, wh)[0])
