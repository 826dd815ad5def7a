"""CPU pins of oracle/rope_cache.py: rotary embedding and the paged cache write.

DecodeKernels has neither op (vLLM runs them), so there is no reference code
or golden vector; the oracle is pinned by an independent complex-number
formulation of the rotation, by rotation invariants in float64, and by an
``index_put_`` scatter, with planted mistakes shown to fail a pin.
"""

import pytest
import torch

from oracle.reference import gather_kv
from oracle.rope_cache import reshape_and_cache_reference, rope_cos_sin_cache, rotary_embedding_reference


def _rope_complex(x, positions, cache, head_size, is_neox):
    """(x1 + i x2) * exp(i theta) in complex128 (an independent route)."""
    t = x.shape[0]
    x3 = x.reshape(t, -1, head_size).double()
    rot = cache.shape[1]
    half = rot // 2
    tab = cache.double()[positions]
    z = torch.complex(tab[:, :half], tab[:, half:])[:, None, :]
    r = x3[..., :rot]
    if is_neox:
        c = torch.complex(r[..., :half], r[..., half:])
    else:
        c = torch.view_as_complex(r.reshape(t, r.shape[1], half, 2).contiguous())
    rc = c * z
    out = x3.clone()
    if is_neox:
        out[..., :half] = rc.real
        out[..., half:rot] = rc.imag
    else:
        out[..., :rot] = torch.view_as_real(rc).reshape(t, r.shape[1], rot)
    return out.reshape(x.shape)


CASES = [(True, 128, 128), (False, 128, 128), (True, 64, 128), (False, 32, 96), (True, 256, 256)]


@pytest.mark.parametrize("is_neox,rot_dim,head_size", CASES)
def test_rope_matches_complex_multiplication(is_neox, rot_dim, head_size):
    g = torch.Generator().manual_seed(rot_dim + head_size)
    t, hq, hkv = 7, 4, 2
    cache = rope_cos_sin_cache(4096, rot_dim)
    pos = torch.randint(0, 4096, (t,), generator=g)
    q = torch.randn(t, hq * head_size, generator=g)
    k = torch.randn(t, hkv, head_size, generator=g)
    oq, ok = rotary_embedding_reference(pos, q, k, head_size, cache, is_neox)
    torch.testing.assert_close(oq.double(), _rope_complex(q, pos, cache, head_size, is_neox), atol=2e-6, rtol=0)
    torch.testing.assert_close(ok.double(), _rope_complex(k, pos, cache, head_size, is_neox), atol=2e-6, rtol=0)
    assert torch.equal(oq.reshape(t, hq, head_size)[..., rot_dim:], q.reshape(t, hq, head_size)[..., rot_dim:])


@pytest.mark.parametrize("is_neox", [True, False])
def test_rope_scores_depend_only_on_relative_position(is_neox):
    g = torch.Generator().manual_seed(3)
    d = 128
    cache = rope_cos_sin_cache(8192, d)
    q = torch.randn(1, d, generator=g)
    k = torch.randn(1, d, generator=g)

    def score(pq, pk):
        rq, _ = rotary_embedding_reference(torch.tensor([pq]), q, None, d, cache, is_neox)
        rk, _ = rotary_embedding_reference(torch.tensor([pk]), k, None, d, cache, is_neox)
        return float((rq.double() * rk.double()).sum())

    for pq, pk, shift in ((10, 3, 100), (500, 900, 2000), (0, 4000, 4000)):
        assert abs(score(pq, pk) - score(pq + shift, pk + shift)) < 1e-3


@pytest.mark.parametrize("is_neox", [True, False])
def test_rope_inverse_rotation_restores_input(is_neox):
    g = torch.Generator().manual_seed(4)
    d = 64
    cache = rope_cos_sin_cache(1024, d)
    inverse = torch.cat([cache[:, : d // 2], -cache[:, d // 2 :]], dim=1)
    pos = torch.randint(0, 1024, (5,), generator=g)
    x = torch.randn(5, 3 * d, generator=g)
    once, _ = rotary_embedding_reference(pos, x, None, d, cache, is_neox)
    back, _ = rotary_embedding_reference(pos, once, None, d, inverse, is_neox)
    torch.testing.assert_close(back, x, atol=2e-6, rtol=0)
    # Each rotated pair keeps its length.
    n0 = x.reshape(5, 3, d).double().pow(2).sum(-1)
    n1 = once.reshape(5, 3, d).double().pow(2).sum(-1)
    torch.testing.assert_close(n1, n0, atol=1e-4, rtol=1e-6)


def test_rope_position_zero_and_out_of_range_leave_tokens_unchanged():
    d = 64
    cache = rope_cos_sin_cache(100, d)
    x = torch.randn(3, 2 * d).to(torch.bfloat16)
    out, _ = rotary_embedding_reference(torch.tensor([0, -1, 100]), x, None, d, cache, True)
    assert torch.equal(out, x)


def test_rope_rounds_once_to_the_input_dtype():
    g = torch.Generator().manual_seed(6)
    d = 128
    cache = rope_cos_sin_cache(2048, d)
    pos = torch.randint(0, 2048, (16,), generator=g)
    x = torch.randn(16, 8 * d, generator=g).to(torch.bfloat16)
    out, _ = rotary_embedding_reference(pos, x, None, d, cache, True)
    want = _rope_complex(x.float(), pos, cache, d, True).float().to(torch.bfloat16)
    # fp32 and float64 intermediates may round a halfway case differently: at most 1 ulp.
    diff = (out.view(torch.int16).int() - want.view(torch.int16).int()).abs()
    assert int(diff.max()) <= 1
    assert (diff == 0).float().mean() > 0.99


@pytest.mark.parametrize("mistake", ["sin_sign", "pairing", "past_rot_dim"])
def test_rope_pins_catch_planted_mistakes(mistake):
    g = torch.Generator().manual_seed(7)
    d, rot = 128, 64
    cache = rope_cos_sin_cache(1024, rot)
    pos = torch.randint(1, 1024, (4,), generator=g)
    x = torch.randn(4, 2 * d, generator=g)
    if mistake == "sin_sign":
        bad, _ = rotary_embedding_reference(pos, x, None, d, torch.cat([cache[:, :32], -cache[:, 32:]], 1), True)
    elif mistake == "pairing":
        bad, _ = rotary_embedding_reference(pos, x, None, d, cache, False)
    else:
        full = rope_cos_sin_cache(1024, d)
        bad, _ = rotary_embedding_reference(pos, x, None, d, full, True)
    good = _rope_complex(x, pos, cache, d, True)
    assert (bad.double() - good).abs().max() > 1e-2


@pytest.mark.parametrize("layout", ["nhd", "hnd", "vllm"])
def test_cache_write_matches_index_put_and_gathers_back(layout):
    g = torch.Generator().manual_seed(8)
    nb, bs, hkv, d, t = 12, 16, 2, 64, 9
    if layout == "nhd":
        kc = torch.randn(nb, bs, hkv, d, generator=g)
        vc = torch.randn(nb, bs, hkv, d, generator=g)
    elif layout == "hnd":
        kc = torch.randn(nb, hkv, bs, d, generator=g).transpose(1, 2)
        vc = torch.randn(nb, hkv, bs, d, generator=g).transpose(1, 2)
    else:
        kv = torch.randn(nb, hkv, bs, 2 * d, generator=g)
        kc, vc = kv.transpose(1, 2).split(d, dim=-1)
    key = torch.randn(t, hkv, d, generator=g)
    value = torch.randn(t, hkv, d, generator=g)
    slots = torch.randperm(nb * bs, generator=g)[:t]
    slots[2] = -1  # padding token
    nk, nv = reshape_and_cache_reference(key, value, kc, vc, slots)
    # index_put_ on a flat [slots, heads, d] copy.
    live = slots >= 0
    fk = kc.contiguous().reshape(nb * bs, hkv, d).clone()
    fk.index_put_((slots[live],), key[live])
    assert torch.equal(nk.reshape(nb * bs, hkv, d), fk)
    # Gathering the written tokens back through a block table returns them.
    bt = torch.arange(nb, dtype=torch.int32)
    whole = gather_kv(nv, bt, nb * bs)
    assert torch.equal(whole[slots[live]], value[live])
    # Untouched slots keep their contents; the padding token wrote nothing.
    keep = torch.ones(nb * bs, dtype=torch.bool)
    keep[slots[live]] = False
    assert torch.equal(gather_kv(nk, bt, nb * bs)[keep], gather_kv(kc, bt, nb * bs)[keep])


def test_cache_write_skips_slots_past_the_cache():
    kc = torch.zeros(2, 4, 1, 8)
    vc = torch.zeros(2, 4, 1, 8)
    key = torch.ones(2, 1, 8)
    nk, nv = reshape_and_cache_reference(key, key, kc, vc, torch.tensor([8, 3]))
    assert nk.sum() == 8 and nk[0, 3].sum() == 8 and nv[0, 3].sum() == 8
