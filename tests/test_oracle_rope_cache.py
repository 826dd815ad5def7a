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


# ---------------------------------------------------------------------------
# fp8 (e4m3fn) cache write: quantize_e4m3 against a brute-force nearest search
# ---------------------------------------------------------------------------
def _e4m3_table():
    """(values, codes) of every finite e4m3fn encoding, by decoding the 8 bits."""
    codes = torch.arange(256, dtype=torch.int32)
    vals = codes.to(torch.uint8).view(torch.float8_e4m3fn).float()
    keep = torch.isfinite(vals)
    return vals[keep].double(), codes[keep]


def _brute_e4m3(x: torch.Tensor, scale: float, ties_even: bool = True) -> torch.Tensor:
    """Nearest finite e4m3fn value to fp32(x / scale); ties go to the even
    encoding (last mantissa bit 0) -- or away from zero with ties_even=False,
    a planted mistake; beyond +-448 saturate; NaN stays NaN."""
    vals, codes = _e4m3_table()
    y = (x.float() / torch.tensor(scale, dtype=torch.float32)).double()
    out = torch.empty_like(y)
    for i, v in enumerate(y.tolist()):
        if v != v:
            out[i] = float("nan")
            continue
        v = max(min(v, 448.0), -448.0)
        d = (vals - v).abs()
        best = d.min()
        ties = (d == best).nonzero().flatten()
        if len(ties) == 1:
            pick = ties[0]
        elif ties_even:
            pick = next(t for t in ties if int(codes[t]) % 2 == 0)
        else:
            pick = max(ties.tolist(), key=lambda t: abs(float(vals[t])))
        out[i] = vals[pick]
    return out


def _fp8_probe_values():
    vals, _ = _e4m3_table()
    fin = vals.float().unique()
    mids = (fin[1:] + fin[:-1]) / 2
    extra = torch.tensor([449.0, 464.0, 500.0, 1e6, float("inf"), 1e-12, 2.0**-10, 3 * 2.0**-11, float("nan")])
    up = torch.nextafter(mids, torch.full_like(mids, 1e9))
    down = torch.nextafter(mids, torch.full_like(mids, -1e9))
    g = torch.Generator().manual_seed(3)
    rnd = torch.randn(400, generator=g) * 40
    x = torch.cat([fin, mids, up, down, extra, rnd])
    return torch.cat([x, -x])


@pytest.mark.parametrize("scale", [1.0, 0.37, 2.5])
def test_fp8_quantization_matches_brute_force(scale):
    from oracle.rope_cache import quantize_e4m3

    x = _fp8_probe_values() * scale  # the midpoints land back on midpoints after / scale (up to fp32 rounding)
    got = quantize_e4m3(x, scale).double()
    want = _brute_e4m3(x, scale)
    same = (got == want) | (got.isnan() & want.isnan())
    assert same.all(), [(float(x[i]), float(got[i]), float(want[i])) for i in (~same).nonzero().flatten()[:5]]


@pytest.mark.parametrize("mistake", ["ties_away_from_zero", "multiply_by_scale", "no_saturation"])
def test_fp8_quantization_pins_catch_planted_mistakes(mistake):
    """Each wrong quantizer differs from the pinned oracle on the probe values."""
    from oracle.rope_cache import quantize_e4m3

    x = _fp8_probe_values()
    if mistake == "ties_away_from_zero":
        got = _brute_e4m3(x, 1.0, ties_even=False)
        want = quantize_e4m3(x, 1.0).double()
    elif mistake == "multiply_by_scale":
        got = (x.float() * 2.5).clamp(-448, 448).to(torch.float8_e4m3fn).double()
        want = _brute_e4m3(x, 2.5)
    else:  # torch's cast alone turns values past the range into NaN
        got = x.float().to(torch.float8_e4m3fn).double()
        want = _brute_e4m3(x, 1.0)
    same = (got == want) | (got.isnan() & want.isnan())
    assert not same.all(), f"the brute-force pin does not catch {mistake}"


def test_fp8_cache_write_reference_quantizes_rows():
    from oracle.rope_cache import quantize_e4m3

    nb, bs, h, d, t = 6, 16, 2, 64, 5
    kc = torch.zeros(nb, bs, h, d, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    g = torch.Generator().manual_seed(4)
    key = torch.randn(t, h, d, generator=g, dtype=torch.bfloat16) * 100
    value = torch.randn(t, h * d, generator=g, dtype=torch.bfloat16)
    slots = torch.tensor([3, -1, 40, 95, 96 * 2])
    got_k, got_v = reshape_and_cache_reference(key, value, kc, vc, slots, k_scale=0.5, v_scale=0.01)
    for i, s in enumerate(slots.tolist()):
        if 0 <= s < nb * bs:
            assert torch.equal(got_k[s // bs, s % bs].view(torch.uint8), quantize_e4m3(key[i], 0.5).view(torch.uint8))
            assert torch.equal(got_v[s // bs, s % bs].view(torch.uint8),
                               quantize_e4m3(value[i].view(h, d), 0.01).view(torch.uint8))
    untouched = torch.ones(nb * bs, dtype=torch.bool)
    untouched[[3, 40, 95]] = False
    assert (got_k.view(nb * bs, h, d)[untouched].float() == 0).all()
