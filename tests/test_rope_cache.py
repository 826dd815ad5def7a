"""GPU parity tests of rotary_embedding and reshape_and_cache against
``oracle/rope_cache.py``.

Rotary embedding: bit-exact against the oracle (both round each fp32 product
and sum on its own, then once to the model dtype; the kernel is built without
fused multiply-adds for this), including columns past rot_dim and tokens
whose position is outside the table, which stay as they were. Cache write:
bit-exact. Cases: NeoX and GPT-J pairing, partial rot_dim, float32 and
model-dtype tables, flat / 3-D / strided q and k (the vector and the scalar
paths), key None, the three cache layouts paged attention reads, padding and
out-of-range slots, and a decode step that appends a token through
reshape_and_cache and attends over it. rotary_embedding_and_cache (both steps
in one launch) must equal the two ops in sequence bit for bit, and the oracle.
"""

import ctypes

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from decodekernels_amd.testing import make_paged_kv
from oracle.rope_cache import reshape_and_cache_reference, rope_cos_sin_cache, rotary_embedding_reference
from parity import assert_max_abs, assert_ulp, attention_f32

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
FP8 = torch.float8_e4m3fn


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _qkv(t, hq, hkv, d, dtype, seed, pad=0):
    """Query and key as the column slices of a fused qkv projection output
    ([t, (hq + 2 hkv) d + pad]), the layout a decode step hands to RoPE."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    width = (hq + 2 * hkv) * d + pad
    qkv = torch.randn(t, width, generator=g, device="cuda", dtype=dtype)
    return qkv, qkv[:, : hq * d], qkv[:, hq * d : (hq + hkv) * d]


def _positions(t, max_position, seed, out_of_range=True):
    g = torch.Generator(device="cpu").manual_seed(seed)
    pos = torch.randint(0, max_position, (t,), generator=g)
    if out_of_range and t >= 3:
        pos[0], pos[t // 2], pos[-1] = -1, max_position, 0
    return pos.cuda()


def _check_rope(pos, q, k, head_size, cache, is_neox):
    want_q, want_k = rotary_embedding_reference(
        pos.cpu(), q.cpu(), None if k is None else k.cpu(), head_size, cache.cpu(), is_neox
    )
    q0 = q.clone()
    dk.rotary_embedding(pos, q, k, head_size, cache, is_neox)
    torch.cuda.synchronize()
    assert_ulp(q, want_q, 0, "rotary_embedding(query)")
    rot = cache.shape[1]
    t = q.shape[0]
    assert torch.equal(q.reshape(t, -1, head_size)[..., rot:], q0.reshape(t, -1, head_size)[..., rot:])
    bad = (pos < 0) | (pos >= cache.shape[0])
    assert torch.equal(q[bad], q0[bad])
    if k is not None:
        assert_ulp(k, want_k, 0, "rotary_embedding(key)")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("head_size,rot_dim", [(64, 64), (128, 128), (256, 256), (128, 64), (128, 32)])
def test_rope_fused_qkv_slices(dtype, is_neox, head_size, rot_dim):
    t, hq, hkv = 37, 8, 2
    cache = rope_cos_sin_cache(4096, rot_dim).cuda()
    qkv, q, k = _qkv(t, hq, hkv, head_size, dtype, seed=head_size + rot_dim + is_neox)
    v0 = qkv[:, (hq + hkv) * head_size :].clone()
    _check_rope(_positions(t, 4096, 1), q, k, head_size, cache, is_neox)
    assert torch.equal(qkv[:, (hq + hkv) * head_size :], v0), "value columns must be untouched"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
def test_rope_model_dtype_table_and_3d_views(dtype, is_neox):
    t, hq, hkv, d = 64, 32, 8, 128
    cache = rope_cos_sin_cache(8192, d, base=500000.0, dtype=dtype).cuda()
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn(t, hq, d, generator=g, device="cuda", dtype=dtype)
    k = torch.randn(t, hkv, 2, d, generator=g, device="cuda", dtype=dtype)[:, :, 1]  # head stride 2d
    _check_rope(_positions(t, 8192, 2), q, k, d, cache, is_neox)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("case", ["odd_stride", "rot_dim_20", "head_size_80"])
def test_rope_scalar_path(dtype, is_neox, case):
    """Layouts the vector path cannot take: token strides not a multiple of
    the vector, rot_dim / 2 not a multiple of 4."""
    t, hq, hkv = 19, 4, 2
    if case == "odd_stride":
        d, rot, pad = 128, 128, 2
    elif case == "rot_dim_20":
        d, rot, pad = 64, 20, 0
    else:
        d, rot, pad = 80, 40, 0
    cache = rope_cos_sin_cache(1000, rot).cuda()
    _, q, k = _qkv(t, hq, hkv, d, dtype, seed=7, pad=pad)
    _check_rope(_positions(t, 1000, 3), q, k, d, cache, is_neox)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_without_key_and_large_batch(dtype):
    t, hq, d = 4096, 32, 128
    cache = rope_cos_sin_cache(131072, d, base=500000.0).cuda()
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(t, hq * d, generator=g, device="cuda", dtype=dtype)
    _check_rope(_positions(t, 131072, 4), q, None, d, cache, True)


def test_rope_no_tokens_is_a_no_op():
    q = torch.empty(0, 128, device="cuda", dtype=torch.bfloat16)
    dk.rotary_embedding(torch.empty(0, dtype=torch.long, device="cuda"), q, None, 128, torch.zeros(8, 128, device="cuda"))
    torch.cuda.synchronize()


def test_rope_rejects_bad_arguments():
    q = torch.zeros(4, 256, device="cuda", dtype=torch.bfloat16)
    pos = torch.zeros(4, dtype=torch.long, device="cuda")
    with pytest.raises(RuntimeError, match="rot_dim"):
        dk.rotary_embedding(pos, q, None, 128, torch.zeros(8, 130, device="cuda"))
    with pytest.raises(RuntimeError, match="float32 or the query dtype"):
        dk.rotary_embedding(pos, q, None, 128, torch.zeros(8, 128, device="cuda", dtype=torch.float16))
    with pytest.raises(RuntimeError, match="int64"):
        dk.rotary_embedding(pos.int(), q, None, 128, torch.zeros(8, 128, device="cuda"))
    with pytest.raises(RuntimeError, match="multiple of head_size"):
        dk.rotary_embedding(pos, q, None, 96, torch.zeros(8, 96, device="cuda"))


@pytest.mark.parametrize("is_neox", [True, False])
def test_rope_capi_matches_torch_op(is_neox):
    dtype = torch.bfloat16
    t, hq, hkv, d = 33, 8, 2, 128
    cache = rope_cos_sin_cache(2048, d).cuda()
    _, q, k = _qkv(t, hq, hkv, d, dtype, seed=11)
    q2, k2 = q.clone(), k.clone()
    pos = _positions(t, 2048, 5)
    p = capi.rotary_params(pos, q2, k2, d, cache, is_neox)
    rc = capi.lib().dk_rotary_embedding(ctypes.byref(p), capi.dtype_code(dtype), _stream())
    assert rc == 0, capi.last_error()
    dk.rotary_embedding(pos, q, k, d, cache, is_neox)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(k, k2)


# ---------------------------------------------------------------------------
# reshape_and_cache
# ---------------------------------------------------------------------------
def _slots(num_blocks, block_size, t, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    slots = torch.randperm(num_blocks * block_size, generator=g)[:t].clone()
    if t >= 4:
        slots[1] = -1  # padding token
        slots[t // 2] = num_blocks * block_size + 3  # past the cache: skipped
    return slots.cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["nhd", "hnd", "vllm"])
@pytest.mark.parametrize("head_dim,block_size", [(64, 16), (128, 16), (128, 32), (256, 16)])
def test_cache_write_layouts(dtype, layout, head_dim, block_size):
    hkv, t = 4, 150
    kv = make_paged_kv([700, 300], hkv, head_dim, block_size, dtype, "cuda", layout=layout, seed=head_dim)
    g = torch.Generator(device="cuda").manual_seed(12)
    key = torch.randn(t, hkv, head_dim, generator=g, device="cuda", dtype=dtype)
    value = torch.randn(t, hkv * head_dim, generator=g, device="cuda", dtype=dtype)
    slots = _slots(kv.k_cache.shape[0], block_size, t, 13)
    want_k, want_v = reshape_and_cache_reference(key.cpu(), value.cpu(), kv.k_cache.cpu(), kv.v_cache.cpu(), slots.cpu())
    dk.reshape_and_cache(key, value, kv.k_cache, kv.v_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(kv.k_cache.cpu(), want_k)
    assert torch.equal(kv.v_cache.cpu(), want_v)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", ["misaligned_rows", "head_size_36"])
def test_cache_write_scalar_path(dtype, case):
    hkv, t, bs, nb = 2, 40, 16, 8
    d = 36 if case == "head_size_36" else 64
    g = torch.Generator(device="cuda").manual_seed(14)
    kc = torch.randn(nb, bs, hkv, d, generator=g, device="cuda", dtype=dtype)
    vc = torch.randn(nb, bs, hkv, d, generator=g, device="cuda", dtype=dtype)
    buf = torch.randn(t, 2 * hkv * d + 1, generator=g, device="cuda", dtype=dtype)
    off = 1 if case == "misaligned_rows" else 0
    key = buf[:, off : off + hkv * d]
    value = buf[:, off + hkv * d : off + 2 * hkv * d]
    slots = _slots(nb, bs, t, 15)
    want_k, want_v = reshape_and_cache_reference(key.cpu(), value.cpu(), kc.cpu(), vc.cpu(), slots.cpu())
    dk.reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), want_k) and torch.equal(vc.cpu(), want_v)


def test_cache_write_capi_matches_torch_op():
    dtype = torch.float16
    kv = make_paged_kv([900], 8, 128, 16, dtype, "cuda", layout="vllm", seed=3)
    kc2, vc2 = kv.k_cache.clone(), kv.v_cache.clone()
    g = torch.Generator(device="cuda").manual_seed(16)
    key = torch.randn(64, 8, 128, generator=g, device="cuda", dtype=dtype)
    value = torch.randn(64, 8, 128, generator=g, device="cuda", dtype=dtype)
    slots = _slots(kv.k_cache.shape[0], 16, 64, 17)
    p = capi.cache_write_params(key, value, kc2, vc2, slots)
    rc = capi.lib().dk_reshape_and_cache(ctypes.byref(p), capi.dtype_code(dtype), _stream())
    assert rc == 0, capi.last_error()
    dk.reshape_and_cache(key, value, kv.k_cache, kv.v_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(kv.k_cache, kc2) and torch.equal(kv.v_cache, vc2)


def test_cache_write_rejects_bad_arguments():
    kc = torch.zeros(4, 16, 2, 64, device="cuda", dtype=torch.bfloat16)
    key = torch.zeros(3, 2, 64, device="cuda", dtype=torch.bfloat16)
    slots = torch.zeros(3, dtype=torch.long, device="cuda")
    with pytest.raises(RuntimeError, match="int64"):
        dk.reshape_and_cache(key, key, kc, kc.clone(), slots.int())
    with pytest.raises(RuntimeError, match="heads"):
        dk.reshape_and_cache(torch.zeros(3, 4, 64, device="cuda", dtype=torch.bfloat16), key, kc, kc.clone(), slots)
    with pytest.raises(RuntimeError, match="one key / value row"):
        dk.reshape_and_cache(key, key, kc, kc.clone(), slots[:2])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["nhd", "vllm"])
def test_decode_step_appends_and_attends(dtype, layout):
    """One decode step: RoPE on the new token's q / k, the k / v row written at
    the next slot of each sequence, then attention over the grown cache."""
    hq, hkv, d, bs = 16, 4, 128, 16
    lens = [5, 300, 1100, 47]  # none a multiple of the block size: room in the last block
    kv = make_paged_kv(lens, hkv, d, bs, dtype, "cuda", layout=layout, seed=18)
    n = len(lens)
    qkv, q, k = _qkv(n, hq, hkv, d, dtype, seed=19)
    v = qkv[:, (hq + hkv) * d :]
    cache = rope_cos_sin_cache(4096, d).cuda()
    pos = torch.tensor(lens, device="cuda")  # the new token's position
    want_q, want_k = rotary_embedding_reference(pos.cpu(), q.cpu(), k.cpu(), d, cache.cpu(), True)
    dk.rotary_embedding(pos, q, k, d, cache, True)
    bt = kv.block_tables.cpu()
    slots = torch.tensor([int(bt[s, lens[s] // bs]) * bs + lens[s] % bs for s in range(n)], device="cuda")
    dk.reshape_and_cache(k, v, kv.k_cache, kv.v_cache, slots)
    new_lens = (kv.seq_lens + 1).contiguous()
    q3 = q.reshape(n, hq, d)
    out = dk.paged_attention_decode(q3, kv.k_cache, kv.v_cache, kv.block_tables, new_lens)
    torch.cuda.synchronize()
    assert_ulp(q, want_q, 0, "rotary_embedding(query)")
    assert_ulp(k, want_k, 0, "rotary_embedding(key)")
    ref = attention_f32(q3, kv.k_cache, kv.v_cache, kv.block_tables, new_lens)
    assert_max_abs(out, ref, dtype, "paged_attention_decode after the cache write")


# ---------------------------------------------------------------------------
# rotary_embedding_and_cache: both steps in one launch, bit-identical to the
# two ops in sequence and to the oracle
# ---------------------------------------------------------------------------
def _fused_inputs(dtype, is_neox, head_size, rot_dim, layout, seed, t=61, hq=8, hkv=2, bs=16, misalign=False,
                  cache_dtype=None):
    kv = make_paged_kv([700, 300], hkv, head_size, bs, cache_dtype or dtype, "cuda", layout=layout, seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    width = (hq + 2 * hkv) * head_size
    buf = torch.randn(t, width + 1, generator=g, device="cuda", dtype=dtype)
    qkv = buf[:, 1:] if misalign else buf[:, :width]  # misaligned rows take the scalar path
    q, k = qkv[:, : hq * head_size], qkv[:, hq * head_size : (hq + hkv) * head_size]
    v = qkv[:, (hq + hkv) * head_size :]
    table_dtype = torch.float32 if is_neox else dtype
    cache = rope_cos_sin_cache(4096, rot_dim).to(table_dtype).cuda()
    pos = _positions(t, 4096, seed + 2)
    slots = _slots(kv.k_cache.shape[0], bs, t, seed + 3)
    return kv, buf, q, k, v, cache, pos, slots


def _run_fused_and_pair(kv, buf, q, k, v, cache, pos, slots, head_size, is_neox, **scales):
    """(fused results, two-op results): q, k, k_cache, v_cache of each
    (fp8 caches as their bytes)."""
    kc2, vc2 = kv.k_cache.clone(), kv.v_cache.clone()
    buf2 = buf.clone()
    off = q.data_ptr() - buf.data_ptr()
    el = buf.element_size()
    q2 = buf2.view(-1)[off // el :].as_strided(q.shape, q.stride())
    k2 = buf2.view(-1)[(k.data_ptr() - buf.data_ptr()) // el :].as_strided(k.shape, k.stride())
    v2 = buf2.view(-1)[(v.data_ptr() - buf.data_ptr()) // el :].as_strided(v.shape, v.stride())
    dk.rotary_embedding(pos, q2, k2, head_size, cache, is_neox)
    dk.reshape_and_cache(k2, v2, kc2, vc2, slots, **scales)
    dk.rotary_embedding_and_cache(pos, q, k, v, head_size, cache, is_neox, kv.k_cache, kv.v_cache, slots, **scales)
    torch.cuda.synchronize()
    b = lambda c: c.view(torch.uint8) if c.dtype == FP8 else c  # noqa: E731
    return (q, k, b(kv.k_cache), b(kv.v_cache)), (q2, k2, b(kc2), b(vc2))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("head_size,rot_dim", [(128, 128), (128, 64), (64, 64), (256, 256)])
@pytest.mark.parametrize("layout", ["nhd", "hnd", "vllm"])
def test_fused_rope_and_cache_equals_the_two_ops(dtype, is_neox, head_size, rot_dim, layout):
    seed = head_size + rot_dim + 3 * is_neox
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(dtype, is_neox, head_size, rot_dim, layout, seed)
    kc0, vc0 = kv.k_cache.cpu(), kv.v_cache.cpu()
    q0, k0, v0 = q.cpu(), k.cpu(), v.cpu()
    fused, pair = _run_fused_and_pair(kv, buf, q, k, v, cache, pos, slots, head_size, is_neox)
    for name, a, b in zip(("query", "key", "key_cache", "value_cache"), fused, pair):
        assert torch.equal(a, b), f"fused {name} differs from rotary_embedding + reshape_and_cache"
    want_q, want_k = rotary_embedding_reference(pos.cpu(), q0, k0, head_size, cache.cpu(), is_neox)
    want_kc, want_vc = reshape_and_cache_reference(want_k.reshape(k0.shape[0], -1, head_size), v0, kc0, vc0,
                                                   slots.cpu())
    assert_ulp(q, want_q, 0, "fused rotary(query)")
    assert_ulp(k, want_k, 0, "fused rotary(key)")
    assert torch.equal(kv.k_cache.cpu(), want_kc) and torch.equal(kv.v_cache.cpu(), want_vc)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("case", ["misaligned_rows", "rot_dim_36"])
def test_fused_rope_and_cache_scalar_path(dtype, is_neox, case):
    rot = 36 if case == "rot_dim_36" else 64  # rot_dim % 8 != 0 keeps the copies element-wise
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(dtype, is_neox, 64, rot, "vllm", seed=40 + rot,
                                                        misalign=case == "misaligned_rows")
    fused, pair = _run_fused_and_pair(kv, buf, q, k, v, cache, pos, slots, 64, is_neox)
    for name, a, b in zip(("query", "key", "key_cache", "value_cache"), fused, pair):
        assert torch.equal(a, b), f"fused {name} differs ({case})"


def test_fused_rope_and_cache_capi_and_errors():
    dtype = torch.bfloat16
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(dtype, True, 128, 128, "vllm", seed=50)
    kv2 = make_paged_kv([700, 300], 2, 128, 16, dtype, "cuda", layout="vllm", seed=50)
    buf2 = buf.clone()
    q2, k2, v2 = buf2[:, : 8 * 128], buf2[:, 8 * 128 : 10 * 128], buf2[:, 10 * 128 : 12 * 128]
    r = capi.rotary_params(pos, q2, k2, 128, cache, True)
    c = capi.cache_write_params(k2, v2, kv2.k_cache, kv2.v_cache, slots)
    rc = capi.lib().dk_rotary_embedding_and_cache(ctypes.byref(r), ctypes.byref(c), capi.dtype_code(dtype), _stream())
    assert rc == 0, capi.last_error()
    dk.rotary_embedding_and_cache(pos, q, k, v, 128, cache, True, kv.k_cache, kv.v_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(buf, buf2) and torch.equal(kv.k_cache, kv2.k_cache) and torch.equal(kv.v_cache, kv2.v_cache)
    with pytest.raises(RuntimeError, match="one key / value row"):
        dk.rotary_embedding_and_cache(pos, q, k, v, 128, cache, True, kv.k_cache, kv.v_cache, slots[:5])
    with pytest.raises(RuntimeError, match="heads must match the cache"):
        small = make_paged_kv([100], 2, 64, 16, dtype, "cuda", seed=51)
        dk.rotary_embedding_and_cache(pos, q, k, v, 128, cache, True, small.k_cache, small.v_cache, slots)
    dk.rotary_embedding_and_cache(pos[:0], q[:0], k[:0], v[:0], 128, cache, True, kv.k_cache, kv.v_cache, slots[:0])


# ---------------------------------------------------------------------------
# Cache write into an fp8 (e4m3fn) cache: x / scale, saturated, nearest even
# ---------------------------------------------------------------------------


def _fp8_rows(t, hkv, d, dtype, seed):
    """Rows mixing ordinary values, exact e4m3 midpoints and values past +-448 (x scale later)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(t, hkv, d, generator=g) * 3
    table = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(FP8).float()
    fin = table[torch.isfinite(table)].unique()
    mids = (fin[1:] + fin[:-1]) / 2
    pick = torch.randint(0, len(mids), (t, hkv, d // 4), generator=g)
    x[..., : d // 4] = mids[pick]
    x[:, 0, -2:] = torch.tensor([900.0, -2000.0])
    return x.to(dtype).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["nhd", "hnd", "vllm"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.37, 2.5)])
def test_fp8_cache_write_matches_oracle(dtype, layout, head_dim, k_scale, v_scale):
    hkv, t, bs = 2, 70, 16
    kv = make_paged_kv([700, 300], hkv, head_dim, bs, FP8, "cuda", layout=layout, seed=head_dim)
    key = _fp8_rows(t, hkv, head_dim, dtype, seed=1) * k_scale
    value = _fp8_rows(t, hkv, head_dim, dtype, seed=2).reshape(t, hkv * head_dim) * v_scale
    slots = _slots(kv.k_cache.shape[0], bs, t, 21)
    want_k, want_v = reshape_and_cache_reference(key.cpu(), value.cpu(), kv.k_cache.cpu(), kv.v_cache.cpu(),
                                                 slots.cpu(), k_scale, v_scale)
    dk.reshape_and_cache(key, value, kv.k_cache, kv.v_cache, slots, k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    assert torch.equal(kv.k_cache.cpu().view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(kv.v_cache.cpu().view(torch.uint8), want_v.view(torch.uint8))


@pytest.mark.parametrize("case", ["misaligned_rows", "head_size_36"])
def test_fp8_cache_write_scalar_path(case):
    dtype, hkv, t, bs, nb = torch.bfloat16, 2, 40, 16, 8
    d = 36 if case == "head_size_36" else 64
    kc = torch.zeros(nb, bs, hkv, d, device="cuda", dtype=FP8)
    vc = torch.zeros_like(kc)
    buf = torch.cat([_fp8_rows(t, hkv, d, dtype, seed=3).reshape(t, -1), _fp8_rows(t, hkv, d, dtype, seed=4).reshape(t, -1),
                     torch.zeros(t, 1, device="cuda", dtype=dtype)], dim=1)
    off = 1 if case == "misaligned_rows" else 0
    key = buf[:, off : off + hkv * d]
    value = buf[:, off + hkv * d : off + 2 * hkv * d]
    slots = _slots(nb, bs, t, 22)
    want_k, want_v = reshape_and_cache_reference(key.cpu(), value.cpu(), kc.cpu(), vc.cpu(), slots.cpu(), 0.5, 0.75)
    dk.reshape_and_cache(key, value, kc, vc, slots, k_scale=0.5, v_scale=0.75)
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu().view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(vc.cpu().view(torch.uint8), want_v.view(torch.uint8))


@pytest.mark.parametrize("dtype", DTYPES)
def test_fp8_decode_step_writes_then_attends(dtype):
    """RoPE, the new token quantized into the fp8 cache, then fp8 attention
    over the grown cache, against the fp32 oracle on the dequantized cache."""
    hq, hkv, d, bs = 16, 4, 128, 16
    lens = [5, 300, 1100, 47]
    kv = make_paged_kv(lens, hkv, d, bs, FP8, "cuda", layout="vllm", seed=23)
    n = len(lens)
    qkv, q, k = _qkv(n, hq, hkv, d, dtype, seed=24)
    v = qkv[:, (hq + hkv) * d :]
    cache = rope_cos_sin_cache(4096, d).cuda()
    pos = torch.tensor(lens, device="cuda")
    dk.rotary_embedding(pos, q, k, d, cache, True)
    bt = kv.block_tables.cpu()
    slots = torch.tensor([int(bt[s, lens[s] // bs]) * bs + lens[s] % bs for s in range(n)], device="cuda")
    ks, vs = 0.05, 0.02
    want_k, want_v = reshape_and_cache_reference(k.cpu(), v.cpu(), kv.k_cache.cpu(), kv.v_cache.cpu(), slots.cpu(), ks, vs)
    dk.reshape_and_cache(k, v, kv.k_cache, kv.v_cache, slots, k_scale=ks, v_scale=vs)
    new_lens = (kv.seq_lens + 1).contiguous()
    q3 = q.reshape(n, hq, d)
    out = dk.paged_attention_decode(q3, kv.k_cache, kv.v_cache, kv.block_tables, new_lens, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert torch.equal(kv.k_cache.cpu().view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(kv.v_cache.cpu().view(torch.uint8), want_v.view(torch.uint8))
    ref = attention_f32(q3, kv.k_cache.float() * ks, kv.v_cache.float() * vs, kv.block_tables, new_lens)
    assert_max_abs(out, ref, dtype, "fp8 attention after the fp8 cache write")


# ---------------------------------------------------------------------------
# rotary_embedding_and_cache into fp8 caches: equal to rotary_embedding then
# the fp8 cache write, and to the oracle. Small scales push part of k / v
# past +-448 so the saturation is exercised.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("head_size,rot_dim", [(128, 128), (128, 64), (256, 256)])
@pytest.mark.parametrize("layout", ["nhd", "vllm"])
@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.004, 0.01)])
def test_fused_rope_and_fp8_cache_equals_the_two_ops(dtype, is_neox, head_size, rot_dim, layout, k_scale, v_scale):
    seed = head_size + rot_dim + 3 * is_neox + 7
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(dtype, is_neox, head_size, rot_dim, layout, seed,
                                                        cache_dtype=FP8)
    kc0, vc0 = kv.k_cache.cpu(), kv.v_cache.cpu()
    q0, k0, v0 = q.cpu(), k.cpu(), v.cpu()
    fused, pair = _run_fused_and_pair(kv, buf, q, k, v, cache, pos, slots, head_size, is_neox, k_scale=k_scale,
                                      v_scale=v_scale)
    for name, a, b in zip(("query", "key", "key_cache", "value_cache"), fused, pair):
        assert torch.equal(a, b), f"fused {name} differs from rotary_embedding + fp8 reshape_and_cache"
    want_q, want_k = rotary_embedding_reference(pos.cpu(), q0, k0, head_size, cache.cpu(), is_neox)
    want_kc, want_vc = reshape_and_cache_reference(want_k.reshape(k0.shape[0], -1, head_size), v0, kc0, vc0,
                                                   slots.cpu(), k_scale, v_scale)
    assert_ulp(q, want_q, 0, "fused rotary(query)")
    assert_ulp(k, want_k, 0, "fused rotary(key)")
    assert torch.equal(fused[2].cpu(), want_kc.view(torch.uint8))
    assert torch.equal(fused[3].cpu(), want_vc.view(torch.uint8))
    if k_scale != 1.0:
        assert (want_kc.float().abs() == 448).any(), "no saturated key in the case"


@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("case", ["misaligned_rows", "rot_dim_36"])
def test_fused_rope_and_fp8_cache_scalar_path(is_neox, case):
    rot = 36 if case == "rot_dim_36" else 64
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(torch.bfloat16, is_neox, 64, rot, "vllm", seed=60 + rot,
                                                        misalign=case == "misaligned_rows", cache_dtype=FP8)
    fused, pair = _run_fused_and_pair(kv, buf, q, k, v, cache, pos, slots, 64, is_neox, k_scale=0.01, v_scale=0.5)
    for name, a, b in zip(("query", "key", "key_cache", "value_cache"), fused, pair):
        assert torch.equal(a, b), f"fused {name} differs ({case})"


def test_fused_rope_and_fp8_cache_capi():
    dtype = torch.float16
    kv, buf, q, k, v, cache, pos, slots = _fused_inputs(dtype, False, 128, 128, "hnd", seed=70, cache_dtype=FP8)
    kv2 = make_paged_kv([700, 300], 2, 128, 16, FP8, "cuda", layout="hnd", seed=70)
    buf2 = buf.clone()
    q2, k2, v2 = buf2[:, : 8 * 128], buf2[:, 8 * 128 : 10 * 128], buf2[:, 10 * 128 : 12 * 128]
    r = capi.rotary_params(pos, q2, k2, 128, cache, False)
    c = capi.cache_write_params(k2, v2, kv2.k_cache, kv2.v_cache, slots)
    rc = capi.lib().dk_rotary_embedding_and_cache_fp8(ctypes.byref(r), ctypes.byref(c), capi.dtype_code(dtype), 0.02,
                                                      0.03, _stream())
    assert rc == 0, capi.last_error()
    dk.rotary_embedding_and_cache(pos, q, k, v, 128, cache, False, kv.k_cache, kv.v_cache, slots, k_scale=0.02,
                                  v_scale=0.03)
    torch.cuda.synchronize()
    assert torch.equal(buf, buf2)
    assert torch.equal(kv.k_cache.view(torch.uint8), kv2.k_cache.view(torch.uint8))
    assert torch.equal(kv.v_cache.view(torch.uint8), kv2.v_cache.view(torch.uint8))
    with pytest.raises(RuntimeError, match="float8_e4m3fn"):
        torch.ops.decode_kernels.rotary_embedding_and_cache_fp8(pos, q, k, v, 128, cache, False, kv.k_cache.view(
            torch.uint8), kv.v_cache.view(torch.uint8), slots, 1.0, 1.0)
