"""CPU tests of the host side: the C-ABI library, its argument validation and
the Python wrappers' host logic. No kernel is launched: every C-ABI call here
fails validation (or is a documented no-op) before any HIP call."""

import ctypes
import subprocess

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi, ops
from decodekernels_amd.testing import make_paged_kv


def test_library_exports_every_declared_symbol():
    declared = capi.declared_functions()
    assert set(declared) >= {
        "dk_paged_attention_decode",
        "dk_paged_attention_decode_fp8",
        "dk_gemm_tn",
        "dk_gemm_tn_workspace_bytes",
        "dk_gemm_tn_plan",
        "dk_gemm_tn_ws",
        "dk_rms_norm",
        "dk_fused_add_rms_norm",
        "dk_silu_and_mul",
        "dk_rotary_embedding",
        "dk_reshape_and_cache",
        "dk_rotary_embedding_and_cache",
        "dk_reshape_and_cache_fp8",
        "dk_rotary_embedding_and_cache_fp8",
        "dk_last_error",
        "dk_error_string",
        "dk_version",
    }
    lib = capi.lib()
    for name in declared:
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if line.strip()}
    assert set(declared) <= exported
    assert b"gfx950" in capi.lib().dk_version()


def test_params_struct_matches_header_layout():
    # 9 pointers, 11 int64 strides, 5 int32 and a float: 9*8 + 11*8 + 5*4 + 4 = 184 bytes.
    assert ctypes.sizeof(capi.PagedAttnParams) == 184
    # 4 pointers, 5 int64 strides, 8 int32: 32 + 40 + 32 = 104 bytes.
    assert ctypes.sizeof(capi.RotaryParams) == 104
    # 5 pointers, 10 int64 strides, 5 int32 = 140, padded to 8: 144 bytes.
    assert ctypes.sizeof(capi.CacheWriteParams) == 144
    assert capi.RotaryParams.cache_dtype.offset == 100
    assert capi.CacheWriteParams.num_blocks.offset == 136


def _attn_params(num_q_heads=8, num_kv_heads=2, block_size=16, max_partitions=1):
    p = capi.PagedAttnParams()
    fake = 0x10000  # never dereferenced: validation fails or returns first
    p.out = p.q = p.k_cache = p.v_cache = p.block_tables = p.seq_lens = fake
    p.q_stride_seq, p.q_stride_head = num_q_heads * 128, 128
    p.out_stride_seq, p.out_stride_head = num_q_heads * 128, 128
    p.k_stride_block, p.k_stride_token, p.k_stride_head = block_size * num_kv_heads * 128, num_kv_heads * 128, 128
    p.v_stride_block, p.v_stride_token, p.v_stride_head = p.k_stride_block, p.k_stride_token, p.k_stride_head
    p.bt_stride = 4
    p.num_seqs, p.num_q_heads, p.num_kv_heads, p.block_size = 1, num_q_heads, num_kv_heads, block_size
    p.max_partitions = max_partitions
    p.scale = 0.1
    return p


@pytest.mark.parametrize(
    "kwargs,head_dim,max_len,dtype,message",
    [
        (dict(num_q_heads=64, num_kv_heads=2), 128, 10, capi.DK_BFLOAT16, "GQA group"),
        (dict(num_q_heads=6, num_kv_heads=4), 128, 10, capi.DK_BFLOAT16, "multiple of num_kv_heads"),
        (dict(), 80, 10, capi.DK_FLOAT16, "head_dim"),
        (dict(), 128, 10, 7, "float16 or bfloat16"),
        (dict(block_size=0), 128, 10, capi.DK_FLOAT16, "block_size"),
        (dict(), 128, -1, capi.DK_FLOAT16, "non-negative"),
        (dict(), 128, 2000, capi.DK_FLOAT16, "workspace"),
    ],
)
def test_capi_attention_validation(kwargs, head_dim, max_len, dtype, message):
    p = _attn_params(**kwargs)
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), dtype, head_dim, max_len, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert message in capi.last_error()


def test_capi_attention_workspace_too_small_and_misaligned():
    p = _attn_params(max_partitions=2)
    p.tmp_out = p.max_logits = p.exp_sums = 0x20000
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.DK_FLOAT16, 128, 2000, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "ceil(max_seq_len / 512)" in capi.last_error()
    p = _attn_params()
    p.k_stride_token = 130  # 260 bytes: not 8-byte aligned rows at head_dim 128
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.DK_FLOAT16, 128, 10, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "aligned" in capi.last_error()


@pytest.mark.parametrize("field,value", [("k_stride_token", 2**31), ("q_stride_seq", -128), ("bt_stride", 2**40),
                                         ("out_stride_head", 2**31 + 128), ("v_stride_block", -(2**33))])
def test_capi_attention_rejects_strides_outside_int32(field, value):
    """The kernels take element strides as 32-bit arguments (addresses formed
    in 64 bits), so a stride of 2^31 elements or more, or a negative one, is
    refused before any launch."""
    p = _attn_params()
    setattr(p, field, value)
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.DK_FLOAT16, 128, 10, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "strides must be in [0, 2^31)" in capi.last_error()


def test_capi_attention_fp8_validation():
    L = capi.lib()
    p = _attn_params()
    p.k_stride_token = 132  # bytes: not a multiple of 8
    rc = L.dk_paged_attention_decode_fp8(ctypes.byref(p), capi.DK_BFLOAT16, 128, 10, 1.0, 1.0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "multiples of 8 bytes" in capi.last_error()
    p = _attn_params()
    rc = L.dk_paged_attention_decode_fp8(ctypes.byref(p), capi.DK_BFLOAT16, 128, 10, float("nan"), 1.0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "finite" in capi.last_error()
    rc = L.dk_paged_attention_decode_fp8(ctypes.byref(p), 5, 128, 10, 1.0, 1.0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "float16 or bfloat16" in capi.last_error()
    p.num_seqs = 0
    assert L.dk_paged_attention_decode_fp8(ctypes.byref(p), capi.DK_FLOAT16, 128, 10, 1.0, 1.0, None) == 0


def test_capi_attention_zero_seqs_is_a_no_op():
    p = _attn_params()
    p.num_seqs = 0
    assert capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.DK_FLOAT16, 128, 10, None) == 0
    assert capi.last_error() == ""


def test_capi_gemm_validation():
    L = capi.lib()
    rc = L.dk_gemm_tn(capi.DK_FLOAT16, 0x1000, 0x1000, None, 0x1000, 4, 8, 100, 100, 100, 8, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "multiples of 8" in capi.last_error()
    rc = L.dk_gemm_tn(capi.DK_FLOAT16, 0x1008, 0x1000, None, 0x1000, 4, 8, 64, 64, 64, 8, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "16-byte aligned" in capi.last_error()
    assert L.dk_gemm_tn(capi.DK_FLOAT16, 0x1000, 0x1000, None, 0x1000, 0, 8, 64, 64, 64, 8, None) == 0
    assert L.dk_gemm_tn(capi.DK_BFLOAT16, 0x1000, 0x1000, None, 0x1000, 4, 0, 64, 64, 64, 8, None) == 0
    rc = L.dk_gemm_tn(5, 0x1000, 0x1000, None, 0x1000, 4, 8, 64, 64, 64, 8, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "float16 or bfloat16" in capi.last_error()
    # Row strides below the row lengths (overlapping rows; C written out of bounds) are refused,
    # negative ones included.
    for lda, ldb, ldc in [(56, 64, 16), (64, 56, 16), (64, 64, 8), (-64, 64, 16), (64, 64, -16)]:
        rc = L.dk_gemm_tn(capi.DK_BFLOAT16, 0x1000, 0x1000, None, 0x1000, 4, 16, 64, lda, ldb, ldc, None)
        assert rc == capi.HIP_ERROR_INVALID_VALUE and "at least the row lengths" in capi.last_error(), (lda, ldb, ldc)
    rc = L.dk_gemm_tn_ws(capi.DK_BFLOAT16, 0x1000, 0x1000, None, 0x1000, 64, 4096, 14336, 14336, 14336, 4000,
                         None, 0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "at least the row lengths" in capi.last_error()


def test_capi_gemm_workspace_sizes_and_validation():
    """Split-K workspace sizes (splits x M x N fp32) for decode shapes the plan
    splits, 0 for the rest; argument errors of dk_gemm_tn_ws."""
    L = capi.lib()
    for M, N, K, splits in [(64, 4096, 14336, 8), (32, 4096, 14336, 8), (16, 4096, 14336, 2), (64, 4096, 4096, 4),
                            (64, 6144, 4096, 4), (17, 1000, 8200, 4), (8, 4096, 14336, 0), (16, 4096, 4096, 0),
                            (32, 4096, 4096, 4), (16, 6144, 4096, 0), (32, 6144, 4096, 4), (64, 28672, 4096, 0),
                            (64, 37888, 3584, 0), (0, 8, 64, 0),
                            (256, 4096, 14336, 8), (512, 4096, 14336, 4), (256, 28672, 4096, 0),
                            (4096, 4096, 4096, 0)]:
        assert L.dk_gemm_tn_workspace_bytes(M, N, K) == splits * M * N * 4, (M, N, K)
    rc = L.dk_gemm_tn_ws(capi.DK_BFLOAT16, 0x1000, 0x1000, None, 0x1000, 64, 4096, 14336, 14336, 14336, 4096,
                         0x1008, 1 << 23, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "workspace must be 16-byte aligned" in capi.last_error()
    rc = L.dk_gemm_tn_ws(capi.DK_BFLOAT16, 0x1000, 0x1000, None, 0x1000, 64, 4096, 14336, 14336, 14336, 4096,
                         0x1000, -1, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "non-negative" in capi.last_error()
    rc = L.dk_gemm_tn_ws(capi.DK_FLOAT16, 0x1000, 0x1000, None, 0x1000, 4, 8, 100, 100, 100, 8, None, 0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "multiples of 8" in capi.last_error()
    assert L.dk_gemm_tn_ws(capi.DK_FLOAT16, 0x1000, 0x1000, None, 0x1000, 0, 8, 64, 64, 64, 8, None, 0, None) == 0


def test_capi_norm_validation():
    L = capi.lib()
    assert L.dk_rms_norm(capi.DK_FLOAT16, 0x1000, 0x1000, 0x1000, 0, 4096, 4096, 4096, 1e-6, None) == 0
    rc = L.dk_rms_norm(9, 0x1000, 0x1000, 0x1000, 1, 4096, 4096, 4096, 1e-6, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "rms_norm" in capi.last_error()
    rc = L.dk_fused_add_rms_norm(capi.DK_BFLOAT16, None, 0x1000, 0x1000, 1, 64, 64, 64, 1e-6, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert L.dk_silu_and_mul(capi.DK_FLOAT16, 0x1000, 0x1000, 5, 0, 0, 0, None) == 0
    rc = L.dk_silu_and_mul(capi.DK_FLOAT16, 0x1000, 0x1000, -1, 8, 16, 8, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    # Written rows may not overlap and no stride may be negative (a read-only input may repeat a row).
    for rc in (L.dk_rms_norm(capi.DK_BFLOAT16, 0x1000, 0x1000, 0x1000, 4, 64, 64, 32, 1e-6, None),
               L.dk_rms_norm(capi.DK_BFLOAT16, 0x1000, 0x1000, 0x1000, 4, 64, -64, 64, 1e-6, None),
               L.dk_fused_add_rms_norm(capi.DK_BFLOAT16, 0x1000, 0x1000, 0x1000, 4, 64, 0, 64, 1e-6, None),
               L.dk_fused_add_rms_norm(capi.DK_BFLOAT16, 0x1000, 0x1000, 0x1000, 4, 64, 64, 8, 1e-6, None),
               L.dk_silu_and_mul(capi.DK_FLOAT16, 0x1000, 0x1000, 4, 8, 16, 4, None),
               L.dk_silu_and_mul(capi.DK_FLOAT16, 0x1000, 0x1000, 4, 8, -16, 8, None)):
        assert rc == capi.HIP_ERROR_INVALID_VALUE and "overlap" in capi.last_error()
    assert capi.lib().dk_error_string(1)


def _rotary_params(**kw):
    p = capi.RotaryParams()
    p.positions = p.query = p.key = p.cos_sin_cache = 0x10000  # never dereferenced
    p.q_stride_token, p.q_stride_head = 4 * 128, 128
    p.k_stride_token, p.k_stride_head = 2 * 128, 128
    p.cache_stride = 128
    p.num_tokens, p.num_q_heads, p.num_kv_heads, p.head_size = 3, 4, 2, 128
    p.rot_dim, p.max_position, p.is_neox, p.cache_dtype = 128, 4096, 1, capi.DK_FLOAT32
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize(
    "kwargs,dtype,message",
    [
        (dict(), 3, "float16 or bfloat16"),
        (dict(cache_dtype=capi.DK_FLOAT16), capi.DK_BFLOAT16, "float32 or the query dtype"),
        (dict(rot_dim=130), capi.DK_BFLOAT16, "rot_dim"),
        (dict(rot_dim=63, head_size=64), capi.DK_BFLOAT16, "rot_dim"),
        (dict(rot_dim=0), capi.DK_FLOAT16, "rot_dim"),
        (dict(num_q_heads=-1), capi.DK_FLOAT16, "non-negative"),
        (dict(query=None), capi.DK_FLOAT16, "NULL"),
    ],
)
def test_capi_rotary_validation(kwargs, dtype, message):
    p = _rotary_params(**kwargs)
    rc = capi.lib().dk_rotary_embedding(ctypes.byref(p), dtype, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert message in capi.last_error()


def test_capi_rotary_and_cache_write_no_tokens_are_no_ops():
    L = capi.lib()
    assert L.dk_rotary_embedding(ctypes.byref(_rotary_params(num_tokens=0)), capi.DK_BFLOAT16, None) == 0
    assert L.dk_rotary_embedding(None, capi.DK_BFLOAT16, None) == capi.HIP_ERROR_INVALID_VALUE
    c = capi.CacheWriteParams()
    c.num_tokens, c.num_kv_heads, c.head_size, c.block_size, c.num_blocks = 0, 2, 128, 16, 4
    assert L.dk_reshape_and_cache(ctypes.byref(c), capi.DK_FLOAT16, None) == 0
    assert capi.last_error() == ""


@pytest.mark.parametrize(
    "field,value,dtype,message",
    [
        (None, None, 4, "float16 or bfloat16"),
        ("block_size", 0, capi.DK_FLOAT16, "positive"),
        ("num_kv_heads", 0, capi.DK_FLOAT16, "positive"),
        ("value", None, capi.DK_BFLOAT16, "NULL"),
        ("slot_mapping", None, capi.DK_BFLOAT16, "NULL"),
    ],
)
def test_capi_cache_write_validation(field, value, dtype, message):
    c = capi.CacheWriteParams()
    c.key = c.value = c.key_cache = c.value_cache = c.slot_mapping = 0x10000
    c.num_tokens, c.num_kv_heads, c.head_size, c.block_size, c.num_blocks = 2, 2, 128, 16, 4
    if field is not None:
        setattr(c, field, value)
    rc = capi.lib().dk_reshape_and_cache(ctypes.byref(c), dtype, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert message in capi.last_error()


def _fused_pair(num_tokens=2):
    r = _rotary_params(num_tokens=num_tokens)
    c = capi.CacheWriteParams()
    c.key, c.value, c.key_cache, c.value_cache, c.slot_mapping = r.key, 0x20000, 0x30000, 0x40000, 0x50000
    c.k_stride_token, c.k_stride_head = r.k_stride_token, r.k_stride_head
    c.num_tokens, c.num_kv_heads, c.head_size, c.block_size, c.num_blocks = num_tokens, r.num_kv_heads, r.head_size, 16, 4
    return r, c


def test_capi_fused_rotary_and_cache_validation():
    L = capi.lib()
    r, c = _fused_pair(num_tokens=0)
    assert L.dk_rotary_embedding_and_cache(ctypes.byref(r), ctypes.byref(c), capi.DK_BFLOAT16, None) == 0
    for mutate, message in (
        (lambda r, c: setattr(c, "num_tokens", 3), "token counts"),
        (lambda r, c: setattr(c, "key", 0x60000), "same tensor"),
        (lambda r, c: setattr(c, "k_stride_token", r.k_stride_token + 8), "same tensor"),
        (lambda r, c: setattr(c, "num_kv_heads", r.num_kv_heads + 1), "head counts"),
        (lambda r, c: setattr(r, "rot_dim", 3), "rot_dim"),
        (lambda r, c: setattr(c, "block_size", 0), "positive"),
    ):
        r, c = _fused_pair()
        mutate(r, c)
        rc = L.dk_rotary_embedding_and_cache(ctypes.byref(r), ctypes.byref(c), capi.DK_BFLOAT16, None)
        assert rc == capi.HIP_ERROR_INVALID_VALUE, message
        assert message in capi.last_error()
    assert L.dk_rotary_embedding_and_cache(None, None, capi.DK_FLOAT16, None) == capi.HIP_ERROR_INVALID_VALUE


def test_capi_fused_rotary_and_cache_fp8_validation():
    L = capi.lib()
    r, c = _fused_pair(num_tokens=0)
    assert L.dk_rotary_embedding_and_cache_fp8(ctypes.byref(r), ctypes.byref(c), capi.DK_BFLOAT16, 0.5, 2.0, None) == 0
    for ks, vs, message in ((0.0, 1.0, "positive and finite"), (1.0, float("inf"), "positive and finite")):
        rc = L.dk_rotary_embedding_and_cache_fp8(ctypes.byref(r), ctypes.byref(c), capi.DK_BFLOAT16, ks, vs, None)
        assert rc == capi.HIP_ERROR_INVALID_VALUE and message in capi.last_error()
    r, c = _fused_pair()
    c.key = 0x60000
    rc = L.dk_rotary_embedding_and_cache_fp8(ctypes.byref(r), ctypes.byref(c), capi.DK_BFLOAT16, 1.0, 1.0, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE and "same tensor" in capi.last_error()
    assert "rotary_embedding_and_cache_fp8" in capi.last_error()


@pytest.mark.parametrize("ks,vs", [(0.0, 1.0), (1.0, -2.0), (float("inf"), 1.0), (1.0, float("nan"))])
def test_capi_fp8_cache_write_rejects_bad_scales(ks, vs):
    c = capi.CacheWriteParams()
    c.key = c.value = c.key_cache = c.value_cache = c.slot_mapping = 0x10000
    c.num_tokens, c.num_kv_heads, c.head_size, c.block_size, c.num_blocks = 2, 2, 128, 16, 4
    rc = capi.lib().dk_reshape_and_cache_fp8(ctypes.byref(c), capi.DK_BFLOAT16, ks, vs, None)
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert "positive and finite" in capi.last_error()
    c.num_tokens = 0
    assert capi.lib().dk_reshape_and_cache_fp8(ctypes.byref(c), capi.DK_BFLOAT16, 1.0, 1.0, None) == 0


def test_cache_write_scales_need_an_fp8_cache():
    kc = torch.zeros(1, 4, 1, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="fp8"):
        ops.reshape_and_cache(torch.zeros(2, 1, 8, dtype=torch.bfloat16), torch.zeros(2, 1, 8, dtype=torch.bfloat16), kc,
                              kc.clone(), torch.zeros(2, dtype=torch.long), k_scale=0.5)
    with pytest.raises(ValueError, match="fp8"):
        ops.rotary_embedding_and_cache(torch.zeros(2, dtype=torch.long), torch.zeros(2, 8, dtype=torch.bfloat16),
                                       torch.zeros(2, 8, dtype=torch.bfloat16), torch.zeros(2, 8, dtype=torch.bfloat16),
                                       8, torch.zeros(4, 8), True, kc, kc.clone(), torch.zeros(2, dtype=torch.long),
                                       v_scale=2.0)


def test_capi_fill_helpers_read_tensor_layouts():
    pos = torch.arange(5)
    q = torch.zeros(5, 3 * 64, dtype=torch.bfloat16)
    k = torch.zeros(5, 2, 8, 64, dtype=torch.bfloat16)[:, :, 3]  # strided [T, H, D]
    cache = torch.zeros(100, 32)
    p = capi.rotary_params(pos, q, k, 64, cache, False)
    assert (p.q_stride_token, p.q_stride_head, p.num_q_heads) == (192, 64, 3)
    assert (p.k_stride_token, p.k_stride_head, p.num_kv_heads) == (1024, 512, 2)
    assert (p.rot_dim, p.max_position, p.cache_stride, p.is_neox, p.cache_dtype) == (32, 100, 32, 0, capi.DK_FLOAT32)
    kv = torch.zeros(6, 2, 16, 2 * 64, dtype=torch.float16)
    kc, vc = kv.transpose(1, 2).split(64, dim=-1)
    key = torch.zeros(4, 2 * 64, dtype=torch.float16)
    c = capi.cache_write_params(key, key.view(4, 2, 64), kc, vc, torch.arange(4))
    assert (c.kc_stride_block, c.kc_stride_token, c.kc_stride_head) == (2 * 16 * 128, 128, 16 * 128)
    assert c.value_cache - c.key_cache == 64 * 2
    assert (c.k_stride_token, c.k_stride_head, c.v_stride_token, c.v_stride_head) == (128, 64, 128, 64)
    assert (c.num_blocks, c.block_size, c.num_kv_heads, c.head_size, c.num_tokens) == (6, 16, 2, 64, 4)


# ---------------------------------------------------------------------------
# Python wrappers (host logic only)
# ---------------------------------------------------------------------------
def test_constants_and_partitions():
    assert dk.PARTITION_SIZE == 512 and dk.MAX_GQA_GROUP == 16 and dk.SUPPORTED_HEAD_DIMS == (64, 96, 128, 192, 256)
    assert [dk.num_partitions(n) for n in (0, 1, 512, 513, 131072)] == [1, 1, 1, 2, 256]


def test_alloc_workspace_shapes():
    empty = dk.alloc_workspace(4, 32, 128, 512, "cpu")
    assert all(t.numel() == 0 and t.dtype == torch.float32 for t in empty)
    tmp, ml, es = dk.alloc_workspace(4, 32, 128, 513, "cpu")
    assert tmp.shape == (4, 32, 2, 128) and ml.shape == (4, 32, 2) and es.shape == (4, 32, 2)
    assert tmp.is_contiguous() and ml.is_contiguous() and es.dtype == torch.float32


def test_ops_are_registered_with_reference_schemas():
    assert ops._AVAILABLE, "the torch binding must import on the CPU"
    schemas = {
        "paged_attention_decode": "paged_attention_decode(Tensor(a0!) out, Tensor q, Tensor k_cache, Tensor v_cache, "
        "Tensor block_tables, Tensor seq_lens, float scale, int max_seq_len, Tensor(a1!) tmp_out, "
        "Tensor(a2!) max_logits, Tensor(a3!) exp_sums) -> ()",
        "gemm_tn": "gemm_tn(Tensor(a0!) c, Tensor a, Tensor b, Tensor? bias) -> ()",
        "rms_norm": "rms_norm(Tensor(a0!) out, Tensor input, Tensor weight, float eps) -> ()",
        "fused_add_rms_norm": "fused_add_rms_norm(Tensor(a0!) input, Tensor(a1!) residual, Tensor weight, float eps) -> ()",
        "silu_and_mul": "silu_and_mul(Tensor(a0!) out, Tensor input) -> ()",
        "paged_attention_decode_fp8": "paged_attention_decode_fp8(Tensor(a0!) out, Tensor q, Tensor k_cache, "
        "Tensor v_cache, Tensor block_tables, Tensor seq_lens, float scale, int max_seq_len, Tensor(a1!) tmp_out, "
        "Tensor(a2!) max_logits, Tensor(a3!) exp_sums, float k_scale, float v_scale) -> ()",
        "rotary_embedding": "rotary_embedding(Tensor positions, Tensor(a0!) query, Tensor(a1!)? key, int head_size, "
        "Tensor cos_sin_cache, bool is_neox) -> ()",
        "reshape_and_cache": "reshape_and_cache(Tensor key, Tensor value, Tensor(a0!) key_cache, "
        "Tensor(a1!) value_cache, Tensor slot_mapping) -> ()",
        "reshape_and_cache_fp8": "reshape_and_cache_fp8(Tensor key, Tensor value, Tensor(a0!) key_cache, "
        "Tensor(a1!) value_cache, Tensor slot_mapping, float k_scale, float v_scale) -> ()",
        "rotary_embedding_and_cache": "rotary_embedding_and_cache(Tensor positions, Tensor(a0!) query, "
        "Tensor(a1!) key, Tensor value, int head_size, Tensor cos_sin_cache, bool is_neox, Tensor(a2!) key_cache, "
        "Tensor(a3!) value_cache, Tensor slot_mapping) -> ()",
        "rotary_embedding_and_cache_fp8": "rotary_embedding_and_cache_fp8(Tensor positions, Tensor(a0!) query, "
        "Tensor(a1!) key, Tensor value, int head_size, Tensor cos_sin_cache, bool is_neox, Tensor(a2!) key_cache, "
        "Tensor(a3!) value_cache, Tensor slot_mapping, float k_scale, float v_scale) -> ()",
    }
    for name, schema in schemas.items():
        got = str(getattr(torch.ops.decode_kernels, name).default._schema).replace("decode_kernels::", "")
        # torch prints alias sets as ($N! -> ); normalise both spellings.
        import re

        norm = lambda s: re.sub(r"\(\$?a?(\d+)! -> \)|\(a(\d+)!\)", "(!)", s)  # noqa: E731
        assert norm(got) == norm(schema), got


def test_ops_reject_cpu_tensors():
    """The ops exist only for GPU tensors, as in the reference (CUDA dispatch key)."""
    x = torch.randn(2, 64, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        torch.ops.decode_kernels.rms_norm(torch.empty_like(x), x, torch.ones(64, dtype=torch.float16), 1e-6)


def test_wrappers_fail_loudly_without_extension(monkeypatch):
    monkeypatch.setattr(ops, "_AVAILABLE", False)
    monkeypatch.setattr(ops, "_IMPORT_ERROR", ImportError("simulated"))
    assert not ops.is_available()
    kv = make_paged_kv([4], 1, 64)
    with pytest.raises(RuntimeError, match="not built"):
        ops.paged_attention_decode(torch.zeros(1, 1, 64, dtype=torch.float16), kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    for call in (
        lambda: ops.gemm(torch.zeros(2, 8), torch.zeros(4, 8)),
        lambda: ops.rms_norm(torch.zeros(2, 8), torch.ones(8)),
        lambda: ops.fused_add_rms_norm(torch.zeros(2, 8), torch.zeros(2, 8), torch.ones(8)),
        lambda: ops.silu_and_mul(torch.zeros(2, 8)),
        lambda: ops.rotary_embedding(torch.zeros(2, dtype=torch.long), torch.zeros(2, 8), None, 8, torch.zeros(4, 8)),
        lambda: ops.reshape_and_cache(torch.zeros(2, 1, 8), torch.zeros(2, 1, 8), torch.zeros(1, 4, 1, 8),
                                      torch.zeros(1, 4, 1, 8), torch.zeros(2, dtype=torch.long)),
        lambda: ops.rotary_embedding_and_cache(torch.zeros(2, dtype=torch.long), torch.zeros(2, 8), torch.zeros(2, 8),
                                               torch.zeros(2, 8), 8, torch.zeros(4, 8), True, torch.zeros(1, 4, 1, 8),
                                               torch.zeros(1, 4, 1, 8), torch.zeros(2, dtype=torch.long)),
    ):
        with pytest.raises(RuntimeError, match="not built"):
            call()
