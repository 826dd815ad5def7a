"""GPU test of ``dk_paged_attention_decode_noalloc`` through the C ABI.

The allocation-free entry point runs the kernels of
``dk_paged_attention_decode`` with its split-K workspace in the library's
static device array instead of a caller buffer: its output must equal the
existing entry point's bit for bit (same kernels, same inputs) and meet the
parity bar against the oracle. Two calls in a row, the second with a smaller
input, so the second runs over what the first left in the array; plus a
single-pass call (no workspace use) and the size limit.
"""

import ctypes

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from decodekernels_amd.testing import make_paged_kv
from parity import assert_max_abs, attention_f32

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(lens, hkv, group, d, dtype, layout, seed):
    kv = make_paged_kv(lens, hkv, d, 16, dtype, "cuda", layout=layout, seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn(len(lens), hkv * group, d, generator=g, device="cuda", dtype=dtype)
    return kv, q


def _both(kv, q, dtype, max_len):
    """(output of dk_paged_attention_decode with a caller workspace,
    output of dk_paged_attention_decode_noalloc)."""
    n, hq, d = q.shape
    ws = dk.alloc_workspace(n, hq, d, max_len, "cuda")
    want = torch.empty_like(q)
    p = capi.attn_params(want, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, d**-0.5, ws)
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.dtype_code(dtype), d, max_len, _stream())
    assert rc == 0, capi.last_error()
    got = torch.full_like(q, float("nan"))
    p = capi.attn_params(got, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, d**-0.5, None)
    rc = capi.lib().dk_paged_attention_decode_noalloc(ctypes.byref(p), capi.dtype_code(dtype), d, max_len, _stream())
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    return want, got


@pytest.mark.parametrize("schedule", ["auto", "grid", "balanced", "partitions"])
def test_noalloc_matches_workspace_entry_point(schedule, monkeypatch):
    if schedule != "auto":
        monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    dtype = torch.bfloat16
    # First call: the Llama-3-8B batch shape (64 sequences, 8 KV heads).
    lens1 = torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    kv, q = _case(lens1, 8, 4, 128, dtype, "vllm", seed=1)
    want, got = _both(kv, q, dtype, max(lens1))
    assert torch.equal(got, want), "noalloc output differs from dk_paged_attention_decode"
    assert_max_abs(got[:4], attention_f32(q[:4], kv.k_cache, kv.v_cache, kv.block_tables[:4], kv.seq_lens[:4]), dtype,
                   "noalloc, call 1")
    # Second call, smaller: fewer sequences, other lengths and head count; the
    # array still holds the first call's rows.
    lens2 = [1, 700, 513, 0, 2100]
    kv2, q2 = _case(lens2, 2, 8, 64, torch.float16, "nhd", seed=2)
    want2, got2 = _both(kv2, q2, torch.float16, max(lens2))
    assert torch.equal(got2, want2), "noalloc output differs on the second, smaller call"
    assert_max_abs(got2, attention_f32(q2, kv2.k_cache, kv2.v_cache, kv2.block_tables, kv2.seq_lens), torch.float16,
                   "noalloc, call 2")
    assert (got2[3] == 0).all()


def test_noalloc_single_pass_and_size_limit():
    dtype = torch.float16
    kv, q = _case([5, 300, 512], 2, 4, 128, dtype, "hnd", seed=3)
    want, got = _both(kv, q, dtype, 512)
    assert torch.equal(got, want)
    # 2048 sequences x 32 query heads x 256 partitions x 130 x 4 bytes: far past 64 MiB.
    p = capi.attn_params(got, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, 128**-0.5, None)
    p.num_seqs, p.num_q_heads, p.num_kv_heads = 2048, 32, 8
    rc = capi.lib().dk_paged_attention_decode_noalloc(ctypes.byref(p), capi.dtype_code(dtype), 128, 131072, _stream())
    assert rc == capi.HIP_ERROR_INVALID_VALUE
    assert "scratch" in capi.last_error()
