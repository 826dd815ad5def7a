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
        "dk_gemm_tn",
        "dk_rms_norm",
        "dk_fused_add_rms_norm",
        "dk_silu_and_mul",
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
        (dict(num_q_heads=32, num_kv_heads=2), 128, 10, capi.DK_BFLOAT16, "GQA group"),
        (dict(num_q_heads=6, num_kv_heads=4), 128, 10, capi.DK_BFLOAT16, "multiple of num_kv_heads"),
        (dict(), 96, 10, capi.DK_FLOAT16, "head_dim"),
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
    assert capi.lib().dk_error_string(1)


# ---------------------------------------------------------------------------
# Python wrappers (host logic only)
# ---------------------------------------------------------------------------
def test_constants_and_partitions():
    assert dk.PARTITION_SIZE == 512 and dk.MAX_GQA_GROUP == 8 and dk.SUPPORTED_HEAD_DIMS == (64, 128, 256)
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
    ):
        with pytest.raises(RuntimeError, match="not built"):
            call()
