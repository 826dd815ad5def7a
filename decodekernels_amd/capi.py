"""ctypes handle on the C ABI (``include/decodekernels_amd.h``) of
``libdecodekernels_amd.so``.

For callers that hold raw device pointers rather than torch tensors (other
runtimes, FFI bindings), and for tests that exercise the boundary without the
torch binding. ``torch`` is imported first on purpose: the library then binds
to the HIP runtime torch already loaded instead of a second copy.
"""

from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before ours; see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libdecodekernels_amd.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "decodekernels_amd.h"

DK_FLOAT16 = 0
DK_BFLOAT16 = 1
DK_FLOAT32 = 2
HIP_ERROR_INVALID_VALUE = 1


class PagedAttnParams(ctypes.Structure):
    """Mirror of ``dk_paged_attn_params``."""

    _fields_ = [
        ("out", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("tmp_out", ctypes.c_void_p),
        ("max_logits", ctypes.c_void_p),
        ("exp_sums", ctypes.c_void_p),
        ("q_stride_seq", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("out_stride_seq", ctypes.c_int64),
        ("out_stride_head", ctypes.c_int64),
        ("k_stride_block", ctypes.c_int64),
        ("k_stride_token", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("v_stride_block", ctypes.c_int64),
        ("v_stride_token", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("bt_stride", ctypes.c_int64),
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_partitions", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


class RotaryParams(ctypes.Structure):
    """Mirror of ``dk_rotary_params``."""

    _fields_ = [
        ("positions", ctypes.c_void_p),
        ("query", ctypes.c_void_p),
        ("key", ctypes.c_void_p),
        ("cos_sin_cache", ctypes.c_void_p),
        ("q_stride_token", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("k_stride_token", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("cache_stride", ctypes.c_int64),
        ("num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("rot_dim", ctypes.c_int32),
        ("max_position", ctypes.c_int32),
        ("is_neox", ctypes.c_int32),
        ("cache_dtype", ctypes.c_int32),
    ]


class CacheWriteParams(ctypes.Structure):
    """Mirror of ``dk_cache_write_params``."""

    _fields_ = [
        ("key", ctypes.c_void_p),
        ("value", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p),
        ("value_cache", ctypes.c_void_p),
        ("slot_mapping", ctypes.c_void_p),
        ("k_stride_token", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("v_stride_token", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("kc_stride_block", ctypes.c_int64),
        ("kc_stride_token", ctypes.c_int64),
        ("kc_stride_head", ctypes.c_int64),
        ("vc_stride_block", ctypes.c_int64),
        ("vc_stride_token", ctypes.c_int64),
        ("vc_stride_head", ctypes.c_int64),
        ("num_tokens", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
    ]


_LIB: ctypes.CDLL | None = None

_SIGNATURES = {
    "dk_paged_attention_decode": (
        ctypes.c_int,
        [ctypes.POINTER(PagedAttnParams), ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p],
    ),
    "dk_paged_attention_decode_fp8": (
        ctypes.c_int,
        [ctypes.POINTER(PagedAttnParams), ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        + [ctypes.c_void_p],
    ),
    "dk_paged_attention_decode_noalloc": (
        ctypes.c_int,
        [ctypes.POINTER(PagedAttnParams), ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p],
    ),
    "dk_gemm_tn": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        + [ctypes.c_int] * 6
        + [ctypes.c_void_p],
    ),
    "dk_gemm_tn_workspace_bytes": (ctypes.c_int64, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "dk_gemm_tn_plan": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int)],
    ),
    "dk_gemm_tn_ws": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        + [ctypes.c_int] * 6
        + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
    "dk_rms_norm": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        + [ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p],
    ),
    "dk_fused_add_rms_norm": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        + [ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p],
    ),
    "dk_silu_and_mul": (
        ctypes.c_int,
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
        + [ctypes.c_void_p],
    ),
    "dk_rotary_embedding": (
        ctypes.c_int,
        [ctypes.POINTER(RotaryParams), ctypes.c_int, ctypes.c_void_p],
    ),
    "dk_reshape_and_cache": (
        ctypes.c_int,
        [ctypes.POINTER(CacheWriteParams), ctypes.c_int, ctypes.c_void_p],
    ),
    "dk_reshape_and_cache_fp8": (
        ctypes.c_int,
        [ctypes.POINTER(CacheWriteParams), ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_void_p],
    ),
    "dk_rotary_embedding_and_cache": (
        ctypes.c_int,
        [ctypes.POINTER(RotaryParams), ctypes.POINTER(CacheWriteParams), ctypes.c_int, ctypes.c_void_p],
    ),
    "dk_rotary_embedding_and_cache_fp8": (
        ctypes.c_int,
        [ctypes.POINTER(RotaryParams), ctypes.POINTER(CacheWriteParams), ctypes.c_int, ctypes.c_float, ctypes.c_float]
        + [ctypes.c_void_p],
    ),
    "dk_gemm_tn_add_rms_norm": (
        ctypes.c_int,
        [ctypes.c_int] + [ctypes.c_void_p] * 6 + [ctypes.c_float] + [ctypes.c_int] * 7
        + [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
    "dk_gemm_tn_rotary_embedding_and_cache": (
        ctypes.c_int,
        [ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int] * 6
        + [ctypes.POINTER(RotaryParams), ctypes.POINTER(CacheWriteParams), ctypes.c_void_p, ctypes.c_int64,
           ctypes.c_void_p],
    ),
    "dk_gemm_tn_rotary_embedding_and_cache_fp8": (
        ctypes.c_int,
        [ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int] * 6
        + [ctypes.POINTER(RotaryParams), ctypes.POINTER(CacheWriteParams), ctypes.c_float, ctypes.c_float,
           ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p],
    ),
    "dk_last_error": (ctypes.c_char_p, []),
    "dk_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "dk_version": (ctypes.c_char_p, []),
}


def lib() -> ctypes.CDLL:
    """Loads the C-ABI library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m decodekernels_amd._build`")
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def declared_functions() -> list[str]:
    """Names of every function the C header declares."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(dk_\w+)\s*\(", text, flags=re.M)))


def gemm_plan(M: int, N: int, K: int, with_workspace: bool = True) -> tuple[int, int, int, int]:
    """gemm_tn's launch plan for this shape; host arithmetic only. Skinny
    kernel (M <= 64): (waves along N, waves along K, K splits, columns per
    split); LDS-DMA kernel (M > 64, and the 64-row tiles of some M <= 64
    plans): (tile rows, tile columns, K splits, columns per split)."""
    out = (ctypes.c_int * 4)()
    rc = lib().dk_gemm_tn_plan(M, N, K, int(with_workspace), out)
    if rc != 0:
        raise ValueError(last_error())
    return tuple(out)


def last_error() -> str:
    return lib().dk_last_error().decode()


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DK_FLOAT16
    if dtype == torch.bfloat16:
        return DK_BFLOAT16
    raise ValueError(f"expected float16 or bfloat16, got {dtype}")


def attn_params(out, q, k_cache, v_cache, block_tables, seq_lens, scale, workspace=None) -> PagedAttnParams:
    """Fills ``dk_paged_attn_params`` from tensors (strides in elements)."""
    p = PagedAttnParams()
    p.out, p.q = out.data_ptr(), q.data_ptr()
    p.k_cache, p.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    p.block_tables, p.seq_lens = block_tables.data_ptr(), seq_lens.data_ptr()
    if workspace is not None and workspace[0].numel() > 0:
        p.tmp_out, p.max_logits, p.exp_sums = (t.data_ptr() for t in workspace)
        p.max_partitions = workspace[0].shape[2]
    else:
        p.max_partitions = 1
    p.q_stride_seq, p.q_stride_head = q.stride(0), q.stride(1)
    p.out_stride_seq, p.out_stride_head = out.stride(0), out.stride(1)
    p.k_stride_block, p.k_stride_token, p.k_stride_head = k_cache.stride()[:3]
    p.v_stride_block, p.v_stride_token, p.v_stride_head = v_cache.stride()[:3]
    p.bt_stride = block_tables.stride(0)
    p.num_seqs, p.num_q_heads, _ = q.shape
    p.num_kv_heads = k_cache.shape[2]
    p.block_size = k_cache.shape[1]
    p.scale = scale
    return p


def _token_head_strides(t, head_size):
    if t.dim() == 2:
        return t.stride(0), head_size
    return t.stride(0), t.stride(1)


def _heads(t, head_size):
    return t.shape[1] // head_size if t.dim() == 2 else t.shape[1]


def rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox) -> RotaryParams:
    """Fills ``dk_rotary_params`` from tensors; ``query`` / ``key`` are
    [tokens, heads * head_size] or [tokens, heads, head_size]."""
    p = RotaryParams()
    p.positions, p.query = positions.data_ptr(), query.data_ptr()
    p.q_stride_token, p.q_stride_head = _token_head_strides(query, head_size)
    p.num_q_heads = _heads(query, head_size)
    if key is not None:
        p.key = key.data_ptr()
        p.k_stride_token, p.k_stride_head = _token_head_strides(key, head_size)
        p.num_kv_heads = _heads(key, head_size)
    p.cos_sin_cache = cos_sin_cache.data_ptr()
    p.cache_stride = cos_sin_cache.stride(0)
    p.num_tokens = positions.numel()
    p.head_size = head_size
    p.max_position, p.rot_dim = cos_sin_cache.shape
    p.is_neox = int(bool(is_neox))
    p.cache_dtype = DK_FLOAT32 if cos_sin_cache.dtype == torch.float32 else dtype_code(cos_sin_cache.dtype)
    return p


def cache_write_params(key, value, key_cache, value_cache, slot_mapping) -> CacheWriteParams:
    """Fills ``dk_cache_write_params`` from tensors; the caches are
    [blocks, block_size, kv_heads, head_size] views."""
    p = CacheWriteParams()
    d = key_cache.shape[3]
    p.key, p.value = key.data_ptr(), value.data_ptr()
    p.key_cache, p.value_cache = key_cache.data_ptr(), value_cache.data_ptr()
    p.slot_mapping = slot_mapping.data_ptr()
    p.k_stride_token, p.k_stride_head = _token_head_strides(key, d)
    p.v_stride_token, p.v_stride_head = _token_head_strides(value, d)
    p.kc_stride_block, p.kc_stride_token, p.kc_stride_head = key_cache.stride()[:3]
    p.vc_stride_block, p.vc_stride_token, p.vc_stride_head = value_cache.stride()[:3]
    p.num_tokens = slot_mapping.numel()
    p.num_blocks, p.block_size, p.num_kv_heads, p.head_size = key_cache.shape
    return p
