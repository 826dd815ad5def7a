"""decodekernels_amd: the LLM decode hot path as hand-written HIP kernels for MI355X (gfx950).

    import decodekernels_amd as dk
    out = dk.paged_attention_decode(q, k_cache, v_cache, block_tables, seq_lens)

Same public API as DecodeKernels' ``decode_kernels`` package
(``decode_kernels/__init__.py:7-27``); the ops are registered under the same
``torch.ops.decode_kernels.*`` names. ``rotary_embedding`` and
``reshape_and_cache`` add the two steps around attention that the reference
leaves to vLLM (vLLM's signatures); ``rotary_embedding_and_cache`` runs both
in one launch. ``gemm_add_rms_norm`` and ``gemm_rotary_embedding_and_cache``
fuse a decode GEMM with the op that consumes its output.
"""

from .ops import (
    MAX_GQA_GROUP,
    PARTITION_SIZE,
    SUPPORTED_FP8_HEAD_DIMS,
    SUPPORTED_HEAD_DIMS,
    alloc_workspace,
    fused_add_rms_norm,
    gemm,
    gemm_add_rms_norm,
    gemm_rotary_embedding_and_cache,
    is_available,
    num_partitions,
    paged_attention_decode,
    reshape_and_cache,
    rms_norm,
    rotary_embedding,
    rotary_embedding_and_cache,
    silu_and_mul,
)

__all__ = [
    "MAX_GQA_GROUP",
    "PARTITION_SIZE",
    "SUPPORTED_FP8_HEAD_DIMS",
    "SUPPORTED_HEAD_DIMS",
    "alloc_workspace",
    "fused_add_rms_norm",
    "gemm",
    "gemm_add_rms_norm",
    "gemm_rotary_embedding_and_cache",
    "is_available",
    "num_partitions",
    "paged_attention_decode",
    "reshape_and_cache",
    "rms_norm",
    "rotary_embedding",
    "rotary_embedding_and_cache",
    "silu_and_mul",
]
__version__ = "0.2.0"  # pyproject.toml's [project] version (checked by tests/test_packaging.py)
