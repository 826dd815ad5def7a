"""Swap the decode kernels into vLLM.

Same API and rules as DecodeKernels' ``decode_kernels/vllm_patch.py``
(written against vLLM 0.32): three substitutions, each behind a strict
eligibility check that falls back to vLLM's own code for anything it does not
handle, with counters so a silent fallback cannot pass for a result.

* attention ``forward`` of vLLM's decode backends -- pure-decode batches (one
  query token per request) run ``paged_attention_decode`` on vLLM's KV cache
  in place. The reference patches ``FlashAttentionImpl``; on ROCm builds of
  vLLM the decode path may live in the ROCm or Triton backend instead, so every
  known backend class that exists is patched. The cache layout is read from
  the tensor: the interleaved ``[blocks, kv_heads, block_size, 2*head_dim]``
  buffer (viewed as strided K and V, as the reference does), a stacked
  ``[2, blocks, block_size, kv_heads, head_dim]`` pair or the Triton
  backend's block-major ``[blocks, 2, block_size, kv_heads, head_dim]``.
* ``RMSNorm.forward_cuda`` -- rms_norm / fused_add_rms_norm.
* ``SiluAndMul.forward_cuda`` -- silu_and_mul.

Prefill and mixed batches, sliding windows, ALiBi, soft-capping, attention
sinks, context parallelism, cross/encoder attention and graph capture all go to
vLLM's implementation (reference: decode_kernels/vllm_patch.py:60-99), and so
does every call on a backend whose impl has no ``do_kv_cache_update`` step: the
reference relies on vLLM writing the new token's K/V into the cache before
``forward`` runs (decode_kernels/vllm_patch.py:11-12), and a backend that writes
it inside ``forward`` must keep its own. Unlike
the reference, an fp8 KV cache (``kv_cache_dtype`` "fp8" / "fp8_e4m3", OCP
e4m3fn -- vLLM's fp8 on gfx950) with float scales on the layer runs
``paged_attention_decode_fp8``; other quantized caches (e4m3fnuz, e5m2, ...)
fall back.
"""

from __future__ import annotations

import importlib
import logging

import torch

from . import ops as dk_ops

logger = logging.getLogger("decodekernels_amd.vllm")

_STATS = {
    "attention_kernel_calls": 0,
    "attention_fallback_calls": 0,
    "rms_norm_kernel_calls": 0,
    "rms_norm_fallback_calls": 0,
    "silu_and_mul_kernel_calls": 0,
    "silu_and_mul_fallback_calls": 0,
}
_APPLIED: set[str] = set()
_HALF_TYPES = (torch.float16, torch.bfloat16)

# (module, class) of vLLM attention backends whose decode path can be swapped.
ATTENTION_BACKENDS = (
    ("vllm.v1.attention.backends.flash_attn", "FlashAttentionImpl"),
    ("vllm.v1.attention.backends.rocm_attn", "RocmAttentionImpl"),
    ("vllm.v1.attention.backends.triton_attn", "TritonAttentionImpl"),
)


def stats() -> dict[str, int]:
    """How often each patched op used the decode kernels vs fell back."""
    return dict(_STATS)


def reset_stats() -> None:
    for k in _STATS:
        _STATS[k] = 0


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def _decoder_attention_type():
    """vLLM's AttentionType.DECODER (its value is the string "decoder")."""
    try:
        from vllm.v1.attention.backend import AttentionType

        return AttentionType.DECODER
    except Exception:  # noqa: BLE001  (vLLM absent or moved: compare by value)
        return "decoder"


def split_kv_cache(kv_cache: torch.Tensor, head_size: int, num_kv_heads: int | None = None):
    """K and V views [blocks, block_size, kv_heads, head_dim] of vLLM's cache, or None
    for a layout the kernels do not read.

    * [blocks, kv_heads, block_size, 2*D]: the interleaved buffer, viewed as two
      strided NHD tensors (reference: vllm_patch.py:121-122);
    * [2, blocks, block_size, kv_heads, D]: a K/V-major stacked pair;
    * [blocks, 2, block_size, kv_heads, D]: a block-major pair (vLLM's Triton backend).

    The two 5-D pairs cannot be told apart when both leading dims are 2, so
    that shape falls back. With ``num_kv_heads`` the head axis must match it
    (a token-major buffer, say, would otherwise be read with its axes swapped)."""
    if kv_cache.dim() == 4 and kv_cache.shape[-1] == 2 * head_size:
        k, v = kv_cache.transpose(1, 2).split(head_size, dim=-1)
    elif kv_cache.dim() == 5 and kv_cache.shape[-1] == head_size and 2 in kv_cache.shape[:2]:
        if kv_cache.shape[0] == 2 and kv_cache.shape[1] == 2:
            return None
        k, v = (kv_cache[0], kv_cache[1]) if kv_cache.shape[0] == 2 else (kv_cache[:, 0], kv_cache[:, 1])
    else:
        return None
    if num_kv_heads is not None and k.shape[2] != num_kv_heads:
        return None
    return k, v


def _platform_fp8_is_e4m3fn() -> bool:
    """True when vLLM's fp8 storage format on this platform is OCP e4m3fn (gfx950; gfx942 uses e4m3fnuz)."""
    try:
        from vllm.platforms import current_platform

        return current_platform.fp8_dtype() == torch.float8_e4m3fn
    except Exception:  # noqa: BLE001  (vLLM absent or no such query: not known to be e4m3fn)
        return False


def fp8_kv_scales(impl, kv_cache: torch.Tensor, layer) -> tuple[float, float] | None:
    """(k_scale, v_scale) when vLLM's KV cache is fp8 e4m3fn -- stored as
    float8_e4m3fn, or as uint8 on a platform whose fp8 is e4m3fn -- and the
    layer carries its scales as floats (``_k_scale_float`` / ``_v_scale_float``,
    read without a device sync); None otherwise."""
    if str(getattr(impl, "kv_cache_dtype", "auto")) not in ("fp8", "fp8_e4m3"):
        return None
    if kv_cache.dtype != torch.float8_e4m3fn and not (kv_cache.dtype == torch.uint8 and _platform_fp8_is_e4m3fn()):
        return None
    k_scale = getattr(layer, "_k_scale_float", None)
    v_scale = getattr(layer, "_v_scale_float", None)
    if not all(isinstance(x, float) and 0.0 < x < float("inf") for x in (k_scale, v_scale)):
        return None
    return k_scale, v_scale


def _attention_eligible(impl, query, kv_cache, attn_metadata, output, output_scale, output_block_scale,
                        layer=None) -> bool:
    """The reference's eligibility rules (decode_kernels/vllm_patch.py:60-99), plus a cache-layout check
    and fp8 (e4m3fn) caches with float scales on ``layer``."""
    if attn_metadata is None or output_scale is not None or output_block_scale is not None:
        return False
    if query.is_cuda and torch.cuda.is_current_stream_capturing():
        # The single-pass / split-K choice depends on the host-side max_seq_len,
        # which a captured graph would freeze.
        return False
    # The new tokens' K/V must already be in the cache: vLLM writes them in a
    # separate do_kv_cache_update step before forward (what the reference
    # relies on). A backend without that step writes them inside its own
    # forward, which must then run.
    if not callable(getattr(impl, "do_kv_cache_update", None)):
        return False
    if getattr(impl, "attn_type", _decoder_attention_type()) != _decoder_attention_type():
        return False
    if getattr(attn_metadata, "max_query_len", None) != 1:
        return False
    if getattr(impl, "dcp_world_size", 1) > 1:
        return False
    if str(getattr(impl, "kv_cache_dtype", "auto")) in ("auto", "float16", "bfloat16"):
        if kv_cache.dtype != query.dtype:
            return False
    elif fp8_kv_scales(impl, kv_cache, layer) is None:
        return False
    if query.dtype not in _HALF_TYPES:
        return False
    if getattr(impl, "alibi_slopes", None) is not None or getattr(impl, "logits_soft_cap", None):
        return False
    if getattr(impl, "sliding_window", None) not in (None, (-1, -1)):
        return False
    if getattr(impl, "sinks", None) is not None:
        return False
    fp8 = str(getattr(impl, "kv_cache_dtype", "auto")) not in ("auto", "float16", "bfloat16")
    if impl.head_size not in (dk_ops.SUPPORTED_FP8_HEAD_DIMS if fp8 else dk_ops.SUPPORTED_HEAD_DIMS):
        return False
    if impl.num_heads % impl.num_kv_heads or impl.num_heads // impl.num_kv_heads > dk_ops.MAX_GQA_GROUP:
        return False
    if getattr(attn_metadata, "causal", True) is not True:
        return False
    if getattr(attn_metadata, "mm_prefix_query_range_tensor", None) is not None:
        return False
    if getattr(attn_metadata, "rswa_prefix_lens", None) is not None:
        return False
    n = attn_metadata.num_actual_tokens
    if attn_metadata.seq_lens.shape[0] < n or attn_metadata.block_table.shape[0] < n:
        return False
    if not output.is_contiguous():
        return False
    if split_kv_cache(kv_cache, impl.head_size, impl.num_kv_heads) is None:
        return False
    return True


def _make_attention_forward(original):
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                output_block_scale=None, *args, **kwargs):
        if output is not None and not args and not kwargs and _attention_eligible(
            self, query, kv_cache, attn_metadata, output, output_scale, output_block_scale, layer
        ):
            n = attn_metadata.num_actual_tokens
            key_cache, value_cache = split_kv_cache(kv_cache, self.head_size, self.num_kv_heads)
            scales = {}
            fp8 = fp8_kv_scales(self, kv_cache, layer)
            if fp8 is not None:  # uint8 storage read as e4m3fn, in place
                key_cache = key_cache.view(torch.float8_e4m3fn)
                value_cache = value_cache.view(torch.float8_e4m3fn)
                scales = {"k_scale": fp8[0], "v_scale": fp8[1]}
            q = query[:n].reshape(n, self.num_heads, self.head_size)
            out = output[:n].view(n, self.num_heads, self.head_size)
            dk_ops.paged_attention_decode(
                q,
                key_cache,
                value_cache,
                attn_metadata.block_table,
                attn_metadata.seq_lens,
                scale=self.scale,
                max_seq_len=attn_metadata.max_seq_len,
                out=out,
                **scales,
            )
            _STATS["attention_kernel_calls"] += 1
            return output
        _STATS["attention_fallback_calls"] += 1
        return original(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                        output_block_scale, *args, **kwargs)

    forward.__wrapped__ = original  # type: ignore[attr-defined]
    return forward


def _patch_attention() -> None:
    patched = []
    for module_name, class_name in ATTENTION_BACKENDS:
        try:
            cls = getattr(importlib.import_module(module_name), class_name)
        except Exception:  # noqa: BLE001  (backend not present in this vLLM build)
            continue
        cls.forward = _make_attention_forward(cls.forward)
        patched.append(class_name)
    if not patched:
        raise ImportError("no supported vLLM attention backend found to patch")
    logger.info("decodekernels_amd: attention patched in %s", patched)


# ---------------------------------------------------------------------------
# RMSNorm and SiluAndMul
# ---------------------------------------------------------------------------
def _patch_rms_norm() -> None:
    import vllm.envs as envs
    from vllm.model_executor.layers.layernorm import RMSNorm

    original = RMSNorm.forward_cuda

    def forward_cuda(self, x, residual=None):
        eligible = (
            not getattr(envs, "VLLM_BATCH_INVARIANT", False)
            and not torch.compiler.is_compiling()
            and getattr(self, "variance_size_override", None) is None
            and getattr(self, "has_weight", True)
            and x.dtype in _HALF_TYPES
            and self.weight.dtype == x.dtype
            and x.shape[-1] == self.hidden_size
            and x.stride(-1) == 1
            and (residual is None or (residual.dtype == x.dtype and residual.shape == x.shape))
        )
        if not eligible:
            _STATS["rms_norm_fallback_calls"] += 1
            return original(self, x, residual)
        _STATS["rms_norm_kernel_calls"] += 1
        if residual is None:
            return dk_ops.rms_norm(x, self.weight.data, self.variance_epsilon)
        return dk_ops.fused_add_rms_norm(x, residual, self.weight.data, self.variance_epsilon)

    forward_cuda.__wrapped__ = original  # type: ignore[attr-defined]
    RMSNorm.forward_cuda = forward_cuda


def _patch_silu_and_mul() -> None:
    from vllm.model_executor.layers.activation import SiluAndMul

    original = SiluAndMul.forward_cuda

    def forward_cuda(self, x):
        if x.dtype in _HALF_TYPES and not torch.compiler.is_compiling() and x.stride(-1) == 1:
            _STATS["silu_and_mul_kernel_calls"] += 1
            return dk_ops.silu_and_mul(x)
        _STATS["silu_and_mul_fallback_calls"] += 1
        return original(self, x)

    forward_cuda.__wrapped__ = original  # type: ignore[attr-defined]
    SiluAndMul.forward_cuda = forward_cuda


_PATCHERS = {
    "attention": _patch_attention,
    "rms_norm": _patch_rms_norm,
    "silu_and_mul": _patch_silu_and_mul,
}


def apply(ops: list[str] | None = None) -> None:
    """Install the patches (idempotent) (reference: decode_kernels/vllm_patch.py:200-212)."""
    if not dk_ops.is_available():
        logger.warning("decodekernels_amd: HIP extension unavailable; vLLM left unpatched")
        return
    for name in ops or list(_PATCHERS):
        if name not in _PATCHERS:
            raise ValueError(f"unknown op {name!r}; choose from {sorted(_PATCHERS)}")
        if name in _APPLIED:
            continue
        _PATCHERS[name]()
        _APPLIED.add(name)
    logger.info("decodekernels_amd: patched vLLM ops %s", sorted(_APPLIED))
