"""Fake ``vllm.*`` modules for the vLLM-integration tests (vLLM is not installed).

They hold just the classes and attributes ``decodekernels_amd.vllm_patch``
patches and reads: the attention impls of the FlashAttention, ROCm and Triton
backends (their original ``forward`` records a call and returns), ``RMSNorm``,
``SiluAndMul``, ``vllm.envs`` and, optionally, ``vllm.platforms``.
"""

from __future__ import annotations

import sys
import types
from types import SimpleNamespace

import torch


def install(monkeypatch, fp8_dtype=None) -> SimpleNamespace:
    """Registers the fake modules in ``sys.modules`` (undone by ``monkeypatch``) and
    returns the classes plus the list their original methods append to."""
    calls: list = []

    def module(name, **attrs):
        m = types.ModuleType(name)
        for k, v in attrs.items():
            setattr(m, k, v)
        monkeypatch.setitem(sys.modules, name, m)
        return m

    def impl_class(name):
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                    output_block_scale=None):
            calls.append("vllm_attention")
            return output

        return type(name, (), {"forward": forward})

    flash, rocm, triton = impl_class("FlashAttentionImpl"), impl_class("RocmAttentionImpl"), impl_class(
        "TritonAttentionImpl")

    class RMSNorm:
        def forward_cuda(self, x, residual=None):
            calls.append("vllm_rms_norm")
            return x

    class SiluAndMul:
        def forward_cuda(self, x):
            calls.append("vllm_silu")
            return x

    for name in ("vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends", "vllm.model_executor",
                 "vllm.model_executor.layers"):
        module(name)
    module("vllm.v1.attention.backends.flash_attn", FlashAttentionImpl=flash)
    module("vllm.v1.attention.backends.rocm_attn", RocmAttentionImpl=rocm)
    module("vllm.v1.attention.backends.triton_attn", TritonAttentionImpl=triton)
    module("vllm.envs", VLLM_BATCH_INVARIANT=False)
    module("vllm.model_executor.layers.layernorm", RMSNorm=RMSNorm)
    module("vllm.model_executor.layers.activation", SiluAndMul=SiluAndMul)
    if fp8_dtype is not None:
        module("vllm.platforms", current_platform=SimpleNamespace(fp8_dtype=lambda: fp8_dtype))
    # Patching replaces class attributes: restore them after the test.
    for cls in (flash, rocm, triton, RMSNorm, SiluAndMul):
        for attr in ("forward", "forward_cuda"):
            if attr in vars(cls):
                monkeypatch.setattr(cls, attr, vars(cls)[attr])
    return SimpleNamespace(calls=calls, FlashAttentionImpl=flash, RocmAttentionImpl=rocm, TritonAttentionImpl=triton,
                           RMSNorm=RMSNorm, SiluAndMul=SiluAndMul)


def impl_attrs(head_size, num_heads, num_kv_heads, **over) -> dict:
    """Attributes of a decoder attention impl that the patch's eligibility rules read."""
    base = dict(attn_type="decoder", dcp_world_size=1, kv_cache_dtype="auto", alibi_slopes=None, logits_soft_cap=None,
                sliding_window=None, sinks=None, head_size=head_size, num_heads=num_heads, num_kv_heads=num_kv_heads,
                scale=head_size**-0.5, do_kv_cache_update=lambda *a, **k: None)
    base.update(over)
    return base


def make_impl(cls, **attrs):
    impl = cls()
    for k, v in attrs.items():
        setattr(impl, k, v)
    return impl


__all__ = ["impl_attrs", "install", "make_impl", "torch"]
