"""CPU tests of the vLLM integration (``decodekernels_amd.vllm_patch`` / ``vllm_plugin``).

vLLM is not installed here, so the tests use stub objects for the attention
impl and metadata and fake ``vllm.*`` modules for the patch targets, and record
the calls that reach the decode ops (reference behaviour:
decode_kernels/vllm_patch.py:35-212, vllm_plugin.py:14-20).
"""

import sys
import types
from types import SimpleNamespace

import pytest
import torch

import fake_vllm as fake_vllm_modules
from decodekernels_amd import ops as dk_ops
from decodekernels_amd import vllm_patch, vllm_plugin
from decodekernels_amd.testing import make_paged_kv

D, HQ, HKV, BS = 64, 8, 2, 16


@pytest.fixture(autouse=True)
def fresh_state():
    vllm_patch.reset_stats()
    vllm_patch._APPLIED.clear()
    yield
    vllm_patch._APPLIED.clear()


def _impl(**over):
    base = dict(attn_type="decoder", dcp_world_size=1, kv_cache_dtype="auto", alibi_slopes=None, logits_soft_cap=None,
                sliding_window=None, sinks=None, head_size=D, num_heads=HQ, num_kv_heads=HKV, scale=D**-0.5,
                do_kv_cache_update=lambda *a, **k: None)
    base.update(over)
    return SimpleNamespace(**base)


def _inputs(n=3, dtype=torch.float16):
    kv = torch.randn(10, HKV, BS, 2 * D, dtype=dtype)
    query = torch.randn(n, HQ * D, dtype=dtype)
    output = torch.zeros(n, HQ * D, dtype=dtype)
    meta = SimpleNamespace(max_query_len=1, num_actual_tokens=n, seq_lens=torch.tensor([5] * n, dtype=torch.int32),
                           block_table=torch.zeros(n, 2, dtype=torch.int32), max_seq_len=5, causal=True)
    return query, kv, meta, output


def test_split_kv_cache_layouts():
    kv = make_paged_kv([20, 3], HKV, D, BS, torch.float32, layout="vllm")
    buf = kv.k_cache.as_strided((kv.k_cache.shape[0], HKV, BS, 2 * D), (HKV * BS * 2 * D, BS * 2 * D, 2 * D, 1))
    k, v = vllm_patch.split_kv_cache(buf, D)
    assert torch.equal(k, kv.k_cache) and torch.equal(v, kv.v_cache)
    assert k.stride() == kv.k_cache.stride()
    stacked = torch.randn(2, 7, BS, HKV, D)
    k2, v2 = vllm_patch.split_kv_cache(stacked, D, HKV)
    assert torch.equal(k2, stacked[0]) and torch.equal(v2, stacked[1])
    block_major = torch.randn(7, 2, BS, HKV, D)  # vLLM's Triton backend
    k3, v3 = vllm_patch.split_kv_cache(block_major, D, HKV)
    assert torch.equal(k3, block_major[:, 0]) and torch.equal(v3, block_major[:, 1])
    assert vllm_patch.split_kv_cache(torch.randn(7, BS * HKV * D), D) is None


def test_split_kv_cache_rejects_ambiguous_and_mismatched_layouts():
    # [2, 2, ...]: a stacked pair of 2 blocks or 2 blocks of a block-major pair
    assert vllm_patch.split_kv_cache(torch.randn(2, 2, BS, HKV, D), D, HKV) is None
    # a token-major interleaved buffer [blocks, block_size, kv_heads, 2*D] would
    # be read with block_size as the head axis
    assert vllm_patch.split_kv_cache(torch.randn(10, BS, HKV, 2 * D), D, HKV) is None
    assert vllm_patch.split_kv_cache(torch.randn(2, 7, BS, HKV + 1, D), D, HKV) is None
    q, _, meta, out = _inputs()
    token_major = torch.randn(10, BS, HKV, 2 * D, dtype=q.dtype)
    assert not vllm_patch._attention_eligible(_impl(), q, token_major, meta, out, None, None)


def test_attention_eligible_base_case():
    q, kv, meta, out = _inputs()
    assert vllm_patch._attention_eligible(_impl(), q, kv, meta, out, None, None)


@pytest.mark.parametrize(
    "impl_over,meta_over,other",
    [
        (dict(do_kv_cache_update=None), {}, None),  # the backend writes the cache inside forward
        (dict(attn_type="encoder"), {}, None),
        (dict(dcp_world_size=2), {}, None),
        (dict(kv_cache_dtype="fp8"), {}, None),
        (dict(alibi_slopes=torch.ones(HQ)), {}, None),
        (dict(logits_soft_cap=30.0), {}, None),
        (dict(sliding_window=(128, 0)), {}, None),
        (dict(sinks=torch.zeros(HQ)), {}, None),
        (dict(head_size=80), {}, None),
        (dict(num_heads=HKV * 32), {}, None),
        (dict(num_heads=7), {}, None),
        ({}, dict(max_query_len=4), None),
        ({}, dict(causal=False), None),
        ({}, dict(mm_prefix_query_range_tensor=torch.zeros(1)), None),
        ({}, dict(rswa_prefix_lens=torch.zeros(1)), None),
        ({}, dict(seq_lens=torch.tensor([5], dtype=torch.int32)), None),
        ({}, {}, "no_metadata"),
        ({}, {}, "output_scale"),
        ({}, {}, "fp32"),
        ({}, {}, "kv_dtype_mismatch"),
        ({}, {}, "noncontiguous_output"),
        ({}, {}, "unknown_layout"),
    ],
)
def test_attention_fallback_branches(impl_over, meta_over, other):
    q, kv, meta, out = _inputs()
    for k, v in meta_over.items():
        setattr(meta, k, v)
    scale = None
    if other == "no_metadata":
        meta = None
    elif other == "output_scale":
        scale = torch.ones(1)
    elif other == "fp32":
        q, kv = q.float(), kv.float()
    elif other == "kv_dtype_mismatch":
        kv = kv.bfloat16()
    elif other == "noncontiguous_output":
        out = torch.zeros(3, 2 * HQ * D, dtype=q.dtype)[:, ::2]
    elif other == "unknown_layout":
        kv = torch.randn(10, BS * HKV * D, dtype=q.dtype)
    assert not vllm_patch._attention_eligible(_impl(**impl_over), q, kv, meta, out, scale, None)


# ---------------------------------------------------------------------------
# fp8 (e4m3fn) KV caches
# ---------------------------------------------------------------------------
def _platform(monkeypatch, fp8_dtype):
    """A fake ``vllm.platforms`` whose current_platform stores fp8 as ``fp8_dtype``."""
    for name in ("vllm",):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    mod = types.ModuleType("vllm.platforms")
    mod.current_platform = SimpleNamespace(fp8_dtype=lambda: fp8_dtype)
    monkeypatch.setitem(sys.modules, "vllm.platforms", mod)


def _fp8_inputs(storage=torch.uint8):
    q, kv, meta, out = _inputs()
    kv8 = kv.to(torch.float8_e4m3fn)
    return q, (kv8.view(torch.uint8) if storage == torch.uint8 else kv8), meta, out


def test_fp8_cache_eligible_on_e4m3fn_platform(monkeypatch):
    _platform(monkeypatch, torch.float8_e4m3fn)
    q, kv, meta, out = _fp8_inputs()
    layer = SimpleNamespace(_k_scale_float=0.5, _v_scale_float=2.0)
    impl = _impl(kv_cache_dtype="fp8")
    assert vllm_patch.fp8_kv_scales(impl, kv, layer) == (0.5, 2.0)
    assert vllm_patch._attention_eligible(impl, q, kv, meta, out, None, None, layer)
    # an e4m3fn tensor needs no platform query
    _, kv8, _, _ = _fp8_inputs(torch.float8_e4m3fn)
    assert vllm_patch._attention_eligible(_impl(kv_cache_dtype="fp8_e4m3"), q, kv8, meta, out, None, None, layer)


def test_fp8_cache_head_dim_96_falls_back(monkeypatch):
    """head_dim 96 runs with a 16-bit cache but not an fp8 one (its rows load
    64 columns per lane group): the fp8 call must fall back, not raise."""
    _platform(monkeypatch, torch.float8_e4m3fn)
    d = 96
    kv = torch.randn(10, HKV, BS, 2 * d).to(torch.float8_e4m3fn)
    q = torch.randn(3, HQ * d, dtype=torch.float16)
    out = torch.zeros_like(q)
    meta = SimpleNamespace(max_query_len=1, num_actual_tokens=3, seq_lens=torch.tensor([5] * 3, dtype=torch.int32),
                           block_table=torch.zeros(3, 2, dtype=torch.int32), max_seq_len=5, causal=True)
    layer = SimpleNamespace(_k_scale_float=0.5, _v_scale_float=2.0)
    assert not vllm_patch._attention_eligible(_impl(kv_cache_dtype="fp8", head_size=d, scale=d**-0.5), q, kv, meta,
                                              out, None, None, layer)
    kv16 = torch.randn(10, HKV, BS, 2 * d, dtype=torch.float16)
    assert vllm_patch._attention_eligible(_impl(head_size=d, scale=d**-0.5), q, kv16, meta, out, None, None)


@pytest.mark.parametrize("case", ["fnuz_platform", "no_platform", "no_scales", "tensor_scales", "zero_scale", "e5m2",
                                  "fnuz_tensor", "auto_with_uint8"])
def test_fp8_cache_fallbacks(monkeypatch, case):
    _platform(monkeypatch, torch.float8_e4m3fn)
    q, kv, meta, out = _fp8_inputs()
    layer = SimpleNamespace(_k_scale_float=0.5, _v_scale_float=2.0)
    impl = _impl(kv_cache_dtype="fp8")
    if case == "fnuz_platform":
        _platform(monkeypatch, torch.float8_e4m3fnuz)
    elif case == "no_platform":
        monkeypatch.delitem(sys.modules, "vllm.platforms")
        monkeypatch.setitem(sys.modules, "vllm.platforms", None)  # import fails
    elif case == "no_scales":
        layer = SimpleNamespace()
    elif case == "tensor_scales":
        layer = SimpleNamespace(_k_scale_float=torch.tensor(0.5), _v_scale_float=torch.tensor(2.0))
    elif case == "zero_scale":
        layer = SimpleNamespace(_k_scale_float=0.0, _v_scale_float=2.0)
    elif case == "e5m2":
        impl = _impl(kv_cache_dtype="fp8_e5m2")
    elif case == "fnuz_tensor":
        kv = kv.view(torch.float8_e4m3fnuz)
    elif case == "auto_with_uint8":
        impl = _impl(kv_cache_dtype="auto")
    assert not vllm_patch._attention_eligible(impl, q, kv, meta, out, None, None, layer)


# ---------------------------------------------------------------------------
# Patch mechanics against fake vLLM modules
# ---------------------------------------------------------------------------
@pytest.fixture
def fake_vllm(monkeypatch):
    """Fake vLLM modules with the decode ops replaced by recorders (the GPU
    counterpart, tests/test_vllm_patch_gpu.py, keeps the real ops)."""
    fake = fake_vllm_modules.install(monkeypatch)
    calls = fake.calls
    monkeypatch.setattr(dk_ops, "is_available", lambda: True)
    monkeypatch.setattr(dk_ops, "paged_attention_decode", lambda *a, **k: calls.append(("dk_attention", a, k)))
    monkeypatch.setattr(dk_ops, "rms_norm", lambda *a: calls.append("dk_rms_norm"))
    monkeypatch.setattr(dk_ops, "fused_add_rms_norm", lambda *a: calls.append("dk_fused_add"))
    monkeypatch.setattr(dk_ops, "silu_and_mul", lambda *a: calls.append("dk_silu"))
    return fake


def test_attention_patch_routes_decode_batches(fake_vllm):
    vllm_patch.apply(["attention"])
    impl = fake_vllm.FlashAttentionImpl()
    for k, v in vars(_impl()).items():
        setattr(impl, k, v)
    q, kv, meta, out = _inputs()
    assert impl.forward(None, q, None, None, kv, meta, out) is out
    kind, args, kwargs = fake_vllm.calls[-1]
    assert kind == "dk_attention"
    assert args[0].shape == (3, HQ, D) and args[1].shape == (10, BS, HKV, D) and args[1].stride(-1) == 1
    assert kwargs["max_seq_len"] == 5 and kwargs["out"].data_ptr() == out.data_ptr()
    meta.max_query_len = 2  # prefill / mixed batch
    impl.forward(None, q, None, None, kv, meta, out)
    assert fake_vllm.calls[-1] == "vllm_attention"
    assert vllm_patch.stats()["attention_kernel_calls"] == 1
    assert vllm_patch.stats()["attention_fallback_calls"] == 1


def test_attention_patch_keeps_backends_that_write_the_cache_in_forward(fake_vllm):
    """Without a separate do_kv_cache_update step the backend's forward writes
    the new token's K/V itself, so it must run: every call falls back."""
    vllm_patch.apply(["attention"])
    impl = fake_vllm.FlashAttentionImpl()
    for k, v in vars(_impl()).items():
        if k != "do_kv_cache_update":
            setattr(impl, k, v)
    q, kv, meta, out = _inputs()
    assert impl.forward(None, q, None, None, kv, meta, out) is out
    assert fake_vllm.calls == ["vllm_attention"]
    assert vllm_patch.stats()["attention_kernel_calls"] == 0
    assert vllm_patch.stats()["attention_fallback_calls"] == 1


def test_attention_patch_routes_fp8_caches_with_scales(fake_vllm, monkeypatch):
    _platform(monkeypatch, torch.float8_e4m3fn)
    vllm_patch.apply(["attention"])
    impl = fake_vllm.FlashAttentionImpl()
    for k, v in vars(_impl(kv_cache_dtype="fp8")).items():
        setattr(impl, k, v)
    q, kv, meta, out = _fp8_inputs()
    layer = SimpleNamespace(_k_scale_float=0.25, _v_scale_float=4.0)
    assert impl.forward(layer, q, None, None, kv, meta, out) is out
    kind, args, kwargs = fake_vllm.calls[-1]
    assert kind == "dk_attention"
    assert args[1].dtype == torch.float8_e4m3fn and args[2].dtype == torch.float8_e4m3fn
    assert args[1].data_ptr() == kv.data_ptr() and args[1].shape == (10, BS, HKV, D)
    assert torch.equal(args[2][:, :, 0, :].view(torch.uint8), kv.transpose(1, 2)[:, :, 0, D:])
    assert kwargs["k_scale"] == 0.25 and kwargs["v_scale"] == 4.0
    impl.forward(SimpleNamespace(), q, None, None, kv, meta, out)  # no scales on the layer -> vLLM
    assert fake_vllm.calls[-1] == "vllm_attention"
    assert vllm_patch.stats()["attention_kernel_calls"] == 1
    assert vllm_patch.stats()["attention_fallback_calls"] == 1


def test_norm_and_silu_patches(fake_vllm):
    vllm_patch.apply(["rms_norm", "silu_and_mul"])
    norm = fake_vllm.RMSNorm()
    norm.weight = torch.nn.Parameter(torch.ones(D, dtype=torch.float16))
    norm.hidden_size, norm.variance_epsilon = D, 1e-6
    x = torch.randn(4, D, dtype=torch.float16)
    norm.forward_cuda(x)
    norm.forward_cuda(x, torch.randn(4, D, dtype=torch.float16))
    norm.forward_cuda(x.float())  # dtype mismatch -> vLLM
    act = fake_vllm.SiluAndMul()
    act.forward_cuda(torch.randn(4, 2 * D, dtype=torch.bfloat16))
    act.forward_cuda(torch.randn(4, 2 * D, dtype=torch.float32))
    assert fake_vllm.calls == ["dk_rms_norm", "dk_fused_add", "vllm_rms_norm", "dk_silu", "vllm_silu"]
    s = vllm_patch.stats()
    assert (s["rms_norm_kernel_calls"], s["rms_norm_fallback_calls"]) == (2, 1)
    assert (s["silu_and_mul_kernel_calls"], s["silu_and_mul_fallback_calls"]) == (1, 1)
    vllm_patch.reset_stats()
    assert all(v == 0 for v in vllm_patch.stats().values())


def test_apply_is_idempotent_and_validates(fake_vllm):
    vllm_patch.apply(["silu_and_mul"])
    first = fake_vllm.SiluAndMul.forward_cuda
    vllm_patch.apply(["silu_and_mul"])
    assert fake_vllm.SiluAndMul.forward_cuda is first
    with pytest.raises(ValueError, match="unknown op"):
        vllm_patch.apply(["gemm"])


def test_apply_without_extension_leaves_vllm_alone(fake_vllm, monkeypatch):
    monkeypatch.setattr(dk_ops, "is_available", lambda: False)
    original = fake_vllm.SiluAndMul.forward_cuda
    vllm_patch.apply()
    assert fake_vllm.SiluAndMul.forward_cuda is original and not vllm_patch._APPLIED


def test_plugin_env_gating(monkeypatch):
    seen = []
    monkeypatch.setattr(vllm_patch, "apply", lambda ops: seen.append(ops))
    monkeypatch.delenv("DECODE_KERNELS_VLLM", raising=False)
    vllm_plugin.register()
    assert seen == []
    monkeypatch.setenv("DECODE_KERNELS_VLLM", "1")
    monkeypatch.setenv("DECODE_KERNELS_OPS", " attention , silu_and_mul,")
    vllm_plugin.register()
    assert seen == [["attention", "silu_and_mul"]]
    monkeypatch.delenv("DECODE_KERNELS_OPS")
    vllm_plugin.register()
    assert seen[-1] == ["attention", "rms_norm", "silu_and_mul"]
