"""GPU tests of the vLLM integration with the real HIP ops.

The CPU tests (tests/test_vllm_patch.py) replace the decode ops with
recorders; here the patched methods of fake vLLM classes (tests/fake_vllm.py)
run ``paged_attention_decode`` / ``rms_norm`` / ``fused_add_rms_norm`` /
``silu_and_mul`` on the GPU, on every cache layout the patch reads in place:

* FlashAttention's interleaved ``[blocks, kv_heads, block_size, 2*D]`` buffer
  (the reference's layout, decode_kernels/vllm_patch.py:102-141),
* a stacked ``[2, blocks, block_size, kv_heads, D]`` pair (ROCm backend),
* a block-major ``[blocks, 2, block_size, kv_heads, D]`` pair (Triton backend),
* an fp8 cache stored as uint8 on an e4m3fn platform, with float layer scales,

and compare vLLM's ``output`` buffer with the oracle on the K/V the layout
defines, at the bar of tests/parity.py; the norm and activation patches
against the oracle at 1 ulp (the fused residual bit-exact). The counters must
show that the kernels, not the fallbacks, ran.
"""

from types import SimpleNamespace

import pytest
import torch

import fake_vllm
from decodekernels_amd import vllm_patch
from parity import assert_max_abs, assert_ulp, attention_f32, fused_add_rms_norm_reference, rms_norm_reference
from oracle.reference import silu_and_mul_reference

pytestmark = pytest.mark.gpu

NB, BS = 160, 16


@pytest.fixture
def patched(monkeypatch):
    vllm_patch.reset_stats()
    vllm_patch._APPLIED.clear()
    fake = fake_vllm.install(monkeypatch, fp8_dtype=torch.float8_e4m3fn)
    vllm_patch.apply()
    yield fake
    vllm_patch._APPLIED.clear()


def _block_table(lens, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(NB, generator=g).to(torch.int32)
    width = max(-(-n // BS) for n in lens)
    bt = torch.zeros(len(lens), width, dtype=torch.int32)
    off = 0
    for s, n in enumerate(lens):
        nb = -(-n // BS)
        bt[s, :nb] = perm[off : off + nb]
        off += nb
    assert off <= NB
    return bt.cuda()


def _cache(layout, hkv, d, dtype, seed):
    """(the tensor vLLM hands to forward, K view, V view) in NHD shape."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    store = torch.float16 if dtype in (torch.uint8, torch.float8_e4m3fn) else dtype

    def randn(*shape):
        x = torch.randn(*shape, generator=g, device="cuda", dtype=store)
        return x.to(torch.float8_e4m3fn).view(dtype) if dtype in (torch.uint8, torch.float8_e4m3fn) else x

    if layout == "interleaved":
        buf = randn(NB, hkv, BS, 2 * d)
        k, v = buf.transpose(1, 2)[..., :d], buf.transpose(1, 2)[..., d:]
    elif layout == "stacked":
        buf = randn(2, NB, BS, hkv, d)
        k, v = buf[0], buf[1]
    else:  # block_major
        buf = randn(NB, 2, BS, hkv, d)
        k, v = buf[:, 0], buf[:, 1]
    return buf, k, v


CASES = [
    # (backend class, layout, dtype, cache dtype, hq, hkv, d, lens)
    ("FlashAttentionImpl", "interleaved", torch.bfloat16, None, 32, 8, 128, [700, 1, 513, 40]),
    ("FlashAttentionImpl", "interleaved", torch.float16, None, 8, 2, 64, [100, 300]),
    ("RocmAttentionImpl", "stacked", torch.bfloat16, None, 28, 4, 128, [1000, 17, 512]),
    ("TritonAttentionImpl", "block_major", torch.float16, None, 16, 2, 256, [64, 900]),
    ("FlashAttentionImpl", "interleaved", torch.bfloat16, torch.uint8, 32, 8, 128, [700, 1, 513, 40]),
    ("RocmAttentionImpl", "stacked", torch.float16, torch.uint8, 14, 2, 64, [1200, 5]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-{str(c[2])[6:]}-{'fp8' if c[3] else 'kv16'}")
def test_patched_attention_runs_the_kernel(patched, case):
    cls_name, layout, dtype, cache_dtype, hq, hkv, d, lens = case
    n = len(lens)
    padded = n + 2  # vLLM pads the batch; rows past num_actual_tokens are left alone
    buf, k, v = _cache(layout, hkv, d, cache_dtype or dtype, seed=hq + d)
    bt = _block_table(lens, seed=d)
    meta = SimpleNamespace(max_query_len=1, num_actual_tokens=n, max_seq_len=max(lens), causal=True,
                           seq_lens=torch.tensor(lens, dtype=torch.int32, device="cuda"), block_table=bt)
    g = torch.Generator(device="cuda").manual_seed(5)
    query = torch.randn(padded, hq * d, generator=g, device="cuda", dtype=dtype)
    output = torch.full((padded, hq * d), 7.0, device="cuda", dtype=dtype)
    extra = {}
    layer = SimpleNamespace()
    k_scale = v_scale = 1.0
    if cache_dtype is not None:
        extra["kv_cache_dtype"] = "fp8"
        k_scale, v_scale = 0.25, 1.5
        layer = SimpleNamespace(_k_scale_float=k_scale, _v_scale_float=v_scale)
    impl = fake_vllm.make_impl(getattr(patched, cls_name), **fake_vllm.impl_attrs(d, hq, hkv, **extra))
    ret = impl.forward(layer, query, None, None, buf, meta, output)
    torch.cuda.synchronize()
    assert ret is output
    assert vllm_patch.stats()["attention_kernel_calls"] == 1, vllm_patch.stats()
    assert vllm_patch.stats()["attention_fallback_calls"] == 0
    assert "vllm_attention" not in patched.calls
    if cache_dtype is not None:
        kf = k.view(torch.float8_e4m3fn).float() * k_scale
        vf = v.view(torch.float8_e4m3fn).float() * v_scale
    else:
        kf, vf = k, v
    ref = attention_f32(query[:n].view(n, hq, d), kf, vf, bt, meta.seq_lens, d**-0.5)
    assert_max_abs(output[:n].view(n, hq, d), ref, dtype, f"vLLM {cls_name} {layout}")
    assert (output[n:] == 7.0).all(), "rows past num_actual_tokens must not be written"


def test_patched_attention_falls_back_on_prefill(patched):
    buf, _, _ = _cache("interleaved", 2, 64, torch.float16, seed=1)
    meta = SimpleNamespace(max_query_len=4, num_actual_tokens=2, max_seq_len=40, causal=True,
                           seq_lens=torch.tensor([40, 20], dtype=torch.int32, device="cuda"),
                           block_table=_block_table([40, 20], seed=2))
    impl = fake_vllm.make_impl(patched.FlashAttentionImpl, **fake_vllm.impl_attrs(64, 8, 2))
    q = torch.randn(2, 8 * 64, device="cuda", dtype=torch.float16)
    out = torch.zeros_like(q)
    impl.forward(SimpleNamespace(), q, None, None, buf, meta, out)
    assert patched.calls == ["vllm_attention"]
    assert vllm_patch.stats()["attention_fallback_calls"] == 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_patched_rms_norm_and_silu_run_the_kernels(patched, dtype):
    g = torch.Generator(device="cuda").manual_seed(3)
    h, t, inter = 4096, 64, 14336
    norm = patched.RMSNorm()
    norm.weight = torch.nn.Parameter((1 + 0.1 * torch.randn(h, generator=g, device="cuda")).to(dtype))
    norm.hidden_size, norm.variance_epsilon = h, 1e-5
    x = torch.randn(t, h, generator=g, device="cuda", dtype=dtype)
    r = torch.randn(t, h, generator=g, device="cuda", dtype=dtype)
    y = norm.forward_cuda(x)
    want = rms_norm_reference(x.cpu(), norm.weight.data.cpu(), 1e-5)
    assert_ulp(y, want, 1, "patched RMSNorm")
    want_out, want_res = fused_add_rms_norm_reference(x.cpu(), r.cpu(), norm.weight.data.cpu(), 1e-5)
    out, res = norm.forward_cuda(x.clone(), r.clone())
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), want_res), "fused residual must be bit-exact"
    assert_ulp(out, want_out, 1, "patched fused_add RMSNorm")
    act = patched.SiluAndMul()
    xs = torch.randn(t, 2 * inter, generator=g, device="cuda", dtype=dtype)
    assert_ulp(act.forward_cuda(xs), silu_and_mul_reference(xs.cpu()), 1, "patched SiluAndMul")
    s = vllm_patch.stats()
    assert (s["rms_norm_kernel_calls"], s["rms_norm_fallback_calls"]) == (2, 0)
    assert (s["silu_and_mul_kernel_calls"], s["silu_and_mul_fallback_calls"]) == (1, 0)
    assert patched.calls == []
