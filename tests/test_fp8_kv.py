"""GPU parity tests of paged attention over an fp8 (e4m3fn) KV cache.

The reference has no fp8 path (README.md:185); the oracle is the fp32
reference attention on the dequantised cache (K = k_scale * k8, V = v_scale *
v8) at the 16-bit bar (2e-2 bf16 / 5e-3 fp16 plus the final rounding). A
structural check pins the conversion: with unit scales, an fp8 cache gives
the output of the 16-bit path on the same cache converted to the model dtype
(e4m3fn values are exact in bf16 and fp16) to within 2 ulp -- the fp8 path
sums Q.K^T over the head dimension in another column order, which moves the
fp32 logits by a few ulp of fp32.
"""

import ctypes

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from decodekernels_amd.testing import make_paged_kv
from parity import assert_max_abs, assert_ulp, attention_f32

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
DTYPES = [torch.float16, torch.bfloat16]


def _q(n, hq, d, dtype, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(n, hq, d, generator=g, device="cuda", dtype=dtype)


def _check(q, kv, k_scale, v_scale, dtype, **kw):
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, k_scale=k_scale,
                                    v_scale=v_scale, **kw)
    ref = attention_f32(q, kv.k_cache.float() * k_scale, kv.v_cache.float() * v_scale, kv.block_tables, kv.seq_lens)
    assert_max_abs(out, ref, dtype, "fp8 paged_attention_decode")
    return out


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("group", [1, 4, 8])
@pytest.mark.parametrize("layout", ["nhd", "hnd", "vllm"])
def test_fp8_single_pass_and_split(dtype, head_dim, group, layout):
    lens = [1, 17, 300, 512, 513, 1500, 0, 2100]
    kv = make_paged_kv(lens, 2, head_dim, 16, FP8, "cuda", layout=layout, seed=head_dim + group)
    q = _q(len(lens), 2 * group, head_dim, dtype)
    out = _check(q, kv, 0.05, 0.7, dtype)
    assert (out[6] == 0).all(), "an empty sequence gives zeros"
    short = [1, 17, 300, 512]
    kv_s = make_paged_kv(short, 2, head_dim, 32, FP8, "cuda", layout=layout, seed=head_dim + group + 1)
    _check(_q(len(short), 2 * group, head_dim, dtype, seed=2), kv_s, 0.05, 0.7, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim,group", [(192, 4), (192, 8), (128, 16), (64, 16), (256, 16)])
@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_fp8_head_dim_192_and_group_16(dtype, head_dim, group, schedule, monkeypatch):
    """Past the reference's limits with an fp8 cache: head_dim 192 (the D=256
    class) and GQA groups of 16 (the LDS merge in two passes of 8 heads),
    single pass and split-K under both schedules."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    lens = [1, 17, 300, 512, 513, 1500, 0, 2100]
    kv = make_paged_kv(lens, 2, head_dim, 16, FP8, "cuda", layout="vllm", seed=head_dim + group + 7)
    q = _q(len(lens), 2 * group, head_dim, dtype, seed=3)
    out = _check(q, kv, 0.3, 0.4, dtype)
    assert (out[6] == 0).all(), "an empty sequence gives zeros"
    short = [1, 17, 300, 512]
    kv_s = make_paged_kv(short, 2, head_dim, 16, FP8, "cuda", layout="nhd", seed=head_dim + group + 8)
    _check(_q(len(short), 2 * group, head_dim, dtype, seed=4), kv_s, 0.3, 0.4, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("schedule", ["grid", "balanced", "balanced-lockstep", "partitions"])
def test_fp8_long_contexts_both_schedules(dtype, schedule, monkeypatch):
    """Long ragged contexts under every schedule, including the balanced
    schedule's lockstep groups (not the fp8 default; DK_ATTN_LOCKSTEP=1)."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule.split("-")[0])
    if schedule == "balanced-lockstep":
        monkeypatch.setenv("DK_ATTN_LOCKSTEP", "1")
    lens = [16384, 3000, 7777, 1, 600, 9000, 12000, 5]
    kv = make_paged_kv(lens, 8, 128, 16, FP8, "cuda", layout="vllm", seed=7)
    _check(_q(len(lens), 32, 128, dtype, seed=3), kv, 0.031, 0.25, dtype)


@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_fp8_128k_batch_1(schedule, monkeypatch):
    """The long-context split-K shape with an fp8 cache: one 131072-token
    sequence, 32 query / 8 KV heads, head_dim 128, HND cache, 1% of rows
    scaled up (to 8x the others before the fp8 rounding), bf16 queries. Under
    the balanced schedule each KV stream spans more than 64 workspace rows."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    L = 131072
    kv = make_paged_kv([L], 8, 128, 16, FP8, "cuda", layout="hnd", seed=17)
    g = torch.Generator(device="cuda").manual_seed(18)
    rows = torch.rand(kv.k_cache.shape[0], 16, 8, 1, generator=g, device="cuda") < 0.01
    big = torch.where(rows, 8.0, 1.0)
    kv.k_cache.copy_((kv.k_cache.float() * big).to(FP8))
    kv.v_cache.copy_((kv.v_cache.float() * big).to(FP8))
    q = _q(1, 32, 128, torch.bfloat16, seed=19) * 128**-0.5
    ws = dk.alloc_workspace(1, 32, 128, L, "cuda")
    for t in ws:
        t.fill_(float("nan"))
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=L,
                                    workspace=ws, k_scale=0.5, v_scale=0.5)
    torch.cuda.synchronize()
    ref = attention_f32(q, kv.k_cache.float() * 0.5, kv.v_cache.float() * 0.5, kv.block_tables, kv.seq_lens)
    assert_max_abs(out, ref, torch.bfloat16, f"fp8 cache, 128K batch 1 ({schedule})")
    if schedule == "balanced":
        es = ws[2].cpu()
        filled = ~torch.isnan(es) & (es != 0)
        rows_used = int(torch.cumprod(filled.to(torch.int32), dim=-1).sum(dim=-1).max())
        assert rows_used > 64, f"the longest stream spans {rows_used} rows"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hq,hkv,head_dim", [(28, 4, 128), (14, 2, 64), (6, 2, 128), (10, 2, 64), (12, 2, 256)])
@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_fp8_odd_gqa_groups(dtype, hq, hkv, head_dim, schedule, monkeypatch):
    """GQA groups 3, 5, 6 and 7 (Qwen2.5-7B: 28 / 4, Qwen2.5-0.5B: 14 / 2) over an
    fp8 cache, single pass and split-K."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    lens = [1, 100, 512, 0, 37, 4000, 513, 9000]
    kv = make_paged_kv(lens, hkv, head_dim, 16, FP8, "cuda", layout="vllm", seed=hq + head_dim)
    out = _check(_q(len(lens), hq, head_dim, dtype, seed=hq), kv, 0.2, 0.7, dtype)
    assert (out[3] == 0).all()
    short = [1, 100, 512, 0]
    kv_s = make_paged_kv(short, hkv, head_dim, 16, FP8, "cuda", layout="hnd", seed=hq + 1)
    _check(_q(len(short), hq, head_dim, dtype, seed=hq + 1), kv_s, 0.2, 0.7, dtype)


@pytest.mark.parametrize("layout", ["nhd", "vllm"])
def test_fp8_automatic_schedule_llama_batch(layout):
    """The automatic schedule at the Llama-3-8B batch-64 shape (lengths
    U[512, 4096], 32 / 8 heads) over an fp8 cache: the NHD cache takes the
    1024-token grid, the vLLM cache the balanced schedule; both against the
    oracle on every sequence."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 4097, (64,), generator=g).tolist()
    kv = make_paged_kv(lens, 8, 128, 16, FP8, "cuda", layout=layout, seed=23)
    _check(_q(64, 32, 128, torch.bfloat16, seed=24) * 128**-0.5, kv, 0.5, 0.5, torch.bfloat16)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("split", [False, True])
def test_fp8_equals_16bit_path_on_the_converted_cache(dtype, split):
    lens = [700, 33, 2000, 512] if split else [100, 33, 512, 7]
    kv = make_paged_kv(lens, 4, 128, 16, FP8, "cuda", layout="nhd", seed=11)
    q = _q(len(lens), 16, 128, dtype, seed=4)
    got = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    want = dk.paged_attention_decode(q, kv.k_cache.to(dtype), kv.v_cache.to(dtype), kv.block_tables, kv.seq_lens)
    torch.cuda.synchronize()
    assert_ulp(got, want, 2, "fp8 path vs 16-bit path on the converted cache")


def test_fp8_block_sizes_that_split_tiles():
    lens = [5, 40, 700, 1300]
    for bs in (8, 24):
        kv = make_paged_kv(lens, 2, 64, bs, FP8, "cuda", layout="nhd", seed=bs)
        _check(_q(len(lens), 8, 64, torch.bfloat16, seed=bs), kv, 0.1, 0.1, torch.bfloat16)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_fp8_rows_aligned_to_8_bytes_only(head_dim):
    """Rows 8- but not 16-byte aligned take the paired 8-byte load path."""
    lens = [30, 700, 1500]
    kv = make_paged_kv(lens, 2, head_dim, 16, FP8, "cuda", layout="nhd", seed=head_dim)
    nb, bs, hkv, d = kv.k_cache.shape
    pitch = d + 8  # token stride with 8 bytes of padding: rows alternate 16- and 8-byte alignment
    bufk = torch.zeros(nb * bs * hkv * pitch + 8, dtype=FP8, device="cuda")
    bufv = torch.zeros_like(bufk)
    k = bufk[8:].as_strided((nb, bs, hkv, d), (bs * hkv * pitch, hkv * pitch, pitch, 1))
    v = bufv[8:].as_strided((nb, bs, hkv, d), (bs * hkv * pitch, hkv * pitch, pitch, 1))
    k.copy_(kv.k_cache)
    v.copy_(kv.v_cache)
    kv.k_cache, kv.v_cache = k, v
    _check(_q(len(lens), 8, head_dim, torch.bfloat16, seed=9), kv, 0.3, 0.6, torch.bfloat16)


def test_fp8_graph_replay_follows_new_lengths():
    dtype = torch.bfloat16
    kv = make_paged_kv([2048] * 3, 2, 128, 16, FP8, "cuda", seed=13)
    kv.seq_lens.copy_(torch.tensor([300, 1500, 40], dtype=torch.int32))
    q = _q(3, 8, 128, dtype, seed=5)
    out = torch.empty_like(q)
    ws = dk.alloc_workspace(3, 8, 128, 2048, "cuda")

    def step():
        dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=2048,
                                  out=out, workspace=ws, k_scale=0.2, v_scale=0.3)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for lens in ([300, 1500, 40], [2048, 1, 777], [0, 513, 2047]):
        kv.seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        ref = attention_f32(q, kv.k_cache.float() * 0.2, kv.v_cache.float() * 0.3, kv.block_tables, kv.seq_lens)
        assert_max_abs(out, ref, dtype, f"replay {lens}")


def test_fp8_capi_matches_torch_op():
    dtype = torch.float16
    lens = [3, 200, 512, 1900]
    kv = make_paged_kv(lens, 4, 128, 16, FP8, "cuda", layout="vllm", seed=21)
    q = _q(len(lens), 16, 128, dtype, seed=6)
    ws = dk.alloc_workspace(len(lens), 16, 128, max(lens), "cuda")
    out = torch.empty_like(q)
    p = capi.attn_params(out, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, 128**-0.5, ws)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = capi.lib().dk_paged_attention_decode_fp8(ctypes.byref(p), capi.dtype_code(dtype), 128, max(lens), 0.5, 2.0,
                                                  stream)
    assert rc == 0, capi.last_error()
    via_torch = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens,
                                          max_seq_len=max(lens), k_scale=0.5, v_scale=2.0)
    torch.cuda.synchronize()
    assert torch.equal(out, via_torch)


def test_fp8_rejects_bad_arguments():
    kv = make_paged_kv([10, 20], 2, 128, 16, FP8, "cuda", seed=1)
    q = _q(2, 8, 128, torch.bfloat16)
    with pytest.raises(RuntimeError, match="finite"):
        dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, k_scale=float("inf"))
    with pytest.raises(RuntimeError, match="multiples of 8 bytes"):
        flat = torch.zeros(kv.k_cache.numel() + 4, dtype=FP8, device="cuda")
        k_off = flat[4:].view(kv.k_cache.shape)
        dk.paged_attention_decode(q, k_off, kv.v_cache, kv.block_tables, kv.seq_lens)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        dk.paged_attention_decode(q.float(), kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    with pytest.raises(ValueError, match="fp8"):
        kv16 = make_paged_kv([10], 2, 128, 16, torch.bfloat16, "cuda")
        dk.paged_attention_decode(q[:1], kv16.k_cache, kv16.v_cache, kv16.block_tables, kv16.seq_lens, k_scale=0.5)
