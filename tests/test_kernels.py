"""GPU parity tests: every HIP kernel against the oracle on seeded inputs.

Mirrors DecodeKernels' ``tests/test_kernels.py:36-241`` (same cases: head dims,
GQA groups, block sizes, partition boundaries, strided layouts, empty
sequences, custom scale, graph replay, bad inputs, GEMM shapes, norms,
torch.compile), at the acceptance bar of ``tests/parity.py``, plus cases the
reference does not cover: block sizes that are not multiples of 16, narrowly
aligned KV strides, the Llama-3-8B decode shape and long split-K contexts.
These run only on a GPU; the ops raise if the HIP libraries are missing.
"""

import math

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd.testing import make_paged_kv
from parity import (
    assert_max_abs,
    assert_ulp,
    attention_f32,
    fused_add_rms_norm_reference,
    gemm_f32,
    gemm_f32_gpu,
    rms_norm_reference,
    silu_and_mul_reference,
)

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _q(num_seqs, num_q_heads, head_dim, dtype, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(num_seqs, num_q_heads, head_dim, generator=g, device="cuda", dtype=dtype)


def _check_attention(q, kv, dtype, scale=None, **kw):
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, scale=scale, **kw)
    ref = attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, scale)
    assert_max_abs(out, ref, dtype, "paged_attention_decode")
    return out


def test_extension_is_loaded():
    assert dk.is_available(), "decodekernels_amd._C must load on a GPU box"


# ---------------------------------------------------------------------------
# Paged attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("group", [1, 4, 8])
@pytest.mark.parametrize("block_size", [16, 32])
def test_paged_attention_short(dtype, head_dim, group, block_size):
    """Single-pass path: every sequence fits in one partition."""
    seq_lens = [1, 2, 17, 100, 255, 512]
    kv = make_paged_kv(seq_lens, 2, head_dim, block_size, dtype, "cuda")
    _check_attention(_q(len(seq_lens), 2 * group, head_dim, dtype), kv, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("group", [1, 4, 8])
def test_paged_attention_split_k(dtype, head_dim, group):
    """Split-K: partition boundaries and sequences much shorter than the maximum."""
    seq_lens = [1, 511, 512, 513, 1024, 1025, 3000, 8192]
    kv = make_paged_kv(seq_lens, 2, head_dim, 16, dtype, "cuda")
    _check_attention(_q(len(seq_lens), 2 * group, head_dim, dtype), kv, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("schedule", ["auto", "grid", "balanced", "partitions"])
def test_paged_attention_c1_shape(dtype, schedule, monkeypatch):
    """BASELINE configs[0] on the HIP path: 4 sequences of {1, 511, 512, 513}
    tokens, 8 query / 2 KV heads, head_dim 128, block 16, NHD cache of 160
    physical blocks (98 used + extra_blocks=62), split-K (max_seq_len 513)."""
    if schedule != "auto":
        monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    lens = [1, 511, 512, 513]
    kv = make_paged_kv(lens, 2, 128, 16, dtype, "cuda", layout="nhd", extra_blocks=62, seed=0)
    assert kv.k_cache.shape[0] == 160
    q = _q(4, 8, 128, dtype)
    out = _check_attention(q, kv, dtype, max_seq_len=513)
    ws = dk.alloc_workspace(4, 8, 128, 513, "cuda")
    assert ws[0].shape == (4, 8, 2, 128)
    again = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=513,
                                      workspace=ws)
    assert torch.equal(out, again)


def _workspace_rows(exp_sums: torch.Tensor) -> torch.Tensor:
    """Rows a balanced-schedule call filled per (sequence, query head): the
    workspace starts as NaN, pieces fill rows 0 .. n-1 and the stream's last
    piece marks row n empty (exp-sum 0) when n < max_partitions."""
    es = exp_sums.cpu()
    filled = ~torch.isnan(es) & (es != 0)
    # rows before the first unfilled one
    return torch.cumprod(filled.to(torch.int32), dim=-1).sum(dim=-1)


@pytest.mark.parametrize("seq_len,min_rows", [(140000, 64), (270000, 128)])
@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_paged_attention_reduce_many_rows(seq_len, min_rows, schedule, monkeypatch):
    """One KV head of one long sequence: under the balanced schedule the stream
    is cut into one piece per workgroup share, so the reduce merges more than
    64 (140K tokens) and more than 128 (270K tokens) workspace rows per query
    head -- its second and third lane-parallel passes over the exp-sums. The
    grid schedule merges ceil(L / 1024) + 1 rows, the grid of 512-token units
    ceil(L / 512). All against the oracle."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    dtype = torch.bfloat16
    kv = make_paged_kv([seq_len], 1, 128, 16, dtype, "cuda", layout="nhd", seed=seq_len % 1000)
    q = _q(1, 4, 128, dtype, seed=3)
    ws = dk.alloc_workspace(1, 4, 128, seq_len, "cuda")
    for t in ws:
        t.fill_(float("nan"))
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=seq_len,
                                    workspace=ws)
    torch.cuda.synchronize()
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), dtype,
                   f"{seq_len} tokens, one KV head ({schedule})")
    if schedule == "balanced":
        rows = _workspace_rows(ws[2])
        assert (rows == rows[0, 0]).all(), "every query head of a stream uses the same rows"
        assert int(rows[0, 0]) > min_rows, f"the stream spans {int(rows[0, 0])} rows, expected > {min_rows}"
        assert int(rows[0, 0]) <= ws[2].shape[-1]
    if schedule == "partitions":  # one row per 512-token partition, as the reference's workspace
        assert (_workspace_rows(ws[2]) == -(-seq_len // 512)).all()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lens", [[2048] * 32, [8192] * 8, [700] * 24, [3000, 1, 2047, 0] * 6],
                         ids=["32x2048", "8x8192", "24x700", "mixed24"])
def test_paged_attention_balanced_small_totals(dtype, lens, monkeypatch):
    """Balanced schedule with too little work for the first-dispatched half's
    full share ratio above the 64-tile minimum share: the second half keeps the
    minimum and the first half takes the rest. Against the oracle, and every
    stream's pieces stay inside the workspace's rows."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", "balanced")
    n, ml = len(lens), max(lens)
    kv = make_paged_kv(lens, 8, 128, 16, dtype, "cuda", layout="nhd", seed=n + ml)
    q = _q(n, 32, 128, dtype, seed=ml)
    ws = dk.alloc_workspace(n, 32, 128, ml, "cuda")
    for t in ws:
        t.fill_(float("nan"))
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=ml,
                                    workspace=ws)
    torch.cuda.synchronize()
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), dtype,
                   f"balanced, {n} sequences up to {ml} tokens")
    rows = _workspace_rows(ws[2])
    live = torch.tensor(lens).repeat_interleave(32).view(n, 32) > 0
    assert (rows[live] >= 1).all() and (rows <= ws[2].shape[-1]).all()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lockstep", ["0", "1"])
@pytest.mark.parametrize("hkv", [8, 4, 3, 1])
def test_paged_attention_balanced_lockstep(dtype, lockstep, hkv, monkeypatch):
    """Balanced schedule with one workgroup per share (DK_ATTN_LOCKSTEP=0) and
    with lockstep groups of hkv workgroups sharing each share (=1; 3 KV heads
    do not divide the resident grid, so the host keeps one workgroup per
    share). Ragged lengths with empty sequences, against the oracle; every
    stream's pieces stay inside the workspace rows, and under lockstep all
    query heads of a sequence fill the same number of rows (its KV heads take
    the same pieces)."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", "balanced")
    monkeypatch.setenv("DK_ATTN_LOCKSTEP", lockstep)
    lens = [5000, 0, 1, 777, 2048, 16, 9000, 513, 0, 3100] * 3
    n, ml, hq = len(lens), max(lens), 4 * hkv
    kv = make_paged_kv(lens, hkv, 128, 16, dtype, "cuda", layout="nhd", seed=hkv)
    q = _q(n, hq, 128, dtype, seed=hkv + 1)
    ws = dk.alloc_workspace(n, hq, 128, ml, "cuda")
    for t in ws:
        t.fill_(float("nan"))
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=ml,
                                    workspace=ws)
    torch.cuda.synchronize()
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), dtype,
                   f"balanced, lockstep={lockstep}, {hkv} KV heads")
    assert (out[torch.tensor(lens) == 0] == 0).all(), "empty sequences give zeros"
    rows = _workspace_rows(ws[2])
    live = torch.tensor(lens) > 0
    assert (rows[live] >= 1).all() and (rows <= ws[2].shape[-1]).all()
    if lockstep == "1" and hkv != 3:
        assert (rows == rows[:, :1]).all(), "lockstep: every KV head of a sequence takes the same pieces"


# Qwen2.5-7B (28 query / 4 KV heads, group 7, head_dim 128), Qwen2.5-0.5B
# (14 / 2, group 7, head_dim 64) and groups 3, 5 and 6.
ODD_GROUP_CASES = [(28, 4, 128), (14, 2, 64), (6, 2, 128), (10, 2, 64), (12, 2, 256), (21, 3, 96)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hq,hkv,head_dim", ODD_GROUP_CASES, ids=lambda v: str(v))
@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_paged_attention_odd_gqa_groups(dtype, hq, hkv, head_dim, schedule, monkeypatch):
    """GQA groups that are not powers of two (the reference's benchmark models,
    benchmarks/bench_kernels.py:38-42), single pass and split-K."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    short = [1, 100, 512, 0, 37]
    kv = make_paged_kv(short, hkv, head_dim, 16, dtype, "cuda", layout="vllm", seed=hq)
    out = _check_attention(_q(len(short), hq, head_dim, dtype, seed=hq), kv, dtype)
    assert (out[3] == 0).all()
    lens = _log_uniform_lens(20, 9000, seed=hq + head_dim, zeros=2)
    kv = make_paged_kv(lens, hkv, head_dim, 16, dtype, "cuda", layout="hnd", seed=hq + 1)
    _check_attention(_q(len(lens), hq, head_dim, dtype, seed=hq + 2), kv, dtype, max_seq_len=9000)


@pytest.mark.parametrize("dtype", DTYPES)
def test_paged_attention_split_k_head_dim_256(dtype):
    seq_lens = [0, 700, 1536, 2049]
    kv = make_paged_kv(seq_lens, 2, 256, 32, dtype, "cuda", layout="nhd")
    _check_attention(_q(len(seq_lens), 16, 256, dtype), kv, dtype)


@pytest.mark.parametrize("block_size", [1, 8, 24])
@pytest.mark.parametrize("max_len", [300, 1300])
def test_paged_attention_block_sizes_not_multiple_of_16(block_size, max_len):
    """Block sizes whose 16-token tiles straddle cache blocks."""
    seq_lens = [5, max_len, 47]
    kv = make_paged_kv(seq_lens, 2, 128, block_size, torch.float16, "cuda")
    _check_attention(_q(3, 8, 128, torch.float16), kv, torch.float16)


@pytest.mark.parametrize("head_dim,pad", [(64, 2), (128, 4), (64, 4)])
def test_paged_attention_narrow_kv_alignment(head_dim, pad):
    """KV strides that are multiples of head_dim/32 but not of 8 elements take
    the 8- or 4-byte load variants."""
    seq_lens = [33, 700]
    blocks = 2 + sum(-(-n // 16) for n in seq_lens)
    g = torch.Generator(device="cuda").manual_seed(7)
    raw = torch.randn(blocks, 16, 2, head_dim + pad, generator=g, device="cuda", dtype=torch.bfloat16)
    raw_v = torch.randn(blocks, 16, 2, head_dim + pad, generator=g, device="cuda", dtype=torch.bfloat16)
    k, v = raw[..., :head_dim], raw_v[..., :head_dim]
    kv = make_paged_kv(seq_lens, 2, head_dim, 16, torch.bfloat16, "cuda", extra_blocks=2)
    kv.k_cache, kv.v_cache = k, v
    _check_attention(_q(2, 8, head_dim, torch.bfloat16), kv, torch.bfloat16)


@pytest.mark.parametrize("layout", ["hnd", "vllm"])
@pytest.mark.parametrize("seq_lens", [[5, 300], [700, 2000]])
def test_paged_attention_strided_layouts(layout, seq_lens):
    kv = make_paged_kv(seq_lens, 2, 128, 16, torch.float16, "cuda", layout=layout)
    assert not kv.k_cache.is_contiguous()
    _check_attention(_q(len(seq_lens), 8, 128, torch.float16), kv, torch.float16)


@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_paged_attention_token_stride_beyond_tile_offsets(schedule, monkeypatch):
    """A token stride of 2^26 elements (a [block_size, blocks, heads, D] cache
    viewed as [blocks, block_size, heads, D], 2 GiB per K/V): 16 rows of a tile
    span 2^31 bytes, more than the whole-tile loads' 32-bit buffer offsets
    reach, so the host routes the call to the per-row loads (64-bit
    addresses). Blocks are spread over the whole cache, up to the last one.
    Checked against the oracle on the gathered blocks and, under the grid
    schedule, bit for bit against the same call on a compact copy (whole-tile
    loads). The balanced schedule cuts the streams by the resident workgroup
    count, which differs between the two kernels (the per-row one needs less
    LDS and fits three workgroups per CU, not two), so its pieces, and the
    last bits, differ there."""
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    hkv, d, bs, nb = 2, 128, 16, 2**18
    seq_lens = [37, 700, 1300]
    need = [-(-n // bs) for n in seq_lens]
    g = torch.Generator(device="cuda").manual_seed(11)
    ids = torch.randperm(nb, generator=g, device="cuda")[: sum(need)]
    ids[-1] = nb - 1
    big_k = torch.empty(bs, nb, hkv, d, device="cuda", dtype=torch.bfloat16)
    big_v = torch.empty_like(big_k)
    k_cache, v_cache = big_k.permute(1, 0, 2, 3), big_v.permute(1, 0, 2, 3)
    assert k_cache.stride(1) == 2**26
    kc = torch.randn(len(ids), bs, hkv, d, generator=g, device="cuda", dtype=torch.bfloat16)
    vc = torch.randn(len(ids), bs, hkv, d, generator=g, device="cuda", dtype=torch.bfloat16)
    k_cache[ids], v_cache[ids] = kc, vc
    bt = torch.zeros(len(seq_lens), max(need), dtype=torch.int32, device="cuda")
    bt_c = torch.zeros_like(bt)
    pos = 0
    for s, n in enumerate(need):
        bt[s, :n] = ids[pos : pos + n].to(torch.int32)
        bt_c[s, :n] = torch.arange(pos, pos + n, dtype=torch.int32, device="cuda")
        pos += n
    lens = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    q = _q(len(seq_lens), 8, d, torch.bfloat16, seed=12)
    out = dk.paged_attention_decode(q, k_cache, v_cache, bt, lens)
    compact = dk.paged_attention_decode(q, kc, vc, bt_c, lens)
    torch.cuda.synchronize()
    del big_k, big_v, k_cache, v_cache
    ref = attention_f32(q, kc, vc, bt_c, lens)
    assert_max_abs(out, ref, torch.bfloat16, "token stride 2^26")
    assert_max_abs(compact, ref, torch.bfloat16, "compact copy")
    if schedule == "grid":
        assert torch.equal(out, compact)


@pytest.mark.parametrize("max_seq_len", [100, 2000])
def test_paged_attention_empty_sequences(max_seq_len):
    seq_lens = [0, 50, 0, max_seq_len]
    kv = make_paged_kv(seq_lens, 2, 64, 16, torch.float16, "cuda")
    out = _check_attention(_q(4, 4, 64, torch.float16), kv, torch.float16)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0


def test_paged_attention_custom_scale_and_output_buffer():
    kv = make_paged_kv([64, 900], 1, 128, 16, torch.bfloat16, "cuda")
    q = _q(2, 4, 128, torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, scale=0.05, out=out)
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, 0.05), torch.bfloat16)


def test_paged_attention_strided_q_and_out():
    """q and out are views with non-contiguous head/seq strides."""
    kv = make_paged_kv([40, 600], 2, 128, 16, torch.float16, "cuda")
    big = _q(2, 24, 128, torch.float16)
    q = big[:, ::3]  # head stride 3*128
    out_big = torch.zeros(2, 16, 128, device="cuda", dtype=torch.float16)
    out = out_big[:, ::2]
    dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, out=out)
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), torch.float16)
    assert torch.count_nonzero(out_big[:, 1::2]) == 0


def test_paged_attention_llama3_8b_decode_shape():
    """The Llama-3-8B batch decode shape on vLLM's interleaved cache (8 seqs checked)."""
    g = torch.Generator().manual_seed(11)
    seq_lens = torch.randint(512, 4097, (8,), generator=g).tolist()
    kv = make_paged_kv(seq_lens, 8, 128, 16, torch.bfloat16, "cuda", layout="vllm", seed=12)
    q = _q(8, 32, 128, torch.bfloat16) * 128**-0.5
    _check_attention(q, kv, torch.bfloat16)


def test_paged_attention_long_context_outlier_rows():
    """A 32K context with 1% of K/V rows scaled by 8 stresses the max-logit merge."""
    kv = make_paged_kv([32768], 8, 128, 16, torch.float16, "cuda", layout="hnd", seed=13)
    g = torch.Generator(device="cuda").manual_seed(14)
    nb = kv.k_cache.shape[0]
    mask = torch.rand(nb, 16, 1, 1, generator=g, device="cuda") < 0.01
    kv.k_cache.mul_(torch.where(mask, 8.0, 1.0).to(torch.float16))
    kv.v_cache.mul_(torch.where(mask, 8.0, 1.0).to(torch.float16))
    _check_attention(_q(1, 32, 128, torch.float16), kv, torch.float16)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("group", [9, 12, 16])
def test_paged_attention_groups_above_8(dtype, head_dim, group):
    """GQA groups of 9-16 query heads per KV head (Llama-3.1-405B: 16), which
    the reference rejects; the heads' partial outputs merge in two passes."""
    lens = [1, 300, 512, 513, 2100, 0, 777]
    kv = make_paged_kv(lens, 2, head_dim, 16, dtype, "cuda", layout="vllm", seed=group + head_dim)
    out = _check_attention(_q(len(lens), 2 * group, head_dim, dtype, seed=group), kv, dtype)
    assert (out[5] == 0).all()
    short = [7, 64, 512]
    kv = make_paged_kv(short, 1, head_dim, 32, dtype, "cuda", seed=group)
    _check_attention(_q(len(short), group, head_dim, dtype, seed=group + 1), kv, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [96, 192])
@pytest.mark.parametrize("group", [1, 4, 8, 16])
@pytest.mark.parametrize("layout", ["nhd", "vllm"])
def test_paged_attention_head_dims_96_192(dtype, head_dim, group, layout):
    """Head dims the reference rejects (Phi-3: 96; 192), single pass and split-K."""
    lens = [1, 17, 300, 512, 513, 1500, 0, 2100]
    kv = make_paged_kv(lens, 2, head_dim, 16, dtype, "cuda", layout=layout, seed=head_dim + group)
    out = _check_attention(_q(len(lens), 2 * group, head_dim, dtype, seed=group), kv, dtype)
    assert (out[6] == 0).all()


@pytest.mark.parametrize("head_dim", [96, 192])
@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_paged_attention_head_dims_96_192_long(head_dim, schedule, monkeypatch):
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    lens = _log_uniform_lens(24, 12000, seed=head_dim)
    kv = make_paged_kv(lens, 4, head_dim, 32, torch.bfloat16, "cuda", layout="hnd", seed=head_dim)
    _check_attention(_q(len(lens), 16, head_dim, torch.bfloat16, seed=5), kv, torch.bfloat16, max_seq_len=12000)


def test_paged_attention_head_dim_192_fp8_cache():
    lens = [5, 700, 3000, 1]
    kv = make_paged_kv(lens, 2, 192, 16, torch.float8_e4m3fn, "cuda", layout="vllm", seed=8)
    q = _q(len(lens), 16, 192, torch.float16, seed=6)
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, k_scale=0.2, v_scale=0.9)
    ref = attention_f32(q, kv.k_cache.float() * 0.2, kv.v_cache.float() * 0.9, kv.block_tables, kv.seq_lens)
    assert_max_abs(out, ref, torch.float16, "head_dim 192, fp8 cache")
    kv96 = make_paged_kv(lens, 2, 96, 16, torch.float8_e4m3fn, "cuda", seed=9)
    with pytest.raises(RuntimeError, match="head_dim"):
        dk.paged_attention_decode(_q(len(lens), 4, 96, torch.float16), kv96.k_cache, kv96.v_cache, kv96.block_tables,
                                  kv96.seq_lens)


@pytest.mark.parametrize("schedule", ["grid", "balanced", "partitions"])
def test_paged_attention_group_16_fp8_cache(schedule, monkeypatch):
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    lens = [9000, 40, 3000, 1]
    kv = make_paged_kv(lens, 8, 128, 16, torch.float8_e4m3fn, "cuda", layout="vllm", seed=3)
    q = _q(len(lens), 128, 128, torch.bfloat16, seed=4)
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, k_scale=0.1, v_scale=0.3)
    ref = attention_f32(q, kv.k_cache.float() * 0.1, kv.v_cache.float() * 0.3, kv.block_tables, kv.seq_lens)
    assert_max_abs(out, ref, torch.bfloat16, "group 16, fp8 cache")


def _log_uniform_lens(n, max_len, seed, zeros=4):
    """Lengths log-uniform in [1, max_len], a few empty, the first at max_len."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.exp(torch.rand(n, generator=g) * math.log(max_len)).long().clamp(1, max_len)
    lens[torch.randperm(n, generator=g)[:zeros]] = 0
    lens[0] = max_len
    return lens.tolist()


# (head_dim, num_kv_heads, group, block_size, layout, num_seqs, max_len, dtype)
SCHEDULE_CASES = [
    (256, 2, 8, 32, "nhd", 48, 16384, torch.bfloat16),  # the head-dim-256 / group-8 stress shape, fewer seqs
    (128, 8, 4, 16, "vllm", 24, 9000, torch.float16),
    (64, 4, 2, 16, "hnd", 40, 12000, torch.bfloat16),
    (128, 2, 4, 24, "nhd", 16, 5000, torch.float16),  # blocks that split 16-token tiles
]


@pytest.mark.parametrize("case", SCHEDULE_CASES, ids=lambda c: f"d{c[0]}_hkv{c[1]}_g{c[2]}_bs{c[3]}_{c[4]}")
def test_paged_attention_split_k_schedules(case, monkeypatch):
    """Split-K under the three schedules -- one workgroup per 1024-token unit,
    resident workgroups with equal tile shares of all sequences, one workgroup
    per 512-token partition -- against the oracle. They cut the sequences
    differently (so they may differ in the last bits); each is deterministic
    from call to call."""
    d, hkv, group, bs, layout, n, max_len, dtype = case
    lens = _log_uniform_lens(n, max_len, seed=d + bs)
    kv = make_paged_kv(lens, hkv, d, bs, dtype, "cuda", layout=layout, seed=d + 1)
    q = _q(n, hkv * group, d, dtype)
    ref = attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    for schedule in ("grid", "balanced", "partitions"):
        monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
        run = lambda: dk.paged_attention_decode(  # noqa: E731
            q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=max_len
        )
        out = run()
        again = run()
        torch.cuda.synchronize()
        assert_max_abs(out, ref, dtype, f"{schedule} schedule")
        assert torch.equal(out, again), f"{schedule} schedule is not deterministic"


@pytest.mark.parametrize("num_seqs", [2048, 2049])
def test_paged_attention_split_k_many_sequences(num_seqs, monkeypatch):
    """Split-K at the balanced schedule's sequence limit (its length scan holds
    2048 sequences in LDS) and one past it, where the grid schedule takes over
    even when the balanced one is asked for: both against the oracle, and
    deterministic."""
    g = torch.Generator().manual_seed(num_seqs)
    lens = torch.randint(0, 1101, (num_seqs,), generator=g)
    lens[0] = 1100
    lens = lens.tolist()
    kv = make_paged_kv(lens, 1, 64, 16, torch.bfloat16, "cuda", layout="nhd", seed=3)
    q = _q(num_seqs, 4, 64, torch.bfloat16)
    ref = attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    monkeypatch.setenv("DK_ATTN_SCHEDULE", "balanced")
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=1100)
    again = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=1100)
    torch.cuda.synchronize()
    assert_max_abs(out, ref, torch.bfloat16, f"{num_seqs} sequences")
    assert torch.equal(out, again)
    assert (out[kv.seq_lens == 0] == 0).all()


# (lens, num_kv_heads, max_seq_len): shapes whose tile shares end inside short
# streams, a single long stream, a two-row workspace and mostly-empty batches.
BALANCED_CASES = [
    ([0, 1, 17, 300, 1023, 1024, 1025, 5], 4, 20000),
    ([513, 600, 1000, 1024, 700, 520, 999, 1001] * 8, 8, 1024),
    ([40000], 8, 40000),
    ([0] * 30 + [3000] + [0] * 30, 2, 3000),
    ([511, 512, 513] * 40, 1, 600),
    ([16, 32, 48, 64, 80, 96] * 50, 8, 4096),
]


@pytest.mark.parametrize("case", BALANCED_CASES, ids=lambda c: f"n{len(c[0])}_hkv{c[1]}_max{c[2]}")
def test_paged_attention_balanced_schedule_edge_shapes(case, monkeypatch):
    monkeypatch.setenv("DK_ATTN_SCHEDULE", "balanced")
    lens, hkv, max_len = case
    kv = make_paged_kv(lens, hkv, 128, 16, torch.bfloat16, "cuda", seed=len(lens))
    q = _q(len(lens), 4 * hkv, 128, torch.bfloat16)
    out = _check_attention(q, kv, torch.bfloat16, max_seq_len=max_len)
    if 0 in lens:
        assert (out[torch.tensor(lens) == 0] == 0).all()


@pytest.mark.parametrize("schedule", ["auto", "grid", "balanced", "partitions"])
def test_paged_attention_graph_replay(schedule, monkeypatch):
    """Preallocated buffers make the op capturable; replays track new cache
    contents and lengths (within the captured max_seq_len)."""
    if schedule != "auto":
        monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    dtype = torch.float16
    max_seq_len = 2048
    kv = make_paged_kv([max_seq_len] * 3, 2, 128, 16, dtype, "cuda")
    kv.seq_lens.copy_(torch.tensor([300, 1500, 40], dtype=torch.int32))
    q = _q(3, 8, 128, dtype)
    out = torch.empty_like(q)
    ws = dk.alloc_workspace(3, 8, 128, max_seq_len, "cuda")

    def step():
        dk.paged_attention_decode(
            q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=max_seq_len, out=out, workspace=ws
        )

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()

    for new_lens in ([300, 1500, 40], [2048, 1, 777], [0, 513, 2047]):
        kv.seq_lens.copy_(torch.tensor(new_lens, dtype=torch.int32))
        q.normal_()
        graph.replay()
        torch.cuda.synchronize()
        ref = attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
        assert_max_abs(out, ref, dtype, f"replay {new_lens}")
        step()  # eager call between replays must agree too
        torch.cuda.synchronize()
        assert_max_abs(out, ref, dtype, f"eager {new_lens}")


def test_paged_attention_rejects_bad_inputs():
    kv = make_paged_kv([10], 2, 128, 16, torch.float16, "cuda")
    with pytest.raises(RuntimeError, match="GQA group"):
        dk.paged_attention_decode(_q(1, 64, 128, torch.float16), kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    kv80 = make_paged_kv([10], 2, 80, 16, torch.float16, "cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        dk.paged_attention_decode(_q(1, 2, 80, torch.float16), kv80.k_cache, kv80.v_cache, kv80.block_tables, kv80.seq_lens)
    with pytest.raises(RuntimeError, match="tmp_out must be"):
        ws = dk.alloc_workspace(1, 4, 128, 600, "cuda")
        dk.paged_attention_decode(_q(1, 4, 128, torch.float16), kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens,
                                  max_seq_len=2000, workspace=ws)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        kv32 = make_paged_kv([10], 1, 64, 16, torch.float32, "cuda")
        dk.paged_attention_decode(_q(1, 1, 64, torch.float32), kv32.k_cache, kv32.v_cache, kv32.block_tables, kv32.seq_lens)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
GEMM_SHAPES = [
    (1, 4096, 4096),
    (7, 1000, 520),
    (64, 6144, 4096),
    (65, 512, 256),
    (128, 4096, 4096),
    (200, 300, 72),  # K tail inside the first slice
    (256, 4096, 1024),  # 64x64 tiles
    (333, 1024, 1032),
    (512, 4096, 1032),  # 128x64 tiles
    (512, 6144, 1032),  # 128x128 tiles
    (512, 11008, 4096),
    (902, 10465, 560),  # 256x192 tiles, ragged M and N, N odd (scalar stores)
    (1000, 1000, 136),
    (274, 10917, 520),  # 256x128 tiles, partial in M and N
    (2000, 6000, 264),  # 256x192 tiles, partial in M and N
    (2000, 7000, 264),  # 256x256 tiles, partial in M and N
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm(dtype, M, N, K, with_bias):
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype) if with_bias else None
    assert_max_abs(dk.gemm(a, b, bias), gemm_f32(a, b, bias), dtype, f"gemm {M}x{N}x{K}")


@pytest.mark.parametrize("M", [1, 8, 16, 32, 48, 64, 4096])
@pytest.mark.parametrize("N", [6144, 4096, 28672])
def test_gemm_decode_layer_shapes(M, N):
    """The bf16 decode-layer projections (K=4096, A and B ~ N(0, 0.02)); the
    largest against a GPU fp32 GEMM, the rest against the CPU oracle."""
    g = torch.Generator(device="cuda").manual_seed(M + N)
    a = torch.randn(M, 4096, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
    b = torch.randn(N, 4096, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
    ref = _gemm_f32_gpu(a, b) if M * N >= 4096 * 28672 else gemm_f32(a, b)
    assert_max_abs(dk.gemm(a, b), ref, torch.bfloat16, f"gemm {M}x{N}")


def _gemm_f32_gpu(a, b):
    """Plain torch fp32 GEMM on the GPU, for shapes where the CPU oracle would take minutes."""
    return gemm_f32_gpu(a, b)


@pytest.mark.parametrize("M", [1, 16, 32, 48, 64, 4096])
def test_gemm_down_projection_k14336(M):
    """The decode layer's down projection (N = 4096, K = 14336), bf16."""
    g = torch.Generator(device="cuda").manual_seed(M + 14336)
    a = torch.randn(M, 14336, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
    b = torch.randn(4096, 14336, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
    ref = _gemm_f32_gpu(a, b) if M == 4096 else gemm_f32(a, b)
    assert_max_abs(dk.gemm(a, b), ref, torch.bfloat16, f"gemm down {M}x4096x14336")


# Skinny shapes with ragged N and K around the plan's boundaries (unsplit
# grids of 1 ... 8 waves along N, the wide plan past N = 32768 at M = 64);
# tests/test_gemm_splitk.py runs one shape per plan the launcher can pick.
SKINNY_POLICY_SHAPES = [
    (1, 12328, 520),
    (16, 24600, 136),
    (17, 6152, 1032),
    (32, 12296, 136),
    (33, 1000, 4104),
    (40, 6168, 520),
    (63, 12304, 136),
    (64, 24584, 136),
    (64, 33000, 136),
]


@pytest.mark.parametrize("M,N,K", SKINNY_POLICY_SHAPES)
def test_gemm_skinny_policy_boundaries(M, N, K):
    g = torch.Generator(device="cuda").manual_seed(M * 7 + K)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=torch.bfloat16) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=torch.bfloat16)
    assert_max_abs(dk.gemm(a, b, bias), gemm_f32(a, b, bias), torch.bfloat16, f"gemm {M}x{N}x{K}")


def test_gemm_batched_input_and_strided_rows():
    a = torch.randn(2, 3, 256, device="cuda", dtype=torch.float16)
    b = torch.randn(80, 256, device="cuda", dtype=torch.float16) / 16
    out = dk.gemm(a, b)
    assert out.shape == (2, 3, 80)
    assert_max_abs(out.view(6, 80), gemm_f32(a.reshape(-1, 256), b), torch.float16)
    wide = torch.randn(5, 512, device="cuda", dtype=torch.float16)
    a2 = wide[:, :256]
    assert_max_abs(dk.gemm(a2, b), gemm_f32(a2, b), torch.float16)
    c_wide = torch.zeros(5, 96, device="cuda", dtype=torch.float16)
    torch.ops.decode_kernels.gemm_tn(c_wide[:, :80], a2, b, None)
    assert_max_abs(c_wide[:, :80], gemm_f32(a2, b), torch.float16)
    assert torch.count_nonzero(c_wide[:, 80:]) == 0


@pytest.mark.parametrize("M", [37, 300])
def test_gemm_odd_ldc_and_row_strides(M):
    """C rows of odd stride (no 8-byte stores) and A/B rows padded past K."""
    g = torch.Generator(device="cuda").manual_seed(M)
    a_buf = torch.randn(M, 264, generator=g, device="cuda", dtype=torch.bfloat16)
    b_buf = torch.randn(150, 272, generator=g, device="cuda", dtype=torch.bfloat16) / 16
    a, b = a_buf[:, :200], b_buf[:, :200]
    c_buf = torch.full((M, 153), 3.0, device="cuda", dtype=torch.bfloat16)
    torch.ops.decode_kernels.gemm_tn(c_buf[:, :150], a, b, None)
    assert_max_abs(c_buf[:, :150], gemm_f32(a, b), torch.bfloat16, f"gemm M={M} ldc=153")
    assert (c_buf[:, 150:] == 3.0).all()


def test_gemm_rejects_unaligned_k():
    a = torch.randn(4, 100, device="cuda", dtype=torch.float16)
    b = torch.randn(8, 100, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        dk.gemm(a, b)


# ---------------------------------------------------------------------------
# RMSNorm / fused add / SiLU-and-mul: <= 1 ulp, residual exact
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,H", [(1, 4096), (33, 5120), (7, 8), (4, 100), (128, 8192), (64, 4096), (2, 40000)])
def test_rms_norm(dtype, rows, H):
    x = torch.randn(rows, H, device="cuda", dtype=dtype)
    w = torch.randn(H, device="cuda", dtype=dtype)
    assert_ulp(dk.rms_norm(x, w, 1e-6), rms_norm_reference(x.cpu(), w.cpu(), 1e-6), what=f"rms_norm {rows}x{H}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,H", [(1, 4096), (17, 2048), (5, 100), (64, 4096), (128, 8192), (2, 16384), (3, 40000)])
def test_fused_add_rms_norm(dtype, rows, H):
    x = torch.randn(rows, H, device="cuda", dtype=dtype)
    r = torch.randn(rows, H, device="cuda", dtype=dtype)
    w = (1 + 0.1 * torch.randn(H, device="cuda")).to(dtype)
    ref_out, ref_res = fused_add_rms_norm_reference(x.cpu(), r.cpu(), w.cpu(), 1e-5)
    out, res = dk.fused_add_rms_norm(x.clone(), r.clone(), w, 1e-5)
    assert torch.equal(res.cpu(), ref_res), "residual must be bit-exact"
    assert_ulp(out, ref_out, what="fused_add_rms_norm")


def test_rms_norm_3d_and_strided_rows():
    x = torch.randn(2, 5, 1024, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(1024, device="cuda", dtype=torch.bfloat16)
    assert_ulp(dk.rms_norm(x, w), rms_norm_reference(x.cpu(), w.cpu()))
    wide = torch.randn(6, 1536, device="cuda", dtype=torch.bfloat16)
    xs = wide[:, :1024]
    assert_ulp(dk.rms_norm(xs, w), rms_norm_reference(xs.cpu(), w.cpu()))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,d", [(1, 14336), (64, 11008), (3, 100), (9, 8), (64, 14336)])
def test_silu_and_mul(dtype, rows, d):
    x = torch.randn(rows, 2 * d, device="cuda", dtype=dtype) * 3
    assert_ulp(dk.silu_and_mul(x), silu_and_mul_reference(x.cpu()), what=f"silu_and_mul {rows}x{d}")


def test_empty_and_zero_row_inputs_are_no_ops():
    w = torch.randn(64, device="cuda", dtype=torch.float16)
    assert dk.rms_norm(torch.empty(0, 64, device="cuda", dtype=torch.float16), w).shape == (0, 64)
    assert dk.silu_and_mul(torch.empty(0, 128, device="cuda", dtype=torch.float16)).shape == (0, 64)
    assert dk.gemm(torch.empty(0, 64, device="cuda", dtype=torch.float16), torch.randn(8, 64, device="cuda", dtype=torch.float16)).shape == (0, 8)
    q = torch.empty(0, 4, 64, device="cuda", dtype=torch.float16)
    kv = make_paged_kv([1], 1, 64, 16, torch.float16, "cuda")
    assert dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=0).shape == (0, 4, 64)


def test_ops_work_under_torch_compile():
    """The fake implementations let torch.compile trace the mutating ops."""
    w = torch.randn(256, device="cuda", dtype=torch.float16)

    @torch.compile(fullgraph=True)
    def f(x):
        out = torch.empty_like(x)
        torch.ops.decode_kernels.rms_norm(out, x, w, 1e-6)
        return out * 2

    x = torch.randn(4, 256, device="cuda", dtype=torch.float16)
    assert_ulp(f(x), (rms_norm_reference(x.cpu(), w.cpu()).float() * 2).half())
