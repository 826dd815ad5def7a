"""GPU parity of paged_attention_decode at the benchmark configurations' full sizes.

* C2 -- the Llama-3-8B batch-64 decode: 64 sequences, lengths U[512, 4096]
  (the benchmark's seed), 32 query / 8 KV heads, head_dim 128, block 16,
  vLLM's interleaved cache, bf16; every sequence against the CPU oracle.
* C3 -- 128K-token contexts, batch 4, fp16, HND cache, 1% of K/V rows scaled
  by 8; every sequence against the CPU oracle (one at a time).
* C3 -- the same at batch 1 (one 128K context, 8 KV streams): under the
  balanced schedule with one workgroup per share each stream is cut into one
  piece per share, so the reduce merges more than 64 workspace rows per
  query head (asserted from the workspace contents).
* C5 -- the head-dim-256 / group-8 stress batch: 256 sequences with
  log-uniform lengths in [1, 32768] and 8 empty ones, 16 query / 2 KV heads,
  block 32, bf16 and fp16; every sequence against the CPU oracle. The NHD
  cache is contiguous in one case per dtype and, as BASELINE.json's C5
  states, a strided view in the other: [blocks, 32, 2, 256 + 64][..., :256]
  (token and block strides padded by 64 elements per head row).

The oracle bar is the same as the small-size tests (``tests/parity.py``).
Two properties that hold exactly at any size are checked on top: permuting
the physical cache blocks (and the block table with them) leaves the output
unchanged bit for bit, and doubling V (exact in bf16 / fp16) doubles it bit
for bit wherever the output is a normal number (subnormal outputs round on a
fixed grid, so round(2x) and 2 round(x) may differ there by one spacing).
All three split-K schedules (1024-token grid units, balanced shares, 512-token
partitions) run on every configuration, the balanced one both with its default
grouping (lockstep groups of KV heads for 16-bit caches) and with one
workgroup per share (``balanced-plain``).
"""

import math

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd.testing import make_paged_kv
from parity import assert_max_abs, attention_f32

pytestmark = pytest.mark.gpu


def _llama_lens():
    g = torch.Generator().manual_seed(0)
    return torch.randint(512, 4097, (64,), generator=g).tolist()


def _stress_lens(num_seqs=256, seed=5):
    g = torch.Generator().manual_seed(seed)
    lens = torch.exp(torch.rand(num_seqs, generator=g) * math.log(32768)).long().clamp(1, 32768)
    lens[torch.randperm(num_seqs, generator=g)[:8]] = 0
    return lens.tolist()


def _q(n, hq, d, dtype, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(n, hq, d, generator=g, device="cuda", dtype=dtype) * scale


def _outliers(kv, frac, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    rows = torch.rand(kv.k_cache.shape[0], kv.k_cache.shape[1], kv.k_cache.shape[2], 1, generator=g, device="cuda")
    scale = torch.where(rows < frac, 8.0, 1.0).to(kv.k_cache.dtype)
    kv.k_cache.mul_(scale)
    kv.v_cache.mul_(scale)


def _padded_nhd(kv, pad):
    """The same cache as a strided NHD view: rows of head_dim + pad elements,
    the first head_dim of them used."""
    nb, bs, hkv, d = kv.k_cache.shape
    k = torch.empty(nb, bs, hkv, d + pad, dtype=kv.k_cache.dtype, device="cuda").fill_(float("nan"))
    v = torch.empty_like(k).fill_(float("nan"))
    k[..., :d] = kv.k_cache
    v[..., :d] = kv.v_cache
    kv.k_cache, kv.v_cache = k[..., :d], v[..., :d]
    assert not kv.k_cache.is_contiguous() and kv.k_cache.stride(1) == hkv * (d + pad)


def _workspace_rows(exp_sums):
    """Rows filled per (sequence, query head) in a workspace that started as
    NaN: rows 0 .. n-1 hold pieces, row n (if any) is marked empty (exp-sum 0)."""
    es = exp_sums.cpu()
    filled = ~torch.isnan(es) & (es != 0)
    return torch.cumprod(filled.to(torch.int32), dim=-1).sum(dim=-1)


def _run(q, kv, **kw):
    return dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens,
                                     max_seq_len=kv.max_seq_len, **kw)


def _permuted(kv, seed):
    """The same cache with its physical blocks moved: block b goes to perm[b]."""
    nb = kv.k_cache.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).cuda()
    k = torch.empty_like(kv.k_cache)
    v = torch.empty_like(kv.v_cache)
    k[perm] = kv.k_cache
    v[perm] = kv.v_cache
    bt = perm.to(torch.int32)[kv.block_tables.long()]
    return k, v, bt


CONFIGS = {
    "c2_llama3_8b_b64": dict(lens=_llama_lens, hq=32, hkv=8, d=128, bs=16, dtype=torch.bfloat16, layout="vllm",
                             q_scale=128**-0.5, outlier=0.0),
    "c3_128k_b1": dict(lens=lambda: [131072], hq=32, hkv=8, d=128, bs=16, dtype=torch.float16, layout="hnd",
                       q_scale=1.0, outlier=0.01, min_rows=64),
    "c3_128k_b4": dict(lens=lambda: [131072] * 4, hq=32, hkv=8, d=128, bs=16, dtype=torch.float16, layout="hnd",
                       q_scale=1.0, outlier=0.01),
    "c5_stress_bf16": dict(lens=_stress_lens, hq=16, hkv=2, d=256, bs=32, dtype=torch.bfloat16, layout="nhd",
                           q_scale=1.0, outlier=0.0),
    "c5_stress_bf16_strided": dict(lens=_stress_lens, hq=16, hkv=2, d=256, bs=32, dtype=torch.bfloat16,
                                   layout="nhd", q_scale=1.0, outlier=0.0, pad=64),
    "c5_stress_fp16": dict(lens=_stress_lens, hq=16, hkv=2, d=256, bs=32, dtype=torch.float16, layout="nhd",
                           q_scale=1.0, outlier=0.0),
    "c5_stress_fp16_strided": dict(lens=_stress_lens, hq=16, hkv=2, d=256, bs=32, dtype=torch.float16,
                                   layout="nhd", q_scale=1.0, outlier=0.0, pad=64),
}


@pytest.fixture(scope="module", params=list(CONFIGS))
def case(request):
    c = CONFIGS[request.param]
    lens = c["lens"]()
    kv = make_paged_kv(lens, c["hkv"], c["d"], c["bs"], c["dtype"], "cuda", layout=c["layout"], seed=7)
    if c["outlier"]:
        _outliers(kv, c["outlier"], seed=8)
    if c.get("pad"):
        _padded_nhd(kv, c["pad"])
    q = _q(len(lens), c["hq"], c["d"], c["dtype"], seed=9, scale=c["q_scale"])
    ref = attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    yield request.param, c, kv, q, ref
    del kv, q, ref
    torch.cuda.empty_cache()


@pytest.mark.parametrize("schedule", ["grid", "balanced", "balanced-plain", "partitions"])
def test_full_size_against_oracle(case, schedule, monkeypatch):
    name, c, kv, q, ref = case
    monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule.split("-")[0])
    if schedule == "balanced-plain":
        monkeypatch.setenv("DK_ATTN_LOCKSTEP", "0")
    ws = dk.alloc_workspace(q.shape[0], q.shape[1], q.shape[2], kv.max_seq_len, "cuda")
    for t in ws:
        t.fill_(float("nan"))  # every row the reduce reads must have been written by this call
    out = _run(q, kv, workspace=ws)
    again = _run(q, kv)
    torch.cuda.synchronize()
    assert torch.equal(out, again), f"{name}: {schedule} schedule is not deterministic"
    assert_max_abs(out, ref, c["dtype"], f"{name} ({schedule})")
    empty = kv.seq_lens == 0
    assert (out[empty] == 0).all(), f"{name}: empty sequences must give zeros"
    if schedule == "balanced-plain" and c.get("min_rows"):
        rows = int(_workspace_rows(ws[2]).max())
        assert rows > c["min_rows"], f"{name}: the longest stream spans {rows} workspace rows (> {c['min_rows']} expected)"


def test_full_size_block_placement_and_v_linearity(case):
    name, c, kv, q, _ = case
    out = _run(q, kv)
    k2, v2, bt2 = _permuted(kv, seed=10)
    moved = dk.paged_attention_decode(q, k2, v2, bt2, kv.seq_lens, max_seq_len=kv.max_seq_len)
    del k2, v2
    doubled = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache * 2, kv.block_tables, kv.seq_lens,
                                        max_seq_len=kv.max_seq_len)
    torch.cuda.synchronize()
    assert torch.equal(moved, out), f"{name}: output depends on where the blocks live"
    # Rounding commutes with doubling for normal outputs; below the smallest
    # normal (fp16: 6.1e-5, hit by long contexts) round(2x) and 2 round(x) may
    # differ by one subnormal spacing.
    fi = torch.finfo(c["dtype"])
    normal = out.abs() >= fi.tiny
    assert torch.equal(doubled[normal], out[normal] * 2), f"{name}: doubling V does not double the output exactly"
    sub_gap = (doubled[~normal].float() - 2 * out[~normal].float()).abs()
    assert sub_gap.numel() == 0 or sub_gap.max().item() <= fi.tiny * fi.eps, f"{name}: subnormal outputs off by > 1 ulp"
