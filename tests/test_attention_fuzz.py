"""Seeded random shapes through paged_attention_decode, against the fp32
reference at the parity bar: KV-head counts that do and do not divide the
resident grid (1, 2, 3, 4, 5, 8, 16), GQA groups 1-16, every head dim, block
sizes that split tiles, NHD / HND / vLLM caches, 16-bit and fp8 caches,
ragged lengths with empty sequences, and every split-K schedule (automatic or
forced) with the balanced schedule's lockstep grouping on, off or at its
default. Empty sequences must give zeros."""

import random

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd.testing import make_paged_kv
from parity import assert_max_abs, attention_f32

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _cases(count=40, seed=77):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        hkv = rng.choice([1, 2, 3, 4, 5, 8, 16])
        group = rng.choice([1, 2, 3, 4, 7, 8, 16])
        d = rng.choice([64, 96, 128, 192, 256])
        fp8 = d % 64 == 0 and rng.random() < 0.3
        bs = rng.choice([8, 16, 16, 32, 48])
        layout = rng.choice(["nhd", "hnd", "vllm"])
        S = rng.randint(1, 40)
        mode = rng.random()
        lens = []
        for _ in range(S):
            if rng.random() < 0.1:
                lens.append(0)
            elif mode < 0.5:
                lens.append(rng.randint(1, 6000))
            else:
                lens.append(rng.choice([1, 15, 16, 17, 511, 512, 513, 1023, 1024, 1025, 4096]))
        if max(lens) == 0:
            lens[0] = 1
        schedule = rng.choice(["auto", "grid", "balanced", "partitions"])
        lockstep = rng.choice([None, "0", "1"])
        dtype = rng.choice([torch.float16, torch.bfloat16])
        out.append((hkv, group, d, fp8, bs, layout, lens, schedule, lockstep, dtype))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_random_attention_shapes(case, monkeypatch):
    hkv, group, d, fp8, bs, layout, lens, schedule, lockstep, dtype = CASES[case]
    what = (f"case {case}: {len(lens)} seqs up to {max(lens)}, {hkv} KV heads x group {group}, D={d}, bs={bs}, "
            f"{layout}, {'fp8' if fp8 else '16-bit'} cache, {dtype}, schedule {schedule}, lockstep {lockstep}")
    print(what, flush=True)
    if schedule != "auto":
        monkeypatch.setenv("DK_ATTN_SCHEDULE", schedule)
    if lockstep is not None:
        monkeypatch.setenv("DK_ATTN_LOCKSTEP", lockstep)
    kv = make_paged_kv(lens, hkv, d, bs, FP8 if fp8 else dtype, "cuda", layout=layout, seed=case)
    g = torch.Generator(device="cuda").manual_seed(1000 + case)
    q = torch.randn(len(lens), hkv * group, d, generator=g, device="cuda", dtype=dtype) * d**-0.5
    scales = dict(k_scale=0.5, v_scale=0.75) if fp8 else {}
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, **scales)
    torch.cuda.synchronize()
    k = kv.k_cache.float() * 0.5 if fp8 else kv.k_cache
    v = kv.v_cache.float() * 0.75 if fp8 else kv.v_cache
    assert_max_abs(out, attention_f32(q, k, v, kv.block_tables, kv.seq_lens), dtype, what)
    empty = torch.tensor(lens, device="cuda") == 0
    assert (out[empty] == 0).all(), f"{what}: empty sequences must give zeros"
