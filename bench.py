"""Benchmark of the decode hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras]

Headline (``value``): paged decode attention on the Llama-3-8B batch-64 shape
64 sequences, 32 query / 8 KV heads, head_dim 128,
block_size 16, lengths ~ U[512, 4096] (seed 0), vLLM's interleaved K|V cache,
bf16. A step is one ``paged_attention_decode`` call over the whole batch with
preallocated output and split-K workspace; W untimed steps, then K timed steps
between device synchronisations. ``value`` is algorithmic HBM bytes (every K
and V row once, plus q and out) per second, in TB/s. Every timed op, headline
and extras, is first compared with the oracle (or, for the large GEMMs, an
fp32 GEMM) and the bench stops if one is off.

``value`` and ``roofline`` use the median of the K timed calls, each from cold
caches (1 GiB read before the call, outside its HIP-event interval; events on
torch's current stream, the one the kernels run on), against the 8 TB/s HBM
peak; the mean of K back-to-back calls is reported beside it. ``cpu_baseline``: the oracle (the reference's CPU path,
restated in ``oracle/reference.py``) timed on this host's cores over a bounded
sample of the same workload; the GPU output is checked against it on that
sample before anything is reported.

Each extra also carries ``cpu_path``: the reference's CPU path for that op
(the oracle, torch on all host cores) timed in the same run on the same inputs
(attention: the sequences checked before timing; GEMM: one to three calls;
norms: eleven), with the thread count -- skipped with ``--no-cpu``.

``extras``: the other BASELINE configs -- 128K-token split-K decode (fp16,
batch 1 and 4, HND cache, 1% outlier rows), the head-dim-256 / group-8 stress
batch, gemm_tn at the decode-layer shapes next to hipBLASLt (``F.linear``; the
two timed interleaved, call by call, so that drift moves both alike),
the norm / activation ops, and one Llama-3-8B decoder layer's decode step
end to end, RoPE and the cache write included (eager and HIP graph) -- each op timed as the median of cold-cache calls
(a 1 GiB buffer is read before every call, 4x the 256 MB Infinity
Cache).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch
import torch.nn.functional as F

import decodekernels_amd as dk

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FLUSH_BYTES = 1 << 30


# ---------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------
def paged_cache_on_device(seq_lens, num_kv_heads, head_dim, block_size, dtype, layout, seed, outlier_frac=0.0):
    """Seeded paged KV cache built on the GPU (same layouts and block-table
    rules as ``decodekernels_amd.testing.make_paged_kv``, without a host round trip)."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    nblk = [-(-n // block_size) for n in seq_lens]
    num_blocks = sum(nblk) + 3
    fp8 = dtype == torch.float8_e4m3fn

    def randn(*shape):  # fp8: N(0, 1) drawn in fp16, rounded to e4m3fn
        x = torch.randn(*shape, generator=g, device=dev, dtype=torch.float16 if fp8 else dtype)
        return x.to(dtype) if fp8 else x

    if layout == "vllm":
        kv = randn(num_blocks, num_kv_heads, block_size, 2 * head_dim)
        k, v = kv.transpose(1, 2).split(head_dim, dim=-1)
    elif layout == "hnd":
        k = randn(num_blocks, num_kv_heads, block_size, head_dim).transpose(1, 2)
        v = randn(num_blocks, num_kv_heads, block_size, head_dim).transpose(1, 2)
    else:
        k = randn(num_blocks, block_size, num_kv_heads, head_dim)
        v = randn(num_blocks, block_size, num_kv_heads, head_dim)
    if outlier_frac > 0 and not fp8:
        rows = torch.rand(num_blocks, block_size, num_kv_heads, 1, generator=g, device=dev) < outlier_frac
        scale = torch.where(rows, 8.0, 1.0).to(dtype)
        k.mul_(scale)
        v.mul_(scale)
    perm = torch.randperm(num_blocks, generator=g, device=dev).to(torch.int32)
    width = max(max(nblk), 1)
    bt = torch.zeros(len(seq_lens), width, dtype=torch.int32, device=dev)
    off = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[off : off + n]
        off += n
    lens = torch.tensor(seq_lens, dtype=torch.int32, device=dev)
    return k, v, bt, lens


def attention_case(num_seqs, hq, hkv, d, bs, seq_lens, dtype, layout, seed, q_scale=1.0, outlier_frac=0.0,
                   kv_dtype=None, k_scale=1.0, v_scale=1.0, nhd_pad=0):
    """kv_dtype: the cache's element type (default: dtype); torch.float8_e4m3fn
    runs the fp8-cache op with the given scales. nhd_pad > 0: the NHD cache is
    a strided view whose head rows are nhd_pad elements longer than head_dim."""
    kv_dtype = kv_dtype or dtype
    k, v, bt, lens = paged_cache_on_device(seq_lens, hkv, d, bs, kv_dtype, layout, seed, outlier_frac)
    if nhd_pad:
        assert layout == "nhd"
        kp = torch.empty(*k.shape[:3], d + nhd_pad, dtype=k.dtype, device=k.device)
        vp = torch.empty_like(kp)
        kp[..., :d], vp[..., :d] = k, v
        k, v = kp[..., :d], vp[..., :d]
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    q = torch.randn(num_seqs, hq, d, generator=g, device="cuda", dtype=dtype) * q_scale
    max_len = max(seq_lens)
    out = torch.empty_like(q)
    ws = dk.alloc_workspace(num_seqs, hq, d, max_len, "cuda")
    elt = torch.finfo(dtype).bits // 8
    kv_elt = torch.finfo(kv_dtype).bits // 8
    nbytes = sum(seq_lens) * 2 * hkv * d * kv_elt + 2 * q.numel() * elt
    scales = dict(k_scale=k_scale, v_scale=v_scale) if kv_dtype == torch.float8_e4m3fn else {}

    def run():
        dk.paged_attention_decode(q, k, v, bt, lens, max_seq_len=max_len, out=out, workspace=ws, **scales)

    return dict(q=q, k=k, v=v, bt=bt, lens=lens, out=out, run=run, bytes=nbytes, seq_lens=seq_lens, dtype=dtype,
                k_scale=k_scale, v_scale=v_scale)


def rope_table(max_position, rot_dim, base=500000.0):
    """[max_position, rot_dim] float32 cos | sin table, theta_i = base^(-2i / rot_dim)."""
    inv_freq = base ** (-torch.arange(0, rot_dim, 2, dtype=torch.float64, device="cuda") / rot_dim)
    ang = torch.arange(max_position, dtype=torch.float64, device="cuda")[:, None] * inv_freq[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1).float()


def llama3_8b_decode_case():
    g = torch.Generator().manual_seed(0)
    seq_lens = torch.randint(512, 4097, (64,), generator=g).tolist()
    return attention_case(64, 32, 8, 128, 16, seq_lens, torch.bfloat16, "vllm", seed=0, q_scale=128**-0.5)


def progress(msg: str) -> None:
    """One line per finished stage on stderr (stdout carries only the JSON line)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
_FLUSH: torch.Tensor | None = None


def flush_caches() -> None:
    """Reads 1 GiB (4x the Infinity Cache) so the next call starts cold. A read,
    not a write: dirty lines left behind would be written back during the call."""
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.ones(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    torch.amax(_FLUSH)


def time_back_to_back(fn, steps: int, warmup: int) -> float:
    """Mean ms per call over `steps` back-to-back calls, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_cold(fn, iters: int = 30, warmup: int = 3) -> dict:
    """Median / p10 / p90 / mean microseconds of single calls, caches flushed
    before each (the flush is outside the timed interval)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        flush_caches()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    us = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))
    return {"median_us": round(statistics.median(us), 2), "p10_us": round(us[int(0.1 * (iters - 1))], 2),
            "p90_us": round(us[int(0.9 * (iters - 1))], 2), "mean_us": round(statistics.fmean(us), 2)}


def time_cold_interleaved(fns: dict, iters: int = 30, warmup: int = 3) -> dict:
    """time_cold for several ops at once, the calls interleaved (one call of
    each per round, caches flushed before each), so that clock or thermal
    drift during the run moves every op's figures alike. Returns
    {name: time_cold-style stats}."""
    for _ in range(warmup):
        for fn in fns.values():
            fn()
    torch.cuda.synchronize()
    events = {name: [] for name in fns}
    for _ in range(iters):
        for name, fn in fns.items():
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            flush_caches()
            s.record()
            fn()
            e.record()
            events[name].append((s, e))
    torch.cuda.synchronize()
    out = {}
    for name, lst in events.items():
        us = sorted(s.elapsed_time(e) * 1e3 for s, e in lst)
        out[name] = {"median_us": round(statistics.median(us), 2), "p10_us": round(us[int(0.1 * (iters - 1))], 2),
                     "p90_us": round(us[int(0.9 * (iters - 1))], 2), "mean_us": round(statistics.fmean(us), 2)}
    return out


# ---------------------------------------------------------------------------
# Correctness before timing: every timed op is first compared with the oracle
# ---------------------------------------------------------------------------
# Whether the extras also time the reference's CPU path (off with --no-cpu).
CPU_PATH = True


def cpu_threads() -> int:
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_entry(seconds: float, calls: int, what: str, nbytes: float = 0.0, flops: float = 0.0) -> dict:
    """The reference's CPU path (the oracle, torch on the host's cores) on the
    same op: microseconds per call and the matching rate."""
    us = seconds / calls * 1e6
    out = {"us_per_call": round(us, 1), "threads": torch.get_num_threads(), "sample": what}
    if nbytes:
        out["GB/s"] = round(nbytes / (us * 1e-6) / 1e9, 2)
    if flops:
        out["TFLOP/s"] = round(flops / (us * 1e-6) / 1e12, 3)
    return out


def time_cpu(fn, calls: int, warmup: int = 1) -> float:
    """Median seconds of `calls` host calls after `warmup` untimed ones."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(calls):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def check_attention(c, what: str, sample: int = 4, cpu: dict | None = None) -> float:
    """Runs the case once and compares up to `sample` sequences (the longest
    first) with the CPU oracle at the parity bar (2e-2 bf16 / 5e-3 fp16, or
    half an ulp where that is larger). Returns the max abs error. With `cpu` a
    dict, the oracle calls are timed there too (the reference's CPU path on
    those sequences: seconds, algorithmic bytes, sequences)."""
    from oracle.reference import paged_attention_reference

    c["run"]()
    torch.cuda.synchronize()
    lens = c["lens"].cpu()
    order = sorted(range(len(c["seq_lens"])), key=lambda s: -c["seq_lens"][s])[:sample]
    k, v = c["k"], c["v"]

    def gather(t, blocks, scale):  # this sequence's cache blocks, dequantised, on the host
        if t.dtype == torch.float8_e4m3fn:
            return (t.view(torch.uint8)[blocks].view(torch.float8_e4m3fn).float() * scale).cpu()
        return t[blocks].float().cpu()

    worst = 0.0
    for s in order:
        blocks = c["bt"][s, : -(-c["seq_lens"][s] // k.shape[1])].long()
        ks, vs = gather(k, blocks, c["k_scale"]), gather(v, blocks, c["v_scale"])
        bt = torch.arange(blocks.numel(), dtype=torch.int32)[None]
        qs = c["q"][s : s + 1].float().cpu()
        t0 = time.perf_counter()
        ref = paged_attention_reference(qs, ks, vs, bt, lens[s : s + 1])[0]
        if cpu is not None:
            cpu["s"] = cpu.get("s", 0.0) + time.perf_counter() - t0
            cpu["bytes"] = cpu.get("bytes", 0) + (int(lens[s]) * 2 * k.shape[2] * k.shape[3] * k.element_size()
                                                  + 2 * c["q"].shape[1] * c["q"].shape[2] * c["q"].element_size())
            cpu["seqs"] = cpu.get("seqs", 0) + 1
        got = c["out"][s].float().cpu()
        err = (got - ref).abs()
        bar = half_ulp_bar(ref, c["dtype"])
        if (err > bar).any():
            raise AssertionError(f"{what}: sequence {s} differs from the oracle by {err.max().item():.3e} before timing")
        worst = max(worst, err.max().item())
    return worst


def half_ulp_bar(ref_f32: torch.Tensor, dtype) -> torch.Tensor:
    """max(2e-2 bf16 / 5e-3 fp16, half an ulp of dtype at |ref|), elementwise."""
    a = ref_f32.abs().to(dtype)
    half = 0.5 * (torch.nextafter(a, torch.full_like(a, float("inf"))) - a).float()
    return half.clamp(min=2e-2 if dtype == torch.bfloat16 else 5e-3)


def check_gemm(out: torch.Tensor, a: torch.Tensor, w: torch.Tensor, bias=None, what: str = "gemm") -> float:
    """gemm_tn's output against an fp32 GEMM of the same inputs (the oracle's
    formula, on the GPU for speed) at the parity bar of the tests: max(2e-2
    bf16 / 5e-3 fp16, half an ulp) plus the fp32 accumulation-order slack
    2^-23 sqrt(K) (|A| |W|^T + |bias|). Returns the max abs error."""
    af, wf = a.float(), w.float()
    ref = af @ wf.t()
    slack = af.abs() @ wf.abs().t()
    if bias is not None:
        ref = ref + bias.float()
        slack = slack + bias.float().abs()
    err = (out.float() - ref).abs()
    tol = half_ulp_bar(ref, out.dtype) + slack * (2.0**-23 * a.shape[-1] ** 0.5)
    if (err > tol).any():
        raise AssertionError(f"{what}: differs from an fp32 GEMM by {err.max().item():.3e} (over the bar) before timing")
    worst = err.max().item()
    del ref, slack, err, tol
    return worst


def ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    """Max distance in units in the last place between two 16-bit float tensors."""
    def key(t):
        bits = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        return torch.where(bits >= 0x8000, -(bits & 0x7FFF), bits & 0x7FFF)

    return int((key(a.cpu()) - key(b.cpu())).abs().max().item())


# ---------------------------------------------------------------------------
# Extras
# ---------------------------------------------------------------------------
def attention_cpu_path(cpu: dict, num_seqs: int, fp8: bool = False) -> dict:
    """The `cpu_path` entry of an attention extra from check_attention's timing."""
    if not cpu:
        return {}
    what = (f"oracle.reference.paged_attention_reference (torch CPU, fp32) on the {cpu['seqs']} longest of "
            f"{num_seqs} sequences, one call each ({cpu['bytes'] / 1e6:.0f} MB of "
            f"{'fp8' if fp8 else '16-bit'} KV; the reference has no fp8 path, so its input is the dequantised "
            "cache)" if fp8 else f"oracle.reference.paged_attention_reference (torch CPU, fp32) on the {cpu['seqs']} "
            f"longest of {num_seqs} sequences, one call each ({cpu['bytes'] / 1e6:.0f} MB of KV)")
    entry = cpu_entry(cpu["s"], cpu["seqs"], what, nbytes=cpu["bytes"] / cpu["seqs"])
    entry["us_per_sequence"] = entry.pop("us_per_call")
    return {"cpu_path": entry}


def extras_attention() -> dict:
    res = {}
    for b in (1, 4):
        c = attention_case(b, 32, 8, 128, 16, [131072] * b, torch.float16, "hnd", seed=10 + b, outlier_frac=0.01)
        cpu = {}
        err = check_attention(c, f"128K batch {b}", sample=1, cpu=cpu if CPU_PATH else None)
        t = time_cold(c["run"], iters=20)
        gbs = c["bytes"] / (t["median_us"] * 1e-6) / 1e9
        res[f"split_k_128k_b{b}_fp16"] = {**t, "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                                           "MB": round(c["bytes"] / 1e6, 1), "checked_max_abs_err": err,
                                           **attention_cpu_path(cpu, len(c["seq_lens"]))}
        progress(f"128K batch {b}: {t['median_us']} us (checked, max abs err {err:.2e})")
        del c
    lens = c5_seq_lens()
    for dtype, tag in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        c = attention_case(256, 16, 2, 256, 32, lens, dtype, "nhd", seed=20, nhd_pad=64)
        cpu = {}
        err = check_attention(c, f"D=256 stress {tag}", cpu=cpu if CPU_PATH else None)
        t = time_cold(c["run"], iters=20)
        gbs = c["bytes"] / (t["median_us"] * 1e-6) / 1e9
        res[f"d256_g8_stress_{tag}"] = {**t, "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                                        "MB": round(c["bytes"] / 1e6, 1), "checked_max_abs_err": err,
                                        "kv_layout": "strided NHD [blocks, 32, 2, 256 + 64][..., :256]",
                                        **attention_cpu_path(cpu, len(c["seq_lens"]))}
        progress(f"D=256 stress {tag}: {t['median_us']} us (checked, max abs err {err:.2e})")
        del c
    # fp8 (e4m3fn) KV cache, bf16 queries: the headline batch (vLLM cache, and
    # the reference's default NHD cache, which takes the 1024-token grid) and
    # 128K batch 1 (half the bytes of the 16-bit cache; GB/s counts the fp8 bytes).
    llama_lens = torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    for name, args in (("fp8_kv_llama3_8b_b64", (64, 32, 8, 128, 16, llama_lens, torch.bfloat16, "vllm")),
                       ("fp8_kv_llama3_8b_b64_nhd", (64, 32, 8, 128, 16, llama_lens, torch.bfloat16, "nhd")),
                       ("fp8_kv_128k_b1", (1, 32, 8, 128, 16, [131072], torch.bfloat16, "hnd"))):
        c = attention_case(*args, seed=60, q_scale=128**-0.5, kv_dtype=torch.float8_e4m3fn, k_scale=0.5, v_scale=0.5)
        cpu = {}
        err = check_attention(c, name, sample=1 if len(args[5]) == 1 else 4, cpu=cpu if CPU_PATH else None)
        t = time_cold(c["run"], iters=20)
        gbs = c["bytes"] / (t["median_us"] * 1e-6) / 1e9
        res[name] = {**t, "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
                     "MB": round(c["bytes"] / 1e6, 1), "checked_max_abs_err": err,
                     **attention_cpu_path(cpu, len(c["seq_lens"]), fp8=True)}
        progress(f"{name}: {t['median_us']} us (checked, max abs err {err:.2e})")
        del c
    return res


def extras_gemm() -> dict:
    from oracle.reference import gemm_reference

    torch.backends.cuda.preferred_blas_library("cublaslt")  # hipBLASLt on ROCm
    res = {}
    g = torch.Generator(device="cuda").manual_seed(30)
    ms = (1, 8, 32, 64, 256, 4096)
    for name, n, k in (("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)):
        w = torch.randn(n, k, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
        w_c = w.cpu() if CPU_PATH else None
        for m in ms:
            a = torch.randn(m, k, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
            out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
            torch.ops.decode_kernels.gemm_tn(out, a, w, None)
            err = check_gemm(out, a, w, what=f"gemm {name} M={m}")
            iters = 10 if m == 4096 else 30
            t = time_cold_interleaved({"dk": lambda: torch.ops.decode_kernels.gemm_tn(out, a, w, None),
                                       "hipblaslt": lambda: F.linear(a, w)}, iters=iters)
            t_dk, t_bl = t["dk"], t["hipblaslt"]
            flops = 2.0 * m * n * k
            nbytes = (m * k + n * k + m * n) * 2
            res[f"{name}_M{m}"] = {
                "dk_us": t_dk["median_us"], "hipblaslt_us": t_bl["median_us"],
                "dk_over_hipblaslt": round(t_dk["median_us"] / t_bl["median_us"], 3),
                "TFLOP/s": round(flops / (t_dk["median_us"] * 1e-6) / 1e12, 1),
                "GB/s": round(nbytes / (t_dk["median_us"] * 1e-6) / 1e9, 1),
                "checked_max_abs_err": err,
            }
            if CPU_PATH:
                a_c = a.cpu()
                calls = 1 if m == 4096 else 3
                sec = time_cpu(lambda: gemm_reference(a_c, w_c), calls, warmup=0 if m == 4096 else 1)
                res[f"{name}_M{m}"]["cpu_path"] = cpu_entry(
                    sec, 1, f"oracle.reference.gemm_reference (torch CPU, fp32 F.linear on the bf16 inputs), median "
                    f"of {calls} call{'s' if calls > 1 else ''}", nbytes=nbytes, flops=flops)
            if m == 4096:
                res[f"{name}_M{m}"]["pct_mfma_peak"] = round(100 * res[f"{name}_M{m}"]["TFLOP/s"] / BF16_PEAK_TFLOPS, 1)
        progress(f"gemm {name}: " + ", ".join(f"M={m} {res[f'{name}_M{m}']['dk_over_hipblaslt']}x" for m in ms))
        del w, w_c
    return res


def extras_norms() -> dict:
    g = torch.Generator(device="cuda").manual_seed(40)
    t, h, d = 64, 4096, 14336
    x = torch.randn(t, h, generator=g, device="cuda", dtype=torch.bfloat16)
    r = torch.randn(t, h, generator=g, device="cuda", dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g, device="cuda")).to(torch.bfloat16)
    out = torch.empty_like(x)
    xs = torch.randn(t, 2 * d, generator=g, device="cuda", dtype=torch.bfloat16)
    ys = torch.empty(t, d, device="cuda", dtype=torch.bfloat16)
    from oracle.reference import fused_add_rms_norm_reference, rms_norm_reference, silu_and_mul_reference

    # Checked against the oracle before timing (<= 1 ulp, fused residual bit-exact).
    torch.ops.decode_kernels.rms_norm(out, x, w, 1e-5)
    checked = {"rms_norm_64x4096": ulps(out, rms_norm_reference(x.cpu(), w.cpu(), 1e-5))}
    want_out, want_res = fused_add_rms_norm_reference(x.cpu(), r.cpu(), w.cpu(), 1e-5)
    xc, rc = x.clone(), r.clone()
    torch.ops.decode_kernels.fused_add_rms_norm(xc, rc, w, 1e-5)
    if not torch.equal(rc.cpu(), want_res):
        raise AssertionError("fused_add_rms_norm residual differs from the oracle before timing")
    checked["fused_add_rms_norm_64x4096"] = ulps(xc, want_out)
    torch.ops.decode_kernels.silu_and_mul(ys, xs)
    checked["silu_and_mul_64x2x14336"] = ulps(ys, silu_and_mul_reference(xs.cpu()))
    bad = {k: u for k, u in checked.items() if u > 1}
    if bad:
        raise AssertionError(f"norm / activation ops more than 1 ulp from the oracle before timing: {bad}")
    res = {}
    for name, fn, nbytes in (
        ("rms_norm_64x4096", lambda: torch.ops.decode_kernels.rms_norm(out, x, w, 1e-5), 2 * t * h * 2),
        ("fused_add_rms_norm_64x4096", lambda: torch.ops.decode_kernels.fused_add_rms_norm(x, r, w, 1e-5), 4 * t * h * 2),
        ("silu_and_mul_64x2x14336", lambda: torch.ops.decode_kernels.silu_and_mul(ys, xs), 3 * t * d * 2),
    ):
        tm = time_cold(fn, iters=50)
        res[name] = {**tm, "GB/s": round(nbytes / (tm["median_us"] * 1e-6) / 1e9, 1), "checked_max_ulp": checked[name]}
    if CPU_PATH:
        x_c, r_c, w_c, xs_c = x.cpu(), r.cpu(), w.cpu(), xs.cpu()
        for name, fn, nbytes, ref in (
            ("rms_norm_64x4096", lambda: rms_norm_reference(x_c, w_c, 1e-5), 2 * t * h * 2, "rms_norm_reference"),
            ("fused_add_rms_norm_64x4096", lambda: fused_add_rms_norm_reference(x_c, r_c, w_c, 1e-5), 4 * t * h * 2,
             "fused_add_rms_norm_reference"),
            ("silu_and_mul_64x2x14336", lambda: silu_and_mul_reference(xs_c), 3 * t * d * 2, "silu_and_mul_reference"),
        ):
            sec = time_cpu(fn, 11, warmup=2)
            res[name]["cpu_path"] = cpu_entry(sec, 1, f"oracle.reference.{ref} (torch CPU, fp32), median of 11 calls",
                                              nbytes=nbytes)
    return res


def c5_seq_lens(num_seqs: int = 256, seed: int = 5) -> list:
    """Log-uniform lengths in [1, 32768] with 8 zero-length sequences."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.exp(torch.rand(num_seqs, generator=g) * math.log(32768)).long().clamp(1, 32768)
    lens[torch.randperm(num_seqs, generator=g)[:8]] = 0
    return lens.tolist()


def layer_step(num_seqs, hq, hkv, d, bs, seq_lens, dtype, layout, seed, hidden=4096, inter=14336):
    """One random-init decoder layer's decode step on this path: fused_add_rms_norm
    -> qkv gemm -> rotary embedding of the q and k columns and the new token's
    k and v columns written to its cache slot (one launch,
    rotary_embedding_and_cache) -> paged attention (q read in place from the
    qkv output) -> o gemm -> fused_add_rms_norm -> gate_up gemm -> silu_and_mul
    -> down gemm. The new token is the last of each sequence (position
    len - 1). Returns the step's per-op callables, the two unfused ops the
    fused one replaces (timed for comparison only) and the bytes the step must
    move."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    kw = dict(device="cuda", dtype=dtype)
    nqkv = 6144  # Llama-3-8B's fused q|k|v projection; q is its first hq * d columns
    w_qkv = torch.randn(nqkv, hidden, generator=g, **kw) * 0.02
    w_o = torch.randn(hidden, hq * d, generator=g, **kw) * 0.02
    w_gu = torch.randn(2 * inter, hidden, generator=g, **kw) * 0.02
    w_down = torch.randn(hidden, inter, generator=g, **kw) * 0.02
    ln1 = (1 + 0.1 * torch.randn(hidden, generator=g, device="cuda")).to(dtype)
    ln2 = (1 + 0.1 * torch.randn(hidden, generator=g, device="cuda")).to(dtype)
    case = attention_case(num_seqs, hq, hkv, d, bs, seq_lens, dtype, layout, seed=seed + 1)
    x = torch.randn(num_seqs, hidden, generator=g, **kw)
    resid = torch.randn(num_seqs, hidden, generator=g, **kw)
    qkv = torch.empty(num_seqs, nqkv, **kw)
    attn = torch.empty(num_seqs, hq, d, **kw)
    o = torch.empty(num_seqs, hidden, **kw)
    gu = torch.empty(num_seqs, 2 * inter, **kw)
    act = torch.empty(num_seqs, inter, **kw)
    down = torch.empty(num_seqs, hidden, **kw)
    max_len = max(max(seq_lens), 1)
    ws = dk.alloc_workspace(num_seqs, hq, d, max_len, "cuda")
    q = qkv[:, : hq * d].view(num_seqs, hq, d)
    k_new, v_new = qkv[:, hq * d : (hq + hkv) * d], qkv[:, (hq + hkv) * d : (hq + 2 * hkv) * d]
    rope = rope_table(max_len, d)
    bt_host = case["bt"].cpu()
    positions = torch.tensor([n - 1 for n in seq_lens], device="cuda")
    slots = torch.tensor([int(bt_host[i, (n - 1) // bs]) * bs + (n - 1) % bs if n > 0 else -1
                          for i, n in enumerate(seq_lens)], device="cuda")
    dko = torch.ops.decode_kernels
    ops = {
        "fused_add_rms_norm": lambda: dko.fused_add_rms_norm(x, resid, ln1, 1e-5),
        "qkv_gemm": lambda: dko.gemm_tn(qkv, x, w_qkv, None),
        "rotary_embedding_and_cache": lambda: dko.rotary_embedding_and_cache(
            positions, qkv[:, : hq * d], k_new, v_new, d, rope, True, case["k"], case["v"], slots),
        "attention": lambda: dk.paged_attention_decode(q, case["k"], case["v"], case["bt"], case["lens"],
                                                       max_seq_len=max_len, out=attn, workspace=ws),
        "o_gemm": lambda: dko.gemm_tn(o, attn.view(num_seqs, hq * d), w_o, None),
        "fused_add_rms_norm_2": lambda: dko.fused_add_rms_norm(o, resid, ln2, 1e-5),
        "gate_up_gemm": lambda: dko.gemm_tn(gu, o, w_gu, None),
        "silu_and_mul": lambda: dko.silu_and_mul(act, gu),
        "down_gemm": lambda: dko.gemm_tn(down, act, w_down, None),
    }
    elt = torch.finfo(dtype).bits // 8
    nbytes = case["bytes"] + elt * (w_qkv.numel() + w_o.numel() + w_gu.numel() + w_down.numel())
    nbytes += num_seqs * (2 * (hq + hkv) * d * elt + d * 4 + 4 * hkv * d * elt)  # rope rows + table row, k/v copy
    unfused = {
        "rotary_embedding": lambda: dko.rotary_embedding(positions, qkv[:, : hq * d], k_new, d, rope, True),
        "cache_write": lambda: dko.reshape_and_cache(k_new, v_new, case["k"], case["v"], slots),
    }
    # The same layer with each decode GEMM fused into the op that consumes its
    # output (the split-K sum done by the consumer): qkv -> RoPE + cache write,
    # o -> post-attention norm, down -> the next layer's input norm. The step
    # starts from the normalised input (x) and leaves the next layer's in x,
    # so it runs the same ops per layer as the unfused step: 4 GEMMs, 2 norms,
    # RoPE + cache, attention, SiLU.
    fused = {
        "qkv_gemm_rotary_embedding_and_cache": lambda: dko.gemm_tn_rotary_embedding_and_cache(
            qkv, x, w_qkv, None, positions, qkv[:, : hq * d], k_new, v_new, d, rope, True, case["k"], case["v"], slots),
        "attention": ops["attention"],
        "o_gemm_add_rms_norm": lambda: dko.gemm_tn_add_rms_norm(o, attn.view(num_seqs, hq * d), w_o, None, resid, ln2,
                                                                1e-5),
        "gate_up_gemm": ops["gate_up_gemm"],
        "silu_and_mul": ops["silu_and_mul"],
        "down_gemm_add_rms_norm": lambda: dko.gemm_tn_add_rms_norm(x, act, w_down, None, resid, ln1, 1e-5),
    }

    def check_fused() -> dict:
        """One fused step against the unfused ops from the same state, bit for
        bit: norm1 -> the unfused layer -> norm1 of its down output (the next
        layer's first op) against norm1 (setup) -> the fused layer."""
        x0, r0 = x.clone(), resid.clone()
        kc0, vc0 = case["k"].clone(), case["v"].clone()
        for fn in ops.values():
            fn()
        dko.fused_add_rms_norm(down, resid, ln1, 1e-5)
        want = [t.clone() for t in (qkv, case["k"], case["v"], attn, o, gu, act, down, resid)]
        x.copy_(x0), resid.copy_(r0), case["k"].copy_(kc0), case["v"].copy_(vc0)
        for t in (qkv, attn, o, gu, act, down):
            t.fill_(float("nan"))
        ops["fused_add_rms_norm"]()
        for fn in fused.values():
            fn()
        got = [qkv, case["k"], case["v"], attn, o, gu, act, x, resid]
        torch.cuda.synchronize()
        names = ("qkv", "k_cache", "v_cache", "attention", "o_normed", "gate_up", "act", "next_layer_input", "residual")
        for name, a, b in zip(names, want, got):
            if not torch.equal(a, b):
                raise AssertionError(f"fused layer step: {name} differs from the unfused ops")
        return {"bit_identical_to_unfused": list(names)}

    def check() -> dict:
        """After one step: the stages whose inputs the rest of the step leaves
        intact, each against the oracle on its own inputs -- attention (the
        rotated q, the cache with the new token written; longest sequences),
        gate_up and down against a GPU fp32 GEMM, silu_and_mul at 1 ulp."""
        from oracle.reference import silu_and_mul_reference

        errs = {"attention": check_attention(dict(case, q=q, out=attn, run=ops["attention"]), "layer-step attention",
                                             sample=2)}
        for name, a, w, c in (("gate_up_gemm", o, w_gu, gu), ("down_gemm", act, w_down, down)):
            errs[name] = check_gemm(c, a, w, what=f"layer-step {name}")
        u = ulps(act, silu_and_mul_reference(gu.cpu()))
        if u > 1:
            raise AssertionError(f"layer-step silu_and_mul {u} ulp from the oracle")
        errs["silu_and_mul_ulp"] = u
        return errs

    return ops, unfused, fused, nbytes, check, check_fused


def extras_layer_step() -> dict:
    """The single-layer decode step timed end to end, eager
    (back to back) and as one captured HIP graph replayed back to back, next to
    the sum of its ops timed one by one from cold caches. Hidden 4096 and MLP
    14336 and the projections as Llama-3-8B (qkv N = 6144); attention at the
    head-dim-256 / group-8 stress shape (256 seqs) and at the Llama-3-8B
    batch-64 shape."""
    res = {}
    cases = (
        ("d256_g8_b256_bf16", (256, 16, 2, 256, 32, c5_seq_lens(), torch.bfloat16, "nhd")),
        ("d256_g8_b256_fp16", (256, 16, 2, 256, 32, c5_seq_lens(), torch.float16, "nhd")),
        ("llama3_8b_b64_bf16", (64, 32, 8, 128, 16, torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist(),
                                torch.bfloat16, "vllm")),
    )
    def timed(fns: dict) -> tuple[float, float, float]:
        """Eager (back to back) and HIP-graph replay time of one step, and the
        per-step time of a graph of 8 consecutive steps (8 layers): each graph
        launch starts ~8 us after the previous one ends on the device (a kernel
        trace shows the kernels inside a replay back to back), which one
        step per graph pays in full and 8 steps share."""
        def step():
            for fn in fns.values():
                fn()

        eager = time_back_to_back(step, 20, 3) * 1e3
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        replay = time_back_to_back(graph.replay, 20, 3) * 1e3
        graph8 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph8):
            for _ in range(8):
                step()
        replay8 = time_back_to_back(graph8.replay, 5, 2) * 1e3 / 8
        del graph, graph8
        return eager, replay, replay8

    for name, args in cases:
        ops, unfused, fused, nbytes, check, check_fused = layer_step(*args, seed=50)
        for fn in ops.values():
            fn()
        torch.cuda.synchronize()
        checked = check()
        checked.update(check_fused())
        per_op = {k: time_cold(fn, iters=20)["median_us"] for k, fn in ops.items()}
        fused_per_op = {k: time_cold(fn, iters=20)["median_us"] for k, fn in fused.items()
                        if k not in ("attention", "gate_up_gemm", "silu_and_mul")}
        unfused_us = {k: time_cold(fn, iters=20)["median_us"] for k, fn in unfused.items()}
        eager_us, graph_us, graph8_us = timed(fused)
        u_eager_us, u_graph_us, u_graph8_us = timed(ops)
        res[name] = {
            "eager_us": round(eager_us, 1), "graph_us": round(graph_us, 1),
            "graph_8_steps_us_per_step": round(graph8_us, 1),
            "step": "fused decode GEMMs: qkv -> rotary_embedding_and_cache, o -> post-attention norm, "
                    "down -> next layer's input norm (the split-K sums done by the consumers)",
            "unfused": {"eager_us": round(u_eager_us, 1), "graph_us": round(u_graph_us, 1),
                        "graph_8_steps_us_per_step": round(u_graph8_us, 1),
                        "step": "norm -> qkv -> rotary_embedding_and_cache -> attention -> o -> norm -> gate_up "
                                "-> silu_and_mul -> down, one op per launch"},
            "sum_of_cold_ops_us": round(sum(per_op.values()), 1), "ops_cold_us": per_op,
            "fused_ops_cold_us": fused_per_op,
            "unfused_rope_and_cache_cold_us": unfused_us,
            "weights_plus_kv_MB": round(nbytes / 1e6, 1),
            "eager_GB/s": round(nbytes / (eager_us * 1e-6) / 1e9, 1),
            "graph_GB/s": round(nbytes / (graph_us * 1e-6) / 1e9, 1),
            "checked_before_timing": checked,
        }
        progress(f"layer step {name}: fused eager {eager_us:.1f} us, graph {graph_us:.1f} us "
                 f"(8-step graph {graph8_us:.1f} us/step); unfused eager {u_eager_us:.1f} us, graph {u_graph_us:.1f} us "
                 f"(8-step graph {u_graph8_us:.1f} us/step)")
        del ops, fused
        torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# CPU baseline (the oracle on the host cores) + pre-report correctness check
# ---------------------------------------------------------------------------
def cpu_baseline_and_check(case, budget_s: float = 20.0, min_s: float = 10.0) -> dict:
    """The oracle on the host's cores over the same workload, one sequence per
    call: sequences in order until `budget_s` is spent; if the whole batch
    takes less than `min_s`, further passes over it until `min_s` is reached
    (the GPU output is checked on the first pass)."""
    from oracle.reference import paged_attention_reference

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, bt, lens = case["q"].cpu(), case["bt"].cpu(), case["lens"].cpu()
    k, v = case["k"].cpu(), case["v"].cpu()  # bf16, as the reference's CPU path receives them
    gpu_out = case["out"].float().cpu()
    elt = 2
    hkv, d = case["k"].shape[2], case["k"].shape[3]
    done_bytes, elapsed, seqs, passes = 0, 0.0, 0, 0
    worst = 0.0
    paged_attention_reference(q[:1], k, v, bt[:1], lens[:1])  # warm-up
    while elapsed < min_s and elapsed < budget_s:
        for s in range(q.shape[0]):
            t0 = time.perf_counter()
            ref = paged_attention_reference(q[s : s + 1], k, v, bt[s : s + 1], lens[s : s + 1])
            elapsed += time.perf_counter() - t0
            if passes == 0:
                worst = max(worst, (gpu_out[s] - ref[0].float()).abs().max().item())
                seqs += 1
            done_bytes += int(lens[s]) * 2 * hkv * d * elt + 2 * q.shape[1] * d * elt
            if elapsed >= budget_s:
                break
        passes += 1
    del k, v
    if worst > 2e-2:
        raise AssertionError(f"paged_attention_decode differs from the oracle by {worst:.3e} (> 2e-2)")
    n = q.shape[0]
    what = f"the first {seqs} of {n} sequences" if passes == 1 else f"all {n} sequences, {passes} passes"
    return {
        "value": round(done_bytes / elapsed / 1e12, 6),
        "unit": "TB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"oracle.reference.paged_attention_reference (torch CPU, fp32) on {what} of the same workload "
        f"({done_bytes / 1e6:.0f} MB of bf16 KV read in total, bf16 inputs), one sequence per call, {elapsed:.1f} s; "
        f"GPU output matched to {worst:.2e} max abs on the {seqs} sequences of the first pass",
    }


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "paged_attention_llama3_8b_b64_bf16_traffic.md")
CALIBRATION_BYTES = 256 << 20


def pmc_workload_gemm(calls: int = 3) -> None:
    """What the GEMM counter runs profile: gemm_tn at a prefill shape (M=4096,
    N=K=4096: 256x256 tiles) and a batched-decode shape (M=256, N=6144,
    K=4096: 128x128 tiles, K in 2 splits), `calls` times each, then hipBLASLt
    (torch's F.linear) at the prefill shape for comparison."""
    g = torch.Generator(device="cuda").manual_seed(30)
    for m, n in ((4096, 4096), (256, 6144)):
        a = torch.randn(m, 4096, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
        w = torch.randn(n, 4096, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
        c = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
        for _ in range(calls):
            torch.ops.decode_kernels.gemm_tn(c, a, w, None)
        if m == 4096:
            for _ in range(calls):
                torch.nn.functional.linear(a, w)
    torch.cuda.synchronize()
    print(f"pmc gemm workload done: {calls} calls each at M=4096 N=4096 and M=256 N=6144 (K=4096), "
          f"{calls} hipBLASLt calls at M=4096", flush=True)


def pmc_workload_gemm_skinny(calls: int = 3) -> None:
    """What the decode-GEMM counter runs profile: the decode layer's down
    projection (N=4096, K=14336) at M=1 (the skinny kernel) and M=64 (the
    LDS-DMA kernel's 64-row tile with K in 8 splits), `calls` times each."""
    g = torch.Generator(device="cuda").manual_seed(1)
    w = torch.randn(4096, 14336, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
    for m in (1, 64):
        a = torch.randn(m, 14336, generator=g, device="cuda", dtype=torch.bfloat16) * 0.02
        c = torch.empty(m, 4096, device="cuda", dtype=torch.bfloat16)
        for _ in range(calls):
            torch.ops.decode_kernels.gemm_tn(c, a, w, None)
    torch.cuda.synchronize()
    print(f"pmc decode gemm workload done: {calls} calls each at M=1 and M=64 (N=4096, K=14336)", flush=True)


def pmc_workload_attention_fp8(calls: int = 3) -> None:
    """What the fp8-cache counter runs profile: the headline batch with a bf16
    cache, then the same batch with an fp8 (e4m3fn) cache, `calls` times each."""
    lens = torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    for kv in (torch.bfloat16, torch.float8_e4m3fn):
        c = attention_case(64, 32, 8, 128, 16, lens, torch.bfloat16, "vllm", seed=60, q_scale=128**-0.5, kv_dtype=kv,
                           k_scale=0.5, v_scale=0.5)
        for _ in range(calls):
            c["run"]()
        torch.cuda.synchronize()
        del c
    print(f"pmc fp8 attention workload done: {calls} calls each with a bf16 and an fp8 cache", flush=True)


def pmc_workload_attention_cold(calls: int = 3) -> None:
    """What the cold-cache attention profiles cover: the headline batch, then the
    128K-token batch-1 and batch-4 cases (fp16, HND, 1% outlier rows), `calls`
    times each, every call after a 1 GiB cache flush (the flush is its own
    kernel, `amax`)."""
    lens = torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    cases = (("llama3_8b_b64", (64, 32, 8, 128, 16, lens, torch.bfloat16, "vllm"), dict(seed=0, q_scale=128**-0.5)),
             ("128k_b1", (1, 32, 8, 128, 16, [131072], torch.float16, "hnd"), dict(seed=11, outlier_frac=0.01)),
             ("128k_b4", (4, 32, 8, 128, 16, [131072] * 4, torch.float16, "hnd"), dict(seed=14, outlier_frac=0.01)))
    for name, args, kw in cases:
        c = attention_case(*args, **kw)
        for _ in range(calls):
            flush_caches()
            c["run"]()
        torch.cuda.synchronize()
        print(f"pmc cold attention workload: {calls} calls of {name}", flush=True)
        del c
        torch.cuda.empty_cache()


def pmc_workload_norm(calls: int = 3) -> None:
    """What the norm / activation counter runs profile: rms_norm and
    fused_add_rms_norm at hidden 4096 and silu_and_mul at 2 x 14336, for 64
    tokens (decode) and 16384 tokens (a prefill batch), each call from cold
    caches, then copies of CALIBRATION_BYTES to scale the counters."""
    g = torch.Generator(device="cuda").manual_seed(40)
    w = (1 + 0.1 * torch.randn(4096, generator=g, device="cuda")).to(torch.bfloat16)
    for tokens in (64, 16384):
        x = torch.randn(tokens, 4096, generator=g, device="cuda", dtype=torch.bfloat16)
        r = torch.randn(tokens, 4096, generator=g, device="cuda", dtype=torch.bfloat16)
        out = torch.empty_like(x)
        gu = torch.randn(tokens, 2 * 14336, generator=g, device="cuda", dtype=torch.bfloat16)
        act = torch.empty(tokens, 14336, device="cuda", dtype=torch.bfloat16)
        for _ in range(calls):
            for fn in (lambda: dk.rms_norm(x, w, 1e-5, out=out), lambda: dk.fused_add_rms_norm(x, r, w, 1e-5),
                       lambda: dk.silu_and_mul(gu, out=act)):
                flush_caches()
                fn()
        torch.cuda.synchronize()
        del x, r, out, gu, act
    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(calls):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"pmc norm workload done: {calls} cold calls of each op at 64 and 16384 tokens", flush=True)


# ---------------------------------------------------------------------------
# The reference's benchmark sweep (opt-in: --sweep)
# ---------------------------------------------------------------------------
SWEEP_ATTN_MODELS = (("llama3-8b", 32, 8, 128), ("qwen2.5-7b", 28, 4, 128), ("qwen2.5-0.5b", 14, 2, 64))
SWEEP_GEMM_SHAPES = (("qkv_proj", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up_proj", 28672, 4096),
                     ("down_proj", 4096, 14336))
SWEEP_MAX_KV_BYTES = 6 * 1024**3  # the reference skips attention configs whose KV cache exceeds this


def sweep(dtype, quick: bool, out_path: str | None) -> int:
    """The grid of DecodeKernels' own benchmark (benchmarks/bench_kernels.py:37-54,
    227-230): paged decode attention for 3 models x batch {1, 8, 32, 64} x
    context {512, 2048, 8192, 32768} (every sequence of the context length,
    block 16, NHD cache, KV caches above 6 GiB skipped as there); gemm_tn at the
    4 Llama-3-8B projections x M {1, 8, 32, 64, 128, 512, 2048} next to
    hipBLASLt (F.linear, timed interleaved); rms_norm and fused_add_rms_norm
    (H 4096) and silu_and_mul (d 14336) at {1, 32, 256, 2048} tokens. Every row
    is checked before it is timed -- attention on its 2 longest sequences
    against the CPU oracle at the parity bar, GEMMs against an fp32 GEMM at the
    bar, norms and SiLU at 1 ulp of the oracle -- and timed as the median of
    cold-cache calls, with its roofline fraction (HBM 8 TB/s; GEMM also the
    bf16 / fp16 MFMA peak). One JSON line per row on stdout (and in out_path)."""
    from oracle.reference import fused_add_rms_norm_reference, rms_norm_reference, silu_and_mul_reference

    torch.backends.cuda.preferred_blas_library("cublaslt")  # hipBLASLt on ROCm
    batches = (1, 8) if quick else (1, 8, 32, 64)
    ctxs = (512, 4096) if quick else (512, 2048, 8192, 32768)
    ms = (1, 64, 512) if quick else (1, 8, 32, 64, 128, 512, 2048)
    tokens = (1, 256) if quick else (1, 32, 256, 2048)
    elt = torch.finfo(dtype).bits // 8
    tag = "bf16" if dtype == torch.bfloat16 else "fp16"
    sink = open(out_path, "w") if out_path else None

    def emit(row: dict) -> None:
        row = {"dtype": tag, **row}
        line = json.dumps(row)
        print(line, flush=True)
        if sink:
            sink.write(line + "\n")
            sink.flush()

    def rate(nbytes: float, us: float) -> dict:
        gbs = nbytes / (us * 1e-6) / 1e9
        return {"GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3)}

    for name, hq, hkv, d in SWEEP_ATTN_MODELS:
        for b in batches:
            for ctx in ctxs:
                cfg = f"{name} bs={b} ctx={ctx}"
                kv_bytes = 2 * b * ctx * hkv * d * elt
                if kv_bytes > SWEEP_MAX_KV_BYTES:
                    emit({"op": "attention", "config": cfg, "skipped": f"KV cache {kv_bytes / 1e9:.1f} GB > 6 GiB"})
                    continue
                c = attention_case(b, hq, hkv, d, 16, [ctx] * b, dtype, "nhd", seed=b + ctx)
                err = check_attention(c, f"sweep attention {cfg}", sample=2)
                t = time_cold(c["run"], iters=20)
                emit({"op": "attention", "config": cfg, "us": t["median_us"], "p10_us": t["p10_us"],
                      "p90_us": t["p90_us"], "MB": round(c["bytes"] / 1e6, 2), **rate(c["bytes"], t["median_us"]),
                      "checked_max_abs_err": err})
                progress(f"sweep attention {cfg}: {t['median_us']} us")
                del c
                torch.cuda.empty_cache()
    g = torch.Generator(device="cuda").manual_seed(70)
    peak = BF16_PEAK_TFLOPS
    for name, n, k in SWEEP_GEMM_SHAPES:
        w = torch.randn(n, k, generator=g, device="cuda", dtype=dtype) * k**-0.5
        for m in ms:
            a = torch.randn(m, k, generator=g, device="cuda", dtype=dtype)
            out = torch.empty(m, n, device="cuda", dtype=dtype)
            torch.ops.decode_kernels.gemm_tn(out, a, w, None)
            err = check_gemm(out, a, w, what=f"sweep gemm {name} M={m}")
            t = time_cold_interleaved({"dk": lambda: torch.ops.decode_kernels.gemm_tn(out, a, w, None),
                                       "hipblaslt": lambda: F.linear(a, w)}, iters=10 if m >= 512 else 20)
            us, bl = t["dk"]["median_us"], t["hipblaslt"]["median_us"]
            flops, nbytes = 2.0 * m * n * k, (m * k + n * k + m * n) * elt
            tf = flops / (us * 1e-6) / 1e12
            emit({"op": "gemm_tn", "config": f"{name} M={m} N={n} K={k}", "us": us, "hipblaslt_us": bl,
                  "dk_over_hipblaslt": round(us / bl, 3), "TFLOP/s": round(tf, 1), "mfma_frac": round(tf / peak, 3),
                  **rate(nbytes, us), "checked_max_abs_err": err})
            progress(f"sweep gemm {name} M={m}: {us} us ({us / bl:.3f}x hipBLASLt)")
        del w
    h, dmlp = 4096, 14336
    wt = (1 + 0.1 * torch.randn(h, generator=g, device="cuda")).to(dtype)
    for t_ in tokens:
        x = torch.randn(t_, h, generator=g, device="cuda", dtype=dtype)
        r = torch.randn(t_, h, generator=g, device="cuda", dtype=dtype)
        xs = torch.randn(t_, 2 * dmlp, generator=g, device="cuda", dtype=dtype)
        out, ys = torch.empty_like(x), torch.empty(t_, dmlp, device="cuda", dtype=dtype)
        torch.ops.decode_kernels.rms_norm(out, x, wt, 1e-6)
        u_rms = ulps(out, rms_norm_reference(x.cpu(), wt.cpu(), 1e-6))
        xc, rc = x.clone(), r.clone()
        torch.ops.decode_kernels.fused_add_rms_norm(xc, rc, wt, 1e-6)
        want_x, want_r = fused_add_rms_norm_reference(x.cpu(), r.cpu(), wt.cpu(), 1e-6)
        if not torch.equal(rc.cpu(), want_r):
            raise AssertionError(f"sweep fused_add_rms_norm T={t_}: residual differs from the oracle before timing")
        u_fused = ulps(xc, want_x)
        torch.ops.decode_kernels.silu_and_mul(ys, xs)
        u_silu = ulps(ys, silu_and_mul_reference(xs.cpu()))
        if max(u_rms, u_fused, u_silu) > 1:
            raise AssertionError(f"sweep norms T={t_}: {u_rms} / {u_fused} / {u_silu} ulp from the oracle before timing")
        for op, fn, nbytes, u in (
            ("rms_norm", lambda: torch.ops.decode_kernels.rms_norm(out, x, wt, 1e-6), 2 * t_ * h * elt, u_rms),
            ("fused_add_rms_norm", lambda: torch.ops.decode_kernels.fused_add_rms_norm(xc, rc, wt, 1e-6),
             4 * t_ * h * elt, u_fused),
            ("silu_and_mul", lambda: torch.ops.decode_kernels.silu_and_mul(ys, xs), 3 * t_ * dmlp * elt, u_silu),
        ):
            tm = time_cold(fn, iters=30)
            emit({"op": op, "config": f"T={t_} " + (f"d={dmlp}" if op == "silu_and_mul" else f"H={h}"),
                  "us": tm["median_us"], "p10_us": tm["p10_us"], "p90_us": tm["p90_us"], **rate(nbytes, tm["median_us"]),
                  "checked_max_ulp": u})
        progress(f"sweep norms T={t_} done")
    if sink:
        sink.close()
    return 0


def pmc_workload_layer_graph(steps: int = 20) -> None:
    """What the graph-against-eager kernel trace records: the Llama-3-8B batch-64
    decode-layer step, fused and unfused, `steps` eager steps and then `steps`
    replays of a one-step HIP graph, each phase between two marker kernels (an
    add on a 1-element tensor before it, on a 3-element one after it)."""
    seq_lens = torch.randint(512, 4097, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    ops, _, fused, _, _, _ = layer_step(64, 32, 8, 128, 16, seq_lens, torch.bfloat16, "vllm", seed=50)
    before, after = torch.zeros(1, device="cuda"), torch.zeros(3, device="cuda")
    for name, fns in (("fused", fused), ("unfused", ops)):
        def step():
            for fn in fns.values():
                fn()

        for _ in range(5):
            step()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        for run in (step, graph.replay):
            before.add_(1.0)
            torch.cuda.synchronize()
            for _ in range(steps):
                run()
            torch.cuda.synchronize()
            after.add_(1.0)
            torch.cuda.synchronize()
        del graph
    print(f"layer graph workload done: fused and unfused step, {steps} eager steps then {steps} replays each", flush=True)


def pmc_workload(calls: int = 5) -> None:
    """What the counter runs profile: the headline op `calls` times, then a
    copy of CALIBRATION_BYTES (read once, written once) to scale the counters."""
    case = llama3_8b_decode_case()
    for _ in range(calls):
        case["run"]()
    torch.cuda.synchronize()
    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(calls):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"pmc workload done: {calls} attention calls, {calls} copies of {CALIBRATION_BYTES >> 20} MiB", flush=True)


def environment() -> dict:
    """What the numbers were measured on (the reference records the same,
    benchmarks/bench_utils.py:68-92)."""
    props = torch.cuda.get_device_properties(0)
    return {
        "gpu": props.name, "arch": getattr(props, "gcnArchName", ""), "compute_units": props.multi_processor_count,
        "hbm_GiB": round(props.total_memory / 2**30, 1), "hip": torch.version.hip, "torch": torch.__version__,
        "host_cores": len(os.sched_getaffinity(0)), "date_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
    }


def measured_traffic() -> int | None:
    """HBM bytes per headline call from the committed counter summary, if any."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extras", action="store_true", help="skip the secondary configs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (and its correctness check)")
    ap.add_argument("--sweep", action="store_true",
                    help="run DecodeKernels' benchmark grid instead (one JSON line per row; not the bench line)")
    ap.add_argument("--sweep-dtype", choices=["bf16", "fp16"], default="bf16")
    ap.add_argument("--sweep-quick", action="store_true", help="the reference's --quick grid")
    ap.add_argument("--sweep-out", default=None, help="also write the sweep's JSON lines to this file")
    ap.add_argument("--pmc-workload", nargs="?", const="attention",
                    choices=["attention", "attention_cold", "attention_fp8", "gemm", "gemm_skinny", "norm",
                             "layer_graph"],
                    help="run only what the rocprofv3 --pmc / --kernel-trace passes profile (default: attention)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every work unit of this path fits one MI355X and no multi-GPU "
              "figure is defined (sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        return 2
    if not dk.is_available():
        raise RuntimeError("decodekernels_amd HIP extension not available (build it with __graft_entry__.build())")
    if args.sweep:
        return sweep(torch.bfloat16 if args.sweep_dtype == "bf16" else torch.float16, args.sweep_quick, args.sweep_out)
    if args.pmc_workload == "attention_cold":
        pmc_workload_attention_cold()
        return 0
    if args.pmc_workload == "attention_fp8":
        pmc_workload_attention_fp8()
        return 0
    if args.pmc_workload == "gemm_skinny":
        pmc_workload_gemm_skinny()
        return 0
    if args.pmc_workload == "gemm":
        pmc_workload_gemm()
        return 0
    if args.pmc_workload == "norm":
        pmc_workload_norm()
        return 0
    if args.pmc_workload == "layer_graph":
        pmc_workload_layer_graph()
        return 0
    if args.pmc_workload:
        pmc_workload()
        return 0

    global CPU_PATH
    CPU_PATH = not args.no_cpu
    if CPU_PATH:
        cpu_threads()
    case = llama3_8b_decode_case()
    headline_err = check_attention(case, "headline (Llama-3-8B batch 64)", sample=8)
    # K timed steps, each from cold caches (a 1 GiB read before every call,
    # outside its HIP-event interval); value and roofline use their median.
    cold = time_cold(case["run"], iters=args.steps, warmup=args.warmup)
    ms = cold["median_us"] * 1e-3
    gbs = case["bytes"] / (ms * 1e-3) / 1e9
    b2b_ms = time_back_to_back(case["run"], args.steps, args.warmup)

    result = {
        "metric": "paged-attn decode HBM TB/s (% peak) + µs/call; gemm_tn TFLOP/s; µs per op",
        "value": round(gbs / 1e3, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_call": round(ms * 1e3, 2),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "cold_cache": cold,
        "back_to_back": {"mean_us": round(b2b_ms * 1e3, 2),
                         "TB/s": round(case["bytes"] / (b2b_ms * 1e-3) / 1e12, 4)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V, q scaled by 1/sqrt(128))",
        "config": {
            "workload": "llama3-8b paged decode attention, batch 64",
            "num_seqs": 64, "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128, "block_size": 16,
            "seq_lens": "U[512,4096] seed 0", "total_tokens": sum(case["seq_lens"]), "kv_layout": "vllm interleaved",
            "algorithmic_MB": round(case["bytes"] / 1e6, 1),
            "checked_max_abs_err": headline_err,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": "one paged_attention_decode call: paged_attention_balanced_kernel + paged_attention_reduce_kernel",
            "timing": "median of the K cold-cache calls",
        },
        "env": environment(),
    }
    progress(f"headline: {cold['median_us']} us cold median, {b2b_ms * 1e3:.2f} us back to back")
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_and_check(case)
        progress("cpu baseline done")
    del case
    torch.cuda.empty_cache()
    if not args.no_extras:
        result["extras"] = {"attention": extras_attention(), "gemm_bf16": extras_gemm(), "norm_act_bf16": extras_norms(),
                            "decode_layer_step_bf16": extras_layer_step()}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
