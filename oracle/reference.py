"""CPU restatement of DecodeKernels' ``decode_kernels/reference.py`` (test infrastructure).

Each function keeps the reference's name, signature and result semantics;
arithmetic is torch fp32 on whatever device the inputs live on (the tests and
the CPU baseline use the CPU). Pinned in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def gather_kv(cache: torch.Tensor, block_table_row: torch.Tensor, seq_len: int) -> torch.Tensor:
    """Rows [seq_len, num_kv_heads, head_dim] of one sequence from a paged cache:
    token t lives in physical block ``block_table_row[t // block_size]`` at slot
    ``t % block_size`` (reference: decode_kernels/reference.py:15-20)."""
    block_size = cache.shape[1]
    tok = torch.arange(seq_len, device=cache.device)
    phys = block_table_row[tok // block_size].long()
    return cache[phys, tok % block_size]


def _per_seq_kv(k_cache, v_cache, block_tables, s, seq_len, group):
    """fp32 K and V of sequence ``s`` expanded to one row per query head: query
    head h reads KV head h // group (reference: decode_kernels/reference.py:23-26)."""
    k = gather_kv(k_cache, block_tables[s], seq_len).float().repeat_interleave(group, dim=1)
    v = gather_kv(v_cache, block_tables[s], seq_len).float().repeat_interleave(group, dim=1)
    return k, v  # [L, num_q_heads, head_dim]


def paged_attention_reference(q, k_cache, v_cache, block_tables, seq_lens, scale=None) -> torch.Tensor:
    """Dense softmax attention of each sequence's query token over its whole
    context, in fp32, rounded once to q's dtype; empty sequences give zeros
    (reference: decode_kernels/reference.py:29-43)."""
    num_seqs, num_q_heads, head_dim = q.shape
    group = num_q_heads // k_cache.shape[2]
    scale = head_dim**-0.5 if scale is None else scale
    out = torch.zeros(num_seqs, num_q_heads, head_dim, dtype=torch.float32, device=q.device)
    for s in range(num_seqs):
        seq_len = int(seq_lens[s])
        if seq_len <= 0:
            continue
        k, v = _per_seq_kv(k_cache, v_cache, block_tables, s, seq_len, group)
        qs = q[s].float() * scale  # [H, D]
        logits = (k.transpose(0, 1) @ qs.unsqueeze(-1)).squeeze(-1)  # [H, L]
        probs = torch.softmax(logits, dim=-1)
        out[s] = (probs.unsqueeze(1) @ v.transpose(0, 1)).squeeze(1)  # [H, D]
    return out.to(q.dtype)


def split_k_attention_reference(
    q, k_cache, v_cache, block_tables, seq_lens, scale=None, partition_size: int = 512
) -> torch.Tensor:
    """Flash-decoding math in fp32: per partition of ``partition_size`` tokens,
    (max logit m, exp-sum s, normalised output o); then
    M = max m_p, w_p = s_p * exp(m_p - M), out = sum w_p o_p / sum w_p.
    Returns fp32 (reference: decode_kernels/reference.py:46-79)."""
    num_seqs, num_q_heads, head_dim = q.shape
    group = num_q_heads // k_cache.shape[2]
    scale = head_dim**-0.5 if scale is None else scale
    out = torch.zeros(num_seqs, num_q_heads, head_dim, dtype=torch.float32, device=q.device)
    for s in range(num_seqs):
        seq_len = int(seq_lens[s])
        if seq_len <= 0:
            continue
        k, v = _per_seq_kv(k_cache, v_cache, block_tables, s, seq_len, group)
        qs = q[s].float() * scale
        parts_m, parts_s, parts_o = [], [], []
        for lo in range(0, seq_len, partition_size):
            hi = min(lo + partition_size, seq_len)
            logits = (k[lo:hi].transpose(0, 1) @ qs.unsqueeze(-1)).squeeze(-1)  # [H, n]
            m = logits.amax(dim=-1)
            e = torch.exp(logits - m.unsqueeze(-1))
            ssum = e.sum(dim=-1)
            o = (e.unsqueeze(1) @ v[lo:hi].transpose(0, 1)).squeeze(1) / ssum.unsqueeze(-1)
            parts_m.append(m)
            parts_s.append(ssum)
            parts_o.append(o)
        m = torch.stack(parts_m)  # [P, H]
        ssum = torch.stack(parts_s)
        o = torch.stack(parts_o)  # [P, H, D]
        w = ssum * torch.exp(m - m.amax(dim=0, keepdim=True))
        out[s] = (w.unsqueeze(-1) * o).sum(dim=0) / w.sum(dim=0).unsqueeze(-1)
    return out


def gemm_reference(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """a @ b.T (+ bias) in fp32, rounded once to a's dtype
    (reference: decode_kernels/reference.py:82-86)."""
    c = a.float() @ b.float().t()
    if bias is not None:
        c = c + bias.float()
    return c.to(a.dtype)


def rms_norm_reference(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight in fp32, rounded to x's dtype
    (reference: decode_kernels/reference.py:89-92)."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv * weight.float()).to(x.dtype)


def fused_add_rms_norm_reference(x, residual, weight, eps: float = 1e-6):
    """(normed, new_residual): the residual sum is rounded to x's dtype before
    the norm reads it (reference: decode_kernels/reference.py:95-99)."""
    new_residual = (x.float() + residual.float()).to(x.dtype)
    return rms_norm_reference(new_residual, weight, eps), new_residual


def silu_and_mul_reference(x: torch.Tensor) -> torch.Tensor:
    """silu(x[..., :d]) * x[..., d:] in fp32, rounded to x's dtype
    (reference: decode_kernels/reference.py:102-104)."""
    d = x.shape[-1] // 2
    return (F.silu(x[..., :d].float()) * x[..., d:].float()).to(x.dtype)
