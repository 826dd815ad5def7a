"""Float64 brute force from the definitions, for tiny inputs (test infrastructure).

Independent of ``oracle.reference`` (numpy, explicit loops, no torch
arithmetic), so a shared mistake cannot hide: it walks the block table token by
token, maps query head h to KV head h // group, and evaluates softmax
attention, the flash-decoding merge, A·Bᵀ, RMSNorm and SiLU in float64.
"""

from __future__ import annotations

import math

import numpy as np


def _np(t) -> np.ndarray:
    return t.detach().cpu().double().numpy() if hasattr(t, "detach") else np.asarray(t, dtype=np.float64)


def attention(q, k_cache, v_cache, block_tables, seq_lens, scale=None) -> np.ndarray:
    """[S, Hq, D] float64 decode attention over a paged cache [NB, bs, Hkv, D]."""
    qn, kn, vn = _np(q), _np(k_cache), _np(v_cache)
    bt = np.asarray(block_tables.cpu() if hasattr(block_tables, "cpu") else block_tables).astype(np.int64)
    lens = [int(x) for x in (seq_lens.cpu() if hasattr(seq_lens, "cpu") else seq_lens)]
    S, Hq, D = qn.shape
    bs, Hkv = kn.shape[1], kn.shape[2]
    group = Hq // Hkv
    scale = D**-0.5 if scale is None else scale
    out = np.zeros((S, Hq, D))
    for s in range(S):
        L = lens[s]
        if L <= 0:
            continue
        for h in range(Hq):
            kvh = h // group
            logits = np.empty(L)
            rows_v = np.empty((L, D))
            for t in range(L):
                blk = bt[s, t // bs]
                logits[t] = scale * float(np.dot(qn[s, h], kn[blk, t % bs, kvh]))
                rows_v[t] = vn[blk, t % bs, kvh]
            w = np.exp(logits - logits.max())
            out[s, h] = (w[:, None] * rows_v).sum(axis=0) / w.sum()
    return out


def lse_merge(maxes, sums, outs) -> np.ndarray:
    """Merge partitions (m_p, s_p, o_p) of one head: sum_p s_p e^(m_p - M) o_p / sum_p s_p e^(m_p - M)."""
    M = max(maxes)
    w = [s * math.exp(m - M) for m, s in zip(maxes, sums)]
    return sum(wi * np.asarray(o, dtype=np.float64) for wi, o in zip(w, outs)) / sum(w)


def gemm(a, b, bias=None) -> np.ndarray:
    an, bn = _np(a), _np(b)
    M, K = an.shape
    N = bn.shape[0]
    c = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            c[m, n] = float(np.dot(an[m], bn[n]))
    if bias is not None:
        c += _np(bias)[None, :]
    return c


def rms_norm(x, w, eps) -> np.ndarray:
    xn, wn = _np(x), _np(w)
    ms = (xn * xn).mean(axis=-1, keepdims=True)
    return xn / np.sqrt(ms + eps) * wn


def silu_and_mul(x) -> np.ndarray:
    xn = _np(x)
    d = xn.shape[-1] // 2
    g, u = xn[..., :d], xn[..., d:]
    return g / (1.0 + np.exp(-g)) * u
