"""CPU oracle of the two decode steps around attention (test infrastructure).

DecodeKernels has no rotary embedding or cache write: vLLM runs them (its
``rotary_embedding`` and ``reshape_and_cache_flash`` ops) before paged
attention reads the cache. These restate that published semantics, which the
decodekernels_amd kernels implement, as the expected results:

* rotary embedding (RoFormer's rotary position embedding, in GPT-NeoX's
  rotate-halves or GPT-J's interleaved pairing): for the first ``rot_dim``
  columns of every head, pairs (x, y) become (x cos - y sin, y cos + x sin)
  with cos = cos_sin_cache[pos, i], sin = cos_sin_cache[pos, rot_dim / 2 + i];
  fp32 arithmetic with each product and sum rounded on its own (as separate
  tensor ops do), one rounding to the input dtype; positions outside the
  table leave the token unchanged.
* cache write: key_cache[slot // block_size, slot % block_size] = key[t]
  (same for value), slot = slot_mapping[t], negative or out-of-range slots
  skipped. Into an fp8 (e4m3fn) cache the rows are quantized as vLLM's
  ``reshape_and_cache_flash`` does for ``kv_cache_dtype`` "fp8": x / scale in
  fp32, saturated to the largest finite value (+-448, NaN stays NaN), rounded
  to nearest even.

Pinned in ``tests/test_oracle_rope_cache.py`` by an independent complex-number
route, rotation invariants in float64 and an ``index_put_`` scatter.
"""

from __future__ import annotations

import torch


def rotary_embedding_reference(positions, query, key, head_size, cos_sin_cache, is_neox=True):
    """Rotated copies (query, key) of [tokens, heads * head_size] or
    [tokens, heads, head_size] tensors; ``key`` may be None."""
    rot = cos_sin_cache.shape[1]
    half = rot // 2
    pos = positions.reshape(-1).long()
    valid = (pos >= 0) & (pos < cos_sin_cache.shape[0])
    table = cos_sin_cache.float()[pos.clamp(0, cos_sin_cache.shape[0] - 1)]
    cos, sin = table[:, None, :half], table[:, None, half:]

    def apply(x):
        if x is None:
            return None
        t = x.shape[0]
        x3 = x.reshape(t, -1, head_size).float()
        r = x3[..., :rot]
        if is_neox:
            x1, x2 = r[..., :half], r[..., half:]
        else:
            x1, x2 = r[..., 0::2], r[..., 1::2]
        o1 = x1 * cos - x2 * sin
        o2 = x2 * cos + x1 * sin
        out = x3.clone()
        if is_neox:
            out[..., :half] = o1
            out[..., half:rot] = o2
        else:
            out[..., 0:rot:2] = o1
            out[..., 1:rot:2] = o2
        out = torch.where(valid[:, None, None], out, x3)
        return out.to(x.dtype).reshape(x.shape)

    return apply(query), apply(key)


E4M3_MAX = 448.0


def quantize_e4m3(x: torch.Tensor, scale: float) -> torch.Tensor:
    """x / scale in fp32, saturated to +-448 (NaN kept), rounded to nearest-even e4m3fn."""
    y = x.float() / torch.tensor(scale, dtype=torch.float32)
    return y.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)


def reshape_and_cache_reference(key, value, key_cache, value_cache, slot_mapping, k_scale=1.0, v_scale=1.0):
    """Copies of the caches with each token's key / value row written to its
    slot (quantized with k_scale / v_scale when the caches are e4m3fn)."""
    if key_cache.dtype == torch.float8_e4m3fn:
        key, value = quantize_e4m3(key, k_scale), quantize_e4m3(value, v_scale)
    kc, vc = key_cache.clone(), value_cache.clone()
    num_blocks, block_size = kc.shape[0], kc.shape[1]
    nkv = kc.shape[2]
    k3 = key.reshape(key.shape[0], nkv, -1)
    v3 = value.reshape(value.shape[0], nkv, -1)
    for t, slot in enumerate(slot_mapping.tolist()):
        if slot < 0 or slot >= num_blocks * block_size:
            continue
        kc[slot // block_size, slot % block_size] = k3[t]
        vc[slot // block_size, slot % block_size] = v3[t]
    return kc, vc


def rope_cos_sin_cache(max_position: int, rot_dim: int, base: float = 10000.0, dtype=torch.float32):
    """The standard table: theta_i = base^(-2i / rot_dim), columns cos(pos theta_i) then sin(pos theta_i)."""
    inv_freq = base ** (-torch.arange(0, rot_dim, 2, dtype=torch.float64) / rot_dim)
    ang = torch.arange(max_position, dtype=torch.float64)[:, None] * inv_freq[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1).to(dtype)
