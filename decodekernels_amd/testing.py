"""Seeded paged KV caches for tests and benchmarks.

Same builder as DecodeKernels' ``decode_kernels/testing.py:10-78``
(``PagedKV`` and ``make_paged_kv`` with the ``nhd``, ``hnd`` and ``vllm``
layouts, ``extra_blocks`` and ``seed``): every sequence gets
ceil(len / block_size) physical blocks taken from a random permutation of the
cache's blocks, and block-table entries past a sequence's last block are 0.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class PagedKV:
    k_cache: torch.Tensor  # [num_blocks, block_size, num_kv_heads, head_dim], possibly a strided view
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [num_seqs, max_blocks] int32
    seq_lens: torch.Tensor  # [num_seqs] int32
    block_size: int

    @property
    def max_seq_len(self) -> int:
        return int(self.seq_lens.max().item()) if self.seq_lens.numel() else 0


def _cache(shape, gen, dtype, device):
    if dtype.is_floating_point and dtype.itemsize == 1:  # fp8: N(0, 1) values rounded to the format
        return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype).to(device)
    return torch.randn(*shape, generator=gen, dtype=dtype).to(device)


def make_paged_kv(
    seq_lens: list[int],
    num_kv_heads: int,
    head_dim: int,
    block_size: int = 16,
    dtype: torch.dtype = torch.float16,
    device: str | torch.device = "cpu",
    layout: str = "nhd",
    extra_blocks: int = 3,
    seed: int = 0,
) -> PagedKV:
    """Random paged KV cache whose physical blocks are shuffled.

    layout:
      * ``nhd``  -- contiguous [num_blocks, block_size, num_kv_heads, head_dim].
      * ``hnd``  -- stored [num_blocks, num_kv_heads, block_size, head_dim],
                    returned as the transposed (NHD-shaped) view.
      * ``vllm`` -- one buffer [num_blocks, num_kv_heads, block_size, 2*head_dim]
                    returned as two strided NHD views, K = [..., :D] and
                    V = [..., D:], the way vLLM's FlashAttention backend slices it.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    nblk = [-(-n // block_size) for n in seq_lens]
    num_blocks = sum(nblk) + extra_blocks

    if layout == "nhd":
        shape = (num_blocks, block_size, num_kv_heads, head_dim)
        k = _cache(shape, gen, dtype, device)
        v = _cache(shape, gen, dtype, device)
    elif layout == "hnd":
        shape = (num_blocks, num_kv_heads, block_size, head_dim)
        k = _cache(shape, gen, dtype, device).transpose(1, 2)
        v = _cache(shape, gen, dtype, device).transpose(1, 2)
    elif layout == "vllm":
        kv = _cache((num_blocks, num_kv_heads, block_size, 2 * head_dim), gen, dtype, device)
        k, v = kv.transpose(1, 2).split(head_dim, dim=-1)
    else:
        raise ValueError(f"unknown layout {layout!r}")

    perm = torch.randperm(num_blocks, generator=gen).to(torch.int32)
    width = max(max(nblk, default=1), 1)
    block_tables = torch.zeros(len(seq_lens), width, dtype=torch.int32)
    offsets = [0]
    for n in nblk:
        offsets.append(offsets[-1] + n)
    for s, n in enumerate(nblk):
        block_tables[s, :n] = perm[offsets[s] : offsets[s] + n]

    return PagedKV(
        k_cache=k,
        v_cache=v,
        block_tables=block_tables.to(device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        block_size=block_size,
    )
