"""Python API of the decode kernels: allocation, defaults and torch.compile fakes.

Mirrors DecodeKernels' ``decode_kernels/ops.py`` (same names, arguments,
defaults and errors) over this package's HIP kernels. The raw ops
``torch.ops.decode_kernels.*`` mutate their ``Tensor!`` arguments and can run
on preallocated buffers inside a HIP graph; these wrappers allocate outputs
(and the attention split-K workspace) when the caller does not pass them. All
raw ops but one allocate nothing. ``gemm_tn``, unlike the reference's op, takes
the fp32 workspace of the decode shapes whose plan splits K (splits * M * N * 4
bytes) from PyTorch's caching allocator, stream-ordered, so it still captures
in a graph (private pool). The C ABI's ``dk_gemm_tn_ws`` with a caller
workspace is the allocation-free route.
"""

from __future__ import annotations

import math

import torch

PARTITION_SIZE = 512  # tokens per split-K workspace slot (DK_PARTITION_SIZE in the C ABI)
MAX_GQA_GROUP = 16  # query heads per KV head (DK_MAX_GQA_GROUP; the reference stops at 8)
SUPPORTED_HEAD_DIMS = (64, 96, 128, 192, 256)  # the reference: 64, 128, 256
SUPPORTED_FP8_HEAD_DIMS = (64, 128, 192, 256)  # an fp8 cache row loads 64 columns per 16-byte lane group

try:
    from . import _C  # noqa: F401  (registers torch.ops.decode_kernels.*)

    _AVAILABLE = True
    _IMPORT_ERROR: Exception | None = None
except ImportError as e:  # libraries not built yet
    _AVAILABLE = False
    _IMPORT_ERROR = e


def is_available() -> bool:
    """True when the HIP extension is built and a GPU is visible."""
    return _AVAILABLE and torch.cuda.is_available()


def _require() -> None:
    if not _AVAILABLE:
        raise RuntimeError(
            "decodekernels_amd._C is not built. Run `python -m decodekernels_amd._build` "
            f"(hipcc for gfx950) first. Original error: {_IMPORT_ERROR}"
        )


def _has_op(name: str) -> bool:
    """False for an op a stale build of _C does not define (rebuilding fixes it)."""
    try:
        getattr(torch.ops.decode_kernels, name)
        return True
    except (AttributeError, RuntimeError):
        return False


if _AVAILABLE:
    # Meta implementations so torch.compile can trace through the mutating ops
    # (reference: decode_kernels/ops.py:41-61).
    @torch.library.register_fake("decode_kernels::paged_attention_decode")
    def _(out, q, k_cache, v_cache, block_tables, seq_lens, scale, max_seq_len, tmp_out, max_logits, exp_sums):
        return None

    if _has_op("paged_attention_decode_fp8"):

        @torch.library.register_fake("decode_kernels::paged_attention_decode_fp8")
        def _(out, q, k_cache, v_cache, block_tables, seq_lens, scale, max_seq_len, tmp_out, max_logits, exp_sums,
              k_scale, v_scale):
            return None

    @torch.library.register_fake("decode_kernels::gemm_tn")
    def _(c, a, b, bias):
        return None

    @torch.library.register_fake("decode_kernels::rms_norm")
    def _(out, input, weight, eps):
        return None

    @torch.library.register_fake("decode_kernels::fused_add_rms_norm")
    def _(input, residual, weight, eps):
        return None

    @torch.library.register_fake("decode_kernels::silu_and_mul")
    def _(out, input):
        return None

    if _has_op("rotary_embedding"):

        @torch.library.register_fake("decode_kernels::rotary_embedding")
        def _(positions, query, key, head_size, cos_sin_cache, is_neox):
            return None

    if _has_op("reshape_and_cache"):

        @torch.library.register_fake("decode_kernels::reshape_and_cache")
        def _(key, value, key_cache, value_cache, slot_mapping):
            return None

    if _has_op("reshape_and_cache_fp8"):

        @torch.library.register_fake("decode_kernels::reshape_and_cache_fp8")
        def _(key, value, key_cache, value_cache, slot_mapping, k_scale, v_scale):
            return None

    if _has_op("rotary_embedding_and_cache"):

        @torch.library.register_fake("decode_kernels::rotary_embedding_and_cache")
        def _(positions, query, key, value, head_size, cos_sin_cache, is_neox, key_cache, value_cache, slot_mapping):
            return None

    if _has_op("rotary_embedding_and_cache_fp8"):

        @torch.library.register_fake("decode_kernels::rotary_embedding_and_cache_fp8")
        def _(positions, query, key, value, head_size, cos_sin_cache, is_neox, key_cache, value_cache, slot_mapping,
              k_scale, v_scale):
            return None

    if _has_op("gemm_tn_add_rms_norm"):

        @torch.library.register_fake("decode_kernels::gemm_tn_add_rms_norm")
        def _(out, a, b, bias, residual, weight, eps):
            return None

    if _has_op("gemm_tn_rotary_embedding_and_cache"):

        @torch.library.register_fake("decode_kernels::gemm_tn_rotary_embedding_and_cache")
        def _(qkv, a, b, bias, positions, query, key, value, head_size, cos_sin_cache, is_neox, key_cache,
              value_cache, slot_mapping):
            return None

    if _has_op("gemm_tn_rotary_embedding_and_cache_fp8"):

        @torch.library.register_fake("decode_kernels::gemm_tn_rotary_embedding_and_cache_fp8")
        def _(qkv, a, b, bias, positions, query, key, value, head_size, cos_sin_cache, is_neox, key_cache,
              value_cache, slot_mapping, k_scale, v_scale):
            return None


# ---------------------------------------------------------------------------
# Paged attention
# ---------------------------------------------------------------------------
def num_partitions(max_seq_len: int) -> int:
    """Workspace slots needed for sequences up to ``max_seq_len`` tokens."""
    return max(1, math.ceil(max_seq_len / PARTITION_SIZE))


def alloc_workspace(num_seqs: int, num_q_heads: int, head_dim: int, max_seq_len: int, device) -> tuple:
    """Split-K buffers ``(tmp_out, max_logits, exp_sums)``; empty tensors when
    no sequence can exceed one partition (reference: decode_kernels/ops.py:71-80)."""
    if max_seq_len <= PARTITION_SIZE:
        empty = torch.empty(0, dtype=torch.float32, device=device)
        return empty, empty, empty
    parts = num_partitions(max_seq_len)
    tmp_out = torch.empty(num_seqs, num_q_heads, parts, head_dim, dtype=torch.float32, device=device)
    max_logits = torch.empty(num_seqs, num_q_heads, parts, dtype=torch.float32, device=device)
    exp_sums = torch.empty_like(max_logits)
    return tmp_out, max_logits, exp_sums


def paged_attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
    max_seq_len: int | None = None,
    out: torch.Tensor | None = None,
    workspace: tuple | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Single-token decode attention over a paged KV cache.

    q: [num_seqs, num_q_heads, head_dim]; k_cache / v_cache:
    [num_blocks, block_size, num_kv_heads, head_dim] with any strides on the
    first three dims (NHD, HND and vLLM's interleaved K|V views are read in
    place); block_tables: [num_seqs, max_blocks] int32; seq_lens: [num_seqs]
    int32. ``max_seq_len`` must bound every entry of seq_lens; passing it
    avoids a device-to-host sync (reference: decode_kernels/ops.py:83-116).

    An fp8 cache (``torch.float8_e4m3fn``, vLLM's fp8 KV cache) is read as
    K = k_scale * k_cache and V = v_scale * v_cache with q / out in fp16 or
    bf16 (``paged_attention_decode_fp8``; the reference has no fp8 path).
    """
    _require()
    num_seqs, num_q_heads, head_dim = q.shape
    if scale is None:
        scale = head_dim**-0.5
    if max_seq_len is None:
        max_seq_len = int(seq_lens[:num_seqs].max().item()) if num_seqs > 0 else 0
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = alloc_workspace(num_seqs, num_q_heads, head_dim, max_seq_len, q.device)
    tmp_out, max_logits, exp_sums = workspace
    if k_cache.dtype == torch.float8_e4m3fn:
        torch.ops.decode_kernels.paged_attention_decode_fp8(
            out, q, k_cache, v_cache, block_tables, seq_lens, float(scale), int(max_seq_len), tmp_out, max_logits,
            exp_sums, float(k_scale), float(v_scale)
        )
        return out
    if k_scale != 1.0 or v_scale != 1.0:
        raise ValueError("k_scale / v_scale apply to an fp8 (float8_e4m3fn) KV cache only")
    torch.ops.decode_kernels.paged_attention_decode(
        out, q, k_cache, v_cache, block_tables, seq_lens, float(scale), int(max_seq_len), tmp_out, max_logits, exp_sums
    )
    return out


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def gemm(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """``a @ b.T + bias`` (nn.Linear semantics) on MFMA. a: [..., K], b: [N, K]
    (reference: decode_kernels/ops.py:122-132)."""
    _require()
    lead = a.shape[:-1]
    a2 = a.reshape(-1, a.shape[-1])
    if a2.stride(-1) != 1:
        a2 = a2.contiguous()
    if out is None:
        out = torch.empty(a2.shape[0], b.shape[0], dtype=a.dtype, device=a.device)
    torch.ops.decode_kernels.gemm_tn(out, a2, b, bias)
    return out.view(*lead, b.shape[0])


# ---------------------------------------------------------------------------
# Norm / activation (vLLM-compatible signatures)
# ---------------------------------------------------------------------------
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, out: torch.Tensor | None = None):
    _require()
    if out is None:
        out = torch.empty_like(x)
    torch.ops.decode_kernels.rms_norm(out, x, weight, float(eps))
    return out


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6):
    """In place: residual += x (rounded to the model dtype); x = rms_norm(residual) * weight.
    Returns (x, residual)."""
    _require()
    torch.ops.decode_kernels.fused_add_rms_norm(x, residual, weight, float(eps))
    return x, residual


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None):
    """silu(x[..., :d]) * x[..., d:] with d = x.shape[-1] // 2."""
    _require()
    d = x.shape[-1] // 2
    if out is None:
        out = torch.empty(*x.shape[:-1], d, dtype=x.dtype, device=x.device)
    torch.ops.decode_kernels.silu_and_mul(out, x)
    return out


# ---------------------------------------------------------------------------
# The steps around attention (vLLM's ops of the same names; not part of
# DecodeKernels, which leaves them to the serving engine)
# ---------------------------------------------------------------------------
def rotary_embedding(
    positions: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor | None,
    head_size: int,
    cos_sin_cache: torch.Tensor,
    is_neox: bool = True,
):
    """In place: rotates the first ``cos_sin_cache.shape[1]`` columns of every
    head of ``query`` (and ``key``) by the token's position. ``query`` /
    ``key`` are [tokens, heads * head_size] or [tokens, heads, head_size];
    ``cos_sin_cache`` is [max_position, rot_dim] (cos columns, then sin), in
    float32 or the query dtype. Returns (query, key)."""
    _require()
    torch.ops.decode_kernels.rotary_embedding(positions, query, key, int(head_size), cos_sin_cache, bool(is_neox))
    return query, key


def reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> None:
    """Writes key[t] / value[t] ([tokens, kv_heads, head_size]) into cache slot
    ``slot_mapping[t]`` (int64; negative = skip) of the
    [num_blocks, block_size, kv_heads, head_size] cache views -- the same views
    paged_attention_decode reads (NHD, HND or vLLM's interleaved buffer).

    Into ``torch.float8_e4m3fn`` caches the rows are quantized as vLLM's fp8
    cache write does: x / scale in fp32, saturated to +-448, rounded to
    nearest even (``reshape_and_cache_fp8``); paged_attention_decode then
    reads the cache with the same k_scale / v_scale."""
    _require()
    if key_cache.dtype == torch.float8_e4m3fn:
        torch.ops.decode_kernels.reshape_and_cache_fp8(
            key, value, key_cache, value_cache, slot_mapping, float(k_scale), float(v_scale)
        )
        return
    if k_scale != 1.0 or v_scale != 1.0:
        raise ValueError("k_scale / v_scale apply to an fp8 (float8_e4m3fn) KV cache only")
    torch.ops.decode_kernels.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping)


def rotary_embedding_and_cache(
    positions: torch.Tensor,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    head_size: int,
    cos_sin_cache: torch.Tensor,
    is_neox: bool,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
):
    """``rotary_embedding`` then ``reshape_and_cache`` of the rotated key, in one
    launch: query and key rotated in place, the rotated key and ``value``
    written to the cache slots. Same results as the two calls in sequence,
    also into ``torch.float8_e4m3fn`` caches with k_scale / v_scale.
    Returns (query, key)."""
    _require()
    if key_cache.dtype == torch.float8_e4m3fn:
        torch.ops.decode_kernels.rotary_embedding_and_cache_fp8(
            positions, query, key, value, int(head_size), cos_sin_cache, bool(is_neox), key_cache, value_cache,
            slot_mapping, float(k_scale), float(v_scale)
        )
        return query, key
    if k_scale != 1.0 or v_scale != 1.0:
        raise ValueError("k_scale / v_scale apply to an fp8 (float8_e4m3fn) KV cache only")
    torch.ops.decode_kernels.rotary_embedding_and_cache(
        positions, query, key, value, int(head_size), cos_sin_cache, bool(is_neox), key_cache, value_cache, slot_mapping
    )
    return query, key


# ---------------------------------------------------------------------------
# Decode-layer fusions: a GEMM with the op that consumes its output (no
# counterpart in DecodeKernels). At decode sizes the GEMM splits K and the
# consumer's kernel sums the partial tiles itself; the results equal the two
# calls in sequence bit for bit.
# ---------------------------------------------------------------------------
def gemm_add_rms_norm(
    a: torch.Tensor,
    b: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
):
    """``out = gemm(a, b, bias)`` then ``fused_add_rms_norm(out, residual, weight,
    eps)`` (residual updated in place): the o projection into the
    post-attention norm, or the down projection into the next layer's input
    norm. a: [M, K], b: [N, K], residual: [M, N]. Returns (out, residual)."""
    _require()
    if out is None:
        out = torch.empty(a.shape[0], b.shape[0], dtype=a.dtype, device=a.device)
    torch.ops.decode_kernels.gemm_tn_add_rms_norm(out, a, b, bias, residual, weight, float(eps))
    return out, residual


def gemm_rotary_embedding_and_cache(
    a: torch.Tensor,
    b: torch.Tensor,
    qkv: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    positions: torch.Tensor,
    head_size: int,
    cos_sin_cache: torch.Tensor,
    is_neox: bool,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    bias: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
):
    """``qkv = gemm(a, b, bias)`` (the fused q | k | v projection, [tokens,
    (num_q_heads + 2 num_kv_heads) head_size] or wider), then
    ``rotary_embedding_and_cache`` of its q, k and v columns: q and k rotated
    in place in ``qkv``, the rotated k and v written to the cache slots (also
    ``torch.float8_e4m3fn`` caches with k_scale / v_scale). Returns (query,
    key, value) as views of ``qkv``."""
    _require()
    hq, hkv, d = int(num_q_heads), int(num_kv_heads), int(head_size)
    query = qkv[:, : hq * d]
    key = qkv[:, hq * d : (hq + hkv) * d]
    value = qkv[:, (hq + hkv) * d : (hq + 2 * hkv) * d]
    if key_cache.dtype == torch.float8_e4m3fn:
        torch.ops.decode_kernels.gemm_tn_rotary_embedding_and_cache_fp8(
            qkv, a, b, bias, positions, query, key, value, d, cos_sin_cache, bool(is_neox), key_cache, value_cache,
            slot_mapping, float(k_scale), float(v_scale)
        )
    else:
        if k_scale != 1.0 or v_scale != 1.0:
            raise ValueError("k_scale / v_scale apply to an fp8 (float8_e4m3fn) KV cache only")
        torch.ops.decode_kernels.gemm_tn_rotary_embedding_and_cache(
            qkv, a, b, bias, positions, query, key, value, d, cos_sin_cache, bool(is_neox), key_cache, value_cache,
            slot_mapping
        )
    return query, key, value
