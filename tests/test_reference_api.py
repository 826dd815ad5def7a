"""GPU tests written against the reference's import name and acceptance style.

Everything here goes through ``decode_kernels`` -- the package, ``.ops``,
``.testing`` and the raw ``torch.ops.decode_kernels.*`` ops after
``import decode_kernels._C`` -- as a DecodeKernels caller would, and judges the
results the way the reference's own GPU tests do
(tests/test_kernels.py:22-241 of the reference): ``torch.testing.assert_close``
of the op's output against the oracle's output rounded to the model dtype, with
the reference's tolerances (attention fp16 atol 3e-3 / rtol 1e-2, bf16 2e-2 /
2e-2; GEMM fp16 2e-2 / 2e-2, bf16 6e-2 / 4e-2; norms and SiLU 2e-2 / 2e-2; the
fused residual exact), and the error messages it matches on. The repo's own
parity tests hold the same ops to tighter bars (``tests/parity.py``). The oracle functions have the
reference's names (``oracle.reference``; the reference's tests import them from
``decode_kernels.reference``, which this package does not ship).
"""

import pytest
import torch

import decode_kernels as dk
from decode_kernels.ops import PARTITION_SIZE
from decode_kernels.testing import make_paged_kv
from oracle.reference import (
    fused_add_rms_norm_reference,
    gemm_reference,
    paged_attention_reference,
    rms_norm_reference,
    silu_and_mul_reference,
)

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not dk.is_available(), reason="needs a GPU and the built extension")]


@pytest.fixture(autouse=True, scope="module")
def reference_extension_name():
    """The reference's callers load the ops with ``import decode_kernels._C``."""
    import decode_kernels._C  # noqa: F401

DTYPES = [torch.float16, torch.bfloat16]
ATTN_TOL = {torch.float16: dict(atol=3e-3, rtol=1e-2), torch.bfloat16: dict(atol=2e-2, rtol=2e-2)}


def _q(n, hq, d, dtype, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(n, hq, d, generator=g, device="cuda", dtype=dtype)


def _ref(q, kv, scale=None):
    return paged_attention_reference(q.cpu(), kv.k_cache.cpu(), kv.v_cache.cpu(), kv.block_tables.cpu(),
                                     kv.seq_lens.cpu(), scale)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("lens", [[1, 2, 17, 100, 255, 512], [1, 511, 512, 513, 1024, 1025, 3000, 8192]])
@pytest.mark.parametrize("group,head_dim", [(1, 64), (4, 128), (8, 128), (8, 256)])
def test_attention_through_reference_names(dtype, lens, group, head_dim):
    kv = make_paged_kv(lens, 2, head_dim, 16, dtype, "cuda")
    q = _q(len(lens), 2 * group, head_dim, dtype)
    out = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    torch.testing.assert_close(out.cpu(), _ref(q, kv), **ATTN_TOL[dtype])


@pytest.mark.parametrize("layout", ["hnd", "vllm"])
def test_attention_strided_layouts_raw_op(layout):
    """The raw op with a caller-allocated workspace of the reference's shape."""
    dtype = torch.float16
    lens = [700, 2000, 5]
    kv = make_paged_kv(lens, 2, 128, 16, dtype, "cuda", layout=layout)
    q = _q(3, 8, 128, dtype)
    parts = -(-max(lens) // PARTITION_SIZE)
    tmp = torch.empty(3, 8, parts, 128, device="cuda")
    ml = torch.empty(3, 8, parts, device="cuda")
    es = torch.empty_like(ml)
    out = torch.empty_like(q)
    torch.ops.decode_kernels.paged_attention_decode(out, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens,
                                                    128**-0.5, max(lens), tmp, ml, es)
    torch.testing.assert_close(out.cpu(), _ref(q, kv), **ATTN_TOL[dtype])


def test_attention_errors_match_reference_messages():
    kv = make_paged_kv([10], 2, 128, 16, torch.float16, "cuda")
    with pytest.raises(RuntimeError, match="GQA group"):
        dk.paged_attention_decode(_q(1, 64, 128, torch.float16), kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens)
    kv80 = make_paged_kv([10], 2, 80, 16, torch.float16, "cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        dk.paged_attention_decode(_q(1, 2, 80, torch.float16), kv80.k_cache, kv80.v_cache, kv80.block_tables,
                                  kv80.seq_lens)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (33, 1000, 520), (256, 4096, 1024)])
def test_gemm_through_reference_names(dtype, M, N, K):
    g = torch.Generator(device="cuda").manual_seed(M + N)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype)
    out = dk.gemm(a, b, bias)
    ref = gemm_reference(a.cpu(), b.cpu(), bias.cpu())
    tol = dict(atol=2e-2, rtol=2e-2) if dtype == torch.float16 else dict(atol=6e-2, rtol=4e-2)
    torch.testing.assert_close(out.cpu(), ref, **tol)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        dk.gemm(torch.randn(4, 12, device="cuda", dtype=dtype), torch.randn(8, 12, device="cuda", dtype=dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_norms_and_silu_through_reference_names(dtype):
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(64, 4096, generator=g, device="cuda", dtype=dtype)
    r = torch.randn(64, 4096, generator=g, device="cuda", dtype=dtype)
    w = (1 + 0.1 * torch.randn(4096, generator=g, device="cuda")).to(dtype)
    tol = dict(atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(dk.rms_norm(x, w, 1e-5).cpu(), rms_norm_reference(x.cpu(), w.cpu(), 1e-5), **tol)
    want_out, want_res = fused_add_rms_norm_reference(x.cpu(), r.cpu(), w.cpu(), 1e-5)
    out, res = dk.fused_add_rms_norm(x.clone(), r.clone(), w, 1e-5)
    assert torch.equal(res.cpu(), want_res)
    torch.testing.assert_close(out.cpu(), want_out, **tol)
    xs = torch.randn(64, 2 * 14336, generator=g, device="cuda", dtype=dtype)
    torch.testing.assert_close(dk.silu_and_mul(xs).cpu(), silu_and_mul_reference(xs.cpu()), **tol)


def test_ops_trace_under_torch_compile():
    """The register_fake stubs let torch.compile trace the mutating ops
    (reference: decode_kernels/ops.py:41-61)."""
    dtype = torch.bfloat16
    x = torch.randn(8, 1024, device="cuda", dtype=dtype)
    w = torch.ones(1024, device="cuda", dtype=dtype)

    def f(x, w):
        out = torch.empty_like(x)
        torch.ops.decode_kernels.rms_norm(out, x, w, 1e-6)
        return out * 2

    got = torch.compile(f, backend="aot_eager", fullgraph=True)(x, w)
    torch.testing.assert_close(got, f(x, w))
