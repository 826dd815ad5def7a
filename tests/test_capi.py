"""GPU tests through the C ABI (``include/decodekernels_amd.h``) with ctypes.

The same kernels the torch ops run, called with raw device pointers and
strides on torch's current stream: results must equal the torch-op path bit
for bit and meet the parity bar against the oracle.
"""

import ctypes

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd import capi
from decodekernels_amd.testing import make_paged_kv
from parity import assert_max_abs, assert_ulp, attention_f32, gemm_f32, rms_norm_reference, silu_and_mul_reference

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seq_lens", [[3, 200, 512], [1, 700, 2100, 0]])
def test_capi_paged_attention(dtype, seq_lens):
    kv = make_paged_kv(seq_lens, 4, 128, 16, dtype, "cuda", layout="vllm", seed=21)
    g = torch.Generator(device="cuda").manual_seed(22)
    q = torch.randn(len(seq_lens), 16, 128, generator=g, device="cuda", dtype=dtype)
    max_len = max(seq_lens)
    ws = dk.alloc_workspace(len(seq_lens), 16, 128, max_len, "cuda")
    out = torch.empty_like(q)
    p = capi.attn_params(out, q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, 128**-0.5, ws)
    rc = capi.lib().dk_paged_attention_decode(ctypes.byref(p), capi.dtype_code(dtype), 128, max_len, _stream())
    assert rc == 0, capi.last_error()
    via_torch = dk.paged_attention_decode(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens, max_seq_len=max_len)
    torch.cuda.synchronize()
    assert torch.equal(out, via_torch)
    assert_max_abs(out, attention_f32(q, kv.k_cache, kv.v_cache, kv.block_tables, kv.seq_lens), dtype)


def test_capi_gemm_and_norms():
    dtype = torch.bfloat16
    code = capi.dtype_code(dtype)
    L = capi.lib()
    g = torch.Generator(device="cuda").manual_seed(23)
    a = torch.randn(32, 4096, generator=g, device="cuda", dtype=dtype) * 0.02
    b = torch.randn(6144, 4096, generator=g, device="cuda", dtype=dtype) * 0.02
    c = torch.empty(32, 6144, device="cuda", dtype=dtype)
    rc = L.dk_gemm_tn(code, a.data_ptr(), b.data_ptr(), None, c.data_ptr(), 32, 6144, 4096, 4096, 4096, 6144, _stream())
    assert rc == 0, capi.last_error()
    assert_max_abs(c, gemm_f32(a, b), dtype)

    x = torch.randn(64, 4096, generator=g, device="cuda", dtype=dtype)
    w = (1 + 0.1 * torch.randn(4096, generator=g, device="cuda")).to(dtype)
    y = torch.empty_like(x)
    rc = L.dk_rms_norm(code, y.data_ptr(), x.data_ptr(), w.data_ptr(), 64, 4096, 4096, 4096, 1e-5, _stream())
    assert rc == 0, capi.last_error()
    assert_ulp(y, rms_norm_reference(x.cpu(), w.cpu(), 1e-5))

    r = torch.randn(64, 4096, generator=g, device="cuda", dtype=dtype)
    x2, r2 = x.clone(), r.clone()
    rc = L.dk_fused_add_rms_norm(code, x2.data_ptr(), r2.data_ptr(), w.data_ptr(), 64, 4096, 4096, 4096, 1e-5, _stream())
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    assert torch.equal(r2.cpu(), (x.cpu().float() + r.cpu().float()).to(dtype))

    xs = torch.randn(64, 2 * 14336, generator=g, device="cuda", dtype=dtype)
    ys = torch.empty(64, 14336, device="cuda", dtype=dtype)
    rc = L.dk_silu_and_mul(code, ys.data_ptr(), xs.data_ptr(), 64, 14336, 2 * 14336, 14336, _stream())
    assert rc == 0, capi.last_error()
    assert_ulp(ys, silu_and_mul_reference(xs.cpu()))


@pytest.mark.parametrize("offset,ldc_pad", [(0, 0), (0, 4), (4, 8), (1, 7)])
def test_capi_gemm_strided_output(offset, ldc_pad):
    """Tiled gemm_tn (M > 64) into a C that is a window of a larger buffer:
    row stride N + ldc_pad and a start offset of `offset` elements select the
    16-byte (aligned, ldc % 8 == 0), 8-byte and element-wise store paths. Each
    must give the contiguous result's bits and leave every element outside the
    window untouched."""
    dtype = torch.bfloat16
    code = capi.dtype_code(dtype)
    L = capi.lib()
    M, N, K = 300, 520, 264
    g = torch.Generator(device="cuda").manual_seed(24)
    a = torch.randn(M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(N, K, generator=g, device="cuda", dtype=dtype) / K**0.5
    bias = torch.randn(N, generator=g, device="cuda", dtype=dtype)
    want = torch.empty(M, N, device="cuda", dtype=dtype)
    rc = L.dk_gemm_tn(code, a.data_ptr(), b.data_ptr(), bias.data_ptr(), want.data_ptr(), M, N, K, K, K, N, _stream())
    assert rc == 0, capi.last_error()
    ldc = N + ldc_pad
    buf = torch.full((offset + M * ldc + 64,), -7.0, device="cuda", dtype=dtype)
    c_ptr = buf.data_ptr() + offset * buf.element_size()
    rc = L.dk_gemm_tn(code, a.data_ptr(), b.data_ptr(), bias.data_ptr(), c_ptr, M, N, K, K, K, ldc, _stream())
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    window = buf[offset:offset + M * ldc].view(M, ldc)
    assert torch.equal(window[:, :N], want)
    outside = torch.ones_like(buf, dtype=torch.bool)
    outside[offset:offset + M * ldc].view(M, ldc)[:, :N] = False
    assert bool((buf[outside] == -7.0).all())
    assert_max_abs(want, gemm_f32(a, b, bias), dtype)
