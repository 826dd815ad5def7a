"""Shared helpers of the GPU parity tests: oracle evaluation on the CPU and the
tolerances of the acceptance bar.

* attention and GEMM: abs error against the *unrounded* fp32 oracle of at
  most max(2e-2, half an ulp) for bf16 and max(5e-3, half an ulp) for fp16,
  the ulp of the model dtype taken at the reference value. Half an ulp is the
  final rounding to bf16/fp16 that the reference itself performs
  (``.to(q.dtype)``); it exceeds 5e-3 only once |out| >= 16 in fp16 (attention
  over outlier V rows), where a correctly rounded result may sit that far from
  the fp32 value;
* GEMM, in addition: the spread of two fp32 accumulations of the same dot
  products in different orders (the kernel's K walk against the oracle's),
  2^-23 * sqrt(K) * (|A| |B|^T + |bias|) elementwise -- a random-walk bound
  on the K roundings of each of the two sums. It matters only where the exact
  value sits within that distance of a rounding midpoint of the model dtype
  and |C| >= 8 (bf16), where half an ulp is the bar: there two correct fp32
  sums may round to the two neighbours;
* norms and activation: at most 1 ulp of the model dtype from the oracle's
  (rounded) output; the fused residual is bit-exact.
"""

from __future__ import annotations

import os

import torch

from oracle.reference import (
    fused_add_rms_norm_reference,
    gemm_reference,
    paged_attention_reference,
    rms_norm_reference,
    silu_and_mul_reference,
)

MAX_ABS = {torch.bfloat16: 2e-2, torch.float16: 5e-3}

# Every assert_max_abs call appends (what, dtype, max abs error, worst error / bar);
# tests/conftest.py prints them at the end of the run and, when DK_PARITY_REPORT
# names a file, writes them there as JSON lines.
ERRORS: list[dict] = []


def attention_f32(q, k_cache, v_cache, block_tables, seq_lens, scale=None) -> torch.Tensor:
    """fp32 oracle output (no final rounding), computed on the CPU."""
    return paged_attention_reference(
        q.float().cpu(), k_cache.float().cpu(), v_cache.float().cpu(), block_tables.cpu(), seq_lens.cpu(), scale
    )


def gemm_slack(a, b, bias=None) -> torch.Tensor:
    """2^-23 sqrt(K) (|A| |B|^T + |bias|): the fp32 accumulation-order slack of A B^T + bias."""
    k = a.shape[-1]
    mag = a.float().abs().reshape(-1, k) @ b.float().abs().t()
    if bias is not None:
        mag = mag + bias.float().abs()
    return mag * (2.0**-23 * k**0.5)


def _with_slack(ref: torch.Tensor, slack: torch.Tensor) -> torch.Tensor:
    ref.dk_slack = slack  # read by assert_max_abs
    return ref


def gemm_f32(a, b, bias=None) -> torch.Tensor:
    """fp32 oracle A B^T (+ bias) on the CPU, carrying its accumulation slack."""
    ac, bc = a.float().cpu(), b.float().cpu()
    biasc = None if bias is None else bias.float().cpu()
    return _with_slack(gemm_reference(ac, bc, biasc), gemm_slack(ac, bc, biasc))


def gemm_f32_gpu(a, b, bias=None) -> torch.Tensor:
    """fp32 A B^T (+ bias) on the GPU (a 2-D mm of contiguous fp32 operands), for
    shapes where the CPU oracle would take minutes; carries the same slack."""
    ref = torch.mm(a.float().reshape(-1, a.shape[-1]), b.float().t().contiguous())
    if bias is not None:
        ref = ref + bias.float()
    return _with_slack(ref, gemm_slack(a, b, bias))


def half_ulp(ref_f32: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Half the spacing of `dtype` at |ref| (the worst-case rounding of a correct result)."""
    a = ref_f32.float().abs().to(dtype)
    return 0.5 * (torch.nextafter(a, torch.full_like(a, float("inf"))) - a).float()


def bar(ref_f32: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Elementwise acceptance bar: max(MAX_ABS[dtype], half an ulp of dtype at |ref|)."""
    return half_ulp(ref_f32, dtype).clamp(min=MAX_ABS[dtype])


def assert_max_abs(got: torch.Tensor, ref_f32: torch.Tensor, dtype: torch.dtype, what: str = "") -> float:
    """Asserts |got - ref| <= max(MAX_ABS[dtype], half_ulp(ref)) (+ a GEMM
    reference's accumulation slack) elementwise; returns the max abs error."""
    assert torch.isfinite(got).all(), f"{what} non-finite output"
    if got.numel() == 0:
        return 0.0
    slack = getattr(ref_f32, "dk_slack", None)
    ref = ref_f32.float().cpu()
    diff = (got.float().cpu() - ref).abs()
    tol = bar(ref, dtype)
    if slack is not None:
        tol = tol + slack.float().cpu().reshape(tol.shape)
    ratio = diff / tol
    worst = int(ratio.argmax())
    ERRORS.append({"what": what or "(unnamed)", "dtype": str(dtype).replace("torch.", ""),
                   "max_abs_err": diff.max().item(), "worst_err_over_bar": ratio.flatten()[worst].item(),
                   "test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]})
    assert ratio.flatten()[worst].item() <= 1.0, (
        f"{what} abs error {diff.flatten()[worst].item():.3e} at |ref| = {ref.flatten()[worst].abs().item():.3g} "
        f"exceeds max({MAX_ABS[dtype]:.0e}, half an ulp){' + slack' if slack is not None else ''} = "
        f"{tol.flatten()[worst].item():.3e} ({dtype})"
    )
    return diff.max().item()


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Elementwise distance in units in the last place between two 16-bit float tensors."""
    assert a.dtype == b.dtype and a.dtype in (torch.float16, torch.bfloat16)

    def key(t):
        bits = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        mag = bits & 0x7FFF
        return torch.where(bits >= 0x8000, -mag, mag)

    return (key(a.cpu()) - key(b.cpu())).abs()


def assert_ulp(got: torch.Tensor, ref: torch.Tensor, max_ulp: int = 1, what: str = "") -> int:
    d = int(ulp_distance(got, ref).max().item()) if got.numel() else 0
    assert d <= max_ulp, f"{what} {d} ulp from the oracle (> {max_ulp})"
    return d


__all__ = [
    "ERRORS",
    "MAX_ABS",
    "bar",
    "assert_max_abs",
    "assert_ulp",
    "attention_f32",
    "fused_add_rms_norm_reference",
    "gemm_f32",
    "gemm_f32_gpu",
    "rms_norm_reference",
    "silu_and_mul_reference",
    "ulp_distance",
]
