"""Shared helpers of the GPU parity tests: oracle evaluation on the CPU and the
tolerances of the acceptance bar.

* attention and GEMM: abs error against the *unrounded* fp32 oracle of at
  most max(2e-2, half an ulp) for bf16 and max(5e-3, half an ulp) for fp16,
  the ulp of the model dtype taken at the reference value. Half an ulp is the
  final rounding to bf16/fp16 that the reference itself performs
  (``.to(q.dtype)``). It exceeds 5e-3 only once |out| >= 16 in fp16: the
  spacing of fp16 in [16, 32) is 2^-6, so a correctly rounded output sits up
  to 2^-7 = 7.8125e-3 from the fp32 value, and no fp16 output there can meet
  5e-3 unless the fp32 value happens to lie near an fp16 number. Attention
  over the x8 outlier V rows of the long-context configs produces such
  outputs (bf16: |out| >= 8);
* attention, in addition, where the half-ulp bar is in force: the spread of
  two correct fp32 evaluations, s = (2^-23 (sqrt(L) + 64) + rho) E_p|v|, added
  to the half ulp: max(MAX_ABS, half_ulp + s). E_p|v| is the oracle's output
  for |V| (the softmax-weighted mean of |v|, the attention analogue of
  |A| |B|^T below); sqrt(L) 2^-23 is the random-walk bound on the roundings of
  the weighted sum over the sequence's L tokens; 64 fp32 ulps cover the
  relative error of each weight exp2(x - m) from the rounded logit x (|x| up
  to ~90 in log2 units) and the exp; rho is the relative error of the weights
  as the kernel feeds them to the P.V MFMA in the model dtype, P_hi + P_lo:
  2^-17 for bf16 (two 8-bit roundings), below fp32's for fp16. Without it an
  fp32 result 1.5e-6 on the other side of an fp16 rounding midpoint than the
  oracle's fails the bar although both are correct (the 128K fp16 config sat
  at 1.000 of the half-ulp bar). s stays below half an ulp wherever it is
  used (asserted), so an output a whole ulp off the correctly rounded value
  still fails unless the exact value lies within s of a midpoint;
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


# Relative error of the softmax weights as the attention kernel multiplies them
# by V: P_hi + P_lo in the model dtype (bf16: two roundings of 2^-9 each, within
# 2^-17; fp16: within 2^-22, below the fp32 terms of the slack).
P_SPLIT_REL = {torch.bfloat16: 2.0**-17, torch.float16: 0.0}


def attention_slack(abs_v_mean: torch.Tensor, seq_lens: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """s = (2^-23 (sqrt(L) + 64) + rho) E_p|v| for outputs [S, Hq, D] of sequences
    of lengths L (E_p|v| = the oracle's output for |V|)."""
    root = seq_lens.cpu().clamp(min=1).double().sqrt().float()
    root = root.view(-1, *([1] * (abs_v_mean.dim() - 1)))
    return abs_v_mean.float() * (2.0**-23 * (root + 64.0) + P_SPLIT_REL[dtype])


def attention_f32(q, k_cache, v_cache, block_tables, seq_lens, scale=None) -> torch.Tensor:
    """fp32 oracle output (no final rounding), computed on the CPU. It carries
    the fp32 evaluation slack (``attention_slack``), computed only when the
    half-ulp bar is in force for some output (an oracle pass over |V|)."""
    qc, kc, vc = q.float().cpu(), k_cache.float().cpu(), v_cache.float().cpu()
    bt, sl = block_tables.cpu(), seq_lens.cpu()
    ref = paged_attention_reference(qc, kc, vc, bt, sl, scale)

    abs_v_mean: list[torch.Tensor] = []  # the |V| pass, run at most once per reference

    def slack(dtype: torch.dtype) -> torch.Tensor:
        if not abs_v_mean:
            abs_v_mean.append(paged_attention_reference(qc, kc, vc.abs(), bt, sl, scale))
        return attention_slack(abs_v_mean[0], sl, dtype)

    ref.dk_attn_slack = slack  # read by assert_max_abs
    return ref


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


def bar(ref_f32: torch.Tensor, dtype: torch.dtype, slack: torch.Tensor | None = None) -> torch.Tensor:
    """Elementwise acceptance bar: max(MAX_ABS[dtype], half an ulp of dtype at
    |ref| (+ an attention reference's fp32 slack))."""
    hu = half_ulp(ref_f32, dtype)
    if slack is not None:
        hu = hu + slack.float().reshape(hu.shape)
    return hu.clamp(min=MAX_ABS[dtype])


def attention_bar(ref_f32: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The bar of an ``attention_f32`` reference: max(MAX_ABS, half_ulp + s).
    The slack is evaluated only where half an ulp exceeds MAX_ABS / 2; elsewhere
    half_ulp + s < MAX_ABS, since s < MAX_ABS / 2 (asserted)."""
    ref = ref_f32.float().cpu()
    hu = half_ulp(ref, dtype)
    fn = getattr(ref_f32, "dk_attn_slack", None)
    if fn is None or not bool((hu > MAX_ABS[dtype] / 2).any()):
        return hu.clamp(min=MAX_ABS[dtype])
    s = fn(dtype).reshape(hu.shape)
    assert float(s.max()) < MAX_ABS[dtype] / 2, f"attention slack {float(s.max()):.3e} is not small"
    used = hu + s > MAX_ABS[dtype]
    assert bool((s[used] < hu[used]).all()), "attention slack reaches half an ulp"
    return (hu + s).clamp(min=MAX_ABS[dtype])


def assert_max_abs(got: torch.Tensor, ref_f32: torch.Tensor, dtype: torch.dtype, what: str = "") -> float:
    """Asserts |got - ref| <= max(MAX_ABS[dtype], half_ulp(ref) (+ an attention
    reference's slack)) (+ a GEMM reference's accumulation slack) elementwise;
    returns the max abs error."""
    assert torch.isfinite(got).all(), f"{what} non-finite output"
    if got.numel() == 0:
        return 0.0
    slack = getattr(ref_f32, "dk_slack", None)
    ref = ref_f32.float().cpu()
    diff = (got.float().cpu() - ref).abs()
    tol = attention_bar(ref_f32, dtype) if hasattr(ref_f32, "dk_attn_slack") else bar(ref, dtype)
    if slack is not None:
        tol = tol + slack.float().cpu().reshape(tol.shape)
    ratio = diff / tol
    worst = int(ratio.argmax())
    rec = {"what": what or "(unnamed)", "dtype": str(dtype).replace("torch.", ""),
           "max_abs_err": diff.max().item(), "worst_err_over_bar": ratio.flatten()[worst].item(),
           "test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]}
    if hasattr(ref_f32, "dk_attn_slack"):  # the same error against the bar without the slack
        rec["worst_err_over_bar_without_slack"] = (diff / bar(ref, dtype)).max().item()
    ERRORS.append(rec)
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
    "P_SPLIT_REL",
    "attention_bar",
    "attention_slack",
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
