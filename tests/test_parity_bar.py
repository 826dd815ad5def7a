"""CPU tests of the attention acceptance bar (``tests/parity.py``).

The bar is max(MAX_ABS, half_ulp(ref) + s), where s is the fp32 evaluation
slack of attention. These tests check both directions at an fp16 rounding
midpoint. A correct fp32 result that lies a few fp32 ulps on the other side
of the midpoint from the oracle's rounds to the other neighbour, and that
output passes. An output a whole ulp off the correctly rounded value fails.
The same holds away from midpoints and for bf16.
"""

import math

import pytest
import torch

from parity import (
    ERRORS,
    MAX_ABS,
    P_SPLIT_REL,
    assert_max_abs,
    attention_bar,
    attention_f32,
    attention_slack,
    bar,
)


@pytest.fixture(autouse=True)
def _keep_report_clean():
    """These checks fail on purpose; keep them out of the run's parity report."""
    n = len(ERRORS)
    yield
    del ERRORS[n:]


FP16_ULP_16 = 2.0**-6  # spacing of fp16 in [16, 32)
BF16_ULP_8 = 2.0**-4  # spacing of bf16 in [8, 16)


def _ref(values, lens, abs_v_mean, calls=None):
    """A stand-in oracle output [S, 1, n] carrying the slack hook of attention_f32."""
    ref = torch.tensor(values, dtype=torch.float32).view(len(lens), 1, -1)
    e = torch.tensor(abs_v_mean, dtype=torch.float32).view_as(ref)
    sl = torch.tensor(lens, dtype=torch.int32)

    def slack(dtype):
        if calls is not None:
            calls.append(dtype)
        return attention_slack(e, sl, dtype)

    ref.dk_attn_slack = slack
    return ref


def test_fp16_midpoint_crossing_passes_with_slack_only():
    # The oracle's fp32 value lies 1.5e-6 above the midpoint of 16 and
    # 16 + 2^-6. A correct fp32 result 1e-6 below the midpoint rounds to 16.
    mid = 16.0 + FP16_ULP_16 / 2
    ref = _ref([mid + 1.5e-6], [131072], [16.0])
    got = torch.tensor([16.0], dtype=torch.float16).view(1, 1, 1)
    plain = bar(ref, torch.float16)
    assert (got.float() - ref).abs().item() > plain.item(), "case must fail without the slack"
    assert_max_abs(got, ref, torch.float16, "midpoint crossing")


@pytest.mark.parametrize("offset", [0.0, 1.5e-6, 0.001, FP16_ULP_16 / 2 - 1e-4])
def test_fp16_one_ulp_off_fails(offset):
    # The correctly rounded output is 16 + 2^-6 (ref at or above the midpoint,
    # ties to even excluded by the offsets). One ulp above it is wrong.
    ref = _ref([16.0 + FP16_ULP_16 / 2 + offset], [131072], [16.0])
    correct = ref.to(torch.float16)
    assert correct.item() == 16.0 + FP16_ULP_16 or offset == 0.0
    wrong = torch.tensor([16.0 + 2 * FP16_ULP_16], dtype=torch.float16).view(1, 1, 1)
    with pytest.raises(AssertionError):
        assert_max_abs(wrong, ref, torch.float16, "one ulp off")
    assert_max_abs(correct, ref, torch.float16, "correctly rounded")


def test_fp16_one_ulp_off_away_from_midpoint_fails():
    ref = _ref([16.001], [4096], [16.0])
    assert_max_abs(torch.tensor([16.0], dtype=torch.float16).view(1, 1, 1), ref, torch.float16)
    with pytest.raises(AssertionError):
        assert_max_abs(torch.tensor([16.0 + FP16_ULP_16], dtype=torch.float16).view(1, 1, 1), ref, torch.float16)


def test_bf16_midpoint_and_one_ulp_off():
    mid = 8.0 + BF16_ULP_8 / 2
    ref = _ref([mid + 2e-6], [32768], [8.0])
    assert bar(ref, torch.bfloat16).item() == pytest.approx(BF16_ULP_8 / 2)
    assert_max_abs(torch.tensor([8.0], dtype=torch.bfloat16).view(1, 1, 1), ref, torch.bfloat16)
    with pytest.raises(AssertionError):
        assert_max_abs(torch.tensor([8.0 + 2 * BF16_ULP_8], dtype=torch.bfloat16).view(1, 1, 1), ref, torch.bfloat16)


def test_slack_stays_below_half_ulp_and_max_abs():
    # The largest slack the benchmark configurations can ask for: 128K tokens,
    # outputs (and E_p|v|) up to 8 x the N(0,1) tail.
    for dtype, hu in ((torch.float16, FP16_ULP_16 / 2), (torch.bfloat16, BF16_ULP_8 / 2)):
        s = attention_slack(torch.tensor([[[40.0]]]), torch.tensor([131072]), dtype).item()
        assert s < MAX_ABS[dtype] / 2 and s < hu / 2, (dtype, s)


def test_slack_only_evaluated_where_half_ulp_is_in_force():
    calls = []
    small = _ref([1.0, -3.5, 7.9], [100], [1.0, 3.5, 7.9], calls)  # fp16 half ulp <= 2^-8 < 5e-3 / 2
    assert torch.equal(attention_bar(small, torch.float16), torch.full((1, 1, 3), MAX_ABS[torch.float16]))
    assert calls == []
    large = _ref([1.0, 20.0], [100], [1.0, 20.0], calls)
    attention_bar(large, torch.float16)
    assert calls == [torch.float16]


def test_attention_f32_slack_matches_its_definition():
    # One KV head of two sequences: the first has one token (E_p|v| = |v|),
    # the second two tokens with q = 0 (equal weights: E_p|v| = mean |v|).
    d, bs = 64, 16
    g = torch.Generator().manual_seed(0)
    k = torch.randn(2, bs, 1, d, generator=g, dtype=torch.float16)
    v = (torch.randn(2, bs, 1, d, generator=g) * 20).to(torch.float16)
    q = torch.zeros(2, 1, d, dtype=torch.float16)
    q[0] = torch.randn(d, generator=g).to(torch.float16)
    bt = torch.tensor([[0], [1]], dtype=torch.int32)
    lens = torch.tensor([1, 2], dtype=torch.int32)
    ref = attention_f32(q, k, v, bt, lens)
    s = ref.dk_attn_slack(torch.float16)
    vf = v.float()
    want0 = vf[0, 0, 0].abs() * (2.0**-23 * (1 + 64))
    want1 = (vf[1, 0, 0].abs() + vf[1, 1, 0].abs()) / 2 * (2.0**-23 * (math.sqrt(2) + 64))
    torch.testing.assert_close(s[0, 0], want0, rtol=1e-6, atol=0)
    torch.testing.assert_close(s[1, 0], want1, rtol=1e-6, atol=0)
    sb = ref.dk_attn_slack(torch.bfloat16)
    torch.testing.assert_close(sb[0, 0], vf[0, 0, 0].abs() * (2.0**-23 * 65 + P_SPLIT_REL[torch.bfloat16]),
                               rtol=1e-6, atol=0)
