"""Pins oracle.envelope: hand-computed limits and a planted error that must fail."""

import torch

from oracle.envelope import gradient_limit, quantization_atol, rel_frobenius


def test_quantization_term_is_fp32_roundtrip_of_point_three():
    ref = torch.tensor([0.0, 1.0, -2.0])
    # (x + 0.3 - 0.3) - x in fp32 is at most one ulp of |x| + 0.3
    q = quantization_atol(ref)
    assert 0 <= q <= 2 * 2.0 ** -21
    assert quantization_atol(torch.zeros(4)) == 2 * abs(float(torch.tensor(0.3) - 0.3))


def test_gradient_limit_is_twice_baseline_plus_quantization():
    ref = torch.tensor([1.0, -1.0, 0.5])
    base = ref + torch.tensor([0.01, -0.02, 0.0])
    lim = gradient_limit(ref, base)
    assert abs(lim - (2 * 0.02 + quantization_atol(ref))) < 1e-7


def test_planted_error_fails_the_rule():
    g = torch.Generator().manual_seed(0)
    ref = torch.randn(1000, generator=g)
    base = ref + 1e-3 * torch.randn(1000, generator=g)
    good = ref + 1e-3 * torch.randn(1000, generator=g)
    bad = good.clone()
    bad[17] += 0.1
    lim = gradient_limit(ref, base)
    assert (good - ref).abs().max() <= lim
    assert (bad - ref).abs().max() > lim


def test_rel_frobenius():
    ref = torch.tensor([3.0, 4.0])
    assert rel_frobenius(ref, ref) == 0
    assert abs(rel_frobenius(torch.tensor([3.0, 5.0]), ref) - 0.2) < 1e-12
