"""Numerical acceptance envelopes -- TEST INFRASTRUCTURE ONLY.

Restates the reference's M1 envelopes:

* local forward: O ``atol=0.03125, rtol=0.02``; LSE ``atol=0.125``
  (tests/test_h100_fa4.py:15-17);
* global forward: O ``atol=0.0625, rtol=0.03``; LSE ``atol=0.25``
  (tests/test_h100_fa4.py:18-20; scripts/probe_h100_global_backward.py:14-16);
* gradients, upstream-relative rule: ``max|g - g_ref| <= 2 * max|g_bf16 - g_ref|
  + 2 * max|(g_ref + 0.3 - 0.3) - g_ref|`` where ``g_ref`` is the fp32/fp64
  reference and ``g_bf16`` an independent bf16 attention
  (scripts/probe_h100_local_backward.py:263-320;
  scripts/probe_h100_global_backward.py:167-196).

``rel_frobenius`` is the extra reported metric ``||x - ref||_F / ||ref||_F``.

Pinned by ``tests/test_oracle_envelope.py`` (hand-computed limits, and a planted
error that must fail the rule).
"""

from __future__ import annotations

import torch

LOCAL_OUT_ATOL = 0.03125
LOCAL_OUT_RTOL = 0.02
LOCAL_LSE_ATOL = 0.125
GLOBAL_OUT_ATOL = 0.0625
GLOBAL_OUT_RTOL = 0.03
GLOBAL_LSE_ATOL = 0.25
UPSTREAM_ERROR_MULTIPLIER = 2.0


def quantization_atol(reference: torch.Tensor) -> float:
    ref = reference.float()
    return 2.0 * ((ref + 0.3 - 0.3) - ref).abs().max().item()


def gradient_limit(reference: torch.Tensor, bf16_baseline: torch.Tensor) -> float:
    """Upstream-relative max-abs limit for one gradient tensor."""
    baseline = (bf16_baseline.float() - reference.float()).abs().max().item()
    return UPSTREAM_ERROR_MULTIPLIER * baseline + quantization_atol(reference)


def rel_frobenius(x: torch.Tensor, reference: torch.Tensor) -> float:
    ref = reference.double()
    denom = torch.linalg.vector_norm(ref).item()
    num = torch.linalg.vector_norm(x.double() - ref).item()
    return num / denom if denom > 0 else num
