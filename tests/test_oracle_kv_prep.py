"""Pins of the K/V preparation oracle (oracle/kv_prep.py) on the CPU.

* The reference test's explicit formulation (tests/test_reference.py:370-407):
  float64 source (1, 2, 3, 512), weight linspace(0.75, 1.25), RoPE angles
  linspace(0.01, 0.91) over 128 rotary dims; K and V and the autograd
  gradients of source and weight for linspace output gradients.
* torch autograd of the float64 forward equals the explicit adjoint.
* Closed forms: unit weight with cos = 1, sin = 0 makes K equal V; the rotation
  keeps the norm of every (x_i, x_{i+64}) pair; V rows have unit RMS at eps = 0.
* The dtype-faithful restatement equals the float64 map on float64 inputs.
"""

import pytest
import torch

from oracle.kv_prep import kv_prep_backward_fp64, kv_prep_fp64, reference_kv_prep


def _explicit_global_kv(source, weight, cos, sin):
    # the formulation of the reference test, written out independently
    inverse_rms = torch.rsqrt(source.float().square().mean(dim=-1, keepdim=True) + 1e-6)
    normalized = source * inverse_rms
    k_before_rope = normalized * weight.float()
    k_rotary, k_pass = k_before_rope[..., :128], k_before_rope[..., 128:]
    first, second = k_rotary.chunk(2, dim=-1)
    rotated_half = torch.cat((-second, first), dim=-1)
    expected_k = torch.cat((k_rotary * cos[:, None] + rotated_half * sin[:, None], k_pass), dim=-1)
    return expected_k.to(source.dtype), normalized.to(source.dtype)


def _case():
    source = torch.randn(1, 2, 3, 512, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    weight = torch.linspace(0.75, 1.25, 512, dtype=torch.float64)
    angles = torch.linspace(0.01, 0.91, 3 * 128, dtype=torch.float64).reshape(1, 3, 128)
    return source, weight, torch.cos(angles), torch.sin(angles)


def test_reference_test_forward_values():
    source, weight, cos, sin = _case()
    for fn in (reference_kv_prep, kv_prep_fp64):
        k, v = fn(source, k_norm_weight=weight, cos=cos, sin=sin, partial_rotary_factor=0.25)
        ek, ev = _explicit_global_kv(source, weight, cos, sin)
        torch.testing.assert_close(k, ek)
        torch.testing.assert_close(v, ev)


def test_explicit_adjoint_matches_the_reference_test_and_autograd():
    source, weight, cos, sin = _case()
    k_shape = source.shape
    grad_k = torch.linspace(-1.0, 1.0, source.numel(), dtype=torch.float64).reshape(k_shape)
    grad_v = torch.linspace(0.5, 1.5, source.numel(), dtype=torch.float64).reshape(k_shape)
    dz, dw = kv_prep_backward_fp64(source, grad_k, grad_v, k_norm_weight=weight, cos=cos, sin=sin)
    # the reference test's route: autograd through its explicit formulation
    s_ref = source.clone().requires_grad_(True)
    w_ref = weight.clone().requires_grad_(True)
    ek, ev = _explicit_global_kv(s_ref, w_ref, cos, sin)
    torch.autograd.backward((ek, ev), (grad_k, grad_v))
    # that formulation takes the inverse RMS of an fp32 copy of the source
    # (source.float()), so it agrees with the float64 adjoint to fp32 precision
    torch.testing.assert_close(dz, s_ref.grad, rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(dw, w_ref.grad, rtol=1e-5, atol=1e-7)
    # and autograd through the oracle's own forward, at other shapes and widths
    gen = torch.Generator().manual_seed(9)
    for shape, factor in (((2, 3, 5, 512), 0.25), ((1, 1, 7, 512), 0.5), ((1, 2, 4, 512), 0.0)):
        z = torch.randn(shape, dtype=torch.float64, generator=gen).requires_grad_(True)
        w = torch.rand(512, dtype=torch.float64, generator=gen).add_(0.5).requires_grad_(True)
        rot = int(512 * factor)
        ang = torch.rand(shape[0], shape[2], max(rot, 2), dtype=torch.float64, generator=gen)[..., :rot]
        c, s = torch.cos(ang), torch.sin(ang)
        k, v = kv_prep_fp64(z, k_norm_weight=w, cos=c, sin=s, partial_rotary_factor=factor)
        gk = torch.randn(shape, dtype=torch.float64, generator=gen)
        gv = torch.randn(shape, dtype=torch.float64, generator=gen)
        torch.autograd.backward((k, v), (gk, gv))
        dz, dw = kv_prep_backward_fp64(z.detach(), gk, gv, k_norm_weight=w.detach(), cos=c, sin=s,
                                       partial_rotary_factor=factor)
        torch.testing.assert_close(dz, z.grad)
        torch.testing.assert_close(dw, w.grad)


def test_closed_forms():
    gen = torch.Generator().manual_seed(4)
    z = torch.randn(1, 2, 6, 512, dtype=torch.float64, generator=gen)
    ones = torch.ones(512, dtype=torch.float64)
    k, v = kv_prep_fp64(z, k_norm_weight=ones, cos=torch.ones(1, 6, 128, dtype=torch.float64),
                        sin=torch.zeros(1, 6, 128, dtype=torch.float64), eps=0.0)
    torch.testing.assert_close(k, v)
    torch.testing.assert_close(v.square().mean(dim=-1), torch.ones(1, 2, 6, dtype=torch.float64))
    ang = torch.rand(1, 6, 64, dtype=torch.float64, generator=gen)
    cos = torch.cat((torch.cos(ang), torch.cos(ang)), dim=-1)  # RoPE tables repeat over halves
    sin = torch.cat((torch.sin(ang), torch.sin(ang)), dim=-1)
    k, v = kv_prep_fp64(z, k_norm_weight=ones, cos=cos, sin=sin)
    pair_k = k[..., :64].square() + k[..., 64:128].square()
    pair_v = v[..., :64].square() + v[..., 64:128].square()
    torch.testing.assert_close(pair_k, pair_v)
    torch.testing.assert_close(k[..., 128:], v[..., 128:])


def test_rotary_width_must_be_even():
    source, weight, cos, sin = _case()
    with pytest.raises(ValueError, match="even integer"):
        reference_kv_prep(source, k_norm_weight=weight, cos=cos, sin=sin,
                          partial_rotary_factor=0.3)
