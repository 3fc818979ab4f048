"""Global-layer K/V preparation oracle -- TEST INFRASTRUCTURE ONLY.

Restates the reference's ``prepare_global_kv_from_projection_source``
(``src/gemma4_fa4/reference.py:306-328``) with its helpers ``rms_norm`` (276-281),
``rotate_half`` (284-286) and ``apply_partial_rotary`` (289-303):

* ``reference_kv_prep`` runs the same torch operations in the same dtypes, so a
  bf16 source with fp32 cos / sin gives the reference's bf16 V and fp32 K;
* ``kv_prep_fp64`` is the same map in float64 with the explicit adjoint
  ``kv_prep_backward_fp64`` (dZ and dweight for given dK, dV):
    r = (mean(z^2) + eps)^(-1/2), n = z r, V = n, kn = n w,
    K = kn with RoPE on its first R dims (x cos + rotate_half(x) sin),
    g_k = RoPE adjoint of dK, g_n = g_k w + dV, dw = sum g_k n,
    dz = r g_n - (r^3 / D) z sum(g_n z).

Pinned by ``tests/test_oracle_kv_prep.py``: the reference test's explicit
formulation (tests/test_reference.py:370-407: forward values and the autograd
gradients of source and weight), torch autograd of the fp64 forward against the
explicit adjoint, and closed forms (unit weight with cos = 1, sin = 0 gives
K = V; the rotation keeps each (x_i, x_{i+R/2}) pair's norm; V rows have unit
RMS at eps = 0).
"""

from __future__ import annotations

import torch


def _rotary_dim(head_dim: int, partial_rotary_factor: float) -> int:
    width = head_dim * partial_rotary_factor
    if int(width) != width or int(width) % 2:
        raise ValueError("partial rotary width must be an even integer")
    return int(width)


def _broadcast_rope(t: torch.Tensor, ndim: int) -> torch.Tensor:
    while t.ndim < ndim:
        t = t.unsqueeze(1)
    return t


def reference_kv_prep(source, *, k_norm_weight, cos, sin, partial_rotary_factor=0.25, eps=1e-6):
    """The reference's operations in the reference's dtypes (reference.py:276-328)."""
    rot = _rotary_dim(source.shape[-1], partial_rotary_factor)

    def rms(x, w):
        ms = x.float().pow(2).mean(dim=-1, keepdim=True) + eps
        y = x * torch.pow(ms, -0.5)
        if w is not None:
            y = y * w.float()
        return y.to(x.dtype)

    k = rms(source, k_norm_weight)
    if rot:
        x_rot, x_pass = k[..., :rot], k[..., rot:]
        c = _broadcast_rope(cos, x_rot.ndim)
        s = _broadcast_rope(sin, x_rot.ndim)
        x1, x2 = x_rot.chunk(2, dim=-1)
        rotated = x_rot * c + torch.cat((-x2, x1), dim=-1) * s
        k = torch.cat((rotated, x_pass), dim=-1)
    v = rms(source, None)
    return k, v


def kv_prep_fp64(source, *, k_norm_weight, cos, sin, partial_rotary_factor=0.25, eps=1e-6):
    """K, V of the same map in float64 (no intermediate rounding)."""
    z = source.double()
    rot = _rotary_dim(z.shape[-1], partial_rotary_factor)
    r = torch.rsqrt(z.square().mean(dim=-1, keepdim=True) + eps)
    n = z * r
    kn = n * k_norm_weight.double()
    k = kn.clone()
    if rot:
        c = _broadcast_rope(cos.double(), z.ndim)
        s = _broadcast_rope(sin.double(), z.ndim)
        h = rot // 2
        x1, x2 = kn[..., :h], kn[..., h:rot]
        k[..., :h] = x1 * c[..., :h] - x2 * s[..., :h]
        k[..., h:rot] = x2 * c[..., h:] + x1 * s[..., h:]
    return k, n


def kv_prep_backward_fp64(source, dk, dv, *, k_norm_weight, cos, sin, partial_rotary_factor=0.25,
                          eps=1e-6):
    """(dZ, dweight) of kv_prep_fp64 for output gradients (dK, dV), explicitly."""
    z = source.double()
    d = z.shape[-1]
    rot = _rotary_dim(d, partial_rotary_factor)
    w = k_norm_weight.double()
    r = torch.rsqrt(z.square().mean(dim=-1, keepdim=True) + eps)
    n = z * r
    gk = dk.double().clone()
    if rot:
        c = _broadcast_rope(cos.double(), z.ndim)
        s = _broadcast_rope(sin.double(), z.ndim)
        h = rot // 2
        d1, d2 = dk.double()[..., :h], dk.double()[..., h:rot]
        gk[..., :h] = d1 * c[..., :h] + d2 * s[..., h:]
        gk[..., h:rot] = d2 * c[..., h:] - d1 * s[..., :h]
    gn = gk * w + dv.double()
    dw = (gk * n).reshape(-1, d).sum(dim=0)
    dot = (gn * z).sum(dim=-1, keepdim=True)
    dz = r * gn - (r ** 3 / d) * z * dot
    return dz, dw
