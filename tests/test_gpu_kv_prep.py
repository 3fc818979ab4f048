"""GPU parity of the fused global K/V preparation (g4_kv_prep_fwd / g4_kv_prep_bwd).

Forward against the reference's own operations in the reference's dtypes
(oracle ``reference_kv_prep``: bf16 source, fp32 cos / sin give bf16 V and fp32
K), run on the CPU on the same inputs: the kernel reduces the row's squares in
another order, so its inverse RMS may differ from torch's by an fp32 ulp and
move a bf16 rounding; the bar is bit-identical on at least 99.5% of the
elements and every element within one bf16 ulp of its magnitude.  Backward
against the float64 adjoint (oracle ``kv_prep_backward_fp64``) of the same
inputs: dZ is rounded to bf16 once, dweight is summed in fp32.  Also: strided
(BSHD-as-BHSD-view) sources, bf16 tables (K in bf16), per-batch tables, the
autograd route, bitwise repeatability, and K/V fed to the global attention.
"""

import pytest
import torch

from oracle.kv_prep import kv_prep_backward_fp64, reference_kv_prep

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, b, h, s, *, table_batch=1, table_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(b, h, s, 512, generator=g) * 2.0).to(torch.bfloat16)
    w = torch.rand(512, generator=g) * 0.5 + 0.75
    pos = torch.arange(s, dtype=torch.float64)[None, :, None] + 17 * torch.arange(
        table_batch, dtype=torch.float64)[:, None, None]
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float64) / 512)  # proportional RoPE
    ang = pos * torch.cat((inv, inv))[None, None, :]
    cos, sin = torch.cos(ang).to(table_dtype), torch.sin(ang).to(table_dtype)
    return z, w, cos, sin


def _k_magnitude(z, w, cos, sin):
    """Per element of K, |kn_i cos_i| + |kn_partner sin_i| (rotary dims) or |kn_i|.

    A one-ulp change of the bf16 RMSNorm output kn moves K by at most one bf16
    ulp of these terms, however much the rotation's sum cancels.
    """
    kn, _ = reference_kv_prep(z, k_norm_weight=w, cos=cos, sin=sin, partial_rotary_factor=0.0)
    kn = kn.float()
    mag = kn.abs().clone()
    c = cos.float()[:, None].abs()
    s = sin.float()[:, None].abs()
    partner = torch.cat((kn[..., 64:128], kn[..., :64]), dim=-1).abs()
    mag[..., :128] = kn[..., :128].abs() * c + partner * s
    return mag


def _ulp_check(got, want, label, min_equal=0.995, mag=None):
    got, want = got.float().cpu(), want.float().cpu()
    equal = (got == want).float().mean().item()
    # one bf16 ulp (2^-7 relative) of the value, or of the terms it sums
    lim = (want.abs() if mag is None else mag) * 2.0 ** -7 + 1e-6
    bad = int(((got - want).abs() > lim).sum())
    assert bad == 0, f"{label}: {bad} elements beyond one bf16 ulp"
    assert equal >= min_equal, f"{label}: only {equal:.4f} bit-identical"
    return equal


def _run(z, w, cos, sin, *, grads=None):
    import gemma4_fa4_amd as g

    zd = z.to(DEV).requires_grad_(grads is not None)
    wd = w.to(DEV).requires_grad_(grads is not None)
    k, v = g.prepare_global_kv_from_projection_source(zd, k_norm_weight=wd, cos=cos.to(DEV),
                                                      sin=sin.to(DEV))
    if grads is not None:
        torch.autograd.backward((k, v), tuple(t.to(DEV) for t in grads))
    torch.cuda.synchronize()
    return k, v, zd.grad, wd.grad


@pytest.mark.parametrize("b,h,s", [(1, 4, 700), (2, 3, 129), (1, 1, 1)])
def test_forward_matches_the_reference_operations(b, h, s):
    z, w, cos, sin = _inputs(40 + s, b, h, s)
    k, v, _, _ = _run(z, w, cos, sin)
    rk, rv = reference_kv_prep(z, k_norm_weight=w, cos=cos, sin=sin)
    assert k.dtype == rk.dtype == torch.float32 and v.dtype == rv.dtype == torch.bfloat16
    assert k.shape == v.shape == z.shape and k.data_ptr() != v.data_ptr()
    _ulp_check(v, rv, "V")
    _ulp_check(k, rk, "K", mag=_k_magnitude(z, w, cos, sin))


def test_bf16_tables_and_per_batch_tables():
    z, w, cos, sin = _inputs(7, 2, 2, 300, table_batch=2, table_dtype=torch.bfloat16)
    k, v, _, _ = _run(z, w, cos, sin)
    assert k.dtype == torch.bfloat16
    # bf16 tables: the kernel rounds each product and the sum to bf16, as the
    # reference's bf16 operations do, so K agrees as V does
    rk, rv = reference_kv_prep(z, k_norm_weight=w, cos=cos, sin=sin)
    _ulp_check(v, rv, "V")
    mag = _k_magnitude(z, w, cos.float(), sin.float())
    _ulp_check(k, rk, "K (three bf16 roundings)", mag=mag)


def test_strided_source_layout():
    # a (B, S, H, D) buffer viewed as (B, H, S, D): the kernel takes the strides
    z, w, cos, sin = _inputs(8, 1, 4, 257)
    bshd = z.permute(0, 2, 1, 3).contiguous()
    view = bshd.to(DEV).permute(0, 2, 1, 3)
    import gemma4_fa4_amd as g

    k, v = g.prepare_global_kv_from_projection_source(view, k_norm_weight=w.to(DEV),
                                                      cos=cos.to(DEV), sin=sin.to(DEV))
    k2, v2, _, _ = _run(z, w, cos, sin)
    assert torch.equal(k, k2) and torch.equal(v, v2)


@pytest.mark.parametrize("b,h,s", [(1, 4, 700), (2, 2, 65)])
def test_backward_matches_the_fp64_adjoint(b, h, s):
    z, w, cos, sin = _inputs(60 + s, b, h, s)
    g = torch.Generator().manual_seed(s)
    dk = torch.randn(b, h, s, 512, generator=g)
    dv = torch.randn(b, h, s, 512, generator=g).to(torch.bfloat16)
    _, _, dz, dw = _run(z, w, cos, sin, grads=(dk, dv))
    rz, rw = kv_prep_backward_fp64(z, dk, dv, k_norm_weight=w, cos=cos, sin=sin)
    assert dz.dtype == torch.bfloat16 and dw.dtype == torch.float32
    dz, dw = dz.double().cpu(), dw.double().cpu()
    # dZ: fp32 arithmetic, one bf16 rounding
    lim = rz.abs() * 2.0 ** -8 + 1e-4 * rz.abs().max()
    assert int(((dz - rz).abs() > lim).sum()) == 0
    assert ((dz - rz).norm() / rz.norm()).item() < 4e-3
    # dweight: sums over all rows in fp32
    assert ((dw - rw).abs() <= rw.abs() * 1e-4 + 1e-4 * rw.abs().max()).all()


def test_backward_is_bitwise_repeatable():
    z, w, cos, sin = _inputs(5, 1, 4, 1000)
    g = torch.Generator().manual_seed(1)
    grads = (torch.randn(1, 4, 1000, 512, generator=g), torch.randn(1, 4, 1000, 512, generator=g)
             .to(torch.bfloat16))
    a = _run(z, w, cos, sin, grads=grads)
    b = _run(z, w, cos, sin, grads=grads)
    assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])


def test_prepared_kv_feed_the_global_attention():
    # K, V of a shared source through the packed global adapter: the two
    # tensors are distinct, as the attention's K/V-distinctness check requires
    import gemma4_fa4_amd as g

    s = 300
    z, w, cos, sin = _inputs(11, 1, 4, s)
    k, v, _, _ = _run(z, w, cos, sin)
    kt = k.to(torch.bfloat16)[0].transpose(0, 1).contiguous()  # (S, 4, 512)
    vt = v[0].transpose(0, 1).contiguous()
    q = (torch.randn(s, 32, 512, generator=torch.Generator().manual_seed(2)) * 512 ** -0.25) \
        .to(torch.bfloat16).to(DEV)
    cu = torch.tensor([0, s], dtype=torch.int32, device=DEV)
    o, lse = g.fa4_global_varlen_forward_only(q, kt, vt, cu, cu, max_seqlen_q=s, max_seqlen_k=s)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
