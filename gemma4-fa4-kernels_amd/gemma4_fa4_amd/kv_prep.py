"""Global-layer K/V preparation from the shared projection source, on gfx950.

Drop-in for the reference's ``prepare_global_kv_from_projection_source``
(``src/gemma4_fa4/reference.py:306-328``; helpers ``rms_norm`` 276-281 and
``apply_partial_rotary`` 289-303; design note ``docs/design.md:202-213``): from
the source Z of each (batch, KV head, token) row, K = partial RoPE of the
weighted RMSNorm and V = the unweighted RMSNorm, two distinct tensors.  One
fused HIP kernel computes both (``g4_kv_prep_fwd``); the autograd backward
applies both preparation adjoints in one kernel and returns dZ and the
weight's gradient (``g4_kv_prep_bwd``; no atomics, bitwise repeatable).

Same signature and result dtypes as the reference: the source is
``(B, H, S, D)`` (any strides with a unit last-dim stride), cos / sin are
``(B, S, R)`` or ``(S, R)`` with ``R = D * partial_rotary_factor``; V has the
source's dtype and K the promoted dtype of source and cos / sin (fp32 for the
usual bf16 source with fp32 tables).  The kernel computes the RMSNorm in fp32
and the rotation in K's dtype the way the reference's tensor operations do:
with fp32 tables two rounded fp32 products and a rounded sum, with bf16 tables
each product and the sum rounded to bf16.

``prepare_rows_into`` is the same kernel without autograd, for the inference
boundaries (the compiled layer and StaticCache decode operators): it writes
the RMSNorm + RoPE of query or key rows, and the unweighted RMSNorm of value
rows, of head_dim 512 or 256 straight into caller-provided views (a cache
slot, a BSHD buffer seen as BHSD).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import G4KvPrep, G4Layout
from .errors import UnsupportedMI355XPath

_HEAD_DIM = 512


def _rotary_dim(head_dim: int, partial_rotary_factor: float) -> int:
    width = head_dim * partial_rotary_factor
    if int(width) != width or int(width) % 2:
        raise ValueError("partial rotary width must be an even integer")
    return int(width)


def _layout(t: torch.Tensor) -> G4Layout:
    # (B, H, S, D) -> element strides of batch, token and head
    return G4Layout(t.stride(0), t.stride(2), t.stride(1))


def _tables(cos: torch.Tensor, sin: torch.Tensor, batch: int, seqlen: int, rot: int):
    if cos.shape != sin.shape:
        raise ValueError("cos and sin must have the same shape")
    if cos.ndim == 2:
        cos, sin = cos[None], sin[None]
    if cos.ndim != 3 or cos.shape[1:] != (seqlen, rot) or cos.shape[0] not in (1, batch):
        raise ValueError(f"cos and sin must be (B, S, {rot}) or (S, {rot})")
    c = cos.to(torch.float32).contiguous()
    s = sin.to(torch.float32).contiguous()
    stride = 0 if c.shape[0] == 1 else c.stride(0)
    return c, s, stride


def _check(source, weight, cos, sin) -> None:
    if source.ndim != 4:
        raise ValueError("the projection source must be a rank-4 (B, H, S, D) tensor")
    if source.dtype != torch.bfloat16:
        raise UnsupportedMI355XPath("the MI355X K/V preparation takes a BF16 projection source")
    if source.device.type != "cuda":
        raise UnsupportedMI355XPath("the MI355X K/V preparation needs GPU tensors")
    if source.shape[-1] != _HEAD_DIM:
        raise UnsupportedMI355XPath("the MI355X K/V preparation covers head_dim 512")
    if source.stride(-1) != 1 or any(s % 8 for s in source.stride()[:-1]) or \
            source.data_ptr() % 16:
        raise ValueError("source needs a unit last-dim stride, outer strides that are "
                         "multiples of 8 and a 16-byte aligned base")
    if weight.shape != (source.shape[-1],):
        raise ValueError("k_norm_weight must have shape (head_dim,)")
    if any(t.device != source.device for t in (weight, cos, sin)):
        raise ValueError("source, k_norm_weight, cos and sin must share a device")
    if cos.requires_grad or sin.requires_grad:
        raise UnsupportedMI355XPath("gradients of cos / sin are not produced")


def _problem(source, rot, eps, stride, k_fp32) -> G4KvPrep:
    b, h, s, d = source.shape
    return G4KvPrep(num_batches=b, seqlen=s, num_heads=h, head_dim=d, rotary_dim=rot,
                    k_fp32=1 if k_fp32 else 0, eps=float(eps), cs_batch_stride=stride)


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


class _KvPrepFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, source, weight, cos, sin, rot, eps, k_dtype):
        lib = _lib.load()
        w = weight.to(torch.float32).contiguous()
        c, s, stride = _tables(cos, sin, source.shape[0], source.shape[2], rot)
        k_fp32 = k_dtype == torch.float32
        prob = _problem(source, rot, eps, stride, k_fp32)
        k = torch.empty(source.shape, dtype=k_dtype, device=source.device)
        v = torch.empty(source.shape, dtype=source.dtype, device=source.device)
        with torch.cuda.device(source.device):
            _lib.check(lib.g4_kv_prep_fwd(
                ctypes.byref(prob), source.data_ptr(), _layout(source), w.data_ptr(),
                c.data_ptr(), s.data_ptr(), k.data_ptr(), _layout(k), v.data_ptr(),
                _layout(v), _stream(source.device)))
        ctx.save_for_backward(source, w, c, s)
        ctx.prob = prob
        ctx.weight_dtype = weight.dtype
        ctx.k_dtype = k_dtype
        ctx.set_materialize_grads(False)
        return k, v

    @staticmethod
    def backward(ctx, dk, dv):
        source, w, c, s = ctx.saved_tensors
        lib = _lib.load()
        if dk is None:
            dk = torch.zeros(source.shape, dtype=ctx.k_dtype, device=source.device)
        if dv is None:
            dv = torch.zeros_like(source)
        dk = dk.to(ctx.k_dtype).contiguous()
        dv = dv.to(source.dtype).contiguous()
        dz = torch.empty_like(source, memory_format=torch.contiguous_format)
        dw = torch.empty(source.shape[-1], dtype=torch.float32, device=source.device)
        prob = ctx.prob
        ws = torch.empty(max(lib.g4_kv_prep_workspace_bytes(ctypes.byref(prob)), 16),
                         dtype=torch.uint8, device=source.device)
        with torch.cuda.device(source.device):
            _lib.check(lib.g4_kv_prep_bwd(
                ctypes.byref(prob), source.data_ptr(), _layout(source), w.data_ptr(),
                c.data_ptr(), s.data_ptr(), dk.data_ptr(), _layout(dk), dv.data_ptr(),
                _layout(dv), dz.data_ptr(), _layout(dz), dw.data_ptr(), ws.data_ptr(), ws.numel(),
                _stream(source.device)))
        return dz, dw.to(ctx.weight_dtype), None, None, None, None, None


def prepare_global_kv_from_projection_source(
    source: torch.Tensor,
    *,
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    partial_rotary_factor: float = 0.25,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """K = partial RoPE of RMSNorm(Z) * w, V = RMSNorm(Z): distinct tensors (autograd-capable)."""
    rot = _rotary_dim(source.shape[-1], partial_rotary_factor)
    _check(source, k_norm_weight, cos, sin)
    k_dtype = torch.promote_types(source.dtype, torch.promote_types(cos.dtype, sin.dtype)) \
        if rot else source.dtype
    if k_dtype not in (torch.bfloat16, torch.float32):
        raise UnsupportedMI355XPath("K is produced as BF16 or FP32 (cos / sin in BF16 or FP32)")
    return _KvPrepFunction.apply(source, k_norm_weight, cos, sin, rot, eps, k_dtype)


def prepare_rows_into(
    source: torch.Tensor,
    *,
    weight: torch.Tensor,
    cos: torch.Tensor | None = None,
    sin: torch.Tensor | None = None,
    rotary_dim: int = 0,
    eps: float = 1e-6,
    k: torch.Tensor | None = None,
    v: torch.Tensor | None = None,
) -> None:
    """Inference-only preparation of (B, H, S, D) rows into the views ``k`` / ``v``.

    ``k`` receives RoPE(RMSNorm(source) * weight) over the first ``rotary_dim``
    dims (bf16 with bf16 tables, fp32 with fp32 tables), ``v`` the unweighted
    RMSNorm (bf16); either may be None.  Every tensor is (B, H, S, D) with a
    unit last-dim stride (views of BSHD buffers and of cache slots included);
    no gradients are produced.
    """
    if k is None and v is None:
        raise ValueError("at least one of k and v must be given")
    if source.ndim != 4 or source.dtype != torch.bfloat16:
        raise ValueError("the projection source must be a rank-4 BF16 (B, H, S, D) tensor")
    if source.device.type != "cuda":
        raise UnsupportedMI355XPath("the MI355X K/V preparation needs GPU tensors")
    d = source.shape[-1]
    if d not in (256, 512):
        raise UnsupportedMI355XPath("the MI355X row preparation covers head_dim 512 and 256")
    if rotary_dim < 0 or rotary_dim > d or rotary_dim % 16:
        raise ValueError("rotary_dim must be a multiple of 16 in [0, head_dim]")
    if weight.shape != (d,):
        raise ValueError("the norm weight must have shape (head_dim,)")
    for name, t in (("source", source), ("k", k), ("v", v)):
        if t is None:
            continue
        if t.shape != source.shape or t.device != source.device:
            raise ValueError(f"{name} must match the source's shape and device")
        if t.stride(-1) != 1 or any(s <= 0 or s % 8 for s in t.stride()[:-1]) or \
                t.data_ptr() % 16:
            raise ValueError(f"{name} needs a unit last-dim stride, positive outer strides "
                             "that are multiples of 8 and a 16-byte aligned base")
    if v is not None and v.dtype != torch.bfloat16:
        raise ValueError("v is written as BF16")
    b, _, s, _ = source.shape
    c = sn = None
    stride = 0
    k_fp32 = False
    if k is not None:
        if k.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("k is written as BF16 or FP32")
        k_fp32 = k.dtype == torch.float32
        if rotary_dim:
            if cos is None or sin is None:
                raise ValueError("cos and sin are required for a rotary k")
            table_dtype = torch.promote_types(cos.dtype, sin.dtype)
            if torch.promote_types(source.dtype, table_dtype) != k.dtype:
                raise ValueError("k's dtype must be the promoted dtype of source, cos and sin")
            c, sn, stride = _tables(cos, sin, b, s, rotary_dim)
    w = weight.to(torch.float32).contiguous()
    lib = _lib.load()
    prob = _problem(source, rotary_dim, eps, stride, k_fp32)
    null = G4Layout(0, 0, 0)
    with torch.cuda.device(source.device):
        _lib.check(lib.g4_kv_prep_fwd(
            ctypes.byref(prob), source.data_ptr(), _layout(source), w.data_ptr(),
            c.data_ptr() if c is not None else None, sn.data_ptr() if sn is not None else None,
            k.data_ptr() if k is not None else None, _layout(k) if k is not None else null,
            v.data_ptr() if v is not None else None, _layout(v) if v is not None else null,
            _stream(source.device)))
