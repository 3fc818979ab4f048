"""Prepared-Q/K/V attention oracle (forward and explicit backward) -- TEST INFRASTRUCTURE ONLY.

Restates the reference's high-precision attention:

* ``reference_attention`` follows ``src/gemma4_fa4/reference.py:23-75``:
  ``S = (q k^T) * scale`` (57), masked to -inf (70), ``lse = logsumexp`` (71),
  ``P = exp(S - lse)`` zeroed on fully masked rows (72-73), ``O = P v`` cast to the
  input dtype (74); LSE returned as fp32 (75).  GQA expands K/V heads (15-20).
* ``reference_attention_varlen`` follows ``reference.py:78-198``: per packed
  segment, lower-right ``q_start = Sk - Sq`` (189), metadata sliced from the K
  stream (174-179), ``Sq == 0`` segments skipped (172-173), ``cu`` validation
  (78-93, 170-171).
* ``attention_fwd_bwd`` is a chunked forward plus explicit backward
  (dV = P^T dO, dP = dO V^T, delta = rowsum(O*dO) - dLSE, dS = P*(dP - delta),
  dQ = dS K, dK = dS^T Q) used at sizes where dense autograd does not fit.
  It runs on whatever device its inputs live on.
* ``bf16_baseline_fwd_bwd`` is the independent BF16 attention the reference's
  gradient envelope is relative to (scripts/probe_h100_local_backward.py:125-167,
  scripts/probe_h100_global_backward.py:105-127): bf16 products, fp32
  logsumexp, softmax rounded to bf16, autograd-style bf16 rounding of every
  product in the backward.

Pinned by ``tests/test_oracle_attention.py``: the reference's known answers
(window-1 returns V, scale 1.0 vs 1/sqrt(d), O = 1.5 lower-right vision truth
table, O = 1/1024 strict W1024 edge, all-masked row gives O = 0 and LSE = -inf,
GQA equals materialised MHA in forward and backward, mixed-empty segments give
exact-zero dK/dV), the explicit backward against torch autograd on small shapes,
and the analytic uniform-score case (Q = 0 gives O = mean of allowed V and
LSE = ln(count)).  ``bf16_baseline_fwd_bwd`` is pinned by
``tests/test_oracle_bf16_baseline.py`` against the reference probe's dense bf16
autograd path run on small CPU shapes (bit-identical on >= 99% of the elements of
O, dQ, dK and dV), and that comparison fails when any one of its rounding points
(``_SKIP_ROUNDING``) is left out.
"""

from __future__ import annotations

import math

import torch

from .masks import gemma4_attention_mask


def expand_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """Expand ``(B, Hkv, S, D)`` to ``(B, Hkv * n_rep, S, D)`` (reference.py:15-20)."""
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def reference_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    softmax_scale: float = 1.0,
    sliding_window: int | None = None,
    vision_block_ids: torch.Tensor | None = None,
    document_ids: torch.Tensor | None = None,
    key_padding_mask: torch.Tensor | None = None,
    allow_vision_bidirectional: bool = False,
    q_start: int | None = None,
    upcast: torch.dtype = torch.float64,
    return_lse: bool = False,
):
    """Dense BHSD attention with the Gemma mask; differentiable through autograd."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must be rank-4 B/H/S/D tensors")
    b, hq, q_len, d = q.shape
    bk, hkv, kv_len, dk = k.shape
    bv, hv, vv_len, _dv = v.shape
    if (bk, bv) != (b, b) or hkv != hv or kv_len != vv_len or d != dk:
        raise ValueError("incompatible q/k/v shapes")
    if hq % hkv:
        raise ValueError("query heads must be divisible by KV heads")
    out_dtype = q.dtype
    qf, kf, vf = (t.to(upcast) for t in (q, k, v))
    kf = expand_kv(kf, hq // hkv)
    vf = expand_kv(vf, hq // hkv)
    scores = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * float(softmax_scale)
    mask = gemma4_attention_mask(
        batch_size=b,
        q_len=q_len,
        kv_len=kv_len,
        sliding_window=sliding_window,
        vision_block_ids=vision_block_ids,
        document_ids=document_ids,
        key_padding_mask=key_padding_mask,
        q_start=q_start,
        allow_vision_bidirectional=allow_vision_bidirectional,
    ).to(q.device)
    scores = scores.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.exp(scores - lse[..., None])
    probs = torch.where(torch.isfinite(lse)[..., None], probs, torch.zeros_like(probs))
    out = torch.matmul(probs, vf).to(out_dtype)
    return (out, lse.to(torch.float32)) if return_lse else out


def _cumulative(values, total: int, name: str) -> list[int]:
    if isinstance(values, torch.Tensor):
        if values.ndim != 1 or values.numel() < 2:
            raise ValueError(f"{name} must be rank-1 with at least two entries")
        if values.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name} must use an integer dtype")
        values = [int(x) for x in values.detach().cpu().tolist()]
    values = [int(x) for x in values]
    if len(values) < 2:
        raise ValueError(f"{name} must be rank-1 with at least two entries")
    if values[0] != 0 or values[-1] != total:
        raise ValueError(f"{name} must start at zero and end at the packed total")
    if any(e < s for s, e in zip(values[:-1], values[1:])):
        raise ValueError(f"{name} must be nondecreasing")
    return values


def reference_attention_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    softmax_scale: float = 1.0,
    sliding_window: int | None = None,
    vision_block_ids: torch.Tensor | None = None,
    document_ids: torch.Tensor | None = None,
    allow_vision_bidirectional: bool = False,
    upcast: torch.dtype = torch.float64,
    return_lse: bool = False,
):
    """Packed THD attention; each Q segment is the lower-right suffix of its K segment."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("packed q, k, and v must be rank-3 T/H/D tensors")
    if k.shape[:2] != v.shape[:2] or q.shape[-1] != k.shape[-1]:
        raise ValueError("incompatible packed q/k/v shapes")
    if q.shape[1] % k.shape[1]:
        raise ValueError("query heads must be divisible by KV heads")
    if q.shape[0] <= 0 or k.shape[0] <= 0:
        raise ValueError("packed Q and K totals must be positive")
    cq = _cumulative(cu_seqlens_q, q.shape[0], "cu_seqlens_q")
    ck = _cumulative(cu_seqlens_k, k.shape[0], "cu_seqlens_k")
    if len(cq) != len(ck):
        raise ValueError("packed Q and K must have the same batch count")
    for name, meta in (("vision_block_ids", vision_block_ids), ("document_ids", document_ids)):
        if meta is None:
            continue
        if tuple(meta.shape) != (k.shape[0],):
            raise ValueError(f"packed {name} must match Tk")
        if meta.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"packed {name} must use an integer dtype")
    outs, lses = [], []
    for i, (qs, qe, ks, ke) in enumerate(zip(cq[:-1], cq[1:], ck[:-1], ck[1:])):
        lq, lk = qe - qs, ke - ks
        if lq > lk:
            raise ValueError(f"packed sequence {i} has Sq greater than Sk")
        if lq == 0:
            continue
        vid = vision_block_ids[ks:ke].unsqueeze(0) if vision_block_ids is not None else None
        doc = document_ids[ks:ke].unsqueeze(0) if document_ids is not None else None
        o, l = reference_attention(
            q[qs:qe].transpose(0, 1).unsqueeze(0),
            k[ks:ke].transpose(0, 1).unsqueeze(0),
            v[ks:ke].transpose(0, 1).unsqueeze(0),
            softmax_scale=softmax_scale,
            sliding_window=sliding_window,
            vision_block_ids=vid,
            document_ids=doc,
            allow_vision_bidirectional=allow_vision_bidirectional,
            q_start=lk - lq,
            upcast=upcast,
            return_lse=True,
        )
        outs.append(o.squeeze(0).transpose(0, 1))
        lses.append(l.squeeze(0))
    out = torch.cat(outs, dim=0)
    lse = torch.cat(lses, dim=1)
    return (out, lse) if return_lse else out


def _chunk_mask(
    q_abs: torch.Tensor,
    k_abs: torch.Tensor,
    *,
    window: int | None,
    vision: torch.Tensor | None,
    documents: torch.Tensor | None,
    bidirectional: bool,
) -> torch.Tensor:
    """Bool ``(len(q_abs), len(k_abs))`` block of the Gemma predicate (masks.py:46-71)."""
    keep = k_abs[None, :] <= q_abs[:, None]
    if bidirectional and vision is not None:
        vq = vision[q_abs][:, None]
        keep = keep | ((vq == vision[k_abs][None, :]) & (vq >= 0))
    if window is not None:
        keep = keep & (k_abs[None, :] > q_abs[:, None] - window)
    if documents is not None:
        keep = keep & (documents[q_abs][:, None] == documents[k_abs][None, :])
    return keep


def attention_fwd_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    do: torch.Tensor | None = None,
    dlse: torch.Tensor | None = None,
    sliding_window: int | None = None,
    vision_block_ids: torch.Tensor | None = None,
    document_ids: torch.Tensor | None = None,
    allow_vision_bidirectional: bool = False,
    softmax_scale: float = 1.0,
    compute_dtype: torch.dtype = torch.float64,
    q_chunk: int = 256,
    heads: list[int] | None = None,
):
    """Chunked packed attention forward and explicit backward.

    ``q`` is ``(Tq, Hq, D)``, ``k``/``v`` are ``(Tk, Hkv, D)``, ``do`` matches
    ``q``'s ``(Tq, Hq, Dv)`` and ``dlse`` is ``(Hq, Tq)``.  Returns
    ``(O, LSE, dQ, dK, dV)`` in ``compute_dtype`` (LSE fp32; gradients ``None``
    when ``do`` is None).  ``heads`` restricts the computation to a subset of
    query heads (other rows/heads are left zero) so large configurations can be
    spot-checked.  The backward uses the exact (unrounded) O for delta.
    """
    dev = q.device
    tq, hq, d = q.shape
    tk, hkv, _ = k.shape
    dv_dim = v.shape[-1]
    rep = hq // hkv
    cq = _cumulative(cu_seqlens_q, tq, "cu_seqlens_q")
    ck = _cumulative(cu_seqlens_k, tk, "cu_seqlens_k")
    vision = vision_block_ids.to(dev, torch.int64) if vision_block_ids is not None else None
    docs = document_ids.to(dev, torch.int64) if document_ids is not None else None
    heads = list(range(hq)) if heads is None else list(heads)
    want_grad = do is not None

    out = torch.zeros(tq, hq, dv_dim, dtype=compute_dtype, device=dev)
    lse = torch.full((hq, tq), float("-inf"), dtype=torch.float32, device=dev)
    dq = torch.zeros(tq, hq, d, dtype=compute_dtype, device=dev) if want_grad else None
    dk = torch.zeros(tk, hkv, d, dtype=compute_dtype, device=dev) if want_grad else None
    dv = torch.zeros(tk, hkv, dv_dim, dtype=compute_dtype, device=dev) if want_grad else None
    scale = float(softmax_scale)

    for qs, qe, ks, ke in zip(cq[:-1], cq[1:], ck[:-1], ck[1:]):
        lq, lk = qe - qs, ke - ks
        if lq > lk:
            raise ValueError("packed sequence has Sq greater than Sk")
        if lq == 0:
            continue
        k_abs_all = torch.arange(ks, ke, device=dev)
        for h in heads:
            g = h // rep
            kh = k[ks:ke, g].to(compute_dtype)
            vh = v[ks:ke, g].to(compute_dtype)
            for c0 in range(0, lq, q_chunk):
                c1 = min(lq, c0 + q_chunk)
                # absolute K-stream position of each query (lower-right alignment)
                q_abs = torch.arange(ks + (lk - lq) + c0, ks + (lk - lq) + c1, device=dev)
                keep = _chunk_mask(
                    q_abs,
                    k_abs_all,
                    window=sliding_window,
                    vision=vision,
                    documents=docs,
                    bidirectional=allow_vision_bidirectional,
                )
                cols = torch.nonzero(keep.any(dim=0)).flatten()
                if cols.numel() == 0:
                    continue
                k0, k1 = int(cols[0]), int(cols[-1]) + 1
                keep = keep[:, k0:k1]
                qh = q[qs + c0 : qs + c1, h].to(compute_dtype)
                kc, vc = kh[k0:k1], vh[k0:k1]
                s = (qh @ kc.T) * scale
                s = s.masked_fill(~keep, float("-inf"))
                m = torch.logsumexp(s, dim=-1)
                finite = torch.isfinite(m)
                p = torch.exp(s - m[:, None])
                p = torch.where(finite[:, None], p, torch.zeros_like(p))
                o = p @ vc
                out[qs + c0 : qs + c1, h] = o
                lse[h, qs + c0 : qs + c1] = m.to(torch.float32)
                if not want_grad:
                    continue
                doh = do[qs + c0 : qs + c1, h].to(compute_dtype)
                delta = (doh * o).sum(dim=-1)
                if dlse is not None:
                    delta = delta - dlse[h, qs + c0 : qs + c1].to(compute_dtype)
                dp = doh @ vc.T
                ds = p * (dp - delta[:, None])
                dv[ks + k0 : ks + k1, g] += p.T @ doh
                dq[qs + c0 : qs + c1, h] = (ds @ kc) * scale
                dk[ks + k0 : ks + k1, g] += (ds.T @ qh) * scale
    return out, lse, dq, dk, dv


# Rounding points of the bf16 baseline left unrounded.  Empty in normal use;
# the pinning tests plant a mistake here to show that their comparison with the
# reference's bf16 autograd path notices a missing rounding.
_SKIP_ROUNDING: frozenset = frozenset()


def _bf(x: torch.Tensor, point: str = "") -> torch.Tensor:
    if point in _SKIP_ROUNDING:
        return x
    return x.to(torch.bfloat16).to(torch.float32)


def bf16_baseline_fwd_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    do: torch.Tensor,
    dlse: torch.Tensor | None = None,
    sliding_window: int | None = None,
    vision_block_ids: torch.Tensor | None = None,
    document_ids: torch.Tensor | None = None,
    allow_vision_bidirectional: bool = False,
    q_chunk: int = 256,
    heads: list[int] | None = None,
):
    """Independent BF16 attention gradients (the envelope's baseline).

    Mirrors the reference's upstream-style bf16 path
    (probe_h100_local_backward.py:125-167): scores are a bf16 product, LSE is an
    fp32 logsumexp of them, probabilities are softmax rounded to bf16, O is a bf16
    product.  Its autograd backward rounds every product and the softmax backward
    to bf16; this restatement applies the same rounding points with fp32
    arithmetic (so it can run on CPU or GPU without bf16 batched products).
    Returns ``(O, dQ, dK, dV)`` as fp32 tensors holding bf16 values.
    """
    dev = q.device
    tq, hq, d = q.shape
    tk, hkv, _ = k.shape
    rep = hq // hkv
    cq = _cumulative(cu_seqlens_q, tq, "cu_seqlens_q")
    ck = _cumulative(cu_seqlens_k, tk, "cu_seqlens_k")
    vision = vision_block_ids.to(dev, torch.int64) if vision_block_ids is not None else None
    docs = document_ids.to(dev, torch.int64) if document_ids is not None else None
    heads = list(range(hq)) if heads is None else list(heads)
    f32 = torch.float32
    out = torch.zeros(tq, hq, v.shape[-1], dtype=f32, device=dev)
    dq = torch.zeros(tq, hq, d, dtype=f32, device=dev)
    # per-query-head K/V gradients are rounded to bf16 and then summed over the
    # GQA group (the backward of a repeat of K/V heads)
    dk_heads = torch.zeros(tk, hq, d, dtype=f32, device=dev)
    dv_heads = torch.zeros(tk, hq, v.shape[-1], dtype=f32, device=dev)
    for qs, qe, ks, ke in zip(cq[:-1], cq[1:], ck[:-1], ck[1:]):
        lq, lk = qe - qs, ke - ks
        if lq == 0:
            continue
        k_abs_all = torch.arange(ks, ke, device=dev)
        for h in heads:
            g = h // rep
            kh = k[ks:ke, g].to(f32)
            vh = v[ks:ke, g].to(f32)
            # the dense bf16 path computes dK/dV over all queries of the segment
            dk_acc = torch.zeros(lk, d, dtype=f32, device=dev)
            dv_acc = torch.zeros(lk, v.shape[-1], dtype=f32, device=dev)
            for c0 in range(0, lq, q_chunk):
                c1 = min(lq, c0 + q_chunk)
                q_abs = torch.arange(ks + (lk - lq) + c0, ks + (lk - lq) + c1, device=dev)
                keep = _chunk_mask(
                    q_abs,
                    k_abs_all,
                    window=sliding_window,
                    vision=vision,
                    documents=docs,
                    bidirectional=allow_vision_bidirectional,
                )
                qh = q[qs + c0 : qs + c1, h].to(f32)
                s = _bf(qh @ kh.T, "S").masked_fill(~keep, float("-inf"))
                lse = torch.logsumexp(s, dim=-1)
                p32 = torch.softmax(s, dim=-1)
                p32 = torch.nan_to_num(p32, nan=0.0)
                p = _bf(p32, "P")
                o = _bf(p @ vh, "O")
                out[qs + c0 : qs + c1, h] = o
                doh = do[qs + c0 : qs + c1, h].to(f32)
                dv_acc += p.T @ doh
                dp = _bf(doh @ vh.T, "dP")
                # softmax backward of the bf16 probabilities, rounded to bf16
                ds = _bf(p * (dp - (dp * p).sum(dim=-1, keepdim=True)), "dS")
                if dlse is not None:
                    plse = torch.exp(s - lse[:, None])
                    plse = torch.where(torch.isfinite(lse)[:, None], plse, torch.zeros_like(plse))
                    ds = _bf(ds + _bf(plse * dlse[h, qs + c0 : qs + c1].to(f32)[:, None], "dLSE"), "dS")
                dq[qs + c0 : qs + c1, h] = _bf(ds @ kh, "dQ")
                dk_acc += ds.T @ qh
            dk_heads[ks:ke, h] = _bf(dk_acc, "dK")
            dv_heads[ks:ke, h] = _bf(dv_acc, "dV")
    dk = _bf(dk_heads.view(tk, hkv, rep, d).sum(dim=2), "dK")
    dv = _bf(dv_heads.view(tk, hkv, rep, v.shape[-1]).sum(dim=2), "dV")
    return out, dq, dk, dv


def analytic_uniform_lse(count: int) -> float:
    """LSE of ``count`` equal zero scores: ``ln(count)``."""
    return math.log(count)
