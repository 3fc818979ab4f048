"""Shared helpers for the GPU parity tests (inputs, oracle runs, envelope checks)."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd
from oracle.envelope import (
    GLOBAL_LSE_ATOL,
    GLOBAL_OUT_ATOL,
    GLOBAL_OUT_RTOL,
    LOCAL_LSE_ATOL,
    LOCAL_OUT_ATOL,
    LOCAL_OUT_RTOL,
    gradient_limit,
    rel_frobenius,
)

LOCAL = dict(hq=32, hkv=16, d=256, window=1024)
GLOBAL = dict(hq=32, hkv=4, d=512, window=None)


def qkv(seed: int, tq: int, tk: int, hq: int, hkv: int, d: int, *, unit_logits: bool = True,
        grad: bool = False):
    """Packed (T, H, D) bf16 q, k, v, dO and fp32 dLSE, drawn on the CPU from a seeded generator.

    unit_logits: Q, K ~ N(0, 1/sqrt(d)); otherwise N(0, 1).
    """
    g = torch.Generator().manual_seed(seed)
    sd = d ** -0.25 if unit_logits else 1.0
    q = (torch.randn(tq, hq, d, generator=g) * sd).to(torch.bfloat16)
    k = (torch.randn(tk, hkv, d, generator=g) * sd).to(torch.bfloat16)
    v = torch.randn(tk, hkv, d, generator=g).to(torch.bfloat16)
    do = torch.randn(tq, hq, d, generator=g).to(torch.bfloat16)
    dlse = torch.randn(hq, tq, generator=g)
    return q, k, v, do, dlse


def cu(lengths) -> torch.Tensor:
    return torch.tensor([0, *np.cumsum(lengths).tolist()], dtype=torch.int32)


def oracle_fwd_bwd(q, k, v, cu_q, cu_k, *, window, vision=None, docs=None, do=None, dlse=None,
                   device="cpu", dtype=torch.float64, heads=None):
    """fp64 oracle (on `device`) for packed inputs; returns CPU tensors."""
    args = [t.to(device) for t in (q, k, v)]
    res = attention_fwd_bwd(
        *args, cu_q.tolist(), cu_k.tolist(),
        do=None if do is None else do.to(device),
        dlse=None if dlse is None else dlse.to(device),
        sliding_window=window,
        vision_block_ids=None if vision is None else vision.to(device),
        document_ids=None if docs is None else docs.to(device),
        allow_vision_bidirectional=window is not None and vision is not None,
        compute_dtype=dtype, heads=heads,
    )
    return tuple(None if t is None else t.cpu() for t in res)


def check_forward(o, lse, o_ref, lse_ref, *, local: bool, label: str = "", rows=None):
    """Reference M1 forward envelope plus a tighter rel-Frobenius bound."""
    atol = LOCAL_OUT_ATOL if local else GLOBAL_OUT_ATOL
    rtol = LOCAL_OUT_RTOL if local else GLOBAL_OUT_RTOL
    latol = LOCAL_LSE_ATOL if local else GLOBAL_LSE_ATOL
    o = o.float().cpu()
    lse = lse.float().cpu()
    o_ref = o_ref.float()
    lse_ref = lse_ref.float()
    torch.testing.assert_close(o, o_ref, atol=atol, rtol=rtol, msg=f"{label} O envelope")
    torch.testing.assert_close(lse, lse_ref, atol=latol, rtol=0, msg=f"{label} LSE envelope")
    fro = rel_frobenius(o, o_ref)
    lse_err = (lse - lse_ref).abs().max().item()
    assert fro < 1e-2, f"{label} O rel-Frobenius {fro:.3e}"
    assert lse_err < 1e-2, f"{label} LSE max abs {lse_err:.3e}"
    return fro, lse_err


GRAD_ABS_FLOOR = 1e-4


def check_gradients(grads, refs, bf16_refs, *, label: str = ""):
    """Upstream-relative M1 gradient rule against the fp64 reference.

    Where the reference gradient is identically zero (e.g. dQ of a single-key
    row, where dP equals delta exactly) the rule's limit degenerates to 0; a
    1e-4 absolute floor then admits fp32 summation-order differences between
    delta = rowsum(O dO) and dP = dO V^T.
    """
    report = {}
    for name, g, r, b in zip(("dQ", "dK", "dV"), grads, refs, bf16_refs):
        g = g.float().cpu()
        assert torch.isfinite(g).all(), f"{label} {name} non-finite"
        err = (g.double() - r.double()).abs().max().item()
        lim = max(gradient_limit(r.double(), b.double()), GRAD_ABS_FLOOR)
        fro = rel_frobenius(g, r)
        report[name] = (err, lim, fro)
        assert err <= lim, f"{label} {name} max_abs={err:.4e} exceeds limit={lim:.4e}"
        assert fro < 2e-2, f"{label} {name} rel-Frobenius {fro:.3e}"
    return report


def vision_blocks(seed: int, length: int, nblocks: int, lo: int, hi: int) -> torch.Tensor:
    """int32 IDs with `nblocks` non-overlapping runs of U[lo, hi] tokens; -1 elsewhere."""
    rng = np.random.default_rng(seed)
    ids = np.full(length, -1, dtype=np.int32)
    lengths = rng.integers(lo, hi + 1, size=nblocks)
    lengths = np.minimum(lengths, max(1, length // (2 * nblocks)))
    free = length - int(lengths.sum())
    cuts = np.sort(rng.integers(0, free + 1, size=nblocks))
    pos = 0
    prev = 0
    for b, (c, ln) in enumerate(zip(cuts, lengths)):
        pos += int(c - prev)
        prev = c
        ids[pos:pos + ln] = b
        pos += int(ln)
    return torch.from_numpy(ids)
