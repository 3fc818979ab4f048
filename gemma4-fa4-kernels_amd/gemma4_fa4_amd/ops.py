"""Lower-level entry points over the C ABI: mask materialisation and scheduler ranges.

These expose the exact device predicate and the device tile scheduler so the
mask contract (bit-exact boolean masks) and the scheduler's coverage can be
checked directly, independent of any attention arithmetic.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .attention import _Plan


def make_plan(
    *,
    num_seqs: int,
    seqlen_q: int,
    seqlen_k: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    window: int | None,
    vision: torch.Tensor | None = None,
    documents: torch.Tensor | None = None,
    bidirectional: bool = True,
    cu_q: torch.Tensor | None = None,
    cu_k: torch.Tensor | None = None,
    total_q: int | None = None,
    total_k: int | None = None,
) -> _Plan:
    packed = cu_q is not None
    return _Plan(
        packed=packed,
        num_seqs=num_seqs,
        seqlen_q=seqlen_q,
        seqlen_k=seqlen_k,
        num_q_heads=num_q_heads,
        num_kv_heads=num_kv_heads,
        head_dim=head_dim,
        window=window or 0,
        bidirectional=bidirectional and vision is not None,
        total_q=total_q if total_q is not None else num_seqs * seqlen_q,
        total_k=total_k if total_k is not None else num_seqs * seqlen_k,
        cu_q=cu_q,
        cu_k=cu_k,
        vision=None if vision is None else vision.to(torch.int32).contiguous(),
        documents=None if documents is None else documents.to(torch.int32).contiguous(),
    )


def mask_materialize(plan: _Plan, device) -> torch.Tensor:
    """Bool ``(num_seqs, seqlen_q, seqlen_k)`` evaluation of the device predicate."""
    lib = _lib.load()
    out = torch.empty((plan.num_seqs, plan.seqlen_q, plan.seqlen_k), dtype=torch.uint8, device=device)
    prob = plan.problem()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        _lib.check(lib.g4_mask_materialize(ctypes.byref(prob), out.data_ptr(), None, 0, stream))
    return out.bool()


def tile_ranges(plan: _Plan, direction: int, row_tile: int, device) -> torch.Tensor:
    """``(num_seqs, ntiles, 2)`` int32 [lo, hi) ranges of the device scheduler."""
    lib = _lib.load()
    length = plan.seqlen_q if direction == 0 else plan.seqlen_k
    ntiles = (length + row_tile - 1) // row_tile
    out = torch.empty((plan.num_seqs, ntiles, 2), dtype=torch.int32, device=device)
    ws = torch.empty(max(plan.workspace_bytes(0), 256), dtype=torch.uint8, device=device)
    prob = plan.problem()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        _lib.check(
            lib.g4_tile_ranges(
                ctypes.byref(prob), direction, row_tile, out.data_ptr(), ws.data_ptr(),
                ws.numel(), stream,
            )
        )
    return out
