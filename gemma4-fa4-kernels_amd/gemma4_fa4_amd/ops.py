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
    ds_budget: int = 0,
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
        ds_budget=ds_budget,
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


class Stages:
    """The forward kernel and the three backward stages as separate launches.

    Used to time each kernel on its own stream position (the adapters launch
    them back to back).  Buffers are allocated once; every call is a single
    stream-ordered library call on the current stream.
    """

    def __init__(self, plan: _Plan, q, k, v, dout, dlse=None, *, forward_only: bool = False):
        """``forward_only``: size the workspace for the forward launch alone."""
        from .attention import _layout

        self.plan = plan
        self.q, self.k, self.v, self.dout, self.dlse = q, k, v, dout, dlse
        dev = q.device
        self.o = torch.empty_like(q)
        self.lse = torch.empty(plan.lse_shape(), dtype=torch.float32, device=dev)
        self.dq = torch.empty_like(q)
        self.dk = torch.empty_like(k)
        self.dv = torch.empty_like(v)
        phase = 0 if forward_only else 1
        self.ws = torch.empty(max(plan.workspace_bytes(phase), 256), dtype=torch.uint8, device=dev)
        self.prob = plan.problem()
        self.lay = {name: _layout(t, plan.packed) for name, t in (
            ("q", q), ("k", k), ("v", v), ("o", self.o), ("do", dout), ("dq", self.dq),
            ("dk", self.dk), ("dv", self.dv))}
        self.lib = _lib.load()

    def _stream(self):
        return torch.cuda.current_stream(self.q.device).cuda_stream

    def forward(self):
        L = self.lay
        _lib.check(self.lib.g4_attn_fwd(
            ctypes.byref(self.prob), self.q.data_ptr(), L["q"], self.k.data_ptr(), L["k"],
            self.v.data_ptr(), L["v"], self.o.data_ptr(), L["o"], self.lse.data_ptr(),
            self.ws.data_ptr(), self.ws.numel(), self._stream()))

    def delta(self):
        L = self.lay
        _lib.check(self.lib.g4_attn_bwd_delta(
            ctypes.byref(self.prob), self.o.data_ptr(), L["o"], self.dout.data_ptr(), L["do"],
            None if self.dlse is None else self.dlse.data_ptr(), self.ws.data_ptr(),
            self.ws.numel(), self._stream()))

    def dkdv(self):
        L = self.lay
        _lib.check(self.lib.g4_attn_bwd_dkdv(
            ctypes.byref(self.prob), self.q.data_ptr(), L["q"], self.k.data_ptr(), L["k"],
            self.v.data_ptr(), L["v"], self.dout.data_ptr(), L["do"], self.lse.data_ptr(),
            self.dk.data_ptr(), L["dk"], self.dv.data_ptr(), L["dv"], self.ws.data_ptr(),
            self.ws.numel(), self._stream()))

    def backward(self):
        """The whole backward through g4_attn_bwd (delta, then dK/dV and dQ; a
        striped problem interleaves the two per stripe)."""
        L = self.lay
        _lib.check(self.lib.g4_attn_bwd(
            ctypes.byref(self.prob), self.q.data_ptr(), L["q"], self.k.data_ptr(), L["k"],
            self.v.data_ptr(), L["v"], self.o.data_ptr(), L["o"], self.dout.data_ptr(), L["do"],
            self.lse.data_ptr(), None if self.dlse is None else self.dlse.data_ptr(),
            self.dq.data_ptr(), L["dq"], self.dk.data_ptr(), L["dk"], self.dv.data_ptr(),
            L["dv"], self.ws.data_ptr(), self.ws.numel(), self._stream()))

    def dq_stage(self):
        L = self.lay
        _lib.check(self.lib.g4_attn_bwd_dq(
            ctypes.byref(self.prob), self.q.data_ptr(), L["q"], self.k.data_ptr(), L["k"],
            self.v.data_ptr(), L["v"], self.dout.data_ptr(), L["do"], self.lse.data_ptr(),
            self.dq.data_ptr(), L["dq"], self.ws.data_ptr(), self.ws.numel(), self._stream()))
