"""Transformers attention + mask backend for the Gemma 4 31B attention path on MI355X.

Mirrors the reference's HF integration (src/gemma4_fa4/transformers_integration.py):

* ``register_gemma4_mi355x()`` registers ``gemma4_fa4_attention_forward`` in
  ``ALL_ATTENTION_FUNCTIONS`` and the mask callback in
  ``ALL_MASK_ATTENTION_FUNCTIONS`` under one backend name, idempotently, and
  refuses a name already taken by other callables (ti.py:3500-3547).
* The mask callback returns a ``Gemma4MaskPlan`` (ti.py:73-84) that keeps the
  composed Transformers mask callable instead of materialising a tensor.
* ``gemma4_fa4_prepared`` routes prepared BHSD q/k/v to the native kernels
  (ti.py:1702-2075) and returns a ``Gemma4DispatchResult`` naming the route.

Admission is exact: a plan runs natively only when its mask is proven to be
the native predicate (ti.py:543-647 states the same contract).  Two proofs:

1. Structural: the callable is a composition of the installed
   ``transformers.masking_utils`` combinators, recognised by code-object
   identity (not by name), whose canonical form is exactly
   ``causal [AND packed]`` (global layers) or
   ``window(1024) AND (causal [OR vision]) [AND packed]`` (local layers), with
   its captured vision/packed tensors checked against the metadata the
   kernels receive.  Cost O(metadata); any sequence length.
2. Exhaustive: any other callable is evaluated on the device over the whole
   ``(B, Sq, Sk)`` grid and compared with the kernels' own device predicate
   (``g4_mask_materialize``), for grids of at most ``_EVAL_PROOF_MAX_PAIRS``.

Everything else fails closed with ``UnsupportedMI355XPath``.  The reference
instead falls back to FlexAttention for forward-only calls (ti.py:1607-1699,
with a RuntimeWarning), which on ROCm is a Triton kernel outside this library;
this build has one code path, the native one, so it behaves as the reference
does with ``allow_flex_fallback=False`` (the same exception class, raised
before any launch).  The argument is accepted for signature compatibility.

The reference's budget fallback (ti.py:1950-1961: when the native global
backward exceeds its HBM budget, re-run a low-memory composition) lives in the
adapters here: the backward stores dS tiles only while they fit the budget and
otherwise recomputes S and dP, so every caller gets it, and
``GlobalBackwardBudgetExceeded`` is raised only when even that route does not
fit.

Padded query rows (2D padding mask) are returned as zeros with LSE ``-inf``,
as the reference's unpacking does (ti.py:1418-1447).

An eager ``StaticCache`` hands over its whole physical K/V backing, whose tail
past the written positions is unwritten.  With the reference's contract (B=1,
no gradient, text only, no documents, no explicit packed lengths, K offset 0,
a contiguous valid K prefix) the call is trimmed to the active prefix
``q_offset + Sq - kv_offset`` before routing (ti.py:1020-1110, 1815-1845); a
mask callable that is not the native plan must also mask every trimmed key.

Under ``torch.compile`` or with FakeTensor inputs, a text-only single
sequence (B = 1, S <= 1024, the layer's causal / sliding-causal mask, explicit
position_ids) is routed to one opaque custom operator of ``torch_ops``
(ti.py:761-921); everything else fails closed there.  The reference further
requires the exact pinned Transformers ``Gemma4TextAttention`` class and its
own compile-origin mask markers, which belong to a Transformers revision that
is not installed here; this route checks the mask callable structurally
instead.
"""

from __future__ import annotations

import types
from dataclasses import dataclass, replace
from typing import Any, Callable

import torch

from .attention import (
    fa4_global_forward_only,
    fa4_global_text_forward,
    fa4_global_varlen_forward,
    fa4_global_varlen_forward_only,
    fa4_local_forward,
    fa4_local_varlen_forward,
)
from .errors import UnsupportedMI355XPath
from .model_spec import GEMMA4_31B, AttentionLayerSpec

BACKEND_NAME = "gemma4_mi355x"

# Largest B*Sq*Sk grid proven by exhaustive device evaluation (64 Mi pairs:
# 64 MiB of bools per side, a few milliseconds of device work).
_EVAL_PROOF_MAX_PAIRS = 1 << 26

# Fixed-adapter envelopes (src/gemma4_fa4/h100.py:219-220, 643-644), used to
# pick the fixed routes the same way the reference does (ti.py:1882-1891, 1993-2003).
_FIXED_LOCAL_MAX = 1025
_FIXED_GLOBAL_MAX_GRAD = 2048
_FIXED_GLOBAL_MAX_NOGRAD = 1024


@dataclass(frozen=True)
class Gemma4MaskPlan:
    """The mask information the companion mask callback keeps (ti.py:73-84)."""

    batch_size: int
    q_length: int
    kv_length: int
    q_offset: int | torch.Tensor
    kv_offset: int | torch.Tensor
    mask_function: Callable | None
    attention_mask: torch.Tensor | None


@dataclass(frozen=True)
class Gemma4DispatchResult:
    """Prepared-attention result with the route that produced it (ti.py:86-92)."""

    output: torch.Tensor
    lse: torch.Tensor | None
    path: str


_NATIVE_ORIGIN = object()


def _snapshot_offset(value):
    # A StaticCache offset tensor is updated in place after the mask is built.
    if isinstance(value, torch.Tensor):
        return value.detach().clone()
    return value


def gemma4_fa4_mask(
    batch_size: int,
    q_length: int,
    kv_length: int,
    q_offset: int | torch.Tensor = 0,
    kv_offset: int | torch.Tensor = 0,
    mask_function: Callable | None = None,
    attention_mask: torch.Tensor | None = None,
    **_kwargs: Any,
) -> Gemma4MaskPlan:
    """Mask-interface callback: keep the composed mask for exact routing (ti.py:118-160)."""
    return Gemma4MaskPlan(
        batch_size=int(batch_size),
        q_length=int(q_length),
        kv_length=int(kv_length),
        q_offset=_snapshot_offset(q_offset),
        kv_offset=_snapshot_offset(kv_offset),
        mask_function=mask_function,
        attention_mask=attention_mask,
    )


# --------------------------------------------------------------------------
# Structural recognition of transformers.masking_utils compositions
# --------------------------------------------------------------------------


def _masking_utils():
    try:
        import transformers.masking_utils as masking_utils
    except Exception:  # transformers absent: nothing is recognisable
        return None
    return masking_utils


def _factory_code(masking_utils, factory_name: str, code_name: str):
    factory = getattr(masking_utils, factory_name, None)
    code = getattr(factory, "__code__", None)
    if code is None:
        return None
    for const in code.co_consts:
        if isinstance(const, types.CodeType) and const.co_name == code_name:
            return const
    return None


def _free_vars(fn) -> dict[str, Any]:
    code = fn.__code__
    cells = fn.__closure__ or ()
    return {name: cell.cell_contents for name, cell in zip(code.co_freevars, cells)}


class _Recognizer:
    """Turns a mask callable into a canonical term, collecting captured tensors.

    Terms: ``("causal",)``, ``("window", W)``, ``("vision",)``, ``("packed",)``,
    ``("and", frozenset(terms))``, ``("or", frozenset(terms))``.  Nested
    and/or of the same kind are flattened, so terms compare as boolean
    formulas up to associativity, commutativity and duplicate children.
    """

    def __init__(self, masking_utils):
        self.mu = masking_utils
        self.codes = {
            "and": _factory_code(masking_utils, "and_masks", "and_mask"),
            "or": _factory_code(masking_utils, "or_masks", "or_mask"),
            "window": _factory_code(masking_utils, "sliding_window_overlay", "inner_mask"),
            "vision": _factory_code(masking_utils, "blockwise_overlay", "inner_mask"),
            "packed": _factory_code(masking_utils, "packed_sequence_mask_function", "inner_mask"),
        }
        self.captured: dict[str, list[torch.Tensor]] = {"vision": [], "packed": []}

    def term(self, fn):
        if not callable(fn) or getattr(fn, "__globals__", None) is not vars(self.mu):
            return None
        if fn is self.mu.causal_mask_function:
            return ("causal",)
        code = getattr(fn, "__code__", None)
        kind = next((k for k, c in self.codes.items() if c is not None and c is code), None)
        if kind is None:
            return None
        free = _free_vars(fn)
        if kind in ("and", "or"):
            children = free.get("mask_functions")
            if not isinstance(children, tuple) or not children:
                return None
            parts = set()
            for child in children:
                sub = self.term(child)
                if sub is None:
                    return None
                if sub[0] == kind:
                    parts.update(sub[1])
                else:
                    parts.add(sub)
            if len(parts) == 1:
                return next(iter(parts))
            return (kind, frozenset(parts))
        if kind == "window":
            width = free.get("sliding_window")
            if isinstance(width, bool) or not isinstance(width, int):
                return None
            return ("window", width)
        name = "block_sequence_ids" if kind == "vision" else "packed_sequence_mask"
        tensor = free.get(name)
        if not isinstance(tensor, torch.Tensor) or tensor.ndim != 2:
            return None
        self.captured[kind].append(tensor)
        return (kind,)


def _and(*terms):
    parts = set()
    for t in terms:
        parts.update(t[1] if t[0] == "and" else (t,))
    return ("and", frozenset(parts)) if len(parts) > 1 else next(iter(parts))


def _expected_term(spec: AttentionLayerSpec, *, vision: bool, packed: bool):
    causal = ("causal",)
    if spec.kind == "full_attention":
        base = causal
    else:
        allow = ("or", frozenset({causal, ("vision",)})) if vision else causal
        base = _and(("window", spec.sliding_window), allow)
    return _and(base, ("packed",)) if packed else base


# --------------------------------------------------------------------------
# Input normalisation (ti.py:688-757, 1176-1247)
# --------------------------------------------------------------------------


def _spec_for_module(module: Any) -> AttentionLayerSpec:
    layer_idx = getattr(module, "layer_idx", None)
    if isinstance(layer_idx, bool) or not isinstance(layer_idx, int):
        raise ValueError("Gemma 4 attention module must expose an integer layer_idx")
    try:
        return GEMMA4_31B.spec_for_layer(layer_idx)
    except IndexError as exc:
        raise IndexError(f"Gemma 4 layer index {layer_idx} is outside 0..59") from exc


def _validate_semantics(module, spec, *, dropout, scaling, sliding_window, output_attentions):
    if scaling is None:
        scaling = getattr(module, "scaling", 1.0)
    if scaling != 1.0:
        raise ValueError("Gemma 4 attention scaling must be exactly 1.0")
    if dropout != 0.0:
        raise ValueError("Gemma 4 MI355X attention requires zero dropout")
    if output_attentions:
        raise UnsupportedMI355XPath(
            "output_attentions/attention weights are not exposed by the MI355X integration"
        )
    if sliding_window != spec.sliding_window:
        raise ValueError(
            f"layer {module.layer_idx} requires sliding_window={spec.sliding_window}, "
            f"got {sliding_window}"
        )
    if getattr(module, "scaling", 1.0) != 1.0:
        raise ValueError("the Gemma attention module must have scaling=1.0")
    if getattr(module, "head_dim", spec.head_dim_qk) != spec.head_dim_qk:
        raise ValueError("module head_dim conflicts with the locked layer index")
    if getattr(module, "num_key_value_groups", spec.qhead_per_kvhead) != spec.qhead_per_kvhead:
        raise ValueError("module GQA ratio conflicts with the locked layer index")


def _validate_prepared(q, k, v, spec) -> tuple[int, int, int]:
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("Transformers prepared q, k, and v must be rank-4 BHSD tensors")
    if not (q.device == k.device == v.device):
        raise ValueError("prepared q, k, and v must share one device")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise ValueError("the Gemma 4 MI355X integration accepts BF16 q, k, and v only")
    if any(t.stride(-1) != 1 for t in (q, k, v)):
        raise ValueError("prepared q, k, and v must have unit last-dimension stride")
    if any(s <= 0 for t in (q, k, v) for s in t.stride()):
        raise ValueError("prepared q, k, and v must use positive, non-broadcast layouts")
    batch, q_heads, q_len, q_dim = q.shape
    k_batch, kv_heads, kv_len, k_dim = k.shape
    if batch <= 0 or q_len <= 0 or kv_len <= 0:
        raise ValueError("batch and sequence lengths must be positive")
    if k_batch != batch or v.shape[0] != batch:
        raise ValueError("prepared q, k, and v batch dimensions must match")
    if (q_heads, q_dim) != (spec.num_q_heads, spec.head_dim_qk):
        raise ValueError("prepared q shape does not match the locked layer geometry")
    if (kv_heads, k_dim) != (spec.num_kv_heads, spec.head_dim_qk):
        raise ValueError("prepared k shape does not match the locked layer geometry")
    if tuple(v.shape) != (batch, spec.num_kv_heads, kv_len, spec.head_dim_v):
        raise ValueError("prepared v shape does not match the locked layer geometry")
    if k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr():
        raise ValueError("prepared K and V must be distinct, non-aliasing operands")
    return batch, q_len, kv_len


def _as_int(value, *, name: str) -> int:
    if isinstance(value, bool):
        raise TypeError(f"{name} must be an integer, not bool")
    if isinstance(value, int):
        return value
    if isinstance(value, torch.Tensor) and value.numel() == 1 and not value.is_floating_point():
        if value.dtype == torch.bool:
            raise TypeError(f"{name} scalar tensor must use an integer, non-bool dtype")
        return int(value.detach().item())
    raise TypeError(f"{name} must be a Python integer or scalar integer tensor")


def _rows(values, *, name: str, batch: int, length: int, device, pad: int | None):
    """(1 or B, <= length) INT32/INT64 metadata -> (B, length) int64."""
    if values is None:
        return None
    if values.ndim != 2 or values.shape[0] not in (1, batch):
        raise ValueError(f"{name} must have shape (1 or {batch}, {length})")
    if values.device != device:
        raise ValueError(f"{name} must share the prepared tensor device")
    if values.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must use INT32 or INT64")
    values = values.to(torch.int64).expand(batch, -1)
    if values.shape[1] != length:
        if pad is None or values.shape[1] > length:
            raise ValueError(f"{name} must have shape (1 or {batch}, {length})")
        values = torch.nn.functional.pad(values, (0, length - values.shape[1]), value=pad)
    return values


def _padding(plan: Gemma4MaskPlan, device) -> torch.Tensor | None:
    """2D 0/1 padding mask restricted to this call's keys (ti.py:997-1017)."""
    mask = plan.attention_mask
    if mask is None:
        return None
    if mask.ndim != 2:
        raise UnsupportedMI355XPath("only 2D padding masks are accepted beside a mask plan")
    if mask.shape[0] not in (1, plan.batch_size):
        raise ValueError("2D attention mask batch dimension must be 1 or match prepared q/k/v")
    mask = mask.to(device).expand(plan.batch_size, -1)
    if not bool(((mask == 0) | (mask == 1)).all().item()):
        raise ValueError("2D attention mask must use 0/1 padding values")
    kv_offset = _as_int(plan.kv_offset, name="kv_offset")
    if kv_offset < 0:
        raise ValueError("kv_offset must be nonnegative")
    end = kv_offset + plan.kv_length
    if mask.shape[1] < end:
        mask = torch.nn.functional.pad(mask, (0, end - mask.shape[1]), value=0)
    return mask[:, kv_offset:end].to(torch.bool)


def _lower_right(plan: Gemma4MaskPlan) -> bool:
    try:
        q_off = _as_int(plan.q_offset, name="q_offset")
        kv_off = _as_int(plan.kv_offset, name="kv_offset")
    except TypeError:
        return False
    return q_off - kv_off == plan.kv_length - plan.q_length


def _static_cache_prefix(query, key, value, plan: Gemma4MaskPlan, *, trusted: bool,
                         vision, documents, grad: bool, explicit_packed: bool):
    """Trim an underfilled eager StaticCache to its active K prefix (ti.py:1020-1110).

    A StaticCache layer returns its whole physical K/V backing after the
    update, while the mask plan was built before it: the query offset and
    the K offset give the active length ``q_offset + Sq - kv_offset``.
    Returns ``(key, value, plan, vision, trimmed)``; raises
    ``UnsupportedMI355XPath`` with the reference's messages where its B1
    text-only no-grad contract does not hold.  Nothing is copied: K and V are
    views of the physical backing.
    """
    physical_k = key.shape[2]
    try:
        q_offset = _as_int(plan.q_offset, name="q_offset")
        kv_offset = _as_int(plan.kv_offset, name="kv_offset")
    except TypeError as exc:
        raise UnsupportedMI355XPath(
            "eager StaticCache active-prefix offsets must be real scalar integers"
        ) from exc
    logical_k = q_offset + query.shape[2] - kv_offset
    if logical_k == physical_k:
        return key, value, plan, vision, False
    if logical_k <= 0 or logical_k > physical_k:
        raise UnsupportedMI355XPath(
            "eager StaticCache active K length is outside the physical K/V backing"
        )
    if q_offset < 0 or kv_offset < 0 or q_offset < kv_offset:
        raise UnsupportedMI355XPath(
            "eager StaticCache offsets must describe a nonnegative lower-right prefix"
        )
    if kv_offset != 0:
        raise UnsupportedMI355XPath(
            "an underfilled eager StaticCache prefix must start at physical K offset zero"
        )
    if query.shape[0] != 1:
        raise UnsupportedMI355XPath("eager StaticCache normalization accepts B1 only")
    if grad:
        raise UnsupportedMI355XPath("eager StaticCache normalization is inference-only")
    if explicit_packed:
        raise UnsupportedMI355XPath(
            "eager StaticCache normalization does not accept explicit packed lengths"
        )
    if documents is not None:
        raise UnsupportedMI355XPath(
            "eager StaticCache normalization does not accept document metadata"
        )
    if vision is not None:
        if bool((vision >= 0).any().item()):
            raise UnsupportedMI355XPath(
                "eager StaticCache normalization accepts text-only vision metadata"
            )
        vision = None
    padding = _padding(plan, query.device)
    if padding is not None and (
        padding.shape != (1, physical_k) or not bool(padding[0, :logical_k].all().item())
    ):
        raise UnsupportedMI355XPath("eager StaticCache requires one contiguous valid K prefix")
    if not trusted:
        # The native plan masks every trimmed key (each lies past the last
        # query); another callable must be shown to do so on all of them.
        dev = query.device
        q_pos = torch.arange(q_offset, q_offset + query.shape[2], device=dev)
        tail = torch.arange(kv_offset + logical_k, kv_offset + physical_k, device=dev)
        if bool(_eval_mask_rows(plan.mask_function, 0, q_pos, tail).any().item()):
            raise UnsupportedMI355XPath(
                "the mask admits keys past the eager StaticCache active prefix"
            )
    mask = plan.attention_mask
    trimmed = replace(plan, kv_length=logical_k,
                      attention_mask=None if mask is None else mask[:, :logical_k])
    if getattr(plan, "_g4_origin", None) is _NATIVE_ORIGIN:
        object.__setattr__(trimmed, "_g4_origin", _NATIVE_ORIGIN)
    return key[:, :, :logical_k, :], value[:, :, :logical_k, :], trimmed, vision, True


def _run_starts(*rows: torch.Tensor) -> torch.Tensor:
    """True where any of the equal-length 1-D tensors changes value."""
    start = torch.zeros_like(rows[0], dtype=torch.bool)
    start[:1] = True
    for row in rows:
        start[1:] |= row[1:] != row[:-1]
    return start


def _single_run_per_value(row: torch.Tensor) -> bool:
    if row.numel() == 0:
        return True
    return int(_run_starts(row).sum().item()) == int(torch.unique(row).numel())


# --------------------------------------------------------------------------
# Native segmentation: which tokens form which packed segment
# --------------------------------------------------------------------------


@dataclass
class _Segments:
    """Native packed problem derived from a plan and its metadata.

    ``q_seg``/``k_seg`` give, per (row, position), the segment index or -1 for
    a padded position; segments are numbered in row-major token order, so
    packing the non-negative entries keeps each segment contiguous.
    """

    q_seg: torch.Tensor  # (B, Sq) int64
    k_seg: torch.Tensor  # (B, Sk) int64
    q_lengths: list[int]
    k_lengths: list[int]
    all_valid: bool

    @property
    def count(self) -> int:
        return len(self.q_lengths)


def _split_rows(valid: torch.Tensor, splits: list[torch.Tensor]) -> tuple[torch.Tensor, list[int]]:
    """Number the maximal runs (of every tensor in ``splits``) among valid tokens."""
    batch, length = valid.shape
    seg = torch.full((batch, length), -1, dtype=torch.int64, device=valid.device)
    lengths: list[int] = []
    for b in range(batch):
        idx = torch.nonzero(valid[b], as_tuple=False).flatten()
        if idx.numel() == 0:
            continue
        first, last = int(idx[0].item()), int(idx[-1].item())
        if idx.numel() != last - first + 1:
            raise UnsupportedMI355XPath("holey padding is outside the native packed contract")
        rows = [s[b, first : last + 1] for s in splits] or [idx]
        starts = _run_starts(*rows) if splits else torch.zeros_like(idx, dtype=torch.bool)
        starts[0] = True
        local = starts.to(torch.int64).cumsum(0) - 1
        seg[b, first : last + 1] = local + len(lengths)
        lengths.extend(int(c) for c in torch.bincount(local).tolist())
    return seg, lengths


def _cumulative_list(cu: torch.Tensor, *, name: str) -> list[int]:
    if cu.ndim != 1 or cu.dtype != torch.int32:
        raise ValueError(f"{name} must be a rank-1 INT32 tensor")
    raw = [int(x) for x in cu.detach().cpu().tolist()]
    if len(raw) < 2 or raw[0] != 0:
        raise ValueError(f"{name} must start at zero")
    if any(b < a for a, b in zip(raw[:-1], raw[1:])):
        raise ValueError(f"{name} must describe nondecreasing segments")
    return raw


def _build_segments(
    plan: Gemma4MaskPlan,
    *,
    device,
    padding: torch.Tensor | None,
    splits: list[torch.Tensor],
    cu_q: torch.Tensor | None,
    cu_k: torch.Tensor | None,
    cu_may_split: bool,
) -> _Segments:
    """Prefill (Sq == Sk): runs of ``splits`` among valid tokens; with
    ``cu_may_split`` and no other boundary source, explicit ``cu`` lengths
    define the segments, otherwise they must equal the derived ones
    (ti.py:1325-1352).  Lower-right rows (Sq < Sk): one segment per row."""
    B, Sq, Sk = plan.batch_size, plan.q_length, plan.kv_length
    all_valid = padding is None or bool(padding.all().item())
    if (cu_q is None) != (cu_k is None):
        raise ValueError("cu_seq_lens_q and cu_seq_lens_k must be provided together")
    if Sq > Sk:
        raise UnsupportedMI355XPath("prepared Q is longer than K; no lower-right alignment exists")
    if Sq == Sk:
        valid = torch.ones((B, Sq), dtype=torch.bool, device=device) if padding is None else padding
        if cu_q is not None and cu_may_split and not splits and all_valid:
            raw = _cumulative_list(cu_q, name="cu_seq_lens_q")
            if raw[-1] != B * Sq or not set(range(0, B * Sq + 1, Sq)).issubset(raw):
                raise ValueError("cu_seq_lens_q must end at B*S and keep every batch-row boundary")
            marks = torch.zeros(B * Sq, dtype=torch.int64, device=device)
            marks[torch.tensor(raw[1:-1], dtype=torch.int64, device=device)] = 1
            splits = [marks.cumsum(0).view(B, Sq)]
        seg, q_lengths = _split_rows(valid, splits)
        seg_k, k_lengths = seg.clone(), list(q_lengths)
    else:
        if not all_valid:
            raise UnsupportedMI355XPath("padded lower-right attention is outside the native contract")
        rows = torch.arange(B, dtype=torch.int64, device=device)[:, None]
        seg, seg_k = rows.expand(B, Sq).clone(), rows.expand(B, Sk).clone()
        q_lengths, k_lengths = [Sq] * B, [Sk] * B
    if cu_q is not None:
        for cu, lengths, name in ((cu_q, q_lengths, "cu_seq_lens_q"), (cu_k, k_lengths, "cu_seq_lens_k")):
            raw = _cumulative_list(cu, name=name)
            if [b - a for a, b in zip(raw[:-1], raw[1:])] != lengths:
                raise ValueError(f"{name} conflicts with the segments implied by padding/position_ids/mask")
    return _Segments(seg, seg_k, q_lengths, k_lengths, all_valid)


# --------------------------------------------------------------------------
# Admission proofs
# --------------------------------------------------------------------------


def _captured_rows(tensor: torch.Tensor, plan: Gemma4MaskPlan, *, offset: int, length: int, device):
    if tensor.shape[0] not in (1, plan.batch_size) or tensor.shape[1] < offset + length:
        return None
    return tensor.to(device=device, dtype=torch.int64).expand(plan.batch_size, -1)[
        :, offset : offset + length
    ]


def _structural_proof(plan, spec, *, device, vision):
    """Return (vision, packed_ids) the kernels must use, or None if unproven."""
    mu = _masking_utils()
    if mu is None:
        return None
    rec = _Recognizer(mu)
    term = rec.term(plan.mask_function)
    if term is None:
        return None
    if len(rec.captured["vision"]) > 1 or len(rec.captured["packed"]) > 1:
        return None
    has_vision = bool(rec.captured["vision"])
    has_packed = bool(rec.captured["packed"])
    if has_vision and spec.kind == "full_attention":
        return None
    if term != _expected_term(spec, vision=has_vision, packed=has_packed):
        return None
    if not _lower_right(plan):
        return None
    kv_off = _as_int(plan.kv_offset, name="kv_offset")
    q_off = _as_int(plan.q_offset, name="q_offset")
    if has_vision:
        # The callable indexes its tensor at absolute q and kv positions; under
        # lower-right alignment both land inside [kv_offset, kv_offset + Sk).
        captured = _captured_rows(
            rec.captured["vision"][0], plan, offset=kv_off, length=plan.kv_length, device=device
        )
        if captured is None:
            return None
        if vision is not None and not torch.equal(captured, vision):
            return None
        vision = captured
    elif vision is not None and spec.kind != "full_attention" and bool((vision >= 0).any().item()):
        # Vision metadata was supplied but the mask has no bidirectional overlay.
        return None
    if has_packed:
        if plan.q_length != plan.kv_length or q_off != kv_off:
            return None
        captured = _captured_rows(
            rec.captured["packed"][0], plan, offset=q_off, length=plan.q_length, device=device
        )
        if captured is None:
            return None
        for b in range(plan.batch_size):
            if not _single_run_per_value(captured[b]):
                return None
        packed_ids = captured
    else:
        packed_ids = None
    return vision, packed_ids


def _eval_mask_rows(fn, b: int, q_pos: torch.Tensor, kv_pos: torch.Tensor) -> torch.Tensor:
    bi = torch.full((1, 1), b, dtype=torch.int64, device=q_pos.device)
    hi = torch.zeros((1, 1), dtype=torch.int64, device=q_pos.device)
    out = fn(bi, hi, q_pos[:, None], kv_pos[None, :])
    out = torch.as_tensor(out, device=q_pos.device).to(torch.bool)
    return out.expand(q_pos.numel(), kv_pos.numel())


def _native_mask_rows(segs: _Segments, seg_mask, b, q_local, k_local, rows: slice):
    qs = segs.q_seg[b, rows]
    ks = segs.k_seg[b]
    same = (qs[:, None] == ks[None, :]) & (qs[:, None] >= 0)
    gathered = seg_mask[
        qs.clamp(min=0)[:, None], q_local[b, rows].clamp(min=0)[:, None], k_local[b].clamp(min=0)[None, :]
    ]
    return same & gathered


def _local_positions(seg: torch.Tensor) -> torch.Tensor:
    """Position of each token inside its segment (-1 for padding)."""
    B, S = seg.shape
    pos = torch.full_like(seg, -1)
    for b in range(B):
        row = seg[b]
        valid = row >= 0
        if not bool(valid.any().item()):
            continue
        idx = torch.nonzero(valid, as_tuple=False).flatten()
        vals = row[idx]
        start = torch.ones_like(vals, dtype=torch.bool)
        start[1:] = vals[1:] != vals[:-1]
        first_index = torch.cummax(torch.where(start, torch.arange(idx.numel(), device=seg.device), 0), 0).values
        pos[b, idx] = torch.arange(idx.numel(), device=seg.device) - first_index
    return pos


def _evaluation_proof(plan, spec, segs: _Segments, native_plan, padding, device) -> bool:
    """Exhaustive device comparison of the callable with the native predicate."""
    from .ops import mask_materialize

    if device.type != "cuda":
        return False  # the native predicate is evaluated by the device library only
    if plan.batch_size * plan.q_length * plan.kv_length > _EVAL_PROOF_MAX_PAIRS:
        return False
    try:
        q_off = _as_int(plan.q_offset, name="q_offset")
        kv_off = _as_int(plan.kv_offset, name="kv_offset")
    except TypeError:
        return False
    seg_mask = mask_materialize(native_plan, device)
    # Fixed plans put the single row's segment at index 0 per row as well.
    q_local = _local_positions(segs.q_seg)
    k_local = _local_positions(segs.k_seg)
    q_pos = torch.arange(plan.q_length, device=device, dtype=torch.int64) + q_off
    kv_pos = torch.arange(plan.kv_length, device=device, dtype=torch.int64) + kv_off
    chunk = max(1, (1 << 24) // max(1, plan.kv_length))
    for b in range(plan.batch_size):
        for r0 in range(0, plan.q_length, chunk):
            rows = slice(r0, min(plan.q_length, r0 + chunk))
            try:
                ref = _eval_mask_rows(plan.mask_function, b, q_pos[rows], kv_pos)
            except Exception:
                return False
            if padding is not None:
                ref = ref & padding[b][None, :]
            keep = segs.q_seg[b, rows] >= 0
            nat = _native_mask_rows(segs, seg_mask, b, q_local, k_local, rows)
            if not torch.equal(ref[keep], nat[keep]):
                return False
    return True


# --------------------------------------------------------------------------
# Packing (ti.py:1250-1447)
# --------------------------------------------------------------------------


def _cumulative(lengths: list[int], device) -> torch.Tensor:
    values = [0]
    for n in lengths:
        values.append(values[-1] + n)
    if values[-1] > torch.iinfo(torch.int32).max:
        raise UnsupportedMI355XPath("packed cumulative totals must fit signed INT32")
    return torch.tensor(values, dtype=torch.int32, device=device)


def _pack(t_bshd: torch.Tensor, seg: torch.Tensor, all_valid: bool) -> torch.Tensor:
    if all_valid and t_bshd.shape[0] == 1:
        return t_bshd[0]
    if all_valid:
        return t_bshd.reshape(-1, t_bshd.shape[2], t_bshd.shape[3])
    return t_bshd[seg >= 0]


def _unpack(out, lse, q_seg: torch.Tensor, all_valid: bool, shape):
    B, S, H, D = shape
    if all_valid:
        return out.reshape(B, S, H, D), lse.reshape(H, B, S).permute(1, 0, 2)
    idx = torch.nonzero((q_seg >= 0).reshape(-1), as_tuple=False).flatten()
    out_flat = out.new_zeros((B * S, H, D)).index_copy(0, idx, out)
    lse_flat = lse.new_full((B * S, H), float("-inf")).index_copy(0, idx, lse.transpose(0, 1))
    return out_flat.view(B, S, H, D), lse_flat.view(B, S, H).permute(0, 2, 1)


def _packed_metadata(values, seg, all_valid):
    if values is None:
        return None
    flat = values.reshape(-1) if all_valid else values[seg >= 0]
    return flat.to(torch.int32)


# --------------------------------------------------------------------------
# Routing (ti.py:1702-2075)
# --------------------------------------------------------------------------


# --------------------------------------------------------------------------
# torch.compile / FakeTensor route (ti.py:761-921)
# --------------------------------------------------------------------------


def _is_fake(t: torch.Tensor) -> bool:
    try:
        from torch._subclasses.fake_tensor import FakeTensor
    except ImportError:  # pragma: no cover
        return False
    return isinstance(t, FakeTensor)


def _compiling() -> bool:
    compiler = getattr(torch, "compiler", None)
    is_compiling = getattr(compiler, "is_compiling", None)
    return bool(is_compiling()) if callable(is_compiling) else False


def _compiled_forward(module, query, key, value, plan, spec: AttentionLayerSpec, *,
                      position_ids, vision_block_ids, document_ids, cu_seq_lens_q,
                      cu_seq_lens_k, max_length_q, max_length_k, extra) -> Gemma4DispatchResult:
    """Admit one text sequence as a single opaque custom operator.

    The reference's compiled fixed-forward ABI (ti.py:761-921): an eval-mode
    module, a mask plan without padding or offsets whose mask is the text-only
    predicate of the layer (causal; causal within the window for sliding
    layers), B = 1, Sq = Sk in 1..1024, BF16 prepared q/k/v of the locked
    geometry, explicit position_ids, and no metadata, packed lengths or cache.
    The operator (``gemma4_mi355x::local_fwd`` / ``global_fwd``) is opaque to
    the tracer and checks positions on the device when it runs.
    """
    label = "FakeTensor/torch.compile"
    if getattr(module, "training", False):
        raise UnsupportedMI355XPath(f"{label} routing requires an eval-mode attention module")
    if not isinstance(plan, Gemma4MaskPlan):
        raise UnsupportedMI355XPath(f"Transformers {label} requires a Gemma4MaskPlan")
    if plan.attention_mask is not None:
        raise UnsupportedMI355XPath(f"{label} does not accept padding or explicit masks")
    for name in ("q_offset", "kv_offset"):
        offset = getattr(plan, name)
        if type(offset) is not int or offset != 0:
            raise UnsupportedMI355XPath(f"{label} does not accept {name.split('_')[0].upper()} "
                                        "offsets")
    if plan.mask_function is not None and getattr(plan, "_g4_origin", None) is not _NATIVE_ORIGIN:
        mu = _masking_utils()
        rec = _Recognizer(mu) if mu is not None else None
        term = rec.term(plan.mask_function) if rec is not None else None
        if term is None or rec.captured["vision"] or rec.captured["packed"] or \
                term != _expected_term(spec, vision=False, packed=False):
            raise UnsupportedMI355XPath(f"{label} accepts only the layer's text-only mask "
                                        "(causal, or causal within the sliding window)")
    tensors = (query, key, value)
    if any(t.ndim != 4 for t in tensors):
        raise UnsupportedMI355XPath(f"{label} requires rank-4 prepared BHSD Q/K/V")
    if not (query.device == key.device == value.device) or query.device.type != "cuda":
        raise UnsupportedMI355XPath(f"{label} requires Q/K/V on one CUDA device")
    if any(t.dtype != torch.bfloat16 for t in tensors):
        raise UnsupportedMI355XPath(f"{label} requires BF16 prepared Q/K/V")
    if not _compiling():
        fake = [_is_fake(t) for t in tensors]
        if any(fake) and not all(fake):
            raise UnsupportedMI355XPath(f"{label} requires Q/K/V to share one tensor mode")
    if any(t.requires_grad for t in tensors):
        raise UnsupportedMI355XPath(f"{label} is forward-only and rejects requires_grad inputs")
    b, hq, sq, dq = query.shape
    kb, hkv, sk, dk = key.shape
    if b != 1 or kb != 1 or value.shape[0] != 1:
        raise UnsupportedMI355XPath(f"{label} accepts B1 only")
    if sq != sk or value.shape[2] != sk:
        raise UnsupportedMI355XPath(f"{label} requires equal Q/K/V sequence lengths")
    if not 1 <= sq <= 1024:
        raise UnsupportedMI355XPath(f"{label} requires a sequence length in 1..1024")
    if (hq, dq) != (spec.num_q_heads, spec.head_dim_qk):
        raise UnsupportedMI355XPath(f"{label} Q geometry conflicts with the locked layer")
    if (hkv, dk) != (spec.num_kv_heads, spec.head_dim_qk) or \
            tuple(value.shape[1:]) != (spec.num_kv_heads, sk, spec.head_dim_v):
        raise UnsupportedMI355XPath(f"{label} K/V geometry conflicts with the locked layer")
    if (plan.batch_size, plan.q_length, plan.kv_length) != (b, sq, sk):
        raise UnsupportedMI355XPath("mask plan dimensions do not match prepared Q/K/V")
    if not isinstance(position_ids, torch.Tensor):
        raise UnsupportedMI355XPath(f"{label} requires explicit position_ids")
    if position_ids.ndim != 2 or tuple(position_ids.shape) != (1, sq) or \
            position_ids.device != query.device or \
            position_ids.dtype not in (torch.int32, torch.int64):
        raise UnsupportedMI355XPath("compiled position_ids must be CUDA INT32/INT64 with shape "
                                    "(1, S)")
    if vision_block_ids is not None or document_ids is not None:
        raise UnsupportedMI355XPath(f"{label} accepts text-only requests without metadata")
    if any(x is not None for x in (cu_seq_lens_q, cu_seq_lens_k, max_length_q, max_length_k)):
        raise UnsupportedMI355XPath(f"{label} does not accept packed sequence metadata")
    if any(extra.get(name) is not None for name in ("past_key_values", "cache",
                                                    "cache_position")):
        raise UnsupportedMI355XPath(f"{label} does not accept a cache")
    from . import torch_ops

    if not torch_ops.CUSTOM_OPS_AVAILABLE:  # pragma: no cover
        raise UnsupportedMI355XPath(f"{label} requires torch.library custom_op and register_fake")
    # packed-sequence ids implied by the positions: a new run wherever the
    # position does not advance by one (the operator checks them on the device)
    first = position_ids[:, :1] - 1
    packed = (torch.diff(position_ids, prepend=first, dim=-1) != 1).cumsum(-1)
    if spec.kind == "full_attention":
        out, lse = torch_ops.global_fwd(query, key, value, position_ids, packed)
        return Gemma4DispatchResult(out, lse, "fa4_global_compiled_op")
    out, lse = torch_ops.local_fwd(query, key, value, position_ids, packed)
    return Gemma4DispatchResult(out, lse, "fa4_local_compiled_op")


def gemma4_fa4_prepared(
    module: Any,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Gemma4MaskPlan | torch.Tensor | None,
    *,
    dropout: float = 0.0,
    scaling: float | None = 1.0,
    sliding_window: int | None = None,
    position_ids: torch.Tensor | None = None,
    vision_block_ids: torch.Tensor | None = None,
    document_ids: torch.Tensor | None = None,
    cu_seq_lens_q: torch.Tensor | None = None,
    cu_seq_lens_k: torch.Tensor | None = None,
    max_length_q: int | torch.Tensor | None = None,
    max_length_k: int | torch.Tensor | None = None,
    allow_flex_fallback: bool = True,
    output_attentions: bool = False,
    **_kwargs: Any,
) -> Gemma4DispatchResult:
    """Route Transformers-prepared BHSD q/k/v to the native MI355X kernels."""
    del allow_flex_fallback  # no non-native route exists; see the module docstring
    spec = _spec_for_module(module)
    _validate_semantics(
        module, spec, dropout=dropout, scaling=scaling, sliding_window=sliding_window,
        output_attentions=output_attentions,
    )
    if _compiling() or any(_is_fake(t) for t in (query, key, value)):
        return _compiled_forward(
            module, query, key, value, attention_mask, spec, position_ids=position_ids,
            vision_block_ids=vision_block_ids, document_ids=document_ids,
            cu_seq_lens_q=cu_seq_lens_q, cu_seq_lens_k=cu_seq_lens_k,
            max_length_q=max_length_q, max_length_k=max_length_k, extra=_kwargs,
        )
    B, Sq, Sk = _validate_prepared(query, key, value, spec)
    device = query.device
    local = spec.kind != "full_attention"

    if isinstance(attention_mask, Gemma4MaskPlan):
        plan = attention_mask
        if (plan.batch_size, plan.q_length, plan.kv_length) != (B, Sq, Sk):
            raise ValueError("Gemma4MaskPlan dimensions do not match prepared q/k/v")
    elif attention_mask is None or isinstance(attention_mask, torch.Tensor):
        if attention_mask is not None and attention_mask.ndim != 2:
            raise UnsupportedMI355XPath(
                "a materialised 4D mask cannot be proven equal to the native predicate"
            )
        plan = Gemma4MaskPlan(B, Sq, Sk, Sk - Sq, 0, None, attention_mask)
        object.__setattr__(plan, "_g4_origin", _NATIVE_ORIGIN)
    else:
        raise TypeError("attention_mask must be a Gemma4MaskPlan, tensor, or None")

    if position_ids is not None:
        if position_ids.ndim != 2 or position_ids.shape[1] != Sq or position_ids.shape[0] not in (1, B):
            raise ValueError("position_ids must have shape (1 or B, prepared Q length)")
        if position_ids.device != device:
            raise ValueError("position_ids must share the prepared tensor device")
        position_ids = position_ids.to(torch.int64).expand(B, -1)
    vision = _rows(vision_block_ids, name="vision_block_ids", batch=B, length=Sk, device=device, pad=-1)
    documents = _rows(document_ids, name="document_ids", batch=B, length=Sk, device=device, pad=-1)

    trusted = plan.mask_function is None or getattr(plan, "_g4_origin", None) is _NATIVE_ORIGIN
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value))
    key, value, plan, vision, trimmed = _static_cache_prefix(
        query, key, value, plan, trusted=trusted, vision=vision, documents=documents, grad=grad,
        explicit_packed=any(x is not None for x in (cu_seq_lens_q, cu_seq_lens_k, max_length_q,
                                                       max_length_k)),
    )
    if trimmed:
        Sk = key.shape[2]
        # A cache is present: position_ids restarts are not packing boundaries
        # (ti.py:1831-1835).
        position_ids = None
    padding = _padding(plan, device)

    if trusted and not _lower_right(plan):
        raise UnsupportedMI355XPath("cache/query offsets are not the native lower-right alignment")
    structural = None
    if not trusted:
        structural = _structural_proof(plan, spec, device=device, vision=vision)

    # Boundary sources.  A recognised mask carries its own packed-sequence ids;
    # otherwise position_ids restarts split prefill rows (ti.py:1141-1173).
    splits: list[torch.Tensor] = []
    if structural is not None:
        vision, packed_ids = structural
        if packed_ids is not None:
            splits.append(packed_ids)
    elif Sq == Sk and position_ids is not None:
        restart = torch.zeros_like(position_ids, dtype=torch.bool)
        restart[:, 1:] = position_ids[:, 1:] - position_ids[:, :-1] != 1
        splits.append(restart.to(torch.int64).cumsum(1))
    if vision is not None and (not local or not bool((vision >= 0).any().item())):
        vision = None  # global layers ignore vision; all-text metadata is the text path

    # Documents: local kernels evaluate the document predicate themselves.  A
    # recognised mask has no document term, and global kernels carry no
    # document ids: there the documents must coincide with segment boundaries.
    docs_as_boundaries = documents is not None and (structural is not None or not local)
    base_split = splits[0] if splits else torch.zeros((B, Sq), dtype=torch.int64, device=device)
    if docs_as_boundaries and Sq == Sk and structural is None:
        splits.append(documents)
    segs = _build_segments(
        plan, device=device, padding=padding, splits=splits,
        cu_q=cu_seq_lens_q, cu_k=cu_seq_lens_k, cu_may_split=structural is None,
    )
    if docs_as_boundaries:
        for b in range(B):
            valid = segs.k_seg[b] >= 0
            seg_row, doc_row = segs.k_seg[b][valid], documents[b][valid]
            if Sq == Sk and structural is None:
                seg_row = base_split[b][valid]  # segments before the document split
            if structural is not None or Sq != Sk:
                # Documents must be constant inside every segment.
                if bool((_run_starts(doc_row) & ~_run_starts(seg_row)).any().item()):
                    raise UnsupportedMI355XPath(
                        "document boundaries inside a segment are not part of the proven mask"
                    )
            elif int(_run_starts(seg_row, doc_row).sum().item()) != int(
                torch.unique(torch.stack((seg_row, doc_row)), dim=1).shape[1]
            ):
                raise UnsupportedMI355XPath(
                    "a document id that reappears after another one needs a document "
                    "predicate the global route does not carry"
                )
        documents = None

    if sum(segs.q_lengths) <= 0 or sum(segs.k_lengths) <= 0:
        raise UnsupportedMI355XPath("packed physical Q/K totals must both be positive")
    max_q, max_k = max(segs.q_lengths), max(segs.k_lengths)
    for value_, derived, name in ((max_length_q, max_q, "max_length_q"), (max_length_k, max_k, "max_length_k")):
        if value_ is not None and _as_int(value_, name=name) != derived:
            raise ValueError("max_length_q/max_length_k must equal the cumulative maxima")

    q_bshd, k_bshd, v_bshd = (t.transpose(1, 2) for t in (query, key, value))
    packed_vision = _packed_metadata(vision, segs.k_seg, segs.all_valid)
    packed_docs = _packed_metadata(documents if local else None, segs.k_seg, segs.all_valid)
    cu_q = _cumulative(segs.q_lengths, device)
    cu_k = _cumulative(segs.k_lengths, device)

    if not trusted and structural is None:
        from .ops import make_plan

        native_plan = make_plan(
            num_seqs=segs.count, seqlen_q=max_q, seqlen_k=max_k,
            num_q_heads=spec.num_q_heads, num_kv_heads=spec.num_kv_heads,
            head_dim=spec.head_dim_qk, window=spec.sliding_window if local else None,
            vision=packed_vision, documents=packed_docs, cu_q=cu_q, cu_k=cu_k,
            total_q=sum(segs.q_lengths), total_k=sum(segs.k_lengths),
        )
        if not _evaluation_proof(plan, spec, segs, native_plan, padding, device):
            raise UnsupportedMI355XPath(
                "the mask is not provably the native Gemma 4 predicate "
                "(unrecognised callable, non-lower-right offsets, or missing vision metadata)"
            )

    single = B == 1 and Sq == Sk and segs.count == 1 and segs.all_valid and documents is None

    if not local:
        if single and Sq <= (_FIXED_GLOBAL_MAX_GRAD if grad else _FIXED_GLOBAL_MAX_NOGRAD):
            out, lse = fa4_global_text_forward(q_bshd, k_bshd, v_bshd, spec=spec)
            return Gemma4DispatchResult(out, lse, "fa4_global_fixed")
        rows_only = segs.all_valid and segs.count == B
        if not grad and Sk > _FIXED_GLOBAL_MAX_NOGRAD and rows_only:
            out, lse = fa4_global_forward_only(q_bshd, k_bshd, v_bshd, spec=spec)
            return Gemma4DispatchResult(out, lse, "fa4_global_forward_only")
        q_p, k_p, v_p = (
            _pack(q_bshd, segs.q_seg, segs.all_valid),
            _pack(k_bshd, segs.k_seg, segs.all_valid),
            _pack(v_bshd, segs.k_seg, segs.all_valid),
        )
        run = fa4_global_varlen_forward if grad else fa4_global_varlen_forward_only
        out, lse = run(q_p, k_p, v_p, cu_q, cu_k, max_seqlen_q=max_q, max_seqlen_k=max_k, spec=spec)
        out, lse = _unpack(out, lse, segs.q_seg, segs.all_valid, tuple(q_bshd.shape))
        path = "fa4_global_varlen_native" if grad else "fa4_global_varlen_forward_only"
        return Gemma4DispatchResult(out, lse, path)

    if single and Sq <= _FIXED_LOCAL_MAX and _lower_right(plan):
        ids = None if vision is None else vision.to(torch.int32)
        out, lse = fa4_local_forward(q_bshd, k_bshd, v_bshd, vision_block_ids=ids, spec=spec)
        return Gemma4DispatchResult(out, lse, "fa4_local_fixed")
    q_p, k_p, v_p = (
        _pack(q_bshd, segs.q_seg, segs.all_valid),
        _pack(k_bshd, segs.k_seg, segs.all_valid),
        _pack(v_bshd, segs.k_seg, segs.all_valid),
    )
    out, lse = fa4_local_varlen_forward(
        q_p, k_p, v_p, cu_q, cu_k, max_seqlen_q=max_q, max_seqlen_k=max_k,
        vision_block_ids=packed_vision, document_ids=packed_docs, spec=spec,
    )
    out, lse = _unpack(out, lse, segs.q_seg, segs.all_valid, tuple(q_bshd.shape))
    return Gemma4DispatchResult(out, lse, "fa4_local_varlen")


def gemma4_fa4_attention_forward(
    module: Any,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Gemma4MaskPlan | torch.Tensor | None,
    **kwargs: Any,
) -> tuple[torch.Tensor, None]:
    """Transformers attention-interface entry point: ``(O_bshd, None)`` (ti.py:2078-2098)."""
    result = gemma4_fa4_prepared(module, query, key, value, attention_mask, **kwargs)
    module._gemma4_fa4_last_path = result.path
    return result.output, None


# --------------------------------------------------------------------------
# Registration (ti.py:3493-3547)
# --------------------------------------------------------------------------


def _registered(registry: Any, name: str):
    try:
        return registry[name]
    except (KeyError, TypeError):
        return None


def register_gemma4_mi355x(attention_registry: Any = None, mask_registry: Any = None) -> str:
    """Register the attention and mask callbacks under ``BACKEND_NAME``.

    Idempotent; raises ``RuntimeError`` (registering nothing) when either name
    is already taken by a different callable.  The registries default to
    Transformers' ``ALL_ATTENTION_FUNCTIONS`` and ``ALL_MASK_ATTENTION_FUNCTIONS``.
    """
    if attention_registry is None or mask_registry is None:
        try:
            from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
            from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
        except Exception as exc:
            raise RuntimeError("Transformers is required for backend registration") from exc
        attention_registry = attention_registry or ALL_ATTENTION_FUNCTIONS
        mask_registry = mask_registry or ALL_MASK_ATTENTION_FUNCTIONS
    targets = (
        (attention_registry, gemma4_fa4_attention_forward, "attention"),
        (mask_registry, gemma4_fa4_mask, "mask"),
    )
    for registry, fn, label in targets:
        existing = _registered(registry, BACKEND_NAME)
        if existing is not None and existing is not fn:
            raise RuntimeError(f"Transformers {label} backend {BACKEND_NAME!r} is already registered")
    for registry, fn, _label in targets:
        if _registered(registry, BACKEND_NAME) is None:
            registry.register(BACKEND_NAME, fn)
    return BACKEND_NAME


# The reference's registration name, kept for callers switching over.
register_gemma4_fa4_h100 = register_gemma4_mi355x

__all__ = [
    "BACKEND_NAME",
    "Gemma4DispatchResult",
    "Gemma4MaskPlan",
    "gemma4_fa4_attention_forward",
    "gemma4_fa4_mask",
    "gemma4_fa4_prepared",
    "register_gemma4_fa4_h100",
    "register_gemma4_mi355x",
]
