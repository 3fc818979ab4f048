"""Drop-in MI355X adapters for the Gemma 4 attention hot path.

Same public functions, keyword arguments, return contracts, validation and
error classes as the reference adapters in ``src/gemma4_fa4/h100.py``
(750-1394); underneath, every call launches the hand-written gfx950 kernels of
``libgemma4_attn.so`` on the caller's current stream:

* forward: one launch for the full head dimension (no V slabs, no LSE
  equality sync) plus, with vision IDs, the O(T) device span table;
* backward: delta pre-pass, dK/dV (KV-tile major, GQA group reduced on chip,
  distinct dK and dV) and dQ (Q-tile major); no atomics, so gradients repeat
  bitwise.

Fixed inputs are BSHD ``(B, S, H, D)``; packed inputs are THD ``(T, H, D)``
with int32 ``cu_seqlens``; LSE is fp32 ``(B, Hq, S)`` or ``(Hq, Tq)`` and is
differentiable.  Queries are the lower-right suffix of their key sequence.
"""

from __future__ import annotations

import ctypes
import threading
import time
import weakref
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import G4Layout, G4Problem
from .errors import GlobalBackwardBudgetExceeded, UnsupportedMI355XPath
from .model_spec import GEMMA4_31B, GLOBAL_ATTENTION, SLIDING_ATTENTION, AttentionLayerSpec

_LOCAL_CUSTOM_DENSE_MAX_SEQLEN = 1025
_LOCAL_MODEL_MAX_SEQLEN = GEMMA4_31B.max_position_embeddings
_GLOBAL_FIXED_BACKWARD_MAX_SEQLEN = 2048
_GLOBAL_NATIVE_BACKWARD_MAX_SEQLEN = _LOCAL_MODEL_MAX_SEQLEN
_GLOBAL_BACKWARD_RESERVE_BYTES = 2 * 1024**3
_METADATA_WORKSPACE_MAX_BYTES = 2 * 1024**3
_TARGET_ARCH = "gfx950"


# ---------------------------------------------------------------------------
# validation (mirrors h100.py:131-367, 604-684, 1039-1145)
# ---------------------------------------------------------------------------


_FAKE_TENSOR_TYPE: list = []


def _fake_tensor_type():
    if not _FAKE_TENSOR_TYPE:
        try:
            from torch._subclasses.fake_tensor import FakeTensor
        except ImportError:  # pragma: no cover
            FakeTensor = ()
        _FAKE_TENSOR_TYPE.append(FakeTensor)
    return _FAKE_TENSOR_TYPE[0]


def _is_fake_tensor(tensor: torch.Tensor) -> bool:
    return isinstance(tensor, _fake_tensor_type())


# gcnArchName per device index: a device's architecture does not change while
# the process runs, and the property query costs a few microseconds per call.
_DEVICE_ARCH: dict[int, str] = {}


def _require_gfx950(device: torch.device) -> None:
    if device.type != "cuda":
        raise UnsupportedMI355XPath("MI355X attention inputs must be GPU tensors")
    index = device.index if device.index is not None else torch.cuda.current_device()
    arch = _DEVICE_ARCH.get(index)
    if arch is None:
        arch = torch.cuda.get_device_properties(index).gcnArchName
        _DEVICE_ARCH[index] = arch
    if not arch.startswith(_TARGET_ARCH):
        raise UnsupportedMI355XPath(f"MI355X attention requires {_TARGET_ARCH}, found {arch}")


def _has_proven_nonoverlap(tensor: torch.Tensor) -> bool:
    """Prove a positive-stride layout non-overlapping (mixed-radix argument)."""
    overlap = torch._debug_has_internal_overlap(tensor)
    if overlap == 0:
        return True
    if overlap == 1:
        return False
    covered = 0
    for stride, size in sorted(
        (st, sz) for sz, st in zip(tensor.shape, tensor.stride()) if sz > 1
    ):
        if stride <= covered:
            return False
        covered += (size - 1) * stride
    return True


def _validate_layout(tensor: torch.Tensor, *, name: str) -> None:
    strides = tensor.stride()
    if strides[-1] != 1:
        raise ValueError(f"{name} must have unit last-dimension stride")
    if min(strides) <= 0:
        raise ValueError(f"{name} must use positive, non-broadcast strides")
    for stride in strides[:-1]:
        if stride % 8:
            raise ValueError(f"{name} outer strides must be 16-byte aligned for BF16")
    if not _has_proven_nonoverlap(tensor):
        raise ValueError(f"{name} must use a non-overlapping layout")


def _check_real_operands(tensors, names, *, label: str) -> None:
    fake_type = _fake_tensor_type()
    for t in tensors:
        if isinstance(t, fake_type):
            raise UnsupportedMI355XPath(
                f"{label}: fake tensors are not supported by the MI355X path")
    for t in tensors:
        if t.data_ptr() % 16:
            raise ValueError(f"{label} base pointers must be 16-byte aligned")


def _validate_bshd(q, k, v, spec: AttentionLayerSpec, *, require_device: bool = True) -> None:
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("q, k, and v must be rank-4 B/S/H/D tensors")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, and v must be on one device")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise ValueError("the MI355X path accepts BF16 q, k, and v only")
    for name, tensor in zip(("q", "k", "v"), (q, k, v)):
        _validate_layout(tensor, name=name)
    _check_real_operands((q, k, v), ("q", "k", "v"), label="q, k, and v")
    batch, seqlen, q_heads, q_dim = q.shape
    if batch <= 0 or seqlen <= 0:
        raise ValueError("batch and sequence length must be positive")
    if (q_heads, q_dim) != (spec.num_q_heads, spec.head_dim_qk):
        raise ValueError("q shape does not match the attention spec")
    if k.shape != (batch, seqlen, spec.num_kv_heads, spec.head_dim_qk) or v.shape != (
        batch,
        seqlen,
        spec.num_kv_heads,
        spec.head_dim_v,
    ):
        raise ValueError("k/v shapes do not match the attention spec")
    if spec.qhead_per_kvhead not in {1, 2, 4, 8}:
        raise ValueError("the validated GQA ratios are 1, 2, 4, and 8")
    if k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr():
        raise ValueError("K and V must be distinct, non-aliasing prepared operands")
    if require_device:
        _require_gfx950(q.device)


def _locked_local(spec: AttentionLayerSpec, *, check_kv_heads: bool) -> bool:
    return (
        spec.kind == "sliding_attention"
        and spec.head_dim_qk == 256
        and spec.head_dim_v == 256
        and spec.num_q_heads == 32
        and (not check_kv_heads or spec.num_kv_heads == 16)
        and spec.softmax_scale == 1.0
        and spec.sliding_window == 1024
        and spec.is_causal
    )


def _locked_global(spec: AttentionLayerSpec) -> bool:
    return (
        spec.kind == "full_attention"
        and spec.head_dim_qk == 512
        and spec.head_dim_v == 512
        and spec.num_q_heads == 32
        and spec.num_kv_heads == 4
        and spec.softmax_scale == 1.0
        and spec.sliding_window is None
        and spec.is_causal
    )


def _validate_local_bshd(q, k, v, spec, *, require_device: bool = True) -> None:
    _validate_bshd(q, k, v, spec, require_device=require_device)
    if q.shape[0] != 1 or q.shape[1] > _LOCAL_CUSTOM_DENSE_MAX_SEQLEN:
        raise UnsupportedMI355XPath("fixed local attention covers only B=1 and 1 <= S <= 1025")
    if not _locked_local(spec, check_kv_heads=False):
        raise UnsupportedMI355XPath("only the locked local d256 attention contract is enabled")


def _normalize_int32_metadata(values: torch.Tensor, *, name: str) -> torch.Tensor:
    if values.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{name} must use INT32 or INT64 values")
    if values.requires_grad:
        raise ValueError(f"{name} must not require gradients")
    if values.dtype == torch.int64 and values.numel():
        lo, hi = torch.aminmax(values)
        info = torch.iinfo(torch.int32)
        if lo.item() < info.min or hi.item() > info.max:
            raise ValueError(f"INT64 {name} values must fit exactly in INT32")
    return values.to(dtype=torch.int32).contiguous()


def _prepare_vision_block_ids(vision_block_ids: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    expected = q.shape[:2]
    if vision_block_ids.shape != expected:
        raise ValueError(
            f"vision_block_ids must have shape {expected}, got {tuple(vision_block_ids.shape)}"
        )
    if vision_block_ids.device != q.device:
        raise ValueError("vision_block_ids must be on the same device as q, k, and v")
    return _normalize_int32_metadata(vision_block_ids, name="vision_block_ids").view(-1)


class _CumulativeCheck:
    """The checks that need the values of ``cu_seqlens``, run just before the first launch.

    Reading the arrays is a device-to-host copy, which waits for all earlier
    work on the stream; the reference reads them while validating
    (h100.py:351-352, 1122-1123), so the GPU sits idle for every host step
    that follows.  Here the steps that do not need the values (the checks the
    reference takes after the read, the plan, the HBM preflight, output
    allocation) run first, while the GPU is still busy, and the read happens
    immediately before the launch.  An error from such a step is held back
    until the length checks have passed, so every input raises the error the
    reference's order gives it.
    """

    def __init__(self, lengths):
        self._lengths = lengths
        self._held: Exception | None = None
        self._settled = False

    def later(self, step, *args):
        """Run a step the reference takes after the length checks; hold its error."""
        if self._held is not None:
            return None
        try:
            return step(*args)
        except Exception as exc:  # re-raised by settle(), after the length checks
            self._held = exc
            return None

    @property
    def failed(self) -> bool:
        return self._held is not None

    def settle(self) -> None:
        """Read the arrays, check the lengths, then raise any held error."""
        if self._settled:
            return
        self._settled = True
        self._lengths()
        if self._held is not None:
            raise self._held


class _HostValues:
    """Host copies of small device int32 arrays, reused while the tensor is unchanged.

    Reading ``cu_seqlens`` to the host waits for every earlier launch on the
    stream, so a model that passes the same arrays to each of its attention
    layers would idle the GPU between layers.  A copy is reused only for the
    same tensor object (held weakly) at the same storage address with the same
    version counter; every in-place torch operation on the tensor or a view of
    it increments that counter, so such a change is always read afresh.  Writes
    that bypass torch (a raw pointer handed to other native code) are not
    seen; such callers pass a new tensor.
    """

    def __init__(self, capacity: int = 16):
        self._capacity = capacity
        self._entries: dict[int, tuple] = {}
        self._lock = threading.Lock()

    def _key(self, t: torch.Tensor):
        return (t._version, t.data_ptr(), tuple(t.shape), t.dtype)

    def lookup(self, t: torch.Tensor):
        if t.is_inference():  # inference tensors keep no version counter
            return None
        with self._lock:
            entry = self._entries.get(id(t))
        if entry is not None and entry[0]() is t and entry[1] == self._key(t):
            return entry[2]
        return None

    def store(self, t: torch.Tensor, values: list[int]) -> None:
        if t.is_inference():
            return
        with self._lock:
            if len(self._entries) >= self._capacity:
                self._entries.pop(next(iter(self._entries)))
            self._entries[id(t)] = (weakref.ref(t), self._key(t), values)


_CU_HOST = _HostValues()


def _host_values(cu_q: torch.Tensor, cu_k: torch.Tensor):
    """``cu_q`` and ``cu_k`` as Python lists, with at most one device-to-host copy."""
    q_vals = _CU_HOST.lookup(cu_q)
    k_vals = q_vals if cu_k is cu_q else _CU_HOST.lookup(cu_k)
    if q_vals is not None and k_vals is not None:
        return q_vals, k_vals
    if cu_q.data_ptr() == cu_k.data_ptr() and cu_q.shape == cu_k.shape:
        q_vals = cu_q.detach().cpu().tolist()
        k_vals = q_vals
    else:
        both = torch.cat((cu_q.detach(), cu_k.detach())).cpu().tolist()
        q_vals, k_vals = both[: cu_q.numel()], both[cu_q.numel():]
    _CU_HOST.store(cu_q, q_vals)
    if cu_k is not cu_q:
        _CU_HOST.store(cu_k, k_vals)
    return q_vals, k_vals


def _cumulative_lengths(cu_q, cu_k, q, k, *, label: str):
    q_vals, k_vals = _host_values(cu_q, cu_k)
    if q_vals[0] != 0 or k_vals[0] != 0:
        raise ValueError(f"{label} cumulative arrays must start at zero")
    if q_vals[-1] != q.shape[0] or k_vals[-1] != k.shape[0]:
        raise ValueError(f"{label} cumulative arrays must end at the packed Q/K totals")
    q_lengths = [e - s for s, e in zip(q_vals[:-1], q_vals[1:])]
    k_lengths = [e - s for s, e in zip(k_vals[:-1], k_vals[1:])]
    if min(q_lengths) < 0 or min(k_lengths) < 0:
        raise ValueError(f"{label} cumulative arrays must be nondecreasing")
    return q_lengths, k_lengths


def _is_python_int(x) -> bool:
    return type(x) is int or (isinstance(x, int) and not isinstance(x, bool))


def _validate_packed_common(q, k, v, cu_q, cu_k, max_q, max_k, *, label: str):
    # Written as plain comparisons (no generator expressions): these checks run
    # on every call, ahead of the launch.
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError(f"{label} q, k, and v must be rank-3 T/H/D tensors")
    device = q.device
    if not (device == k.device == v.device):
        raise ValueError(f"{label} q, k, and v must be on one device")
    bf16 = torch.bfloat16
    if q.dtype != bf16 or k.dtype != bf16 or v.dtype != bf16:
        raise ValueError(f"{label} q, k, and v must use BF16")
    if q.shape[0] <= 0 or k.shape[0] <= 0:
        raise ValueError(f"{label} Q and K totals must be positive")
    _validate_layout(q, name="packed q")
    _validate_layout(k, name="packed k")
    _validate_layout(v, name="packed v")
    _check_real_operands((q, k, v), ("q", "k", "v"), label=f"{label} q, k, and v")
    if k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr():
        raise ValueError("K and V must be distinct, non-aliasing prepared operands")
    if not (_is_python_int(max_q) and _is_python_int(max_k)):
        raise TypeError("max_seqlen_q and max_seqlen_k must be Python integers")
    if cu_q.ndim != 1 or cu_q.numel() < 2 or cu_k.ndim != 1 or cu_k.numel() < 2:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must be rank-1 B+1 tensors")
    if cu_q.shape != cu_k.shape:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same batch count")
    if cu_q.device != device or cu_k.device != device:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must share the q/k/v device")
    if cu_q.dtype != torch.int32 or cu_k.dtype != torch.int32:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must use INT32")
    if not (cu_q.is_contiguous() and cu_k.is_contiguous()):
        raise ValueError("cu_seqlens_q and cu_seqlens_k must be contiguous")


def _validate_local_varlen(q, k, v, cu_q, cu_k, max_q, max_k, spec, *, require_device=True):
    _validate_packed_common(q, k, v, cu_q, cu_k, max_q, max_k, label="packed")
    if q.shape[1:] != (spec.num_q_heads, spec.head_dim_qk):
        raise ValueError("packed q shape does not match the attention spec")
    if k.shape[1:] != (spec.num_kv_heads, spec.head_dim_qk):
        raise ValueError("packed k shape does not match the attention spec")
    if v.shape != (k.shape[0], spec.num_kv_heads, spec.head_dim_v):
        raise ValueError("packed v shape does not match the attention spec")
    if not _locked_local(spec, check_kv_heads=True):
        raise UnsupportedMI355XPath("only the locked local d256 GQA-2 varlen contract is enabled")
    if max_q <= 0 or max_k <= 0 or max_k > _LOCAL_MODEL_MAX_SEQLEN:
        raise UnsupportedMI355XPath("varlen local attention requires 1 <= max Sq <= max Sk <= 262144")
    if max_q > max_k:
        raise UnsupportedMI355XPath("varlen local attention requires max Sq <= max Sk")

    def lengths():
        q_lengths, k_lengths = _cumulative_lengths(cu_q, cu_k, q, k, label="packed")
        if any(lq > lk for lq, lk in zip(q_lengths, k_lengths)):
            raise UnsupportedMI355XPath("each packed sequence requires Sq <= Sk")
        if max(q_lengths) != max_q or max(k_lengths) != max_k:
            raise ValueError("max_seqlen_q/max_seqlen_k must equal the cumulative maxima")

    check = _CumulativeCheck(lengths)
    if require_device:
        check.later(_require_gfx950, q.device)
    return check


def _prepare_packed_k_metadata(values, k: torch.Tensor, *, name: str):
    if values is None:
        return None
    if values.shape != (k.shape[0],):
        raise ValueError(f"{name} must have shape ({k.shape[0]},)")
    if values.device != k.device:
        raise ValueError(f"{name} must share the q/k/v device")
    return _normalize_int32_metadata(values, name=name)


def _validate_global_bshd(q, k, v, spec, *, require_device: bool = True) -> None:
    _validate_bshd(q, k, v, spec, require_device=require_device)
    if q.shape[0] != 1 or q.shape[1] > _GLOBAL_FIXED_BACKWARD_MAX_SEQLEN:
        raise UnsupportedMI355XPath("fixed global backward requires B=1 and 1 <= S <= 2048")
    if not _locked_global(spec):
        raise UnsupportedMI355XPath("only the locked global d512 text-forward contract is enabled")


def _validate_global_forward_only_bshd(q, k, v, spec) -> None:
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("global forward-only q, k, and v must be rank-4 B/S/H/D tensors")
    if not (q.device == k.device == v.device):
        raise ValueError("global forward-only q, k, and v must be on one device")
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise ValueError("global forward-only q, k, and v must use BF16")
    for name, tensor in zip(("q", "k", "v"), (q, k, v)):
        _validate_layout(tensor, name=name)
    _check_real_operands((q, k, v), ("q", "k", "v"), label="global forward-only q, k, and v")
    if k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr():
        raise ValueError("global forward-only K and V must be distinct operands")
    batch, q_len, q_heads, q_dim = q.shape
    kv_len = k.shape[1]
    if batch <= 0 or not (1 <= q_len <= kv_len <= _LOCAL_MODEL_MAX_SEQLEN):
        raise UnsupportedMI355XPath("global forward-only requires B>=1 and 1 <= Sq <= Sk <= 262144")
    if (q_heads, q_dim) != (spec.num_q_heads, spec.head_dim_qk):
        raise ValueError("global forward-only q shape conflicts with the locked geometry")
    if k.shape != (batch, kv_len, spec.num_kv_heads, spec.head_dim_qk):
        raise ValueError("global forward-only k shape conflicts with the locked geometry")
    if v.shape != (batch, kv_len, spec.num_kv_heads, spec.head_dim_v):
        raise ValueError("global forward-only v shape conflicts with the locked geometry")
    if not _locked_global(spec):
        raise UnsupportedMI355XPath("only the locked global d512 contract is enabled")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise UnsupportedMI355XPath(
            "global forward-only cannot participate in autograd; use "
            "fa4_global_text_forward for S<=2048 or packed fa4_global_varlen_forward"
        )
    _require_gfx950(q.device)


def _validate_global_varlen(q, k, v, cu_q, cu_k, max_q, max_k, spec, *, allow_backward=False):
    _validate_packed_common(q, k, v, cu_q, cu_k, max_q, max_k, label="global packed")
    if q.shape[1:] != (spec.num_q_heads, spec.head_dim_qk):
        raise ValueError("global packed q shape conflicts with the lock")
    if k.shape[1:] != (spec.num_kv_heads, spec.head_dim_qk):
        raise ValueError("global packed k shape conflicts with the lock")
    if v.shape != (k.shape[0], spec.num_kv_heads, spec.head_dim_v):
        raise ValueError("global packed v shape conflicts with the lock")
    if not _locked_global(spec):
        raise UnsupportedMI355XPath("only the locked global d512 contract is enabled")
    max_supported = _GLOBAL_NATIVE_BACKWARD_MAX_SEQLEN if allow_backward else _LOCAL_MODEL_MAX_SEQLEN
    if not (1 <= max_q <= max_k <= max_supported):
        op = "backward-capable" if allow_backward else "forward-only"
        raise UnsupportedMI355XPath(
            f"global packed {op} maxima must satisfy 1 <= Sq <= Sk <= {max_supported}"
        )
    if not allow_backward and torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise UnsupportedMI355XPath(
            "global packed forward-only cannot participate in autograd; use "
            "fa4_global_varlen_forward"
        )

    def lengths():
        q_lengths, k_lengths = _cumulative_lengths(cu_q, cu_k, q, k, label="global packed")
        if any(lq > lk for lq, lk in zip(q_lengths, k_lengths)):
            raise UnsupportedMI355XPath("global packed segments require 0 <= Sq <= Sk per segment")
        if max(q_lengths) != max_q or max(k_lengths) != max_k:
            raise ValueError("global packed maxima must equal the cumulative segment maxima")

    check = _CumulativeCheck(lengths)
    check.later(_require_int32_totals, q, k)
    check.later(_require_gfx950, q.device)
    return check


def _require_int32_totals(q, k) -> None:
    if q.shape[0] > torch.iinfo(torch.int32).max or k.shape[0] > torch.iinfo(torch.int32).max:
        raise UnsupportedMI355XPath("packed global totals must fit signed INT32")


# ---------------------------------------------------------------------------
# launch plan
# ---------------------------------------------------------------------------


def _layout(t: torch.Tensor, packed: bool) -> G4Layout:
    if packed:
        return G4Layout(0, t.stride(0), t.stride(1))
    return G4Layout(t.stride(0), t.stride(1), t.stride(2))


def _meets_operand_contract(t: torch.Tensor) -> bool:
    """Whether the library accepts ``t`` as a bf16 operand as it stands.

    Unit head-dim stride, positive outer strides that are multiples of 8
    elements (token stride below 2^24), and a 16-byte aligned base.
    """
    strides = t.stride()
    return (
        strides[-1] == 1
        and all(s > 0 and s % 8 == 0 for s in strides[:-1])
        and strides[-3] < (1 << 24)
        and t.data_ptr() % 16 == 0
    )


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@dataclass
class _Plan:
    """Geometry of one attention call, shared by its forward and backward."""

    packed: bool
    num_seqs: int
    seqlen_q: int  # fixed length, or maximum when packed
    seqlen_k: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    window: int
    bidirectional: bool
    total_q: int
    total_k: int
    cu_q: torch.Tensor | None = None
    cu_k: torch.Tensor | None = None
    vision: torch.Tensor | None = None
    documents: torch.Tensor | None = None
    # Bytes of the backward workspace for stored dS tiles (0: library default,
    # negative: none, so the dQ stage recomputes S and dP).  Fitted again to the
    # free HBM at backward time (_refit_backward).
    ds_budget: int = 0
    # Global layers fail closed at backward time when even the recompute route
    # does not fit the guarded budget (GlobalBackwardBudgetExceeded).
    global_backward: bool = False
    # Cumulative-array checks still to run before the first launch.
    pending: _CumulativeCheck | None = field(default=None, repr=False, compare=False)
    # Workspace sizes already asked of the library, by (phase, ds_budget): the
    # geometry above is fixed once the plan is made, the dS budget is not.
    _ws_sizes: dict = field(default_factory=dict, repr=False, compare=False)

    def _settle(self) -> None:
        pending, self.pending = self.pending, None
        if pending is not None:
            pending.settle()

    def problem(self) -> G4Problem:
        p = G4Problem()
        p.num_seqs = self.num_seqs
        p.seqlen_q = self.seqlen_q
        p.seqlen_k = self.seqlen_k
        p.num_q_heads = self.num_q_heads
        p.num_kv_heads = self.num_kv_heads
        p.head_dim = self.head_dim
        p.window = self.window
        p.bidirectional_vision = 1 if self.bidirectional else 0
        p.total_q = self.total_q
        p.total_k = self.total_k
        p.cu_seqlens_q = _ptr(self.cu_q)
        p.cu_seqlens_k = _ptr(self.cu_k)
        p.vision_ids = _ptr(self.vision)
        p.document_ids = _ptr(self.documents)
        if self.packed:
            p.lse_batch_stride = 0
            p.lse_head_stride = self.total_q
        else:
            p.lse_batch_stride = self.num_q_heads * self.seqlen_q
            p.lse_head_stride = self.seqlen_q
        p.ds_budget = self.ds_budget
        return p

    def lse_shape(self) -> tuple[int, ...]:
        if self.packed:
            return (self.num_q_heads, self.total_q)
        return (self.num_seqs, self.num_q_heads, self.seqlen_q)

    def workspace_bytes(self, phase: int, prob: G4Problem | None = None) -> int:
        key = (phase, self.ds_budget)
        nbytes = self._ws_sizes.get(key)
        if nbytes is not None:
            return nbytes
        lib = _lib.load()
        if prob is None:
            prob = self.problem()
        nbytes = int(lib.g4_workspace_bytes(ctypes.byref(prob), phase))
        if nbytes == 0 and lib.g4_last_error():
            _lib.check(_lib.G4_ERR_INVALID)
        self._ws_sizes[key] = nbytes
        return nbytes

    def _workspace(self, phase: int, device, prob: G4Problem | None = None) -> torch.Tensor:
        nbytes = max(self.workspace_bytes(phase, prob), 256)
        return torch.empty(nbytes, dtype=torch.uint8, device=device)

    def forward(self, q, k, v):
        try:
            lib = _lib.load()
            prob = self.problem()
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
            lse = torch.empty(self.lse_shape(), dtype=torch.float32, device=q.device)
            # Most forwards need no workspace (no vision IDs at head dim 256): the
            # library takes NULL for a zero-byte workspace, so none is allocated.
            ws_bytes = self.workspace_bytes(0, prob)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
        except Exception:
            self._settle()  # an invalid cu_seqlens is reported first
            raise
        with _lib.device_scope(q.device):
            stream = _lib.raw_stream(q.device)
            args = (
                ctypes.byref(prob),
                q.data_ptr(), _layout(q, self.packed),
                k.data_ptr(), _layout(k, self.packed),
                v.data_ptr(), _layout(v, self.packed),
                out.data_ptr(), _layout(out, self.packed),
                lse.data_ptr(), None if ws is None else ws.data_ptr(), ws_bytes, stream,
            )
            self._settle()
            rc = lib.g4_attn_fwd(*args)
        _lib.check(rc)
        return out, lse

    def backward(self, q, k, v, out, dout, lse, dlse):
        lib = _lib.load()
        _refit_backward(self, q, k, v)  # before anything is allocated
        if not _meets_operand_contract(dout):
            # e.g. a broadcast gradient of a sum, or a view off 16-byte alignment
            dout = dout.contiguous()
        if dlse is not None:
            dlse = dlse.to(torch.float32).contiguous()
        dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
        dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        prob = self.problem()
        ws = self._workspace(1, q.device, prob)
        with _lib.device_scope(q.device):
            stream = _lib.raw_stream(q.device)
            rc = lib.g4_attn_bwd(
                ctypes.byref(prob),
                q.data_ptr(), _layout(q, self.packed),
                k.data_ptr(), _layout(k, self.packed),
                v.data_ptr(), _layout(v, self.packed),
                out.data_ptr(), _layout(out, self.packed),
                dout.data_ptr(), _layout(dout, self.packed),
                lse.data_ptr(), _ptr(dlse),
                dq.data_ptr(), _layout(dq, self.packed),
                dk.data_ptr(), _layout(dk, self.packed),
                dv.data_ptr(), _layout(dv, self.packed),
                ws.data_ptr(), ws.numel(), stream,
            )
        _lib.check(rc)
        return dq, dk, dv


class _AttentionFunction(torch.autograd.Function):
    """Forward saves (q, k, v, O, LSE); backward accepts dO and dLSE (either may be None)."""

    @staticmethod
    def forward(ctx, q, k, v, plan: _Plan):
        out, lse = plan.forward(q, k, v)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan = plan
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, k, v, out, lse = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv = ctx.plan.backward(q, k, v, out, dout, lse, dlse)
        return dq, dk, dv, None


def _fixed_plan(q, k, spec: AttentionLayerSpec, *, vision=None) -> _Plan:
    b, sq, hq, d = q.shape
    return _Plan(
        packed=False,
        num_seqs=b,
        seqlen_q=sq,
        seqlen_k=k.shape[1],
        num_q_heads=hq,
        num_kv_heads=k.shape[2],
        head_dim=d,
        window=spec.sliding_window or 0,
        bidirectional=bool(spec.vision_bidirectional_within_block and vision is not None),
        total_q=b * sq,
        total_k=b * k.shape[1],
        vision=vision,
    )


def _packed_plan(q, k, cu_q, cu_k, max_q, max_k, spec, *, vision=None, documents=None) -> _Plan:
    return _Plan(
        packed=True,
        num_seqs=cu_q.numel() - 1,
        seqlen_q=max_q,
        seqlen_k=max_k,
        num_q_heads=q.shape[1],
        num_kv_heads=k.shape[1],
        head_dim=q.shape[2],
        window=spec.sliding_window or 0,
        bidirectional=bool(spec.vision_bidirectional_within_block and vision is not None),
        total_q=q.shape[0],
        total_k=k.shape[0],
        cu_q=cu_q,
        cu_k=cu_k,
        vision=vision,
        documents=documents,
    )


# ---------------------------------------------------------------------------
# HBM preflights (fail closed before any launch; policy of h100.py:425-442, 713-746)
# ---------------------------------------------------------------------------


# Free-HBM readings taken by _free_hbm, per torch device: (time, bytes, reader).
_FREE_HBM_READINGS: dict[torch.device, tuple[float, int, object]] = {}
# How long the checks made before a forward's first launch reuse a reading.
_FREE_HBM_REUSE_S = 0.02


def _free_hbm(device) -> int:
    """Free HBM bytes on ``device`` now (hipMemGetInfo)."""
    free, _total = torch.cuda.mem_get_info(device)
    _FREE_HBM_READINGS[device] = (time.monotonic(), free, _free_hbm)
    return free


def _recent_free_hbm(device) -> int:
    """Free HBM bytes read by ``_free_hbm`` within the last 20 ms, else read now.

    hipMemGetInfo takes tens of microseconds once the device has gone idle,
    and the forward-time checks run before the first launch, so a model whose
    layers call the adapters back to back would pay it per layer with the GPU
    waiting.  Those checks (metadata workspace, forward outputs, the
    backward's preliminary dS fit and the global backward budget) take such
    a recent reading instead.  A reading is reused only if the current
    ``_free_hbm`` took it.  The backward's own fit (``_refit_backward``) always
    reads afresh, so a forward admitted on a reading that has since gone stale
    still fails closed, with the same typed error, before the backward
    allocates.
    """
    entry = _FREE_HBM_READINGS.get(device)
    if entry is not None and entry[2] is _free_hbm and time.monotonic() - entry[0] < _FREE_HBM_REUSE_S:
        return entry[1]
    return _free_hbm(device)


def _preflight_metadata_workspace(plan: _Plan, device, free: int | None = None) -> int:
    """The forward's workspace (vision-span tables, raise flags) against free HBM.

    The backward's delta and dS tiles are budgeted by _preflight_backward.  Returns
    the free-HBM reading it used (``free`` when given), so a backward fit made in
    the same call reuses it instead of querying the device again.
    """
    required = plan.workspace_bytes(0)
    if required > _METADATA_WORKSPACE_MAX_BYTES:
        raise UnsupportedMI355XPath(
            f"vision-span workspace requires {required} bytes, above the 2 GiB safety limit"
        )
    if free is None:
        free = _recent_free_hbm(device)
    if required > free // 10:
        raise UnsupportedMI355XPath(
            f"vision-span workspace requires {required} bytes, exceeding the 10% free-HBM "
            f"budget of {free // 10} bytes ({free} bytes free)"
        )
    return free


def _global_backward_budget(free_bytes: int) -> int:
    return min(free_bytes * 4 // 5, max(0, free_bytes - _GLOBAL_BACKWARD_RESERVE_BYTES))


def _check_global_backward_budget(required: int, free: int) -> None:
    budget = _global_backward_budget(free)
    if required > budget:
        raise GlobalBackwardBudgetExceeded(
            f"global backward needs about {required} additional bytes, above the guarded "
            f"budget of {budget} bytes ({free} bytes currently free)"
        )


def _backward_additional_bytes(plan: _Plan, q, k, v) -> int:
    grads = sum(t.numel() * t.element_size() for t in (q, k, v))
    return grads + plan.workspace_bytes(1)


def _fit_ds_budget(plan: _Plan, q, k, v, budget: int) -> int:
    """Fit the backward's stored dS tiles to ``budget`` bytes of additional HBM.

    The MI355X counterpart of the reference's budget fallback
    (transformers_integration.py:1950-1961, which re-runs a low-memory
    composition when the native global backward exceeds its budget): the
    dK/dV stage stores dS tiles only while they fit what the budget leaves after
    the gradients and the O(T) part of the workspace.  Past that, a single
    global sequence is cut into stripes of query rows that fit it (with fp32
    dK / dV sums beside them); other problems, and budgets below the sums plus
    four rows of tiles, have the dQ stage recompute S and dP.  Returns the
    additional bytes the backward will need.
    """
    plan.ds_budget = 0
    full = _backward_additional_bytes(plan, q, k, v)
    if full <= budget:
        return full
    plan.ds_budget = -1
    lean = _backward_additional_bytes(plan, q, k, v)
    room = budget - lean
    if room > 0:
        plan.ds_budget = room  # stores the tiles only if they fit in what is left
        return _backward_additional_bytes(plan, q, k, v)
    return lean


# Stored-dS budget pinned by the caller (None: fitted to the free HBM).
_PINNED_DS_BUDGET: int | None = None


def pin_backward_ds_budget(nbytes: int | None) -> int | None:
    """Pin the backward's stored-dS budget for every later call; returns the previous pin.

    ``None`` (the default) fits the budget to the free HBM at each forward and
    again at each backward: the dK/dV stage stores dS tiles while they fit, a
    single global sequence past that is striped, else the dQ stage recomputes S
    and dP.  The recompute route sums dQ in another order, and the striped
    route adds dK / dV over its stripes in fp32, so with the default the bits of
    the gradients can depend on how much HBM is free.  A pinned budget fixes the
    route: a negative value always recomputes, a positive one stores the tiles
    (or stripes) that fit in that many bytes, 0 is the library's default cap
    (16 GiB).  The global layers still raise
    ``GlobalBackwardBudgetExceeded`` when the pinned route does not fit the
    guarded budget.  A process-wide setting (not per thread).
    """
    global _PINNED_DS_BUDGET
    if nbytes is not None and not isinstance(nbytes, int):
        raise TypeError("nbytes must be an int or None")
    previous, _PINNED_DS_BUDGET = _PINNED_DS_BUDGET, nbytes
    return previous


def _fit_or_pin(plan: _Plan, q, k, v, free: int) -> int:
    if _PINNED_DS_BUDGET is not None:
        plan.ds_budget = _PINNED_DS_BUDGET
        return _backward_additional_bytes(plan, q, k, v)
    return _fit_ds_budget(plan, q, k, v, _global_backward_budget(free))


def _preflight_backward(plan: _Plan, q, k, v) -> None:
    plan.global_backward = True
    free = _recent_free_hbm(q.device)
    required = _fit_or_pin(plan, q, k, v, free)
    _check_global_backward_budget(required, free)


def _fit_local_backward(plan: _Plan, q, k, v, free: int | None = None) -> None:
    # The local backward has no budget error in the reference (FA4's autograd
    # allocates what it needs); its stored-dS band just shrinks to what fits.
    _fit_or_pin(plan, q, k, v, _recent_free_hbm(q.device) if free is None else free)


def _refit_backward(plan: _Plan, q, k, v) -> None:
    """Fit the dS budget again to the HBM free when the backward starts.

    The reference measures free HBM inside the global backward, before it
    allocates its scratch, and fails closed there
    (patches/flash-attention/0002-sm90-gemma4-d512-forward-backward.patch:1164-1181).
    Between a layer's forward and its backward a training step allocates the
    other layers' activations, so the forward's fit can be stale: the route
    (stored dS or recompute) is chosen again here, and a global layer whose
    lean route no longer fits raises GlobalBackwardBudgetExceeded instead of
    running out of memory in the allocation.
    """
    free = _free_hbm(q.device)
    required = _fit_or_pin(plan, q, k, v, free)
    if plan.global_backward:
        _check_global_backward_budget(required, free)


def _preflight_forward_outputs(q: torch.Tensor) -> None:
    out_bytes = q.numel() * q.element_size()
    lse_bytes = q.numel() // q.shape[-1] * 4
    required = 2 * (out_bytes + lse_bytes)
    free = _recent_free_hbm(q.device)
    if required > free * 8 // 10:
        raise UnsupportedMI355XPath(
            f"forward outputs require about {required} bytes, above 80% of the {free} "
            "currently free HBM bytes"
        )


def _requires_backward(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _run(q, k, v, plan: _Plan):
    if _requires_backward(q, k, v):
        return _AttentionFunction.apply(q, k, v, plan)
    return plan.forward(q, k, v)


def _run_checked(q, k, v, check: _CumulativeCheck, prepare, *, autograd: bool = True):
    """Build the plan while the GPU is busy; the cumulative arrays are read at launch."""
    plan = check.later(prepare)
    if check.failed:
        check.settle()  # raises: the length checks' error, else the held one
    plan.pending = check
    return _run(q, k, v, plan) if autograd else plan.forward(q, k, v)


# ---------------------------------------------------------------------------
# public adapters (reference names; h100.py:750-1394)
# ---------------------------------------------------------------------------


def fa4_local_text_forward(q, k, v, *, spec: AttentionLayerSpec = SLIDING_ATTENTION):
    """Fixed-length local text attention (B=1, 1 <= S <= 1025), autograd-capable.

    Mask ``k <= q`` and ``k > q - 1024``; LSE fp32 ``(B, Hq, S)``.
    """
    _validate_local_bshd(q, k, v, spec)
    return _run(q, k, v, _fixed_plan(q, k, spec))


def fa4_local_forward(
    q, k, v, *, vision_block_ids=None, spec: AttentionLayerSpec = SLIDING_ATTENTION
):
    """Fixed-length local attention with the exact vision overlay (B=1, S <= 1025).

    ``vision_block_ids=None`` is the text path.  With ``(1, S)`` IDs the mask is
    ``(k > q - 1024) AND (k <= q OR same non-negative vision block)``.
    """
    if vision_block_ids is None:
        return fa4_local_text_forward(q, k, v, spec=spec)
    _validate_local_bshd(q, k, v, spec)
    ids = _prepare_vision_block_ids(vision_block_ids, q)
    plan = _fixed_plan(q, k, spec, vision=ids)
    free = _preflight_metadata_workspace(plan, q.device)  # one reading for both checks
    if _requires_backward(q, k, v):
        _fit_local_backward(plan, q, k, v, free)
    return _run(q, k, v, plan)


def fa4_local_varlen_forward(
    q,
    k,
    v,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    max_seqlen_q: int,
    max_seqlen_k: int,
    vision_block_ids=None,
    document_ids=None,
    spec: AttentionLayerSpec = SLIDING_ATTENTION,
):
    """Packed local attention; each Q segment is the lower-right suffix of its K segment.

    Vision/document IDs follow the packed K stream.  One launch covers every
    segment; the device scheduler bounds each tile's key range from the window
    and the vision spans (no host schedule, no per-segment launches).
    """
    check = _validate_local_varlen(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec
    )

    def prepare():
        vision = _prepare_packed_k_metadata(vision_block_ids, k, name="vision_block_ids")
        documents = _prepare_packed_k_metadata(document_ids, k, name="document_ids")
        plan = _packed_plan(
            q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec,
            vision=vision, documents=documents,
        )
        free = None  # one free-HBM reading for both checks of this call
        if vision is not None:
            free = _preflight_metadata_workspace(plan, q.device)
        if _requires_backward(q, k, v):
            _fit_local_backward(plan, q, k, v, free)
        return plan

    return _run_checked(q, k, v, check, prepare)


def fa4_global_forward_only(q, k, v, *, spec: AttentionLayerSpec = GLOBAL_ATTENTION):
    """Fixed/rectangular global d512 forward without autograd (lower-right causal)."""
    _validate_global_forward_only_bshd(q, k, v, spec)
    _preflight_forward_outputs(q)
    return _fixed_plan(q, k, spec).forward(q, k, v)


def fa4_global_varlen_forward_only(
    q,
    k,
    v,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    max_seqlen_q: int,
    max_seqlen_k: int,
    spec: AttentionLayerSpec = GLOBAL_ATTENTION,
):
    """Packed lower-right global d512 forward without autograd."""
    check = _validate_global_varlen(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec
    )

    def prepare():
        _preflight_forward_outputs(q)
        return _packed_plan(q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec)

    return _run_checked(q, k, v, check, prepare, autograd=False)


def fa4_global_varlen_forward(
    q,
    k,
    v,
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    max_seqlen_q: int,
    max_seqlen_k: int,
    spec: AttentionLayerSpec = GLOBAL_ATTENTION,
):
    """Packed global d512 forward with the atomic-free MI355X backward."""
    check = _validate_global_varlen(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec,
        allow_backward=True,
    )

    def prepare():
        plan = _packed_plan(q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, spec)
        if _requires_backward(q, k, v):
            _preflight_backward(plan, q, k, v)
        else:
            _preflight_forward_outputs(q)
        return plan

    return _run_checked(q, k, v, check, prepare)


def fa4_global_text_forward(q, k, v, *, spec: AttentionLayerSpec = GLOBAL_ATTENTION):
    """Fixed-length global d512 causal attention (B=1, 1 <= S <= 2048), autograd-capable."""
    _validate_global_bshd(q, k, v, spec)
    plan = _fixed_plan(q, k, spec)
    if _requires_backward(q, k, v):
        _preflight_backward(plan, q, k, v)
    else:
        _preflight_forward_outputs(q)
    return _run(q, k, v, plan)
