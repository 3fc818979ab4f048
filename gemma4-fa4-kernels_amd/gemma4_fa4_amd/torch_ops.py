"""Opaque PyTorch operators for the compiler and StaticCache decode boundaries.

Mirrors the reference's ``src/gemma4_fa4/h100_torch_ops.py`` on gfx950: six
``torch.library`` custom operators with fake (meta) implementations, so that
``torch.compile`` traces a Gemma 4 attention call as one opaque node whose
output metadata is known without running a kernel (h100_torch_ops.py:986-1017).

* ``local_fwd`` / ``global_fwd`` take Transformers-prepared BHSD q, k, v of
  one text sequence (B = 1, 1 <= S <= 1024, ``position_ids == arange(S)``,
  ``packed_sequence_ids`` derived from them) and return BSHD O and fp32 LSE
  ``(1, 32, S)`` (h100_torch_ops.py:39-195).
* ``local_layer_fwd`` / ``global_layer_fwd`` run a whole attention layer
  around those routes with every weight an explicit tensor argument:
  q / k (/ v) projections, RMSNorm and RoPE, the attention, the output
  projection (h100_torch_ops.py:198-475).
* ``global_static_cache_decode_fwd`` / ``local_static_cache_decode_fwd``
  decode one token against a Transformers StaticCache backing, mutating the
  K / V backings (and, for the global layer, the length counter) in place
  (h100_torch_ops.py:479-846).

What runs on the GPU: the projections are plain library GEMMs
(``torch.nn.functional.linear``, hipBLASLt); every RMSNorm and RoPE is the
fused gfx950 row-preparation kernel (``g4_kv_prep_fwd``), which writes the
prepared K / V rows straight into the cache slot during decode; the attention
is this library's own kernels through the adapters (``fa4_*``).  Fake
implementations allocate only fresh outputs and run neither validation nor a
kernel.

Operator names live in the ``gemma4_mi355x`` namespace; the reference's
Python names (``h100_local_fwd``, ``h100_global_layer_op``, ...) are kept as
aliases of the same objects for drop-in callers.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch
from torch import Tensor

from .attention import (
    _require_gfx950,
    fa4_global_forward_only,
    fa4_global_text_forward,
    fa4_local_text_forward,
    fa4_local_varlen_forward,
)
from .errors import UnsupportedMI355XPath
from .kv_prep import prepare_rows_into
from .model_spec import GEMMA4_31B, GLOBAL_ATTENTION, SLIDING_ATTENTION, AttentionLayerSpec

NAMESPACE = "gemma4_mi355x"
LOCAL_OP_NAME = f"{NAMESPACE}::local_fwd"
GLOBAL_OP_NAME = f"{NAMESPACE}::global_fwd"
LOCAL_LAYER_OP_NAME = f"{NAMESPACE}::local_layer_fwd"
GLOBAL_LAYER_OP_NAME = f"{NAMESPACE}::global_layer_fwd"
GLOBAL_STATIC_CACHE_DECODE_OP_NAME = f"{NAMESPACE}::global_static_cache_decode_fwd"
LOCAL_STATIC_CACHE_DECODE_OP_NAME = f"{NAMESPACE}::local_static_cache_decode_fwd"

_HIDDEN = GEMMA4_31B.hidden_size
_MAX_SEQLEN = 1024          # compiled prefill envelope and the sliding cache capacity
_DECODE_MAX_POSITION = _MAX_SEQLEN * 256
_RMS_EPS = 1e-6


@dataclass(frozen=True)
class _Family:
    spec: AttentionLayerSpec
    label: str

    @property
    def q_heads(self) -> int:
        return self.spec.num_q_heads

    @property
    def kv_heads(self) -> int:
        return self.spec.num_kv_heads

    @property
    def head_dim(self) -> int:
        return self.spec.head_dim_qk

    def weight_shapes(self, *, separate_v: bool) -> tuple[tuple[int, ...], ...]:
        q_rows, kv_rows = self.q_heads * self.head_dim, self.kv_heads * self.head_dim
        shapes = [(q_rows, _HIDDEN), (kv_rows, _HIDDEN)]
        if separate_v:
            shapes.append((kv_rows, _HIDDEN))
        shapes += [(_HIDDEN, q_rows), (self.head_dim,), (self.head_dim,)]
        return tuple(shapes)


_LOCAL = _Family(SLIDING_ATTENTION, "local")
_GLOBAL = _Family(GLOBAL_ATTENTION, "global")


# ---------------------------------------------------------------------------
# shared checks
# ---------------------------------------------------------------------------


def _distinct_storage(tensors, *, what: str) -> None:
    pointers = {t.untyped_storage().data_ptr() for t in tensors}
    if len(pointers) != len(tensors):
        raise ValueError(f"compiled MI355X {what} arguments must use distinct storage")


def _same_gpu(tensors, *, what: str) -> torch.device:
    device = tensors[0].device
    if device.type != "cuda" or any(t.device != device for t in tensors):
        raise UnsupportedMI355XPath(f"compiled MI355X {what} tensors must be CUDA tensors "
                                    "on one device")
    _require_gfx950(device)
    return device


def _index_tensor(t: torch.Tensor, shape: tuple[int, ...], *, name: str, what: str) -> None:
    if t.shape != shape or t.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"compiled MI355X {what} {name} must be INT32/INT64 of shape {shape}")


def _text_positions(position_ids, packed_sequence_ids, seqlen: int, *, what: str) -> None:
    """position_ids == arange(S); packed IDs = the runs they imply (h100_torch_ops.py:79-107)."""
    _index_tensor(position_ids, (1, seqlen), name="position_ids", what=what)
    _index_tensor(packed_sequence_ids, (1, seqlen), name="packed_sequence_ids", what=what)
    expected = torch.arange(seqlen, device=position_ids.device, dtype=position_ids.dtype)
    if not torch.equal(position_ids[0], expected):
        raise UnsupportedMI355XPath(f"compiled MI355X {what} position_ids must equal "
                                    "zero-based arange(S)")
    # a new packed sequence starts wherever the position does not advance by one
    breaks = torch.ones(seqlen, dtype=torch.int64, device=position_ids.device)
    breaks[0] = 0
    if seqlen > 1:
        breaks[1:] = (position_ids[0, 1:] - position_ids[0, :-1] != 1).to(torch.int64)
    if not torch.equal(packed_sequence_ids[0].to(torch.int64), breaks.cumsum(0)):
        raise UnsupportedMI355XPath(f"compiled MI355X {what} packed_sequence_ids must be "
                                    "derived exactly from position_ids")


def _check_fresh_outputs(out, lse, inputs, *, out_shape, lse_shape, what: str):
    if out.shape != out_shape or out.dtype != torch.bfloat16:
        raise RuntimeError(f"compiled MI355X {what} returned an invalid BF16 output contract")
    if lse.shape != lse_shape or lse.dtype != torch.float32:
        raise RuntimeError(f"compiled MI355X {what} returned an invalid FP32 LSE contract")
    if out.requires_grad or lse.requires_grad:
        raise RuntimeError(f"compiled MI355X {what} outputs must not require grad")
    held = {t.untyped_storage().data_ptr() for t in inputs}
    o_ptr, l_ptr = out.untyped_storage().data_ptr(), lse.untyped_storage().data_ptr()
    if o_ptr in held or l_ptr in held or o_ptr == l_ptr:
        raise RuntimeError(f"compiled MI355X {what} outputs must use fresh, non-aliasing storage")
    return out, lse


# ---------------------------------------------------------------------------
# prepared-tensor operators (h100_torch_ops.py:39-195)
# ---------------------------------------------------------------------------


def _validate_prepared(q, k, v, position_ids, packed_sequence_ids, family: _Family):
    what = "forward op"
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("compiled MI355X q, k, and v must be rank-4 BHSD tensors")
    if any(t.requires_grad for t in (q, k, v)):
        raise UnsupportedMI355XPath("compiled MI355X forward ops reject every requires_grad input")
    if q.device.type != "cuda" or not (q.device == k.device == v.device):
        raise UnsupportedMI355XPath("compiled MI355X q, k, and v must be CUDA tensors on one "
                                    "device")
    _require_gfx950(q.device)
    if any(t.dtype != torch.bfloat16 for t in (q, k, v)):
        raise ValueError("compiled MI355X q, k, and v must use BF16")
    batch, heads, seqlen, dim = q.shape
    if batch != 1 or not 1 <= seqlen <= _MAX_SEQLEN:
        raise UnsupportedMI355XPath("compiled MI355X forward ops require B=1 and 1 <= S <= 1024")
    if (heads, dim) != (family.q_heads, family.head_dim):
        raise ValueError("compiled MI355X q does not match the locked layer geometry")
    kv_shape = (1, family.kv_heads, seqlen, family.head_dim)
    if k.shape != kv_shape or v.shape != kv_shape:
        raise ValueError("compiled MI355X k/v must match q length and the locked layer geometry")
    for name, t in (("position_ids", position_ids), ("packed_sequence_ids", packed_sequence_ids)):
        if t.ndim != 2 or t.shape != (1, seqlen):
            raise ValueError(f"compiled MI355X {name} must have shape (1, S)")
        if t.device != q.device:
            raise ValueError(f"compiled MI355X {name} must share the q/k/v CUDA device")
    _text_positions(position_ids, packed_sequence_ids, seqlen, what=what)
    _distinct_storage((q, k, v), what="q, k, and v")
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)


def _prepared_outputs(out, lse, q, k, v):
    b, h, s, _ = q.shape
    return _check_fresh_outputs(out, lse, (q, k, v), out_shape=(b, s, h, v.shape[3]),
                                lse_shape=(b, h, s), what="attention")


def _local_impl(q: Tensor, k: Tensor, v: Tensor, position_ids: Tensor,
                packed_sequence_ids: Tensor) -> tuple[Tensor, Tensor]:
    qs, ks, vs = _validate_prepared(q, k, v, position_ids, packed_sequence_ids, _LOCAL)
    out, lse = fa4_local_text_forward(qs, ks, vs)
    return _prepared_outputs(out, lse, q, k, v)


def _global_impl(q: Tensor, k: Tensor, v: Tensor, position_ids: Tensor,
                 packed_sequence_ids: Tensor) -> tuple[Tensor, Tensor]:
    qs, ks, vs = _validate_prepared(q, k, v, position_ids, packed_sequence_ids, _GLOBAL)
    out, lse = fa4_global_text_forward(qs, ks, vs)
    return _prepared_outputs(out, lse, q, k, v)


def _fake_prepared(q: Tensor, _k: Tensor, v: Tensor, _position_ids: Tensor,
                   _packed_sequence_ids: Tensor) -> tuple[Tensor, Tensor]:
    """Fresh BSHD output and FP32 LSE metadata only."""
    b, h, s, _ = q.shape
    out = torch.empty((b, s, h, v.shape[3]), dtype=q.dtype, device=q.device)
    lse = torch.empty((b, h, s), dtype=torch.float32, device=q.device)
    return out, lse


# ---------------------------------------------------------------------------
# whole-layer operators (h100_torch_ops.py:198-475)
# ---------------------------------------------------------------------------


def _validate_layer(hidden_states, cos, sin, position_ids, packed_sequence_ids, weights,
                    family: _Family, *, separate_v: bool) -> int:
    what = "whole-layer"
    if hidden_states.ndim != 3:
        raise ValueError("compiled MI355X whole-layer hidden_states must be rank-3 BSH")
    batch, seqlen, hidden = hidden_states.shape
    if batch != 1 or not 1 <= seqlen <= _MAX_SEQLEN:
        raise UnsupportedMI355XPath("compiled MI355X whole-layer ops require B=1 and "
                                    "1 <= S <= 1024")
    if hidden != _HIDDEN:
        raise ValueError(f"compiled MI355X whole-layer hidden size must equal {_HIDDEN}")
    explicit = (hidden_states, cos, sin, position_ids, packed_sequence_ids, *weights)
    if any(t.device != hidden_states.device for t in explicit):
        raise ValueError("compiled MI355X whole-layer tensors must share one device")
    _same_gpu(explicit, what=what)
    if hidden_states.dtype != torch.bfloat16:
        raise ValueError("compiled MI355X whole-layer hidden_states must use BF16")
    rope_shape = (1, seqlen, family.head_dim)
    if cos.shape != rope_shape or sin.shape != rope_shape:
        raise ValueError("compiled MI355X whole-layer rotary tensors have the wrong shape")
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
        raise ValueError("compiled MI355X whole-layer rotary tensors must use BF16")
    _text_positions(position_ids, packed_sequence_ids, seqlen, what=what)
    shapes = family.weight_shapes(separate_v=separate_v)
    if len(weights) != len(shapes):
        raise AssertionError("whole-layer weight schema and validation table disagree")
    for weight, shape in zip(weights, shapes):
        if weight.shape != shape:
            raise ValueError("compiled MI355X whole-layer weight shape conflicts with the "
                             "locked layer")
        if weight.dtype != torch.bfloat16:
            raise ValueError("compiled MI355X whole-layer weights must use BF16")
        if not weight.is_contiguous():
            raise ValueError("compiled MI355X whole-layer weights must be contiguous")
    flagged = [n for n, t in zip(("hidden_states", "cos", "sin"), (hidden_states, cos, sin))
               if t.requires_grad]
    if flagged:
        raise UnsupportedMI355XPath("compiled MI355X whole-layer ops reject requires_grad "
                                    "activations; found " + ", ".join(flagged))
    if not (hidden_states.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()):
        raise ValueError("compiled MI355X whole-layer activations must be contiguous")
    _distinct_storage(explicit, what="whole-layer")
    return seqlen


def _project(hidden_states, weight, heads: int, head_dim: int) -> torch.Tensor:
    """(1, S, H * D) projection viewed as BSHD."""
    s = hidden_states.shape[1]
    return torch.nn.functional.linear(hidden_states, weight).view(1, s, heads, head_dim)


def _bhsd(t: torch.Tensor) -> torch.Tensor:
    return t.transpose(1, 2)


def _rope_rows(source_bshd, weight, cos, sin, *, out_bhsd=None) -> torch.Tensor:
    """RoPE(RMSNorm(x) w) over the whole head dim, bf16 (the layers' q and k)."""
    out = torch.empty_like(source_bshd) if out_bhsd is None else None
    target = _bhsd(out) if out is not None else out_bhsd
    prepare_rows_into(_bhsd(source_bshd), weight=weight, cos=cos, sin=sin,
                      rotary_dim=source_bshd.shape[-1], eps=_RMS_EPS, k=target)
    return out


def _layer_outputs(out, lse, explicit, seqlen):
    return _check_fresh_outputs(out, lse, explicit, out_shape=(1, seqlen, _HIDDEN),
                                lse_shape=(1, 32, seqlen), what="whole-layer op")


def _output_projection(attention, o_proj_weight, seqlen):
    return torch.nn.functional.linear(attention.reshape(1, seqlen, -1), o_proj_weight)


def _local_layer_impl(hidden_states: Tensor, cos: Tensor, sin: Tensor, position_ids: Tensor,
                      packed_sequence_ids: Tensor, q_proj_weight: Tensor, k_proj_weight: Tensor,
                      v_proj_weight: Tensor, o_proj_weight: Tensor, q_norm_weight: Tensor,
                      k_norm_weight: Tensor) -> tuple[Tensor, Tensor]:
    weights = (q_proj_weight, k_proj_weight, v_proj_weight, o_proj_weight, q_norm_weight,
               k_norm_weight)
    s = _validate_layer(hidden_states, cos, sin, position_ids, packed_sequence_ids, weights,
                        _LOCAL, separate_v=True)
    f = _LOCAL
    query = _rope_rows(_project(hidden_states, q_proj_weight, f.q_heads, f.head_dim),
                       q_norm_weight, cos, sin)
    key = _rope_rows(_project(hidden_states, k_proj_weight, f.kv_heads, f.head_dim),
                     k_norm_weight, cos, sin)
    value_src = _project(hidden_states, v_proj_weight, f.kv_heads, f.head_dim)
    value = torch.empty_like(value_src)
    prepare_rows_into(_bhsd(value_src), weight=k_norm_weight, eps=_RMS_EPS, v=_bhsd(value))
    attention, lse = fa4_local_text_forward(query, key, value)
    out = _output_projection(attention, o_proj_weight, s)
    return _layer_outputs(out, lse, (hidden_states, cos, sin, position_ids, packed_sequence_ids,
                                     *weights), s)


def _global_layer_impl(hidden_states: Tensor, cos: Tensor, sin: Tensor, position_ids: Tensor,
                       packed_sequence_ids: Tensor, q_proj_weight: Tensor, k_proj_weight: Tensor,
                       o_proj_weight: Tensor, q_norm_weight: Tensor,
                       k_norm_weight: Tensor) -> tuple[Tensor, Tensor]:
    weights = (q_proj_weight, k_proj_weight, o_proj_weight, q_norm_weight, k_norm_weight)
    s = _validate_layer(hidden_states, cos, sin, position_ids, packed_sequence_ids, weights,
                        _GLOBAL, separate_v=False)
    f = _GLOBAL
    query = _rope_rows(_project(hidden_states, q_proj_weight, f.q_heads, f.head_dim),
                       q_norm_weight, cos, sin)
    # K and V from the one shared projection, in one pass over it
    source = _project(hidden_states, k_proj_weight, f.kv_heads, f.head_dim)
    key, value = torch.empty_like(source), torch.empty_like(source)
    prepare_rows_into(_bhsd(source), weight=k_norm_weight, cos=cos, sin=sin,
                      rotary_dim=f.head_dim, eps=_RMS_EPS, k=_bhsd(key), v=_bhsd(value))
    attention, lse = fa4_global_text_forward(query, key, value)
    out = _output_projection(attention, o_proj_weight, s)
    return _layer_outputs(out, lse, (hidden_states, cos, sin, position_ids, packed_sequence_ids,
                                     *weights), s)


def _fake_layer(hidden_states, *_args):
    b, s, _ = hidden_states.shape
    out = torch.empty((b, s, _HIDDEN), dtype=hidden_states.dtype, device=hidden_states.device)
    lse = torch.empty((b, 32, s), dtype=torch.float32, device=hidden_states.device)
    return out, lse


# ---------------------------------------------------------------------------
# StaticCache one-token decode (h100_torch_ops.py:479-846)
# ---------------------------------------------------------------------------


def _validate_decode(hidden_states, cos, sin, position_ids, cache_k, cache_v, cache_length,
                     weights, family: _Family, *, separate_v: bool) -> tuple[int, int]:
    """Checks shared by both decode operators; returns (position, cache length)."""
    what = f"{family.label} StaticCache decode"
    explicit = (hidden_states, cos, sin, position_ids, cache_k, cache_v, cache_length, *weights)
    if hidden_states.shape != (1, 1, _HIDDEN):
        raise UnsupportedMI355XPath(f"compiled MI355X {what} requires B1, Q1, and hidden size "
                                    f"{_HIDDEN}")
    _same_gpu(explicit, what=what)
    if any(t.dtype != torch.bfloat16 for t in (hidden_states, cos, sin, cache_k, cache_v,
                                               *weights)):
        raise ValueError(f"compiled MI355X {what} activations, cache, and weights must use BF16")
    if cos.shape != (1, 1, family.head_dim) or sin.shape != (1, 1, family.head_dim):
        raise ValueError(f"compiled MI355X {what} rotary tensors are invalid")
    _index_tensor(position_ids, (1, 1), name="position_ids", what=what)
    if cache_length.ndim != 0 or cache_length.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"compiled MI355X {what} length must be a scalar integer tensor")
    if cache_k.ndim != 4 or cache_k.shape[:2] != (1, family.kv_heads) or \
            cache_k.shape[-1] != family.head_dim:
        raise ValueError(f"compiled MI355X {what} K backing has the wrong geometry")
    if cache_v.shape != cache_k.shape:
        raise ValueError(f"compiled MI355X {what} K/V backings must have equal geometry")
    for weight, shape in zip(weights, family.weight_shapes(separate_v=separate_v)):
        if weight.shape != shape or not weight.is_contiguous():
            raise ValueError(f"compiled MI355X {what} weight conflicts with the locked layer")
    if any(t.requires_grad for t in (hidden_states, cos, sin, cache_k, cache_v)):
        raise UnsupportedMI355XPath(f"compiled MI355X {what} rejects requires_grad "
                                    "activations/cache")
    if any(not t.is_contiguous() for t in explicit[:7]):
        raise ValueError(f"compiled MI355X {what} inputs must be contiguous")
    _distinct_storage(explicit, what=what)
    return int(position_ids.detach().item()), int(cache_length.detach().item())


def _decode_inputs(hidden_states, q_proj_weight, q_norm_weight, cos, sin, family: _Family):
    return _rope_rows(_project(hidden_states, q_proj_weight, family.q_heads, family.head_dim),
                      q_norm_weight, cos, sin)


def _global_static_cache_decode_impl(hidden_states: Tensor, cos: Tensor, sin: Tensor,
                                     position_ids: Tensor, cache_k: Tensor, cache_v: Tensor,
                                     cache_length: Tensor, q_proj_weight: Tensor,
                                     k_proj_weight: Tensor, o_proj_weight: Tensor,
                                     q_norm_weight: Tensor,
                                     k_norm_weight: Tensor) -> tuple[Tensor, Tensor]:
    """Prepare K/V into the next cache slot, advance the length, attend over the prefix."""
    weights = (q_proj_weight, k_proj_weight, o_proj_weight, q_norm_weight, k_norm_weight)
    f = _GLOBAL
    position, length = _validate_decode(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                                        cache_length, weights, f, separate_v=False)
    capacity = cache_k.shape[2]
    if not 1 <= length < _DECODE_MAX_POSITION:
        raise UnsupportedMI355XPath("compiled MI355X global StaticCache decode requires a "
                                    "nonempty in-range prefix")
    if capacity > _DECODE_MAX_POSITION or length + 1 >= capacity:
        raise UnsupportedMI355XPath("compiled MI355X global StaticCache decode requires spare "
                                    "unwritten capacity")
    if position != length:
        raise UnsupportedMI355XPath("compiled MI355X global StaticCache decode position must "
                                    "equal the active prefix length")
    query = _decode_inputs(hidden_states, q_proj_weight, q_norm_weight, cos, sin, f)
    source = _project(hidden_states, k_proj_weight, f.kv_heads, f.head_dim)
    # the kernel writes K and V of the new token into cache slot `length`
    prepare_rows_into(_bhsd(source), weight=k_norm_weight, cos=cos, sin=sin,
                      rotary_dim=f.head_dim, eps=_RMS_EPS,
                      k=cache_k[:, :, length:length + 1], v=cache_v[:, :, length:length + 1])
    cache_length.add_(1)
    active = length + 1
    attention, lse = fa4_global_forward_only(query, _bhsd(cache_k[:, :, :active]),
                                             _bhsd(cache_v[:, :, :active]))
    out = _output_projection(attention, o_proj_weight, 1)
    return _layer_outputs(out, lse, (hidden_states, cos, sin, position_ids, cache_k, cache_v,
                                     cache_length, *weights), 1)


def _local_static_cache_decode_impl(hidden_states: Tensor, cos: Tensor, sin: Tensor,
                                    position_ids: Tensor, cache_k: Tensor, cache_v: Tensor,
                                    cache_length: Tensor, q_proj_weight: Tensor,
                                    k_proj_weight: Tensor, v_proj_weight: Tensor,
                                    o_proj_weight: Tensor, q_norm_weight: Tensor,
                                    k_norm_weight: Tensor) -> tuple[Tensor, Tensor]:
    """Sliding-window cache: append below capacity, else shift left by one and append last."""
    weights = (q_proj_weight, k_proj_weight, v_proj_weight, o_proj_weight, q_norm_weight,
               k_norm_weight)
    f = _LOCAL
    position, length = _validate_decode(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                                        cache_length, weights, f, separate_v=True)
    if cache_k.shape[2] != _MAX_SEQLEN:
        raise ValueError("compiled MI355X local StaticCache decode K/V backings have the wrong "
                         "geometry")
    if not 1 <= position < _DECODE_MAX_POSITION:
        raise UnsupportedMI355XPath("compiled MI355X local StaticCache decode requires a "
                                    "nonempty in-range prefix")
    if length != min(position, _MAX_SEQLEN):
        raise UnsupportedMI355XPath("compiled MI355X local StaticCache tensor length conflicts "
                                    "with the absolute position")
    query = _decode_inputs(hidden_states, q_proj_weight, q_norm_weight, cos, sin, f)
    if position < _MAX_SEQLEN:
        slot, active = position, position + 1
    else:
        # the window is full: drop the oldest token (the backing keeps the
        # Transformers sliding layout, oldest first)
        for backing in (cache_k, cache_v):
            backing.copy_(backing.roll(-1, dims=2))
        slot, active = _MAX_SEQLEN - 1, _MAX_SEQLEN
    key_src = _project(hidden_states, k_proj_weight, f.kv_heads, f.head_dim)
    value_src = _project(hidden_states, v_proj_weight, f.kv_heads, f.head_dim)
    prepare_rows_into(_bhsd(key_src), weight=k_norm_weight, cos=cos, sin=sin,
                      rotary_dim=f.head_dim, eps=_RMS_EPS, k=cache_k[:, :, slot:slot + 1])
    prepare_rows_into(_bhsd(value_src), weight=k_norm_weight, eps=_RMS_EPS,
                      v=cache_v[:, :, slot:slot + 1])
    device = hidden_states.device
    cu_q = torch.tensor([0, 1], dtype=torch.int32, device=device)
    cu_k = torch.tensor([0, active], dtype=torch.int32, device=device)
    attention, lse = fa4_local_varlen_forward(
        query[0], cache_k[0, :, :active].transpose(0, 1), cache_v[0, :, :active].transpose(0, 1),
        cu_q, cu_k, max_seqlen_q=1, max_seqlen_k=active)
    out = _output_projection(attention, o_proj_weight, 1)
    return _layer_outputs(out, lse.unsqueeze(0), (hidden_states, cos, sin, position_ids, cache_k,
                                                  cache_v, cache_length, *weights), 1)


def _fake_decode(hidden_states, *_args):
    b, s, _ = hidden_states.shape
    out = torch.empty((b, s, _HIDDEN), dtype=hidden_states.dtype, device=hidden_states.device)
    lse = torch.empty((b, 32, s), dtype=torch.float32, device=hidden_states.device)
    return out, lse


# ---------------------------------------------------------------------------
# registration (h100_torch_ops.py:966-1017)
# ---------------------------------------------------------------------------


def _inference_only(hidden_states, cos, sin) -> None:
    """Refuse autograd before the custom operator disables grad mode for its body."""
    if torch.is_grad_enabled():
        raise UnsupportedMI355XPath("compiled MI355X whole-layer ops require global "
                                    "inference/no-grad mode")
    flagged = [n for n, t in zip(("hidden_states", "cos", "sin"), (hidden_states, cos, sin))
               if t.requires_grad]
    if flagged:
        raise UnsupportedMI355XPath("compiled MI355X whole-layer ops reject requires_grad "
                                    "activations; found " + ", ".join(flagged))


_library = getattr(torch, "library", None)
_custom_op: Callable | None = getattr(_library, "custom_op", None)
_register_fake: Callable | None = getattr(_library, "register_fake", None)
CUSTOM_OPS_AVAILABLE = callable(_custom_op) and callable(_register_fake)


def _op(name, impl, fake, mutates=()):
    op = _custom_op(name, mutates_args=mutates)(impl)
    _register_fake(op)(fake)
    return op


if CUSTOM_OPS_AVAILABLE:
    local_fwd = _op(LOCAL_OP_NAME, _local_impl, _fake_prepared)
    global_fwd = _op(GLOBAL_OP_NAME, _global_impl, _fake_prepared)
    local_layer_op = _op(LOCAL_LAYER_OP_NAME, _local_layer_impl, _fake_layer)
    global_layer_op = _op(GLOBAL_LAYER_OP_NAME, _global_layer_impl, _fake_layer)
    global_static_cache_decode_op = _op(GLOBAL_STATIC_CACHE_DECODE_OP_NAME,
                                        _global_static_cache_decode_impl, _fake_decode,
                                        {"cache_k", "cache_v", "cache_length"})
    local_static_cache_decode_op = _op(LOCAL_STATIC_CACHE_DECODE_OP_NAME,
                                       _local_static_cache_decode_impl, _fake_decode,
                                       {"cache_k", "cache_v"})

    def local_layer_fwd(hidden_states, cos, sin, position_ids, packed_sequence_ids,
                        q_proj_weight, k_proj_weight, v_proj_weight, o_proj_weight,
                        q_norm_weight, k_norm_weight):
        _inference_only(hidden_states, cos, sin)
        return local_layer_op(hidden_states, cos, sin, position_ids, packed_sequence_ids,
                              q_proj_weight, k_proj_weight, v_proj_weight, o_proj_weight,
                              q_norm_weight, k_norm_weight)

    def global_layer_fwd(hidden_states, cos, sin, position_ids, packed_sequence_ids,
                         q_proj_weight, k_proj_weight, o_proj_weight, q_norm_weight,
                         k_norm_weight):
        _inference_only(hidden_states, cos, sin)
        return global_layer_op(hidden_states, cos, sin, position_ids, packed_sequence_ids,
                               q_proj_weight, k_proj_weight, o_proj_weight, q_norm_weight,
                               k_norm_weight)

    def global_static_cache_decode_fwd(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                                       cache_length, q_proj_weight, k_proj_weight,
                                       o_proj_weight, q_norm_weight, k_norm_weight):
        _inference_only(hidden_states, cos, sin)
        return global_static_cache_decode_op(hidden_states, cos, sin, position_ids, cache_k,
                                             cache_v, cache_length, q_proj_weight,
                                             k_proj_weight, o_proj_weight, q_norm_weight,
                                             k_norm_weight)

    def local_static_cache_decode_fwd(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                                      cache_length, q_proj_weight, k_proj_weight, v_proj_weight,
                                      o_proj_weight, q_norm_weight, k_norm_weight):
        _inference_only(hidden_states, cos, sin)
        return local_static_cache_decode_op(hidden_states, cos, sin, position_ids, cache_k,
                                            cache_v, cache_length, q_proj_weight, k_proj_weight,
                                            v_proj_weight, o_proj_weight, q_norm_weight,
                                            k_norm_weight)

else:  # pragma: no cover - every supported PyTorch provides torch.library.custom_op

    def _unavailable(*_args):
        raise RuntimeError("MI355X opaque forward ops require PyTorch with "
                           "torch.library.custom_op and torch.library.register_fake")

    local_fwd = global_fwd = local_layer_op = global_layer_op = _unavailable
    global_static_cache_decode_op = local_static_cache_decode_op = _unavailable
    local_layer_fwd = global_layer_fwd = _unavailable
    global_static_cache_decode_fwd = local_static_cache_decode_fwd = _unavailable


# the reference's Python names (src/gemma4_fa4/h100_torch_ops.py:1140-1158)
h100_local_fwd = local_fwd
h100_global_fwd = global_fwd
h100_local_layer_op = local_layer_op
h100_global_layer_op = global_layer_op
h100_local_layer_fwd = local_layer_fwd
h100_global_layer_fwd = global_layer_fwd
h100_global_static_cache_decode_op = global_static_cache_decode_op
h100_local_static_cache_decode_op = local_static_cache_decode_op
h100_global_static_cache_decode_fwd = global_static_cache_decode_fwd
h100_local_static_cache_decode_fwd = local_static_cache_decode_fwd
_h100_local_layer_impl = _local_layer_impl
_h100_global_layer_impl = _global_layer_impl
_h100_global_static_cache_decode_impl = _global_static_cache_decode_impl
_h100_local_static_cache_decode_impl = _local_static_cache_decode_impl

__all__ = [
    "CUSTOM_OPS_AVAILABLE",
    "NAMESPACE",
    "GLOBAL_OP_NAME",
    "GLOBAL_LAYER_OP_NAME",
    "GLOBAL_STATIC_CACHE_DECODE_OP_NAME",
    "LOCAL_OP_NAME",
    "LOCAL_LAYER_OP_NAME",
    "LOCAL_STATIC_CACHE_DECODE_OP_NAME",
    "global_fwd",
    "global_layer_fwd",
    "global_layer_op",
    "global_static_cache_decode_fwd",
    "global_static_cache_decode_op",
    "local_fwd",
    "local_layer_fwd",
    "local_layer_op",
    "local_static_cache_decode_fwd",
    "local_static_cache_decode_op",
    "h100_global_fwd",
    "h100_global_layer_fwd",
    "h100_global_layer_op",
    "h100_global_static_cache_decode_fwd",
    "h100_global_static_cache_decode_op",
    "h100_local_fwd",
    "h100_local_layer_fwd",
    "h100_local_layer_op",
    "h100_local_static_cache_decode_fwd",
    "h100_local_static_cache_decode_op",
]
