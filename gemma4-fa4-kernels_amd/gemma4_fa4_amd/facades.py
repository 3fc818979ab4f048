"""Guarded compiled facades: a whole attention layer and StaticCache one-token decode.

Mirrors the reference's compiled facades (src/gemma4_fa4/transformers_integration.py:
2144-2546 for the whole layer, 2547-3492 for StaticCache decode) over this
library's opaque operators (``torch_ops``):

* ``compile_gemma4_mi355x_layer(module)`` validates an eval-mode Transformers
  ``Gemma4TextAttention`` of the locked geometry and returns a facade whose
  calls run ``torch.compile(fullgraph=True)`` of a tensor-only function around
  the layer operator.  Every call re-validates the module, its weights and the
  inputs outside the compiled frame.
* ``compile_gemma4_mi355x_static_cache_decode(module, cache)`` binds the
  module's layer of a Transformers ``StaticCache`` (a ``StaticLayer`` for a
  global layer, a 1024-slot ``StaticSlidingWindowLayer`` for a sliding one) and
  returns a facade that decodes one token per call against it, in place.  The
  global operator advances the layer's length tensor itself; for the sliding
  layer the facade advances the length tensor (while below capacity) and the
  Python length afterwards, the two counters Transformers keeps
  (cache_utils ``StaticSlidingWindowLayer.update``).
* ``gemma4_mi355x_compile_layer`` is the compile-only replacement for a
  ``Gemma4TextAttention.forward`` call (ti.py:2212-2299).

The reference pins one Transformers revision and accepts only its exact
classes, layer 0 / layer 5 and its compile-origin mask markers; this build
checks the installed Transformers classes and any layer whose kind matches,
because the pinned revision is not installed.  The default ``backend`` is
``"eager"``: the traced graph is the one opaque operator plus argument
plumbing, so there is nothing for a code generator to fuse (``"inductor"`` or
a callable backend is accepted as in the reference).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch

from . import torch_ops
from .errors import UnsupportedMI355XPath
from .model_spec import GEMMA4_31B, AttentionLayerSpec

_EPS = 1e-6
_SLIDING_CAPACITY = 1024


def _spec(module: Any) -> AttentionLayerSpec:
    layer_idx = getattr(module, "layer_idx", None)
    if isinstance(layer_idx, bool) or not isinstance(layer_idx, int):
        raise ValueError("Gemma 4 attention module must expose an integer layer_idx")
    return GEMMA4_31B.spec_for_layer(layer_idx)


def _attention_class():
    try:
        from transformers.models.gemma4.modeling_gemma4 import Gemma4TextAttention
    except Exception:  # transformers without Gemma 4
        return None
    return Gemma4TextAttention


def _linear_weight(module: Any, name: str, shape: tuple[int, int]) -> torch.Tensor:
    layer = getattr(module, name, None)
    weight = getattr(layer, "weight", None)
    if not isinstance(layer, torch.nn.Linear) or layer.bias is not None:
        raise UnsupportedMI355XPath(f"{name} must be a bias-free Linear")
    if weight.shape != shape or weight.dtype != torch.bfloat16 or not weight.is_contiguous():
        raise UnsupportedMI355XPath(f"{name} weight must be a contiguous BF16 {shape} tensor")
    return weight


def _norm_weight(module: Any, name: str, dim: int) -> torch.Tensor:
    norm = getattr(module, name, None)
    weight = getattr(norm, "weight", None)
    if getattr(norm, "with_scale", None) is not True or getattr(norm, "eps", None) != _EPS or \
            not isinstance(weight, torch.Tensor):
        raise UnsupportedMI355XPath(f"{name} must be a scaled RMSNorm with eps 1e-6")
    if weight.shape != (dim,) or weight.dtype != torch.bfloat16 or not weight.is_contiguous():
        raise UnsupportedMI355XPath(f"{name} weight must be a contiguous BF16 ({dim},) tensor")
    return weight


def layer_weights(module: Any, spec: AttentionLayerSpec | None = None) -> tuple[torch.Tensor, ...]:
    """The explicit weight tuple of a locked-geometry Gemma 4 text attention module.

    (q_proj, k_proj, [v_proj,] o_proj, q_norm, k_norm) weights, in the layer
    operators' argument order (ti.py:2144-2211).
    """
    spec = _spec(module) if spec is None else spec
    cls = _attention_class()
    if cls is None or type(module) is not cls:
        raise UnsupportedMI355XPath("compiled routing requires a Transformers Gemma4TextAttention")
    global_layer = spec.kind == "full_attention"
    if (getattr(module, "training", None) is not False
            or getattr(module, "is_sliding", None) is global_layer
            or getattr(module, "is_kv_shared_layer", None) is not False
            or getattr(module, "store_full_length_kv", None) is not False
            or getattr(module, "head_dim", None) != spec.head_dim_qk
            or getattr(module, "num_key_value_groups", None) != spec.qhead_per_kvhead
            or getattr(module, "scaling", None) != 1.0
            or getattr(module, "attention_dropout", None) != 0.0):
        raise UnsupportedMI355XPath(
            f"compiled routing requires an eval-mode Gemma4TextAttention of layer kind "
            f"{spec.kind} that neither shares nor exports full-length K/V")
    if getattr(module, "use_alternative_attention", None) is not global_layer:
        raise UnsupportedMI355XPath("the module's K/V projection mode conflicts with its family")
    v_norm = getattr(module, "v_norm", None)
    if getattr(v_norm, "with_scale", None) is not False or getattr(v_norm, "eps", None) != _EPS:
        raise UnsupportedMI355XPath("compiled routing requires the scale-free V RMSNorm")
    hidden = GEMMA4_31B.hidden_size
    q_width = spec.num_q_heads * spec.head_dim_qk
    kv_width = spec.num_kv_heads * spec.head_dim_qk
    weights = [_linear_weight(module, "q_proj", (q_width, hidden)),
               _linear_weight(module, "k_proj", (kv_width, hidden))]
    if global_layer:
        if getattr(module, "v_proj", object()) is not None:
            raise UnsupportedMI355XPath("global routing requires one shared K/V projection")
    else:
        weights.append(_linear_weight(module, "v_proj", (kv_width, hidden)))
    weights += [_linear_weight(module, "o_proj", (hidden, q_width)),
                _norm_weight(module, "q_norm", spec.head_dim_qk),
                _norm_weight(module, "k_norm", spec.head_dim_qk)]
    if len({w.untyped_storage().data_ptr() for w in weights}) != len(weights):
        raise UnsupportedMI355XPath("module weights must use distinct storage")
    return tuple(weights)


def _rotary(position_embeddings) -> tuple[torch.Tensor, torch.Tensor]:
    if type(position_embeddings) is not tuple or len(position_embeddings) != 2:
        raise UnsupportedMI355XPath("compiled routing requires the (cos, sin) tuple")
    return position_embeddings


def _check_backend(backend) -> None:
    if not (backend in {"eager", "aot_eager", "inductor"} if isinstance(backend, str)
            else callable(backend)):
        raise ValueError("backend must be eager, aot_eager, inductor, or a callable")
    if not torch_ops.CUSTOM_OPS_AVAILABLE or not callable(getattr(torch, "compile", None)):
        raise UnsupportedMI355XPath("compiled facades require torch.compile and torch.library "
                                    "custom operators")


# ---------------------------------------------------------------------------
# whole layer (ti.py:2212-2546)
# ---------------------------------------------------------------------------


def _local_layer_tensor_only(hidden_states, cos, sin, position_ids, *weights):
    packed = torch.zeros_like(position_ids)  # one sequence: positions are arange(S)
    out, _ = torch_ops.local_layer_fwd(hidden_states, cos, sin, position_ids, packed, *weights)
    return out


def _global_layer_tensor_only(hidden_states, cos, sin, position_ids, *weights):
    packed = torch.zeros_like(position_ids)
    out, _ = torch_ops.global_layer_fwd(hidden_states, cos, sin, position_ids, packed, *weights)
    return out


def _check_layer_inputs(hidden_states, cos, sin, position_ids, weights, spec) -> None:
    """The facade's per-call contract, checked outside the compiled frame (ti.py:2377-2424)."""
    if torch.is_grad_enabled():
        raise UnsupportedMI355XPath("the compiled layer facade requires inference/no-grad mode")
    if hidden_states.ndim != 3:
        raise UnsupportedMI355XPath("hidden_states must be rank-3 BSH")
    b, s, h = hidden_states.shape
    if b != 1 or not 1 <= s <= 1024 or h != GEMMA4_31B.hidden_size:
        raise UnsupportedMI355XPath("the compiled layer facade requires B1, hidden size 5376, "
                                    "and 1 <= S <= 1024")
    if cos.shape != (1, s, spec.head_dim_qk) or sin.shape != cos.shape:
        raise UnsupportedMI355XPath("rotary tensors conflict with the locked layer")
    if position_ids.shape != (1, s) or position_ids.dtype not in (torch.int32, torch.int64):
        raise UnsupportedMI355XPath("position_ids must be INT32/INT64 of shape (1, S)")
    tensors = (hidden_states, cos, sin, position_ids, *weights)
    if hidden_states.device.type != "cuda" or any(t.device != hidden_states.device
                                                  for t in tensors):
        raise UnsupportedMI355XPath("facade tensors must share one CUDA device")
    if any(t.dtype != torch.bfloat16 for t in (hidden_states, cos, sin)):
        raise UnsupportedMI355XPath("activations must use BF16")
    if any(t.requires_grad for t in (hidden_states, cos, sin)):
        raise UnsupportedMI355XPath("activation tensors must not require grad")
    if any(not t.is_contiguous() for t in tensors):
        raise UnsupportedMI355XPath("facade tensors must be contiguous")
    expected = torch.arange(s, dtype=position_ids.dtype, device=position_ids.device)
    if not torch.equal(position_ids[0], expected):
        raise UnsupportedMI355XPath("the compiled layer facade requires zero-based position_ids")
    if len({t.untyped_storage().data_ptr() for t in tensors}) != len(tensors):
        raise UnsupportedMI355XPath("facade tensors must use distinct storage")


class Gemma4MI355XCompiledLayerFacade:
    """Explicit guarded facade over one compiled layer; not ``torch.compile(layer)`` support."""

    def __init__(self, module: Any, spec: AttentionLayerSpec, compiled_call: Callable) -> None:
        self._module = module
        self._spec = spec
        self._compiled_call = compiled_call
        self._entries = 0

    @property
    def compiled_entry_count(self) -> int:
        return self._entries

    def __call__(self, hidden_states, position_embeddings, *, position_ids):
        weights = layer_weights(self._module, self._spec)
        cos, sin = _rotary(position_embeddings)
        _check_layer_inputs(hidden_states, cos, sin, position_ids, weights, self._spec)
        self._entries += 1
        return self._compiled_call(hidden_states, cos, sin, position_ids, *weights), None


def compile_gemma4_mi355x_layer(module: Any, *, backend: str | Callable = "eager"
                                ) -> Gemma4MI355XCompiledLayerFacade:
    """Build the guarded, tensor-only compiled facade of one attention layer (ti.py:2517-2544)."""
    _check_backend(backend)
    spec = _spec(module)
    layer_weights(module, spec)
    inner = _global_layer_tensor_only if spec.kind == "full_attention" else \
        _local_layer_tensor_only
    compiled = torch.compile(inner, backend=backend, fullgraph=True, dynamic=True)
    return Gemma4MI355XCompiledLayerFacade(module, spec, compiled)


def gemma4_mi355x_compile_layer(module: Any, hidden_states, position_embeddings, attention_mask,
                                shared_kv_states, past_key_values=None, **kwargs):
    """Compile-only whole-layer route for a ``Gemma4TextAttention.forward`` call (ti.py:2212-2299).

    Called while ``torch.compile`` traces the module's forward: rejects caches,
    shared K/V, padding masks and metadata, then emits the opaque layer
    operator.  Returns ``(output, None)`` like the module.
    """
    from .transformers_integration import Gemma4MaskPlan, _compiling

    if not _compiling():
        raise UnsupportedMI355XPath("whole-layer routing is compile-only")
    if past_key_values is not None:
        raise UnsupportedMI355XPath("whole-layer routing rejects every cache")
    if type(shared_kv_states) is not dict or shared_kv_states:
        raise UnsupportedMI355XPath("whole-layer routing rejects shared prepared K/V")
    cos, sin = _rotary(position_embeddings)
    unexpected = set(kwargs) - {"position_ids", "allow_flex_fallback"}
    if unexpected:
        raise UnsupportedMI355XPath("whole-layer routing rejects metadata outside its scope: "
                                    + ", ".join(sorted(unexpected)))
    if kwargs.get("allow_flex_fallback", False) is not False:
        raise UnsupportedMI355XPath("whole-layer routing does not accept a fallback")
    position_ids = kwargs.get("position_ids")
    if not isinstance(position_ids, torch.Tensor):
        raise UnsupportedMI355XPath("whole-layer routing requires explicit position_ids")
    spec = _spec(module)
    weights = layer_weights(module, spec)
    if isinstance(attention_mask, Gemma4MaskPlan):
        if attention_mask.attention_mask is not None:
            raise UnsupportedMI355XPath("whole-layer routing does not accept padding")
    elif attention_mask is not None:
        raise UnsupportedMI355XPath("whole-layer routing requires a Gemma4MaskPlan or no mask")
    inner = _global_layer_tensor_only if spec.kind == "full_attention" else \
        _local_layer_tensor_only
    return inner(hidden_states, cos, sin, position_ids, *weights), None


# ---------------------------------------------------------------------------
# StaticCache one-token decode (ti.py:2547-3492)
# ---------------------------------------------------------------------------


def _cache_classes():
    try:
        from transformers.cache_utils import StaticCache, StaticLayer, StaticSlidingWindowLayer
    except Exception:
        return None
    return StaticCache, StaticLayer, StaticSlidingWindowLayer


@dataclass
class _CacheBinding:
    cache: Any
    layer: Any
    keys: torch.Tensor
    values: torch.Tensor
    length: torch.Tensor
    pointers: tuple[int, int, int]


def _bind(module: Any, cache: Any, spec: AttentionLayerSpec) -> _CacheBinding:
    """Freeze the identities of the module's cache layer and its tensors."""
    classes = _cache_classes()
    if classes is None or not isinstance(cache, classes[0]):
        raise UnsupportedMI355XPath("StaticCache decode requires a Transformers StaticCache")
    if getattr(cache, "offloading", False):
        raise UnsupportedMI355XPath("StaticCache decode requires a non-offloaded cache")
    layers = getattr(cache, "layers", None)
    idx = module.layer_idx
    if type(layers) is not list or not 0 <= idx < len(layers):
        raise UnsupportedMI355XPath("the cache has no layer for this module")
    layer = layers[idx]
    global_layer = spec.kind == "full_attention"
    expected = classes[1] if global_layer else classes[2]
    if type(layer) is not expected:
        raise UnsupportedMI355XPath(f"cache layer {idx} must be a {expected.__name__}")
    if getattr(layer, "is_initialized", None) is not True:
        raise UnsupportedMI355XPath("StaticCache decode requires an initialized cache layer")
    keys, values, length = layer.keys, layer.values, layer.cumulative_length
    if not all(isinstance(t, torch.Tensor) for t in (keys, values, length)):
        raise UnsupportedMI355XPath("cache layer tensors are not initialized")
    shape = (1, spec.num_kv_heads, keys.shape[2], spec.head_dim_qk)
    if keys.shape != shape or values.shape != shape or keys.dtype != torch.bfloat16 or \
            values.dtype != torch.bfloat16 or not keys.is_contiguous() or \
            not values.is_contiguous():
        raise UnsupportedMI355XPath("cache K/V backings conflict with the locked layer geometry")
    if not global_layer and (layer.max_cache_len != _SLIDING_CAPACITY or
                             type(getattr(layer, "cumulative_length_int", None)) is not int):
        raise UnsupportedMI355XPath("sliding decode requires a 1024-slot sliding cache layer")
    pointers = tuple(t.untyped_storage().data_ptr() for t in (keys, values, length))
    return _CacheBinding(cache, layer, keys, values, length, pointers)


def _rebind_check(b: _CacheBinding, module: Any) -> None:
    layer = b.cache.layers[module.layer_idx] if module.layer_idx < len(b.cache.layers) else None
    live = (getattr(layer, "keys", None), getattr(layer, "values", None),
            getattr(layer, "cumulative_length", None))
    if layer is not b.layer or any(x is not y for x, y in zip(live, (b.keys, b.values, b.length))) \
            or tuple(t.untyped_storage().data_ptr() for t in live) != b.pointers:
        raise UnsupportedMI355XPath("the bound cache layer or its storage was replaced")


def _check_decode_inputs(hidden_states, cos, sin, position_ids, spec) -> None:
    if torch.is_grad_enabled():
        raise UnsupportedMI355XPath("StaticCache decode requires inference/no-grad mode")
    if hidden_states.shape != (1, 1, GEMMA4_31B.hidden_size):
        raise UnsupportedMI355XPath("StaticCache decode takes one token: hidden_states "
                                    "(1, 1, 5376)")
    if cos.shape != (1, 1, spec.head_dim_qk) or sin.shape != cos.shape:
        raise UnsupportedMI355XPath("rotary tensors conflict with the locked layer")
    if position_ids.shape != (1, 1) or position_ids.dtype not in (torch.int32, torch.int64):
        raise UnsupportedMI355XPath("position_ids must be INT32/INT64 of shape (1, 1)")
    if hidden_states.device.type != "cuda" or any(t.device != hidden_states.device
                                                  for t in (cos, sin, position_ids)):
        raise UnsupportedMI355XPath("decode tensors must share one CUDA device")
    if any(t.dtype != torch.bfloat16 for t in (hidden_states, cos, sin)):
        raise UnsupportedMI355XPath("decode activations must use BF16")


def _global_decode_tensor_only(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                               cache_length, *weights):
    return torch_ops.global_static_cache_decode_fwd(hidden_states, cos, sin, position_ids,
                                                    cache_k, cache_v, cache_length, *weights)


def _local_decode_tensor_only(hidden_states, cos, sin, position_ids, cache_k, cache_v,
                              cache_length, *weights):
    return torch_ops.local_static_cache_decode_fwd(hidden_states, cos, sin, position_ids,
                                                   cache_k, cache_v, cache_length, *weights)


class _DecodeFacade:
    def __init__(self, module: Any, spec: AttentionLayerSpec, binding: _CacheBinding,
                 compiled_call: Callable) -> None:
        self._module = module
        self._spec = spec
        self._binding = binding
        self._compiled_call = compiled_call
        self._entries = 0
        self._last_lse: torch.Tensor | None = None

    @property
    def compiled_entry_count(self) -> int:
        return self._entries

    @property
    def last_lse(self) -> torch.Tensor | None:
        return self._last_lse

    def _prepare(self, hidden_states, position_embeddings, position_ids):
        weights = layer_weights(self._module, self._spec)
        cos, sin = _rotary(position_embeddings)
        _check_decode_inputs(hidden_states, cos, sin, position_ids, self._spec)
        _rebind_check(self._binding, self._module)
        return weights, cos, sin

    def _run(self, hidden_states, cos, sin, position_ids, weights):
        b = self._binding
        self._entries += 1
        out, lse = self._compiled_call(hidden_states, cos, sin, position_ids, b.keys, b.values,
                                       b.length, *weights)
        self._last_lse = lse
        return out


class Gemma4MI355XCompiledStaticCacheDecodeFacade(_DecodeFacade):
    """One-token decode of a global layer against its ``StaticLayer`` (ti.py:3238-3325)."""

    def __call__(self, hidden_states, position_embeddings, *, position_ids):
        weights, cos, sin = self._prepare(hidden_states, position_embeddings, position_ids)
        length = int(self._binding.length.item())
        if int(position_ids.item()) != length:
            raise UnsupportedMI355XPath("the decode position must equal the cached length")
        out = self._run(hidden_states, cos, sin, position_ids, weights)
        if int(self._binding.length.item()) != length + 1:
            raise RuntimeError("the global decode operator did not advance the cache length")
        return out, None


class Gemma4MI355XCompiledLocalStaticCacheDecodeFacade(_DecodeFacade):
    """One-token decode of a sliding layer against its 1024-slot window (ti.py:3327-3423)."""

    def __call__(self, hidden_states, position_embeddings, *, position_ids):
        weights, cos, sin = self._prepare(hidden_states, position_embeddings, position_ids)
        layer, b = self._binding.layer, self._binding
        absolute = layer.cumulative_length_int
        if int(position_ids.item()) != absolute:
            raise UnsupportedMI355XPath("the decode position must equal the cached length")
        if int(b.length.item()) != min(absolute, _SLIDING_CAPACITY):
            raise UnsupportedMI355XPath("the sliding cache's length tensor and Python length "
                                        "disagree")
        out = self._run(hidden_states, cos, sin, position_ids, weights)
        # the two counters Transformers' sliding layer keeps: the tensor stops
        # at the capacity, the Python length counts every token
        if absolute < _SLIDING_CAPACITY:
            b.length.add_(1)
        layer.cumulative_length_int = absolute + 1
        return out, None


def compile_gemma4_mi355x_static_cache_decode(module: Any, cache: Any, *,
                                              backend: str | Callable = "eager"):
    """Bind a module's StaticCache layer and build its guarded decode facade (ti.py:3425-3490)."""
    _check_backend(backend)
    spec = _spec(module)
    layer_weights(module, spec)
    binding = _bind(module, cache, spec)
    if spec.kind == "full_attention":
        compiled = torch.compile(_global_decode_tensor_only, backend=backend, fullgraph=True)
        return Gemma4MI355XCompiledStaticCacheDecodeFacade(module, spec, binding, compiled)
    compiled = torch.compile(_local_decode_tensor_only, backend=backend, fullgraph=True)
    return Gemma4MI355XCompiledLocalStaticCacheDecodeFacade(module, spec, binding, compiled)


# the reference's public names (src/gemma4_fa4/__init__.py)
Gemma4H100CompiledLayerFacade = Gemma4MI355XCompiledLayerFacade
Gemma4H100CompiledStaticCacheDecodeFacade = Gemma4MI355XCompiledStaticCacheDecodeFacade
Gemma4H100CompiledLocalStaticCacheDecodeFacade = Gemma4MI355XCompiledLocalStaticCacheDecodeFacade
compile_gemma4_fa4_h100_layer = compile_gemma4_mi355x_layer
compile_gemma4_fa4_h100_static_cache_decode = compile_gemma4_mi355x_static_cache_decode
gemma4_fa4_compile_layer = gemma4_mi355x_compile_layer
