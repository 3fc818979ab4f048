"""MI355X-native Gemma 4 attention (forward + backward) for gfx950.

A drop-in for the attention hot path of amazingvince/gemma4-fa4-kernels: the
same adapter names, arguments, return contracts and errors as its
``gemma4_fa4`` package (``src/gemma4_fa4/__init__.py``), backed by hand-written
HIP kernels in ``libgemma4_attn.so``.
"""

from .attention import (
    fa4_global_forward_only,
    fa4_global_text_forward,
    fa4_global_varlen_forward,
    fa4_global_varlen_forward_only,
    fa4_local_forward,
    fa4_local_text_forward,
    fa4_local_varlen_forward,
    pin_backward_ds_budget,
)
from . import torch_ops
from .errors import GlobalBackwardBudgetExceeded, UnsupportedH100Path, UnsupportedMI355XPath
from .facades import (
    Gemma4H100CompiledLayerFacade,
    Gemma4H100CompiledLocalStaticCacheDecodeFacade,
    Gemma4H100CompiledStaticCacheDecodeFacade,
    Gemma4MI355XCompiledLayerFacade,
    Gemma4MI355XCompiledLocalStaticCacheDecodeFacade,
    Gemma4MI355XCompiledStaticCacheDecodeFacade,
    compile_gemma4_fa4_h100_layer,
    compile_gemma4_fa4_h100_static_cache_decode,
    compile_gemma4_mi355x_layer,
    compile_gemma4_mi355x_static_cache_decode,
    gemma4_fa4_compile_layer,
    gemma4_mi355x_compile_layer,
)
from .kv_prep import prepare_global_kv_from_projection_source
from .model_spec import (
    GEMMA4_31B,
    GLOBAL_ATTENTION,
    SLIDING_ATTENTION,
    AttentionLayerSpec,
    Gemma4ModelSpec,
)
from .transformers_integration import (
    BACKEND_NAME,
    Gemma4DispatchResult,
    Gemma4MaskPlan,
    gemma4_fa4_attention_forward,
    gemma4_fa4_mask,
    gemma4_fa4_prepared,
    register_gemma4_fa4_h100,
    register_gemma4_mi355x,
)

__all__ = [
    "AttentionLayerSpec",
    "Gemma4ModelSpec",
    "GEMMA4_31B",
    "SLIDING_ATTENTION",
    "GLOBAL_ATTENTION",
    "fa4_local_forward",
    "fa4_local_text_forward",
    "fa4_local_varlen_forward",
    "fa4_global_text_forward",
    "fa4_global_forward_only",
    "fa4_global_varlen_forward",
    "fa4_global_varlen_forward_only",
    "pin_backward_ds_budget",
    "prepare_global_kv_from_projection_source",
    "GlobalBackwardBudgetExceeded",
    "UnsupportedH100Path",
    "UnsupportedMI355XPath",
    "BACKEND_NAME",
    "Gemma4DispatchResult",
    "Gemma4MaskPlan",
    "gemma4_fa4_attention_forward",
    "gemma4_fa4_mask",
    "gemma4_fa4_prepared",
    "register_gemma4_fa4_h100",
    "register_gemma4_mi355x",
    "torch_ops",
    "Gemma4MI355XCompiledLayerFacade",
    "Gemma4MI355XCompiledStaticCacheDecodeFacade",
    "Gemma4MI355XCompiledLocalStaticCacheDecodeFacade",
    "Gemma4H100CompiledLayerFacade",
    "Gemma4H100CompiledStaticCacheDecodeFacade",
    "Gemma4H100CompiledLocalStaticCacheDecodeFacade",
    "compile_gemma4_mi355x_layer",
    "compile_gemma4_mi355x_static_cache_decode",
    "compile_gemma4_fa4_h100_layer",
    "compile_gemma4_fa4_h100_static_cache_decode",
    "gemma4_mi355x_compile_layer",
    "gemma4_fa4_compile_layer",
]
