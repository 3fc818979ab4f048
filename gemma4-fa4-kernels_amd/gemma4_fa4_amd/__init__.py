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
)
from .errors import GlobalBackwardBudgetExceeded, UnsupportedH100Path, UnsupportedMI355XPath
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
]
