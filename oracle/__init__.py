"""CPU oracle for the Gemma 4 attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch (CPU, fp64 by default) and Python, the
reference's mask builder, prepared-Q/K/V attention (fixed and packed), explicit
backward, tile-incidence schedule, FLOP model and numerical acceptance
envelopes.  It is the checker the HIP kernels are compared against.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package never imports it and never
falls back to it.

Pinning (what fixes each function independently of this restatement) is
recorded per module header; every function here is pinned by the tests in
``tests/test_oracle_*.py``.
"""

from .masks import gemma4_attention_mask, mask_predicate_scalar
from .attention import (
    attention_fwd_bwd,
    bf16_baseline_fwd_bwd,
    expand_kv,
    reference_attention,
    reference_attention_varlen,
)
from .flops import attention_flops, exact_pair_count, valid_pair_count
from .schedule import build_gemma4_local_sparse_schedule, brute_force_tile_rows
from .envelope import (
    GLOBAL_LSE_ATOL,
    GLOBAL_OUT_ATOL,
    GLOBAL_OUT_RTOL,
    LOCAL_LSE_ATOL,
    LOCAL_OUT_ATOL,
    LOCAL_OUT_RTOL,
    gradient_limit,
    rel_frobenius,
)

__all__ = [
    "gemma4_attention_mask",
    "mask_predicate_scalar",
    "attention_fwd_bwd",
    "bf16_baseline_fwd_bwd",
    "expand_kv",
    "reference_attention",
    "reference_attention_varlen",
    "attention_flops",
    "exact_pair_count",
    "valid_pair_count",
    "build_gemma4_local_sparse_schedule",
    "brute_force_tile_rows",
    "GLOBAL_LSE_ATOL",
    "GLOBAL_OUT_ATOL",
    "GLOBAL_OUT_RTOL",
    "LOCAL_LSE_ATOL",
    "LOCAL_OUT_ATOL",
    "LOCAL_OUT_RTOL",
    "gradient_limit",
    "rel_frobenius",
]
