"""Host tests of the Transformers backend: registration, exact mask admission, routing.

Modelled on the reference's tests/test_transformers_integration.py (registration
1782-1800, fail-closed admission 144-253, routing 254-1120).  The native
adapters are replaced by CPU stand-ins that run the oracle on the packed or
fixed inputs they receive, so packing, segmentation and unpacking are checked
end to end against a dense evaluation of the Transformers mask callable
itself; the kernels are covered by the GPU tests.
"""

from __future__ import annotations

import types

import pytest
import torch

from gemma4_fa4_amd import transformers_integration as ti
from gemma4_fa4_amd.errors import UnsupportedH100Path, UnsupportedMI355XPath
from gemma4_fa4_amd.model_spec import GEMMA4_31B
from oracle.attention import expand_kv, reference_attention, reference_attention_varlen

mu = pytest.importorskip("transformers.masking_utils")

LOCAL_LAYER, GLOBAL_LAYER = 0, 5


def _module(layer_idx):
    spec = GEMMA4_31B.spec_for_layer(layer_idx)
    return types.SimpleNamespace(
        layer_idx=layer_idx, scaling=1.0, head_dim=spec.head_dim_qk,
        num_key_value_groups=spec.qhead_per_kvhead, sliding_window=spec.sliding_window,
    )


def _bhsd(layer_idx, b, sq, sk, seed=0, grad=False):
    spec = GEMMA4_31B.spec_for_layer(layer_idx)
    g = torch.Generator().manual_seed(seed)
    scale = spec.head_dim_qk ** -0.25
    q = (torch.randn(b, spec.num_q_heads, sq, spec.head_dim_qk, generator=g) * scale).bfloat16()
    k = (torch.randn(b, spec.num_kv_heads, sk, spec.head_dim_qk, generator=g) * scale).bfloat16()
    v = torch.randn(b, spec.num_kv_heads, sk, spec.head_dim_v, generator=g).bfloat16()
    if grad:
        q, k, v = (t.requires_grad_() for t in (q, k, v))
    return q, k, v


def _kwargs(layer_idx, **extra):
    return dict(dropout=0.0, scaling=1.0,
                sliding_window=GEMMA4_31B.spec_for_layer(layer_idx).sliding_window, **extra)


class _Calls(list):
    pass


@pytest.fixture
def native(monkeypatch):
    """Replace the adapters with oracle-backed CPU stand-ins that record calls."""
    calls = _Calls()

    def fixed(window, bidir):
        def run(q, k, v, *, vision_block_ids=None, spec=None):
            calls.append(("fixed", window, q.shape, None if vision_block_ids is None else vision_block_ids.clone()))
            o, lse = reference_attention(
                q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), sliding_window=window,
                vision_block_ids=vision_block_ids, allow_vision_bidirectional=bidir,
                q_start=k.shape[1] - q.shape[1], upcast=torch.float32, return_lse=True,
            )
            return o.transpose(1, 2), lse
        return run

    def varlen(window, name):
        def run(q, k, v, cu_q, cu_k, *, max_seqlen_q, max_seqlen_k, vision_block_ids=None,
                document_ids=None, spec=None):
            calls.append((name, cu_q.tolist(), cu_k.tolist(), max_seqlen_q, max_seqlen_k,
                          None if vision_block_ids is None else vision_block_ids.tolist(),
                          None if document_ids is None else document_ids.tolist()))
            return reference_attention_varlen(
                q, k, v, cu_q, cu_k, sliding_window=window, vision_block_ids=vision_block_ids,
                document_ids=document_ids, allow_vision_bidirectional=True,
                upcast=torch.float32, return_lse=True,
            )
        return run

    monkeypatch.setattr(ti, "fa4_local_forward", fixed(1024, True))
    monkeypatch.setattr(ti, "fa4_global_text_forward", lambda q, k, v, spec=None: (
        calls.append(("global_fixed", q.shape)), fixed(None, False)(q, k, v))[1])
    monkeypatch.setattr(ti, "fa4_global_forward_only", lambda q, k, v, spec=None: (
        calls.append(("global_forward_only", q.shape)), fixed(None, False)(q, k, v))[1])
    monkeypatch.setattr(ti, "fa4_local_varlen_forward", varlen(1024, "local_varlen"))
    monkeypatch.setattr(ti, "fa4_global_varlen_forward", varlen(None, "global_varlen"))
    monkeypatch.setattr(ti, "fa4_global_varlen_forward_only", varlen(None, "global_varlen_fwd_only"))
    return calls


def _dense_expected(q, k, v, allowed):
    """BHSD fp32 attention under an explicit (B, Sq, Sk) boolean mask."""
    hq, hkv = q.shape[1], k.shape[1]
    qf, kf, vf = q.float(), expand_kv(k.float(), hq // hkv), expand_kv(v.float(), hq // hkv)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous())
    s = s.masked_fill(~allowed[:, None], float("-inf"))
    lse = torch.logsumexp(s, -1)
    p = torch.where(torch.isfinite(lse)[..., None], torch.exp(s - lse[..., None]), torch.zeros_like(s))
    return torch.matmul(p, vf).transpose(1, 2), lse


def _hf_allowed(plan: ti.Gemma4MaskPlan):
    """Dense evaluation of the plan's Transformers callable, with its padding."""
    b = torch.arange(plan.batch_size)[:, None, None]
    qi = torch.arange(plan.q_length)[None, :, None] + int(plan.q_offset)
    ki = torch.arange(plan.kv_length)[None, None, :] + int(plan.kv_offset)
    allowed = torch.as_tensor(plan.mask_function(b, torch.zeros_like(b), qi, ki)).expand(
        plan.batch_size, plan.q_length, plan.kv_length).clone()
    if plan.attention_mask is not None:
        off = int(plan.kv_offset)
        allowed &= plan.attention_mask.bool()[:, None, off: off + plan.kv_length]
    return allowed


def _check_against_dense(result, q, k, v, allowed, valid_q=None):
    exp_o, exp_lse = _dense_expected(q, k, v, allowed)
    out, lse = result.output.float(), result.lse
    if valid_q is not None:
        assert torch.all(out[~valid_q] == 0)
        assert torch.all(torch.isneginf(lse.permute(0, 2, 1)[~valid_q]))
        out, exp_o = out[valid_q], exp_o[valid_q]
        lse, exp_lse = lse.permute(0, 2, 1)[valid_q], exp_lse.permute(0, 2, 1)[valid_q]
    assert torch.allclose(out, exp_o, atol=2e-2, rtol=2e-2)
    assert torch.allclose(lse, exp_lse, atol=1e-3)


def _config(sliding_window=1024):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig

    ti.register_gemma4_mi355x()
    cfg = Gemma4TextConfig(sliding_window=sliding_window)
    cfg._attn_implementation = ti.BACKEND_NAME
    return cfg


def _hf_masks(b, s, *, attention_mask=None, position_ids=None, vision=None, window=1024):
    cfg = _config(window)
    kw = dict(config=cfg, inputs_embeds=torch.zeros(b, s, 8), attention_mask=attention_mask,
              past_key_values=None, position_ids=position_ids)
    if vision is not None:
        from transformers.models.gemma4 import modeling_gemma4 as mg

        masks = mg.create_masks_for_vision_model(block_sequence_ids=vision, **kw)
        return masks["sliding_attention"], masks["full_attention"]
    return mu.create_sliding_window_causal_mask(**kw), mu.create_causal_mask(**kw)


# ----------------------------------------------------------------------------
# Types and registration
# ----------------------------------------------------------------------------


def test_public_contract_types_are_stable():
    assert [f for f in ti.Gemma4MaskPlan.__dataclass_fields__] == [
        "batch_size", "q_length", "kv_length", "q_offset", "kv_offset", "mask_function",
        "attention_mask",
    ]
    assert [f for f in ti.Gemma4DispatchResult.__dataclass_fields__] == ["output", "lse", "path"]
    assert ti.BACKEND_NAME == "gemma4_mi355x"
    assert ti.register_gemma4_fa4_h100 is ti.register_gemma4_mi355x
    assert issubclass(UnsupportedMI355XPath, RuntimeError) and UnsupportedH100Path is UnsupportedMI355XPath


def test_mask_callback_keeps_callable_padding_and_snapshots_offsets():
    pad = torch.tensor([[0, 1, 1]])
    counter = torch.tensor(5)
    plan = ti.gemma4_fa4_mask(1, 3, 3, q_offset=counter, kv_offset=0,
                              mask_function=mu.causal_mask_function, attention_mask=pad,
                              config=None, use_vmap=True, allow_is_causal_skip=False, dtype=None)
    counter += 1
    assert plan.mask_function is mu.causal_mask_function and plan.attention_mask is pad
    assert int(plan.q_offset) == 5


class _Registry(dict):
    def register(self, key, value):
        self[key] = value


def test_registration_is_idempotent_and_pairs_attention_with_mask():
    att, mask = _Registry(), _Registry()
    assert ti.register_gemma4_mi355x(att, mask) == ti.BACKEND_NAME
    assert ti.register_gemma4_mi355x(att, mask) == ti.BACKEND_NAME
    assert att[ti.BACKEND_NAME] is ti.gemma4_fa4_attention_forward
    assert mask[ti.BACKEND_NAME] is ti.gemma4_fa4_mask


@pytest.mark.parametrize("collision", ["attention", "mask"])
def test_registration_rejects_an_existing_different_backend(collision):
    att, mask = _Registry(), _Registry()
    (att if collision == "attention" else mask)[ti.BACKEND_NAME] = lambda *a, **k: None
    with pytest.raises(RuntimeError, match="already registered"):
        ti.register_gemma4_mi355x(att, mask)
    # Nothing is half-registered.
    assert len(att) + len(mask) == 1


def test_transformers_mask_creation_returns_plans_under_the_backend_name():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    sliding, full = _hf_masks(1, 8)
    assert isinstance(sliding, ti.Gemma4MaskPlan) and isinstance(full, ti.Gemma4MaskPlan)
    assert ALL_ATTENTION_FUNCTIONS[ti.BACKEND_NAME] is ti.gemma4_fa4_attention_forward
    assert mu.ALL_MASK_ATTENTION_FUNCTIONS[ti.BACKEND_NAME] is ti.gemma4_fa4_mask


# ----------------------------------------------------------------------------
# Structural recognition
# ----------------------------------------------------------------------------


def _term(fn):
    return ti._Recognizer(mu).term(fn)


def test_recognizer_canonicalises_the_gemma_compositions():
    sliding, full = _hf_masks(1, 16)
    assert _term(full.mask_function) == ti._expected_term(GEMMA4_31B.full, vision=False, packed=False)
    assert _term(sliding.mask_function) == ti._expected_term(GEMMA4_31B.sliding, vision=False, packed=False)
    vis = torch.tensor([[-1, 0, 0, 0, -1, 1, 1, -1] * 2])
    sliding_v, full_v = _hf_masks(1, 16, vision=vis)
    assert _term(sliding_v.mask_function) == ti._expected_term(GEMMA4_31B.sliding, vision=True, packed=False)
    assert _term(full_v.mask_function) == ti._expected_term(GEMMA4_31B.full, vision=False, packed=False)
    pos = torch.cat([torch.arange(10), torch.arange(6)])[None]
    sliding_p, _ = _hf_masks(1, 16, position_ids=pos)
    assert _term(sliding_p.mask_function) == ti._expected_term(GEMMA4_31B.sliding, vision=False, packed=True)


@pytest.mark.parametrize(
    "fn",
    [
        # Vision outside the window: OR(AND(window, causal), vision) is a different predicate.
        mu.or_masks(mu.sliding_window_causal_mask_function(1024), mu.blockwise_overlay(torch.zeros(1, 8, dtype=torch.long))),
        mu.sliding_window_causal_mask_function(512),
        mu.bidirectional_mask_function,
        mu.and_masks(mu.causal_mask_function, mu.sliding_window_bidirectional_overlay(1024)),
        lambda b, h, q, k: k <= q,
    ],
    ids=["vision-escapes-window", "wrong-window", "bidirectional", "bidirectional-window", "foreign-callable"],
)
def test_non_native_compositions_are_not_structurally_admitted(fn):
    plan = ti.Gemma4MaskPlan(1, 8, 8, 0, 0, fn, None)
    assert ti._structural_proof(plan, GEMMA4_31B.sliding, device=torch.device("cpu"), vision=None) is None


def test_forged_function_metadata_is_not_recognised():
    def inner_mask(batch_idx, head_idx, q_idx, kv_idx):
        return kv_idx <= q_idx

    inner_mask.__module__ = "transformers.masking_utils"
    inner_mask.__qualname__ = "causal_mask_function"
    assert _term(inner_mask) is None
    forged = types.FunctionType(mu.causal_mask_function.__code__, {}, "causal_mask_function")
    assert _term(forged) is None  # same code, foreign globals


# ----------------------------------------------------------------------------
# Routing with exact results (oracle-backed stand-ins)
# ----------------------------------------------------------------------------


def test_sixty_layer_pattern_routes_fifty_local_and_ten_global(native):
    local = [i for i in range(60) if GEMMA4_31B.spec_for_layer(i).kind == "sliding_attention"]
    assert len(local) == 50
    for layer in (0, 5, 11, 59):
        q, k, v = _bhsd(layer, 1, 4, 4)
        res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, None, **_kwargs(layer))
        assert res.path == ("fa4_local_fixed" if layer in local else "fa4_global_fixed")


def test_attention_interface_returns_bshd_and_no_weights(native):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 6, 6)
    mod = _module(LOCAL_LAYER)
    out, weights = ti.gemma4_fa4_attention_forward(mod, q, k, v, None, **_kwargs(LOCAL_LAYER))
    assert weights is None and out.shape == (1, 6, 32, 256) and out.dtype == torch.bfloat16
    assert mod._gemma4_fa4_last_path == "fa4_local_fixed"


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER])
def test_hf_text_masks_route_natively_and_match_the_dense_mask(native, layer):
    sliding, full = _hf_masks(1, 24)
    plan = sliding if layer == LOCAL_LAYER else full
    q, k, v = _bhsd(layer, 1, 24, 24, seed=1)
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kwargs(layer))
    assert res.path == ("fa4_local_fixed" if layer == LOCAL_LAYER else "fa4_global_fixed")
    _check_against_dense(res, q, k, v, _hf_allowed(plan))


def test_hf_vision_mask_forwards_the_captured_vision_ids(native):
    vis = torch.tensor([[-1, -1, 0, 0, 0, 0, -1, 1, 1, 1, -1, -1, 2, 2, -1, -1]])
    sliding, full = _hf_masks(1, 16, vision=vis)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 16, 16, seed=2)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_fixed" and native[-1][3].tolist() == vis.tolist()
    _check_against_dense(res, q, k, v, _hf_allowed(sliding))
    # Global layers of the same model ignore vision (causal only).
    qg, kg, vg = _bhsd(GLOBAL_LAYER, 1, 16, 16, seed=2)
    res = ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), qg, kg, vg, full, **_kwargs(GLOBAL_LAYER),
                                 vision_block_ids=vis)
    assert res.path == "fa4_global_fixed"
    _check_against_dense(res, qg, kg, vg, _hf_allowed(full))


def test_conflicting_explicit_vision_ids_fail_closed(native):
    vis = torch.tensor([[-1, 0, 0, 0, -1, -1, -1, -1]])
    sliding, _ = _hf_masks(1, 8, vision=vis)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    other = torch.tensor([[-1, -1, 0, 0, 0, -1, -1, -1]])
    with pytest.raises(UnsupportedMI355XPath):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, vision_block_ids=other,
                               **_kwargs(LOCAL_LAYER))
    assert not native


def test_vision_metadata_without_a_bidirectional_mask_fails_closed(native):
    sliding, _ = _hf_masks(1, 8)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    with pytest.raises(UnsupportedMI355XPath):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding,
                               vision_block_ids=torch.tensor([[-1, 0, 0, -1, -1, -1, -1, -1]]),
                               **_kwargs(LOCAL_LAYER))


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER])
def test_position_id_packing_derives_segments(native, layer):
    pos = torch.cat([torch.arange(7), torch.arange(5), torch.arange(4)])[None]
    sliding, full = _hf_masks(1, 16, position_ids=pos)
    plan = sliding if layer == LOCAL_LAYER else full
    q, k, v = _bhsd(layer, 1, 16, 16, seed=3)
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, position_ids=pos, **_kwargs(layer))
    assert native[-1][1] == [0, 7, 12, 16] and native[-1][3] == 7
    _check_against_dense(res, q, k, v, _hf_allowed(plan))


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER])
def test_padding_packs_valid_tokens_and_scatters_zero_rows(native, layer):
    pad = torch.ones(2, 12, dtype=torch.long)
    pad[0, :4] = 0  # left padding
    pad[1, 9:] = 0  # right padding
    sliding, full = _hf_masks(2, 12, attention_mask=pad)
    plan = sliding if layer == LOCAL_LAYER else full
    q, k, v = _bhsd(layer, 2, 12, 12, seed=4)
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kwargs(layer))
    assert res.path in ("fa4_local_varlen", "fa4_global_varlen_forward_only")
    assert native[-1][1] == [0, 8, 17]
    _check_against_dense(res, q, k, v, _hf_allowed(plan), valid_q=pad.bool())


def test_holey_padding_fails_closed(native):
    pad = torch.ones(1, 8, dtype=torch.long)
    pad[0, 3] = 0
    sliding, _ = _hf_masks(1, 8, attention_mask=pad)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    with pytest.raises(UnsupportedMI355XPath, match="holey"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, **_kwargs(LOCAL_LAYER))


def test_batch_rows_become_segments_and_explicit_cu_cannot_cross_rows(native):
    q, k, v = _bhsd(LOCAL_LAYER, 2, 6, 6, seed=5)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, None, **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen" and native[-1][1] == [0, 6, 12]
    cu = torch.tensor([0, 3, 6, 12], dtype=torch.int32)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, None, cu_seq_lens_q=cu,
                                 cu_seq_lens_k=cu.clone(), **_kwargs(LOCAL_LAYER))
    assert native[-1][1] == [0, 3, 6, 12]
    bad = torch.tensor([0, 4, 12], dtype=torch.int32)
    with pytest.raises(ValueError, match="batch-row boundary"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, None, cu_seq_lens_q=bad,
                               cu_seq_lens_k=bad.clone(), **_kwargs(LOCAL_LAYER))


def test_explicit_cu_must_match_a_recognised_packed_mask(native):
    pos = torch.cat([torch.arange(5), torch.arange(3)])[None]
    sliding, _ = _hf_masks(1, 8, position_ids=pos)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    good = torch.tensor([0, 5, 8], dtype=torch.int32)
    ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, cu_seq_lens_q=good,
                           cu_seq_lens_k=good.clone(), **_kwargs(LOCAL_LAYER))
    bad = torch.tensor([0, 4, 8], dtype=torch.int32)
    with pytest.raises(ValueError, match="conflicts"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, cu_seq_lens_q=bad,
                               cu_seq_lens_k=bad.clone(), **_kwargs(LOCAL_LAYER))


def test_lower_right_query_suffix_routes_varlen_with_the_kv_offset(native):
    # Chunked prefill against a longer K: q positions 10..15 over k 0..15.
    plan = ti.gemma4_fa4_mask(1, 6, 16, q_offset=10, kv_offset=0,
                              mask_function=mu.sliding_window_causal_mask_function(1024))
    q, k, v = _bhsd(LOCAL_LAYER, 1, 6, 16, seed=6)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen" and native[-1][1:3] == ([0, 6], [0, 16])
    _check_against_dense(res, q, k, v, _hf_allowed(plan))


def test_non_lower_right_offsets_fail_closed(native):
    # Queries past the physical K (no lower-right alignment, not a cache
    # prefix), and an under-filled K with gradients (the StaticCache prefix
    # normalisation is inference-only), both fail closed before any launch.
    fn = mu.sliding_window_causal_mask_function(1024)
    plan = ti.gemma4_fa4_mask(1, 6, 16, q_offset=12, kv_offset=0, mask_function=fn)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 6, 16)
    with pytest.raises(UnsupportedMI355XPath, match="outside the physical K/V backing"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    plan = ti.gemma4_fa4_mask(1, 6, 16, q_offset=4, kv_offset=0, mask_function=fn)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 6, 16, grad=True)
    with pytest.raises(UnsupportedMI355XPath, match="inference-only"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert not native


# ----------------------------------------------------------------------------
# Eager StaticCache active prefix (reference tests/test_transformers_integration.py:1180-1465)
# ----------------------------------------------------------------------------


@pytest.fixture
def received(native, monkeypatch):
    """The Q/K/V tensors each (stand-in) adapter receives, in call order."""
    seen = []
    for name in ("fa4_local_forward", "fa4_global_text_forward", "fa4_global_forward_only",
                 "fa4_local_varlen_forward", "fa4_global_varlen_forward",
                 "fa4_global_varlen_forward_only"):
        inner = getattr(ti, name)

        def wrap(*args, _inner=inner, _name=name, **kwargs):
            seen.append((_name, args[:3]))
            return _inner(*args, **kwargs)

        monkeypatch.setattr(ti, name, wrap)
    return seen


def _static_cache(layer, *, sq=2, physical=8, q_offset=3, style="short", callable_=False,
                  seed=21):
    # Under-filled StaticCache: queries at q_offset .. q_offset + sq - 1 over
    # a physical backing whose keys past them were never written (filled here
    # with hostile values that must not reach the kernels).
    q, k, v = _bhsd(layer, 1, sq, physical, seed=seed)
    active = q_offset + sq
    k[:, :, active:] = 127
    v[:, :, active:] = -91
    mask = {
        "short": torch.ones((1, active), dtype=torch.int32),
        "physical-zero-tail": torch.tensor([[1] * active + [0] * (physical - active)],
                                           dtype=torch.int32),
        "physical-all-ones": torch.ones((1, physical), dtype=torch.int32),
    }[style]
    fn = None
    if callable_:
        fn = (mu.sliding_window_causal_mask_function(1024) if layer == LOCAL_LAYER
              else mu.causal_mask_function)
    plan = ti.gemma4_fa4_mask(1, sq, physical,
                              q_offset=torch.tensor(q_offset) if layer == GLOBAL_LAYER else q_offset,
                              kv_offset=0, mask_function=fn, attention_mask=mask)
    return q, k, v, plan, active


def _causal_allowed(sq, sk, q_offset, window=None):
    qi = torch.arange(sq)[:, None] + q_offset
    ki = torch.arange(sk)[None, :]
    allowed = ki <= qi
    if window:
        allowed &= ki > qi - window
    return allowed[None]


@pytest.mark.parametrize("callable_", [False, True], ids=["native-plan", "hf-callable"])
@pytest.mark.parametrize("style", ["short", "physical-zero-tail", "physical-all-ones"])
@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER], ids=["local", "global"])
def test_static_cache_underfilled_prefix_routes_trimmed_views(native, received, layer, style,
                                                             callable_):
    q, k, v, plan, active = _static_cache(layer, style=style, callable_=callable_)
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kwargs(layer))
    name, (q_arg, k_arg, v_arg) = received[-1]
    assert name == ("fa4_local_varlen_forward" if layer == LOCAL_LAYER
                    else "fa4_global_varlen_forward_only")
    # only the active prefix, as views of the cache's own storage
    for phys, arg in ((k, k_arg), (v, v_arg)):
        expected = phys[:, :, :active].transpose(1, 2)[0]
        assert arg.shape == expected.shape and arg.stride() == expected.stride()
        assert arg.storage_offset() == expected.storage_offset()
        assert arg.untyped_storage().data_ptr() == phys.untyped_storage().data_ptr()
    assert q_arg.untyped_storage().data_ptr() == q.untyped_storage().data_ptr()
    assert native[-1][1:5] == ([0, 2], [0, active], 2, active)
    window = 1024 if layer == LOCAL_LAYER else None
    _check_against_dense(res, q, k[:, :, :active], v[:, :, :active],
                         _causal_allowed(2, active, 3, window))
    assert res.output.shape == (1, 2, q.shape[1], q.shape[-1]) and res.lse.shape == (1, q.shape[1], 2)


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER], ids=["local", "global"])
def test_static_cache_hostile_unwritten_tail_is_absent(native, layer):
    q, k, v, plan, active = _static_cache(layer)
    first = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kwargs(layer))
    k[:, :, active:] = -63
    v[:, :, active:] = 119
    second = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kwargs(layer))
    assert torch.equal(first.output, second.output) and torch.equal(first.lse, second.lse)


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER], ids=["local", "global"])
def test_static_cache_trim_does_not_read_position_resets_as_packing(native, layer):
    # The trimmed call has Sq == Sk; with a cache present, position_ids
    # restarts are not sequence boundaries (ti.py:1831-1835).
    q, k, v = _bhsd(layer, 1, 5, 8, seed=22)
    plan = ti.gemma4_fa4_mask(1, 5, 8, q_offset=0, kv_offset=0,
                              attention_mask=torch.ones((1, 8), dtype=torch.int32))
    pos = torch.tensor([[0, 1, 0, 1, 2]])
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, position_ids=pos, **_kwargs(layer))
    assert res.path == ("fa4_local_fixed" if layer == LOCAL_LAYER else "fa4_global_fixed")
    window = 1024 if layer == LOCAL_LAYER else None
    _check_against_dense(res, q, k[:, :, :5], v[:, :, :5], _causal_allowed(5, 5, 0, window))


def test_static_cache_all_negative_vision_metadata_is_text_only(native):
    q, k, v, plan, _active = _static_cache(LOCAL_LAYER)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan,
                                 vision_block_ids=torch.full((1, 8), -1, dtype=torch.int32),
                                 **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen" and native[-1][5] is None


@pytest.mark.parametrize(("extra", "grad", "batch", "error"), [
    ({"vision_block_ids": torch.tensor([[0, -1, -1, -1, -1, -1, -1, -1]])}, False, 1,
     "text-only vision metadata"),
    ({"document_ids": torch.zeros((1, 8), dtype=torch.int32)}, False, 1, "document metadata"),
    ({"cu_seq_lens_q": torch.tensor([0, 2], dtype=torch.int32),
      "cu_seq_lens_k": torch.tensor([0, 5], dtype=torch.int32)}, False, 1,
     "explicit packed lengths"),
    ({}, True, 1, "inference-only"),
    ({}, False, 2, "B1 only"),
], ids=["active-vision", "documents", "explicit-cu", "grad", "batch2"])
def test_static_cache_underfilled_prefix_outside_the_contract_fails_closed(native, extra, grad,
                                                                          batch, error):
    q, k, v = _bhsd(LOCAL_LAYER, batch, 2, 8, grad=grad)
    plan = ti.gemma4_fa4_mask(batch, 2, 8, q_offset=3, kv_offset=0,
                              attention_mask=torch.ones((batch, 8), dtype=torch.int32))
    with pytest.raises(UnsupportedMI355XPath, match=error):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER), **extra)
    assert not native


def test_static_cache_underfilled_prefix_rejects_nonzero_kv_offset(native):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 2, 8)
    plan = ti.gemma4_fa4_mask(1, 2, 8, q_offset=4, kv_offset=1,
                              attention_mask=torch.ones((1, 9), dtype=torch.int32))
    with pytest.raises(UnsupportedMI355XPath, match="physical K offset zero"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert not native


def test_static_cache_prefix_needs_a_contiguous_valid_prefix(native):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 2, 8)
    plan = ti.gemma4_fa4_mask(1, 2, 8, q_offset=3, kv_offset=0,
                              attention_mask=torch.tensor([[1, 1, 0, 1, 1, 0, 0, 0]]))
    with pytest.raises(UnsupportedMI355XPath, match="contiguous valid K prefix"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert not native


def test_static_cache_trim_needs_the_callable_to_mask_the_tail(native):
    # A callable that is not the native predicate and admits a trimmed key
    # (here: everything) must not be trimmed, whatever it does elsewhere.
    q, k, v = _bhsd(LOCAL_LAYER, 1, 2, 8)
    plan = ti.gemma4_fa4_mask(1, 2, 8, q_offset=3, kv_offset=0,
                              mask_function=lambda b, h, qi, ki: torch.ones_like(qi * ki, dtype=torch.bool))
    with pytest.raises(UnsupportedMI355XPath, match="past the eager StaticCache active prefix"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert not native


def test_static_cache_rolled_local_window_keeps_the_full_physical_view(native):
    # A full sliding cache (kv_offset 1 after one roll): the active length is
    # the physical length, so nothing is trimmed.
    q, k, v = _bhsd(LOCAL_LAYER, 1, 1, 1024, seed=23)
    plan = ti.gemma4_fa4_mask(1, 1, 1024, q_offset=1024, kv_offset=1,
                              attention_mask=torch.ones((1, 1025), dtype=torch.int32))
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen" and native[-1][1:5] == ([0, 1], [0, 1024], 1, 1024)


def test_long_global_routes(native):
    # B=1 no-grad above 1024 keys: forward-only fixed route.
    q, k, v = _bhsd(GLOBAL_LAYER, 1, 2, 1030)
    res = ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None, **_kwargs(GLOBAL_LAYER))
    assert res.path == "fa4_global_forward_only"
    # Grad with S <= 2048 takes the fixed autograd route; packed rows take varlen.
    q, k, v = _bhsd(GLOBAL_LAYER, 1, 8, 8, grad=True)
    assert ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None,
                                  **_kwargs(GLOBAL_LAYER)).path == "fa4_global_fixed"
    q, k, v = _bhsd(GLOBAL_LAYER, 2, 8, 8, grad=True)
    res = ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None, **_kwargs(GLOBAL_LAYER))
    assert res.path == "fa4_global_varlen_native"


def test_gradients_flow_through_packing(native):
    pad = torch.ones(2, 6, dtype=torch.long)
    pad[1, :2] = 0
    sliding, _ = _hf_masks(2, 6, attention_mask=pad)
    q, k, v = _bhsd(LOCAL_LAYER, 2, 6, 6, seed=7, grad=True)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, **_kwargs(LOCAL_LAYER))
    res.output.float().sum().backward()
    assert q.grad is not None and torch.all(q.grad[1, :, :2] == 0)
    assert k.grad is not None and v.grad is not None


def test_global_documents_split_segments_and_repeats_fail_closed(native):
    docs = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2]])
    q, k, v = _bhsd(GLOBAL_LAYER, 1, 8, 8, seed=8)
    res = ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None, document_ids=docs,
                                 **_kwargs(GLOBAL_LAYER))
    assert native[-1][1] == [0, 3, 5, 8]
    allowed = torch.tril(torch.ones(8, 8, dtype=torch.bool)) & (docs[0][:, None] == docs[0][None, :])
    _check_against_dense(res, q, k, v, allowed[None])
    with pytest.raises(UnsupportedMI355XPath, match="reappears"):
        ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None,
                               document_ids=torch.tensor([[0, 0, 1, 1, 0, 0, 2, 2]]),
                               **_kwargs(GLOBAL_LAYER))


def test_local_documents_reach_the_kernel_predicate(native):
    docs = torch.tensor([[0, 0, 1, 1, 0, 0, 2, 2]])
    vis = torch.tensor([[-1, 0, 0, -1, 0, -1, -1, -1]])
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8, seed=9)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, None, document_ids=docs,
                                 vision_block_ids=vis, **_kwargs(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen"
    assert native[-1][6] == docs[0].tolist() and native[-1][5] == vis[0].tolist()
    from oracle.masks import gemma4_attention_mask

    allowed = torch.as_tensor(gemma4_attention_mask(
        batch_size=1, q_len=8, kv_len=8, sliding_window=1024, vision_block_ids=vis,
        document_ids=docs, allow_vision_bidirectional=True))[:, 0]
    _check_against_dense(res, q, k, v, allowed)


def test_documents_inside_a_recognised_mask_segment_fail_closed(native):
    sliding, _ = _hf_masks(1, 8)
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    with pytest.raises(UnsupportedMI355XPath, match="document"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding,
                               document_ids=torch.tensor([[0, 0, 0, 0, 1, 1, 1, 1]]),
                               **_kwargs(LOCAL_LAYER))


def test_unrecognised_callables_and_4d_masks_fail_closed_on_the_host(native):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 8, 8)
    plan = ti.gemma4_fa4_mask(1, 8, 8, mask_function=lambda b, h, qi, ki: ki <= qi)
    with pytest.raises(UnsupportedMI355XPath, match="not provably"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kwargs(LOCAL_LAYER))
    with pytest.raises(UnsupportedMI355XPath, match="4D"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, torch.zeros(1, 1, 8, 8),
                               **_kwargs(LOCAL_LAYER))
    assert not native


@pytest.mark.parametrize(
    "kwargs, error",
    [
        (dict(scaling=0.5), ValueError),
        (dict(dropout=0.1), ValueError),
        (dict(output_attentions=True), UnsupportedMI355XPath),
        (dict(sliding_window=512), ValueError),
    ],
)
def test_invalid_attention_semantics_reject_before_dispatch(native, kwargs, error):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 4, 4)
    base = _kwargs(LOCAL_LAYER)
    base.update(kwargs)
    with pytest.raises(error):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, None, **base)
    assert not native


def test_prepared_operand_contract(native):
    q, k, v = _bhsd(LOCAL_LAYER, 1, 4, 4)
    with pytest.raises(ValueError, match="distinct"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, k, None, **_kwargs(LOCAL_LAYER))
    with pytest.raises(ValueError, match="unit last-dimension"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q.transpose(2, 3), k, v, None,
                               **_kwargs(LOCAL_LAYER))
    with pytest.raises(ValueError, match="geometry"):
        ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, None, **_kwargs(GLOBAL_LAYER))
    with pytest.raises(IndexError):
        ti.gemma4_fa4_prepared(types.SimpleNamespace(layer_idx=60), q, k, v, None, **_kwargs(0))
    with pytest.raises(ValueError, match="layer_idx"):
        ti.gemma4_fa4_prepared(types.SimpleNamespace(layer_idx=True), q, k, v, None, **_kwargs(0))
