"""Host contract of the opaque custom operators and the compile route (CPU).

Mirrors the reference's operator tests (tests/test_h100_torch_ops.py:88-330)
where they run without a GPU: operator names and mutation annotations, the
tensor-explicit argument lists, fake (meta) registrations that allocate fresh
outputs and never enter a kernel, a fake trace that holds one opaque node,
explicit failure of real execution off the GPU, the inference-only wrappers,
and the Transformers compile / FakeTensor admission route
(src/gemma4_fa4/transformers_integration.py:761-921).
"""

from __future__ import annotations

import inspect
import types

import pytest
import torch

import gemma4_fa4_amd as g
from gemma4_fa4_amd import torch_ops
from gemma4_fa4_amd import transformers_integration as ti
from gemma4_fa4_amd.errors import UnsupportedMI355XPath

FakeTensorMode = pytest.importorskip("torch._subclasses.fake_tensor").FakeTensorMode


def _prepared(family, s, device, dtype=torch.bfloat16):
    hkv, d = (16, 256) if family == "local" else (4, 512)
    q = torch.empty(1, 32, s, d, dtype=dtype, device=device)
    k = torch.empty(1, hkv, s, d, dtype=dtype, device=device)
    v = torch.empty(1, hkv, s, d, dtype=dtype, device=device)
    pos = torch.arange(s, device=device).unsqueeze(0) if device == "cpu" else \
        torch.empty(1, s, dtype=torch.int64, device=device)
    packed = torch.zeros(1, s, dtype=torch.int64, device=device)
    return q, k, v, pos, packed


def _layer_inputs(family, s, device):
    d, hkv = (256, 16) if family == "local" else (512, 4)
    bf = dict(dtype=torch.bfloat16, device=device)
    out = [torch.empty(1, s, 5376, **bf), torch.empty(1, s, d, **bf), torch.empty(1, s, d, **bf),
           torch.empty(1, s, dtype=torch.int64, device=device),
           torch.empty(1, s, dtype=torch.int64, device=device),
           torch.empty(32 * d, 5376, **bf), torch.empty(hkv * d, 5376, **bf)]
    if family == "local":
        out.append(torch.empty(hkv * d, 5376, **bf))
    out += [torch.empty(5376, 32 * d, **bf), torch.empty(d, **bf), torch.empty(d, **bf)]
    return out


def test_custom_operators_are_registered_with_their_mutations():
    assert torch_ops.CUSTOM_OPS_AVAILABLE
    names = {
        torch_ops.local_fwd: "local_fwd", torch_ops.global_fwd: "global_fwd",
        torch_ops.local_layer_op: "local_layer_fwd", torch_ops.global_layer_op: "global_layer_fwd",
        torch_ops.global_static_cache_decode_op: "global_static_cache_decode_fwd",
        torch_ops.local_static_cache_decode_op: "local_static_cache_decode_fwd",
    }
    for op, name in names.items():
        assert str(op).endswith(f"gemma4_mi355x::{name})>")
        assert hasattr(torch.ops.gemma4_mi355x, name)
    glob = str(torch_ops.global_static_cache_decode_op._schema)
    assert "Tensor(a4!) cache_k" in glob and "Tensor(a5!) cache_v" in glob
    assert "Tensor(a6!) cache_length" in glob
    loc = str(torch_ops.local_static_cache_decode_op._schema)
    assert "Tensor(a4!) cache_k" in loc and "Tensor(a5!) cache_v" in loc
    assert "Tensor cache_length" in loc and "Tensor(a6!) cache_length" not in loc
    for op in (torch_ops.local_fwd, torch_ops.global_fwd, torch_ops.local_layer_op,
               torch_ops.global_layer_op):
        assert "!" not in str(op._schema)
    # the reference's Python names are the same objects
    assert torch_ops.h100_local_fwd is torch_ops.local_fwd
    assert torch_ops.h100_global_static_cache_decode_op is torch_ops.global_static_cache_decode_op
    assert g.compile_gemma4_fa4_h100_layer is g.compile_gemma4_mi355x_layer


def test_whole_layer_and_decode_abis_are_tensor_explicit():
    common = ("hidden_states", "cos", "sin", "position_ids")
    weights_local = ("q_proj_weight", "k_proj_weight", "v_proj_weight", "o_proj_weight",
                     "q_norm_weight", "k_norm_weight")
    weights_global = ("q_proj_weight", "k_proj_weight", "o_proj_weight", "q_norm_weight",
                      "k_norm_weight")
    sig = lambda f: tuple(inspect.signature(f).parameters)  # noqa: E731
    assert sig(torch_ops._h100_local_layer_impl) == common + ("packed_sequence_ids",) + weights_local
    assert sig(torch_ops._h100_global_layer_impl) == \
        common + ("packed_sequence_ids",) + weights_global
    cache = ("cache_k", "cache_v", "cache_length")
    assert sig(torch_ops._h100_global_static_cache_decode_impl) == common + cache + weights_global
    assert sig(torch_ops._h100_local_static_cache_decode_impl) == common + cache + weights_local


@pytest.mark.parametrize("family,hkv,d", [("local", 16, 256), ("global", 4, 512)])
def test_fake_registration_returns_fresh_symbolic_outputs(monkeypatch, family, hkv, d):
    def forbidden(*_a, **_k):
        raise AssertionError("the fake implementation entered a real route")

    monkeypatch.setattr(torch_ops, f"fa4_{family}_text_forward", forbidden)
    op = torch_ops.local_fwd if family == "local" else torch_ops.global_fwd
    with FakeTensorMode():
        inputs = _prepared(family, 33, "cuda")
        out, lse = op(*inputs)
    assert out.shape == (1, 33, 32, d) and out.dtype == torch.bfloat16
    assert lse.shape == (1, 32, 33) and lse.dtype == torch.float32
    assert all(out is not t and lse is not t for t in inputs)


@pytest.mark.parametrize("family", ["local", "global"])
def test_whole_layer_fake_registration_is_shape_only(monkeypatch, family):
    def forbidden(*_a, **_k):
        raise AssertionError("the whole-layer fake implementation entered a real body")

    monkeypatch.setattr(torch_ops, "prepare_rows_into", forbidden)
    fwd = torch_ops.local_layer_fwd if family == "local" else torch_ops.global_layer_fwd
    with FakeTensorMode(), torch.inference_mode():
        inputs = _layer_inputs(family, 33, "cuda")
        out, lse = fwd(*inputs)
    assert out.shape == (1, 33, 5376) and out.dtype == torch.bfloat16
    assert lse.shape == (1, 32, 33) and lse.dtype == torch.float32


@pytest.mark.parametrize("family", ["local", "global"])
def test_static_cache_decode_fake_registration_is_shape_only(family):
    d, hkv, cap = (256, 16, 1024) if family == "local" else (512, 4, 65)
    with FakeTensorMode(), torch.inference_mode():
        bf = dict(dtype=torch.bfloat16, device="cuda")
        inputs = [torch.empty(1, 1, 5376, **bf), torch.empty(1, 1, d, **bf),
                  torch.empty(1, 1, d, **bf), torch.empty(1, 1, dtype=torch.int64, device="cuda"),
                  torch.empty(1, hkv, cap, d, **bf), torch.empty(1, hkv, cap, d, **bf),
                  torch.empty((), dtype=torch.int64, device="cuda"),
                  torch.empty(32 * d, 5376, **bf), torch.empty(hkv * d, 5376, **bf)]
        if family == "local":
            inputs.append(torch.empty(hkv * d, 5376, **bf))
        inputs += [torch.empty(5376, 32 * d, **bf), torch.empty(d, **bf), torch.empty(d, **bf)]
        fwd = torch_ops.local_static_cache_decode_fwd if family == "local" else \
            torch_ops.global_static_cache_decode_fwd
        out, lse = fwd(*inputs)
    assert out.shape == (1, 1, 5376) and lse.shape == (1, 32, 1)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32


def test_fake_trace_holds_one_opaque_operator():
    from torch.fx.experimental.proxy_tensor import make_fx

    def layer(q, k, v, pos, packed):
        return torch_ops.global_fwd(q, k, v, pos, packed)

    gm = make_fx(layer, tracing_mode="fake")(*_prepared("global", 17, "cpu"))
    calls = [n.target for n in gm.graph.nodes if n.op == "call_function"]
    ours = [t for t in calls if "gemma4_mi355x" in str(t)]
    assert len(ours) == 1 and "global_fwd" in str(ours[0])
    assert all("gemma4_mi355x" in str(t) or "getitem" in str(t) for t in calls)


def test_real_cpu_execution_fails_explicitly():
    with pytest.raises(UnsupportedMI355XPath, match="CUDA tensors"):
        torch_ops.local_fwd(*_prepared("local", 1, "cpu"))


def test_prepared_ops_reject_requires_grad_before_anything_else():
    q, k, v, pos, packed = _prepared("local", 2, "cpu", dtype=torch.float32)
    q.requires_grad_(True)
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="requires_grad"):
        torch_ops._local_impl(q, k, v, pos, packed)
    with pytest.raises(ValueError, match="rank-4"):
        torch_ops._local_impl(q[0], k, v, pos, packed)


@pytest.mark.parametrize("family", ["local", "global"])
def test_inference_only_wrappers_refuse_autograd(family):
    inputs = _layer_inputs(family, 2, "cpu")
    fwd = torch_ops.local_layer_fwd if family == "local" else torch_ops.global_layer_fwd
    with pytest.raises(UnsupportedMI355XPath, match="inference/no-grad"):
        fwd(*inputs)
    inputs[0].requires_grad_(True)
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="hidden_states"):
        fwd(*inputs)


# --------------------------------------------------------------------------
# Transformers compile / FakeTensor route
# --------------------------------------------------------------------------

mu = pytest.importorskip("transformers.masking_utils")


def _module(layer):
    spec = g.GEMMA4_31B.spec_for_layer(layer)
    return types.SimpleNamespace(layer_idx=layer, scaling=1.0, head_dim=spec.head_dim_qk,
                                 num_key_value_groups=spec.qhead_per_kvhead, training=False)


def _text_mask(layer):
    if g.GEMMA4_31B.spec_for_layer(layer).kind == "full_attention":
        return mu.causal_mask_function
    return mu.and_masks(mu.sliding_window_overlay(1024), mu.causal_mask_function)


def _kw(layer):
    return dict(dropout=0.0, scaling=1.0,
                sliding_window=g.GEMMA4_31B.spec_for_layer(layer).sliding_window)


@pytest.mark.parametrize("layer,path,d", [(0, "fa4_local_compiled_op", 256),
                                          (5, "fa4_global_compiled_op", 512)])
def test_fake_inputs_route_to_the_compiled_operator(layer, path, d):
    plan = ti.gemma4_fa4_mask(1, 40, 40, 0, 0, mask_function=_text_mask(layer))
    with FakeTensorMode():
        q, k, v, _, _ = _prepared("local" if layer == 0 else "global", 40, "cuda")
        pos = torch.empty(1, 40, dtype=torch.int64, device="cuda")
        res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, position_ids=pos, **_kw(layer))
    assert res.path == path
    assert res.output.shape == (1, 40, 32, d) and res.lse.shape == (1, 32, 40)


@pytest.mark.parametrize("change,match", [
    (dict(attention_mask=True), "padding"),
    (dict(q_offset=3), "Q offsets"),
    (dict(vision=True), "without metadata"),
    (dict(cu=True), "packed sequence metadata"),
    (dict(cache=True), "cache"),
    (dict(mask="bidirectional"), "text-only mask"),
    (dict(position_ids=None), "position_ids"),
    (dict(training=True), "eval-mode"),
])
def test_compile_route_fails_closed(change, match):
    layer, s = 0, 24
    mask_fn = (lambda b, h, qi, ki: qi >= 0) if change.get("mask") else _text_mask(layer)
    pad = torch.ones(1, s, dtype=torch.bool) if change.get("attention_mask") else None
    plan = ti.gemma4_fa4_mask(1, s, s, change.get("q_offset", 0), 0, mask_function=mask_fn,
                              attention_mask=pad)
    module = _module(layer)
    module.training = change.get("training", False)
    with FakeTensorMode():
        q, k, v, _, _ = _prepared("local", s, "cuda")
        pos = None if "position_ids" in change else \
            torch.empty(1, s, dtype=torch.int64, device="cuda")
        extra = {}
        if change.get("vision"):
            extra["vision_block_ids"] = torch.empty(1, s, dtype=torch.int32, device="cuda")
        if change.get("cu"):
            extra["cu_seq_lens_q"] = torch.empty(2, dtype=torch.int32, device="cuda")
        if change.get("cache"):
            extra["past_key_values"] = object()
        with pytest.raises(UnsupportedMI355XPath, match=match):
            ti.gemma4_fa4_prepared(module, q, k, v, plan, position_ids=pos, **extra, **_kw(layer))


def test_compile_route_rejects_long_batched_and_trainable_inputs():
    plan = ti.gemma4_fa4_mask(1, 1025, 1025, 0, 0, mask_function=mu.causal_mask_function)
    with FakeTensorMode():
        q, k, v, _, _ = _prepared("global", 1025, "cuda")
        pos = torch.empty(1, 1025, dtype=torch.int64, device="cuda")
        with pytest.raises(UnsupportedMI355XPath, match="1..1024"):
            ti.gemma4_fa4_prepared(_module(5), q, k, v, plan, position_ids=pos, **_kw(5))
        q2, k2, v2, _, _ = _prepared("global", 8, "cuda")
        qb = torch.cat((q2, q2))
        plan2 = ti.gemma4_fa4_mask(2, 8, 8, 0, 0, mask_function=mu.causal_mask_function)
        with pytest.raises(UnsupportedMI355XPath, match="B1"):
            ti.gemma4_fa4_prepared(_module(5), qb, torch.cat((k2, k2)), torch.cat((v2, v2)),
                                   plan2, position_ids=torch.empty(1, 8, dtype=torch.int64,
                                                                   device="cuda"), **_kw(5))
        q2.requires_grad_(True)
        plan3 = ti.gemma4_fa4_mask(1, 8, 8, 0, 0, mask_function=mu.causal_mask_function)
        with pytest.raises(UnsupportedMI355XPath, match="forward-only"):
            ti.gemma4_fa4_prepared(_module(5), q2, k2, v2, plan3,
                                   position_ids=torch.empty(1, 8, dtype=torch.int64,
                                                            device="cuda"), **_kw(5))
