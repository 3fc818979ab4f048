"""GPU parity of the Transformers backend: HF-built mask plans through the native kernels.

Each case builds the mask with Transformers' own mask factories (registered
under the backend name), runs ``gemma4_fa4_prepared`` on the MI355X kernels,
and compares with fp32 dense attention under the dense evaluation of the same
mask callable (M1 envelopes; oracle/envelope.py).  The exhaustive-evaluation
admission proof, which needs the device predicate, is covered here too.
"""

from __future__ import annotations

import types

import pytest
import torch

from gemma4_fa4_amd import transformers_integration as ti
from gemma4_fa4_amd.errors import UnsupportedMI355XPath
from gemma4_fa4_amd.model_spec import GEMMA4_31B
from oracle.attention import expand_kv
from oracle.envelope import (
    GLOBAL_LSE_ATOL,
    GLOBAL_OUT_ATOL,
    GLOBAL_OUT_RTOL,
    LOCAL_LSE_ATOL,
    LOCAL_OUT_ATOL,
    LOCAL_OUT_RTOL,
)

mu = pytest.importorskip("transformers.masking_utils")
pytestmark = pytest.mark.gpu

LOCAL_LAYER, GLOBAL_LAYER = 0, 5
DEV = "cuda"


def _module(layer):
    spec = GEMMA4_31B.spec_for_layer(layer)
    return types.SimpleNamespace(layer_idx=layer, scaling=1.0, head_dim=spec.head_dim_qk,
                                 num_key_value_groups=spec.qhead_per_kvhead)


def _kw(layer):
    return dict(dropout=0.0, scaling=1.0, sliding_window=GEMMA4_31B.spec_for_layer(layer).sliding_window)


def _bhsd(layer, b, sq, sk, seed, grad=False):
    spec = GEMMA4_31B.spec_for_layer(layer)
    g = torch.Generator().manual_seed(seed)
    s = spec.head_dim_qk ** -0.25
    q = (torch.randn(b, spec.num_q_heads, sq, spec.head_dim_qk, generator=g) * s).bfloat16().to(DEV)
    k = (torch.randn(b, spec.num_kv_heads, sk, spec.head_dim_qk, generator=g) * s).bfloat16().to(DEV)
    v = torch.randn(b, spec.num_kv_heads, sk, spec.head_dim_v, generator=g).bfloat16().to(DEV)
    if grad:
        q, k, v = (t.requires_grad_() for t in (q, k, v))
    return q, k, v


def _masks(b, s, *, attention_mask=None, position_ids=None, vision=None):
    from transformers.models.gemma4 import modeling_gemma4 as mg
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig

    ti.register_gemma4_mi355x()
    cfg = Gemma4TextConfig(sliding_window=1024)
    cfg._attn_implementation = ti.BACKEND_NAME
    kw = dict(config=cfg, inputs_embeds=torch.zeros(b, s, 8, device=DEV),
              attention_mask=attention_mask, past_key_values=None, position_ids=position_ids)
    if vision is not None:
        m = mg.create_masks_for_vision_model(block_sequence_ids=vision, **kw)
        return m["sliding_attention"], m["full_attention"]
    return mu.create_sliding_window_causal_mask(**kw), mu.create_causal_mask(**kw)


def _allowed(plan):
    b = torch.arange(plan.batch_size, device=DEV)[:, None, None]
    qi = torch.arange(plan.q_length, device=DEV)[None, :, None] + int(plan.q_offset)
    ki = torch.arange(plan.kv_length, device=DEV)[None, None, :] + int(plan.kv_offset)
    a = torch.as_tensor(plan.mask_function(b, torch.zeros_like(b), qi, ki), device=DEV)
    a = a.expand(plan.batch_size, plan.q_length, plan.kv_length).clone()
    if plan.attention_mask is not None:
        a &= plan.attention_mask.bool()[:, None, :]
    return a


def _dense(q, k, v, allowed):
    hq, hkv = q.shape[1], k.shape[1]
    qf, kf, vf = q.float(), expand_kv(k.float(), hq // hkv), expand_kv(v.float(), hq // hkv)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous())
    s = s.masked_fill(~allowed[:, None], float("-inf"))
    lse = torch.logsumexp(s, -1)
    p = torch.where(torch.isfinite(lse)[..., None], torch.exp(s - lse[..., None]), torch.zeros_like(s))
    return torch.matmul(p, vf).transpose(1, 2), lse


def _check(res, q, k, v, allowed, layer, valid_q=None):
    local = layer == LOCAL_LAYER
    atol, rtol = (LOCAL_OUT_ATOL, LOCAL_OUT_RTOL) if local else (GLOBAL_OUT_ATOL, GLOBAL_OUT_RTOL)
    lse_atol = LOCAL_LSE_ATOL if local else GLOBAL_LSE_ATOL
    exp_o, exp_lse = _dense(q.detach(), k.detach(), v.detach(), allowed)
    out, lse = res.output.float(), res.lse.permute(0, 2, 1)
    exp_lse = exp_lse.permute(0, 2, 1)
    if valid_q is not None:
        assert torch.all(out[~valid_q] == 0) and torch.all(torch.isneginf(lse[~valid_q]))
        out, exp_o, lse, exp_lse = out[valid_q], exp_o[valid_q], lse[valid_q], exp_lse[valid_q]
    assert torch.all(torch.abs(out - exp_o) <= atol + rtol * torch.abs(exp_o))
    assert torch.all(torch.abs(lse - exp_lse) <= lse_atol)
    rel = torch.linalg.norm(out - exp_o) / torch.linalg.norm(exp_o)
    assert rel < 1e-2


def test_vision_mask_fixed_route_matches_dense():
    s = 300
    vis = torch.full((1, s), -1, dtype=torch.long)
    vis[0, 40:120] = 0
    vis[0, 200:260] = 1
    sliding, _ = _masks(1, s, vision=vis.to(DEV))
    q, k, v = _bhsd(LOCAL_LAYER, 1, s, s, seed=11)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, sliding, **_kw(LOCAL_LAYER))
    assert res.path == "fa4_local_fixed"
    _check(res, q, k, v, _allowed(sliding), LOCAL_LAYER)


@pytest.mark.parametrize("layer", [LOCAL_LAYER, GLOBAL_LAYER])
def test_padded_batch_routes_varlen_with_gradients(layer):
    b, s = 2, 160
    pad = torch.ones(b, s, dtype=torch.long)
    pad[0, :37] = 0
    pad[1, 131:] = 0
    pad = pad.to(DEV)
    sliding, full = _masks(b, s, attention_mask=pad)
    plan = sliding if layer == LOCAL_LAYER else full
    q, k, v = _bhsd(layer, b, s, s, seed=12, grad=True)
    res = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kw(layer))
    assert res.path in ("fa4_local_varlen", "fa4_global_varlen_native")
    allowed = _allowed(plan)
    _check(res, q, k, v, allowed, layer, valid_q=pad.bool())
    # Gradients of the valid rows against fp32 autograd of the dense reference.
    g = torch.Generator().manual_seed(13)
    dout = torch.randn(res.output.shape, generator=g).to(DEV) * pad.bool()[:, :, None, None]
    (res.output.float() * dout).sum().backward()
    qr, kr, vr = (t.detach().float().requires_grad_() for t in (q, k, v))
    o_ref, _ = _dense(qr, kr, vr, allowed)
    (o_ref * dout).sum().backward()
    for got, ref in ((q.grad, qr.grad), (k.grad, kr.grad), (v.grad, vr.grad)):
        rel = torch.linalg.norm(got.float() - ref) / torch.linalg.norm(ref)
        assert rel < 2e-2


def test_position_packed_global_matches_dense():
    pos = torch.cat([torch.arange(90), torch.arange(70), torch.arange(40)])[None].to(DEV)
    _, full = _masks(1, 200, position_ids=pos)
    q, k, v = _bhsd(GLOBAL_LAYER, 1, 200, 200, seed=14)
    res = ti.gemma4_fa4_prepared(_module(GLOBAL_LAYER), q, k, v, full, position_ids=pos,
                                 **_kw(GLOBAL_LAYER))
    assert res.path == "fa4_global_varlen_forward_only"
    _check(res, q, k, v, _allowed(full), GLOBAL_LAYER)


def test_evaluation_proof_admits_an_equal_foreign_callable():
    def window_causal(b, h, qi, ki):
        return (ki <= qi) & (ki > qi - 1024)

    s = 1100  # window boundary inside the grid
    plan = ti.gemma4_fa4_mask(1, s, s, mask_function=window_causal)
    q, k, v = _bhsd(LOCAL_LAYER, 1, s, s, seed=15)
    res = ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kw(LOCAL_LAYER))
    assert res.path == "fa4_local_varlen"
    _check(res, q, k, v, _allowed(plan), LOCAL_LAYER)


def test_evaluation_proof_rejects_a_different_callable():
    def wider(b, h, qi, ki):
        return (ki <= qi) & (ki > qi - 1025)

    s = 1100
    plan = ti.gemma4_fa4_mask(1, s, s, mask_function=wider)
    q, k, v = _bhsd(LOCAL_LAYER, 1, s, s, seed=16)
    with pytest.raises(UnsupportedMI355XPath, match="not provably"):
        ti.gemma4_fa4_prepared(_module(LOCAL_LAYER), q, k, v, plan, **_kw(LOCAL_LAYER))


@pytest.mark.parametrize("layer,physical,active,sq", [
    (LOCAL_LAYER, 2048, 1500, 1),
    (LOCAL_LAYER, 2048, 1500, 4),
    (GLOBAL_LAYER, 4096, 3000, 1),
], ids=["local-decode", "local-chunk", "global-decode"])
def test_static_cache_underfilled_prefix_routes_natively(layer, physical, active, sq):
    # Eager StaticCache: the layer hands over its whole physical backing; keys
    # past the active prefix were never written.  The call is trimmed to the
    # prefix (reference ti.py:1020-1110) and runs on the kernels: the result
    # matches dense attention over the prefix and does not depend on the tail.
    print(f"static cache layer={layer} physical={physical} active={active} sq={sq}", flush=True)
    q, k, v = _bhsd(layer, 1, sq, physical, seed=17)
    fn = mu.sliding_window_causal_mask_function(1024) if layer == LOCAL_LAYER else mu.causal_mask_function
    plan = ti.gemma4_fa4_mask(1, sq, physical, q_offset=active - sq, kv_offset=0,
                              mask_function=fn,
                              attention_mask=torch.ones((1, active), dtype=torch.long, device=DEV))
    k[:, :, active:] = 3e4
    v[:, :, active:] = -3e4
    with torch.no_grad():
        first = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kw(layer))
        k[:, :, active:] = -1e4
        v[:, :, active:] = 7e3
        second = ti.gemma4_fa4_prepared(_module(layer), q, k, v, plan, **_kw(layer))
    torch.cuda.synchronize()
    assert first.path == ("fa4_local_varlen" if layer == LOCAL_LAYER else "fa4_global_forward_only")
    assert torch.equal(first.output, second.output) and torch.equal(first.lse, second.lse)
    qi = torch.arange(sq, device=DEV)[:, None] + active - sq
    ki = torch.arange(active, device=DEV)[None, :]
    allowed = ki <= qi
    if layer == LOCAL_LAYER:
        allowed &= ki > qi - 1024
    _check(first, q, k[:, :, :active], v[:, :, :active], allowed[None], layer)
