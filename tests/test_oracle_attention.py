"""Pins oracle.attention: the reference's known answers, autograd, analytic cases."""

import math

import pytest
import torch

from oracle.attention import (
    attention_fwd_bwd,
    bf16_baseline_fwd_bwd,
    reference_attention,
    reference_attention_varlen,
)


# tests/test_reference.py:34-61
@pytest.mark.parametrize(("hq", "hkv"), [(8, 8), (8, 4), (8, 2), (8, 1), (32, 16), (32, 4)])
def test_gqa_matches_materialized_mha_forward_and_backward(hq, hkv):
    g = torch.Generator().manual_seed(17 + hq + hkv)
    q = torch.randn(1, hq, 5, 8, dtype=torch.float64, generator=g)
    k = torch.randn(1, hkv, 5, 8, dtype=torch.float64, generator=g)
    v = torch.randn(1, hkv, 5, 8, dtype=torch.float64, generator=g)
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    b = [t.clone().requires_grad_(True) for t in (q, k, v)]
    r = hq // hkv
    oa = reference_attention(*a)
    ob = reference_attention(b[0], b[1].repeat_interleave(r, 1), b[2].repeat_interleave(r, 1))
    torch.testing.assert_close(oa, ob)
    go = torch.linspace(-0.75, 1.25, oa.numel(), dtype=torch.float64).reshape_as(oa)
    oa.backward(go)
    ob.backward(go)
    for x, y in zip(a, b):
        torch.testing.assert_close(x.grad, y.grad)


# tests/test_reference.py:64-69
def test_window_one_returns_current_v():
    q, k, v = (torch.randn(1, 2, 4, 8) for _ in range(3))
    torch.testing.assert_close(reference_attention(q, k, v, sliding_window=1), v,
                               atol=1e-6, rtol=1e-6)


# tests/test_reference.py:72-78
def test_scale_one_differs_from_inverse_sqrt_d():
    q, k, v = (torch.randn(1, 2, 4, 8, dtype=torch.float64) for _ in range(3))
    assert not torch.allclose(reference_attention(q, k, v, softmax_scale=1.0),
                              reference_attention(q, k, v, softmax_scale=1 / math.sqrt(8)))


# tests/test_reference.py:81-101
def test_lse_is_fp32_and_bf16_inputs_return_bf16():
    q = torch.randn(1, 2, 4, 8, dtype=torch.bfloat16)
    k = torch.randn(1, 1, 4, 8, dtype=torch.bfloat16)
    v = torch.randn(1, 1, 4, 8, dtype=torch.bfloat16)
    out, lse = reference_attention(q, k, v, return_lse=True)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    assert lse.shape == (1, 2, 4)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()


# tests/test_reference.py:104-137
def test_varlen_matches_individual_lower_right_sequences():
    g = torch.Generator().manual_seed(81)
    q = torch.randn(3, 2, 4, dtype=torch.float64, generator=g)
    k = torch.randn(5, 1, 4, dtype=torch.float64, generator=g)
    v = torch.randn(5, 1, 4, dtype=torch.float64, generator=g)
    out, lse = reference_attention_varlen(q, k, v, torch.tensor([0, 2, 3], dtype=torch.int32),
                                          torch.tensor([0, 3, 5], dtype=torch.int32),
                                          sliding_window=4, return_lse=True)
    eo, el = [], []
    for qs, qe, ks, ke in ((0, 2, 0, 3), (2, 3, 3, 5)):
        o, l = reference_attention(q[qs:qe].transpose(0, 1)[None], k[ks:ke].transpose(0, 1)[None],
                                   v[ks:ke].transpose(0, 1)[None], sliding_window=4,
                                   q_start=(ke - ks) - (qe - qs), return_lse=True)
        eo.append(o[0].transpose(0, 1))
        el.append(l[0])
    torch.testing.assert_close(out, torch.cat(eo))
    torch.testing.assert_close(lse, torch.cat(el, dim=1))


# tests/test_reference.py:140-179
def test_mixed_empty_segments_give_exact_zero_kv_gradients():
    g = torch.Generator().manual_seed(82)
    q = torch.randn(3, 2, 4, dtype=torch.float64, generator=g, requires_grad=True)
    k = torch.randn(5, 1, 4, dtype=torch.float64, generator=g, requires_grad=True)
    v = torch.randn(5, 1, 4, dtype=torch.float64, generator=g, requires_grad=True)
    cu_q = torch.tensor([0, 0, 2, 2, 2, 3, 3], dtype=torch.int32)
    cu_k = torch.tensor([0, 0, 3, 4, 4, 5, 5], dtype=torch.int32)
    out, lse = reference_attention_varlen(q, k, v, cu_q, cu_k, sliding_window=4, return_lse=True)
    (out.square().sum() + lse.sum()).backward()
    assert torch.equal(k.grad[3], torch.zeros_like(k.grad[3]))
    assert torch.equal(v.grad[3], torch.zeros_like(v.grad[3]))
    # the explicit backward gives the same gradients
    do = 2 * out.detach()
    dlse = torch.ones(2, 3, dtype=torch.float64)
    _, _, dq, dk, dv = attention_fwd_bwd(q.detach(), k.detach(), v.detach(), cu_q, cu_k, do=do,
                                         dlse=dlse, sliding_window=4)
    torch.testing.assert_close(dq, q.grad)
    torch.testing.assert_close(dk, k.grad)
    torch.testing.assert_close(dv, v.grad)


# tests/test_reference.py:182-213
@pytest.mark.parametrize(("cu_q", "cu_k", "match"), [
    ([0, 2, 1, 3], [0, 2, 2, 4], "nondecreasing"),
    ([0, 2, 3], [0, 1, 4], "Sq greater than Sk"),
])
def test_varlen_rejects_invalid_contracts(cu_q, cu_k, match):
    q, k = torch.zeros(3, 2, 4), torch.zeros(4, 1, 4)
    with pytest.raises(ValueError, match=match):
        reference_attention_varlen(q, k, torch.zeros_like(k), torch.tensor(cu_q, dtype=torch.int32),
                                   torch.tensor(cu_k, dtype=torch.int32))


def test_varlen_rejects_nonpositive_totals():
    cu = torch.tensor([0, 0, 0], dtype=torch.int32)
    with pytest.raises(ValueError, match="totals must be positive"):
        reference_attention_varlen(torch.empty(0, 2, 4), torch.empty(0, 1, 4),
                                   torch.empty(0, 1, 4), cu, cu)


# tests/test_reference.py:216-248
def test_varlen_composes_vision_and_document_masks():
    q = torch.zeros(4, 2, 4, dtype=torch.float64)
    k = torch.zeros(4, 1, 4, dtype=torch.float64)
    v = torch.zeros(4, 1, 4, dtype=torch.float64)
    v[2] = 16
    cu = torch.tensor([0, 4], dtype=torch.int32)
    vision = torch.zeros(4, dtype=torch.int32)
    docs = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    a = reference_attention_varlen(q, k, v, cu, cu, sliding_window=4, vision_block_ids=vision,
                                   document_ids=docs, allow_vision_bidirectional=True)
    b = reference_attention_varlen(q, k, v, cu, cu, sliding_window=4, vision_block_ids=vision,
                                   allow_vision_bidirectional=True)
    assert torch.count_nonzero(a[1]) == 0
    assert torch.count_nonzero(b[1]) > 0


# tests/test_reference.py:251-285
def test_varlen_isolates_repeated_ids_across_segments():
    q = torch.zeros(4, 2, 4, dtype=torch.float64)
    k = torch.zeros(4, 1, 4, dtype=torch.float64)
    v = torch.zeros(4, 1, 4, dtype=torch.float64)
    cu = torch.tensor([0, 2, 4], dtype=torch.int32)
    z = torch.zeros(4, dtype=torch.int32)
    base = reference_attention_varlen(q, k, v, cu, cu, sliding_window=4, vision_block_ids=z,
                                      document_ids=z, allow_vision_bidirectional=True)
    v2 = v.clone()
    v2[2:] = 1024
    mut = reference_attention_varlen(q, k, v2, cu, cu, sliding_window=4, vision_block_ids=z,
                                     document_ids=z, allow_vision_bidirectional=True)
    assert torch.equal(mut[:2], base[:2])
    assert torch.count_nonzero(mut[2:]) > 0


# tests/test_reference.py:288-304
def test_varlen_rejects_metadata_not_matching_tk():
    with pytest.raises(ValueError, match="match Tk"):
        reference_attention_varlen(torch.zeros(2, 2, 4), torch.zeros(3, 1, 4), torch.zeros(3, 1, 4),
                                   torch.tensor([0, 2], dtype=torch.int32),
                                   torch.tensor([0, 3], dtype=torch.int32),
                                   vision_block_ids=torch.tensor([0, 0], dtype=torch.int32))


# tests/test_reference.py:307-328
def test_lower_right_vision_truth_table_gives_one_point_five():
    q = torch.zeros(3, 1, 1, dtype=torch.float64)
    k = torch.zeros(5, 1, 1, dtype=torch.float64)
    v = torch.arange(5, dtype=torch.float64).reshape(5, 1, 1)
    cu_q, cu_k = torch.tensor([0, 3], dtype=torch.int32), torch.tensor([0, 5], dtype=torch.int32)
    vision = torch.tensor([-1, -1, 7, 7, 8], dtype=torch.int32)
    out = reference_attention_varlen(q, k, v, cu_q, cu_k, sliding_window=1024,
                                     vision_block_ids=vision, allow_vision_bidirectional=True)
    assert out[0, 0, 0].item() == 1.5
    o2, *_ = attention_fwd_bwd(q, k, v, cu_q, cu_k, sliding_window=1024, vision_block_ids=vision,
                               allow_vision_bidirectional=True)
    assert o2[0, 0, 0].item() == 1.5


# tests/test_reference.py:331-356
def test_strict_w1024_lower_edge_gives_one_over_1024():
    q = torch.zeros(1, 1, 1, dtype=torch.float64)
    k = torch.zeros(1025, 1, 1, dtype=torch.float64)
    v = torch.zeros_like(k)
    v[0], v[1] = 100, 1
    cu_q, cu_k = torch.tensor([0, 1], dtype=torch.int32), torch.tensor([0, 1025], dtype=torch.int32)
    vision = torch.zeros(1025, dtype=torch.int32)
    out = reference_attention_varlen(q, k, v, cu_q, cu_k, sliding_window=1024,
                                     vision_block_ids=vision, allow_vision_bidirectional=True)
    assert out[0, 0, 0].item() == pytest.approx(1.0 / 1024.0, abs=1e-15)
    o2, *_ = attention_fwd_bwd(q, k, v, cu_q, cu_k, sliding_window=1024, vision_block_ids=vision,
                               allow_vision_bidirectional=True)
    assert o2[0, 0, 0].item() == pytest.approx(1.0 / 1024.0, abs=1e-15)


# tests/test_reference.py:417-429
def test_all_masked_row_returns_zero_and_negative_infinite_lse():
    q, k, v = (torch.randn(1, 1, 1, 8) for _ in range(3))
    out, lse = reference_attention(q, k, v, key_padding_mask=torch.tensor([[False]]),
                                   return_lse=True)
    assert torch.equal(out, torch.zeros_like(out))
    assert torch.isneginf(lse).all()


def _packed_case(seed, lengths_q, lengths_k, hq, hkv, d, window, vision=None, docs=None):
    g = torch.Generator().manual_seed(seed)
    tq, tk = sum(lengths_q), sum(lengths_k)
    q = torch.randn(tq, hq, d, dtype=torch.float64, generator=g)
    k = torch.randn(tk, hkv, d, dtype=torch.float64, generator=g)
    v = torch.randn(tk, hkv, d, dtype=torch.float64, generator=g)
    do = torch.randn(tq, hq, d, dtype=torch.float64, generator=g)
    dlse = torch.randn(hq, tq, dtype=torch.float64, generator=g)
    cu_q = torch.tensor([0] + torch.tensor(lengths_q).cumsum(0).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + torch.tensor(lengths_k).cumsum(0).tolist(), dtype=torch.int32)
    return q, k, v, do, dlse, cu_q, cu_k


@pytest.mark.parametrize("window,use_meta", [(None, False), (4, False), (4, True), (3, True)])
def test_explicit_backward_matches_autograd(window, use_meta):
    q, k, v, do, dlse, cu_q, cu_k = _packed_case(5, [3, 0, 7, 5], [4, 2, 7, 9], 4, 2, 8, window)
    tk = k.shape[0]
    vision = docs = None
    if use_meta:
        g = torch.Generator().manual_seed(9)
        vision = torch.randint(-1, 2, (tk,), generator=g, dtype=torch.int32)
        docs = torch.randint(0, 2, (tk,), generator=g, dtype=torch.int32)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out, lse = reference_attention_varlen(qa, ka, va, cu_q, cu_k, sliding_window=window,
                                          vision_block_ids=vision, document_ids=docs,
                                          allow_vision_bidirectional=use_meta, return_lse=True)
    (out * do).sum().backward(retain_graph=True)
    o2, l2, dq, dk, dv = attention_fwd_bwd(q, k, v, cu_q, cu_k, do=do, sliding_window=window,
                                           vision_block_ids=vision, document_ids=docs,
                                           allow_vision_bidirectional=use_meta, q_chunk=3)
    torch.testing.assert_close(o2, out)
    torch.testing.assert_close(l2, lse)
    torch.testing.assert_close(dq, qa.grad)
    torch.testing.assert_close(dk, ka.grad)
    torch.testing.assert_close(dv, va.grad)


def test_explicit_backward_lse_gradient_matches_autograd():
    q, k, v, do, dlse, cu_q, cu_k = _packed_case(6, [5, 6], [5, 8], 4, 1, 8, None)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    # fp64 LSE path: differentiate logsumexp of the fp64 scores directly
    outs, lses = [], []
    for (qs, qe, ks, ke) in ((0, 5, 0, 5), (5, 11, 5, 13)):
        qq = qa[qs:qe].transpose(0, 1)
        kk = ka[ks:ke].transpose(0, 1).repeat_interleave(4, 0)
        vv = va[ks:ke].transpose(0, 1).repeat_interleave(4, 0)
        s = qq @ kk.transpose(-1, -2)
        lq, lk = qe - qs, ke - ks
        qi = torch.arange(lk - lq, lk)[:, None]
        ki = torch.arange(lk)[None, :]
        s = s.masked_fill(~(ki <= qi), float("-inf"))
        l = torch.logsumexp(s, -1)
        outs.append((torch.softmax(s, -1) @ vv).transpose(0, 1))
        lses.append(l)
    out, lse = torch.cat(outs), torch.cat(lses, 1)
    ((out * do).sum() + (lse * dlse).sum()).backward()
    _, _, dq, dk, dv = attention_fwd_bwd(q, k, v, cu_q, cu_k, do=do, dlse=dlse)
    torch.testing.assert_close(dq, qa.grad)
    torch.testing.assert_close(dk, ka.grad)
    torch.testing.assert_close(dv, va.grad)


def test_analytic_uniform_scores():
    # probe_h100_global_varlen_backward.py:191-265: Q = 0 gives uniform attention,
    # O = mean of the allowed V rows, LSE = ln(count), dK = 0.
    s = 37
    q = torch.zeros(s, 2, 4, dtype=torch.float64)
    k = torch.ones(s, 1, 4, dtype=torch.float64)
    v = torch.randn(s, 1, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    cu = torch.tensor([0, s], dtype=torch.int32)
    do = torch.ones(s, 2, 4, dtype=torch.float64)
    o, l, dq, dk, dv = attention_fwd_bwd(q, k, v, cu, cu, do=do)
    for i in (0, 5, s - 1):
        torch.testing.assert_close(o[i, 0], v[: i + 1, 0].mean(0))
        assert l[0, i].item() == pytest.approx(math.log(i + 1), abs=1e-6)
    assert torch.count_nonzero(dk) == 0
    # dV of the final key: only the final query sees it, with weight 1/S, twice (2 heads)
    torch.testing.assert_close(dv[s - 1, 0], torch.full((4,), 2.0 / s, dtype=torch.float64))


def test_bf16_baseline_is_close_but_not_exact():
    q, k, v, do, dlse, cu_q, cu_k = _packed_case(7, [40], [40], 4, 2, 16, 8)
    q, k, v = (t.to(torch.bfloat16).double() for t in (q, k, v))
    o, _, dq, dk, dv = attention_fwd_bwd(q, k, v, cu_q, cu_k, do=do, sliding_window=8)
    ob, dqb, dkb, dvb = bf16_baseline_fwd_bwd(q, k, v, cu_q, cu_k, do=do, sliding_window=8)
    for ref, got in ((o, ob), (dq, dqb), (dk, dkb), (dv, dvb)):
        err = (got.double() - ref).abs().max().item()
        assert 0 < err < 0.25 * ref.abs().max().item()
