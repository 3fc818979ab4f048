"""Packed adapters on the GPU: cumulative-array errors raised at launch time.

The packed adapters read ``cu_seqlens`` immediately before the first launch
(the host work that does not need the values runs first).  These cases pass
device tensors through the public functions, with autograd on, and check the
reference's error classes and messages (tests/test_h100_fa4.py validation
cases), that nothing is left pending after a failure, and that a valid call
afterwards runs and repeats bitwise.
"""

import pytest
import torch

import gemma4_fa4_amd as g

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _global_inputs(lengths, seed=0):
    gen = torch.Generator().manual_seed(seed)
    t = sum(lengths)
    q = (torch.randn(t, 32, 512, generator=gen) * 512 ** -0.25).bfloat16()
    k = (torch.randn(t, 4, 512, generator=gen) * 512 ** -0.25).bfloat16()
    v = torch.randn(t, 4, 512, generator=gen).bfloat16()
    cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int32)
    return [x.to(DEV) for x in (q, k, v, cu)]


def _leaf(*ts):
    return [t.detach().clone().requires_grad_(True) for t in ts]


def test_global_packed_errors_at_launch_then_valid_call():
    q, k, v, cu = _global_inputs([40, 24])
    run = g.fa4_global_varlen_forward
    short = torch.tensor([0, 40, 63], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="end at"):
        run(*_leaf(q, k, v), short, short, max_seqlen_q=40, max_seqlen_k=40)
    with pytest.raises(ValueError, match="maxima"):
        run(*_leaf(q, k, v), cu, cu, max_seqlen_q=64, max_seqlen_k=64)
    cq = torch.tensor([0, 30, 64], dtype=torch.int32, device=DEV)  # second segment 34 > 24
    with pytest.raises(g.UnsupportedMI355XPath, match="per segment"):
        run(*_leaf(q, k, v), cq, cu, max_seqlen_q=34, max_seqlen_k=40)

    outs = []
    for _ in range(2):
        qi, ki, vi = _leaf(q, k, v)
        out, lse = run(qi, ki, vi, cu, cu, max_seqlen_q=40, max_seqlen_k=40)
        out.float().square().sum().backward()
        torch.cuda.synchronize()
        outs.append((out.detach(), lse.detach(), qi.grad, ki.grad, vi.grad))
    for a, b in zip(*outs):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b)


def test_global_forward_only_errors_at_launch():
    q, k, v, cu = _global_inputs([17, 30, 5], seed=1)
    bad = torch.tensor([0, 30, 17, 52], dtype=torch.int32, device=DEV)
    with torch.no_grad():
        with pytest.raises(ValueError, match="nondecreasing"):
            g.fa4_global_varlen_forward_only(q, k, v, bad, bad, max_seqlen_q=30,
                                             max_seqlen_k=30)
        out, lse = g.fa4_global_varlen_forward_only(q, k, v, cu, cu, max_seqlen_q=30,
                                                    max_seqlen_k=30)
        torch.cuda.synchronize()
    assert out.shape == q.shape and lse.shape == (32, 52)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()


def test_local_packed_with_vision_errors_at_launch():
    gen = torch.Generator().manual_seed(2)
    lengths = [96, 64]
    t = sum(lengths)
    q = (torch.randn(t, 32, 256, generator=gen) * 256 ** -0.25).bfloat16().to(DEV)
    k = (torch.randn(t, 16, 256, generator=gen) * 256 ** -0.25).bfloat16().to(DEV)
    v = torch.randn(t, 16, 256, generator=gen).bfloat16().to(DEV)
    cu = torch.tensor([0, 96, 160], dtype=torch.int32, device=DEV)
    vis = torch.full((t,), -1, dtype=torch.int32)
    vis[10:40] = 0
    vis[100:130] = 1
    vis = vis.to(DEV)
    with pytest.raises(ValueError, match="maxima"):
        g.fa4_local_varlen_forward(*_leaf(q, k, v), cu, cu, max_seqlen_q=64, max_seqlen_k=96,
                                   vision_block_ids=vis)
    qi, ki, vi = _leaf(q, k, v)
    out, lse = g.fa4_local_varlen_forward(qi, ki, vi, cu, cu, max_seqlen_q=96, max_seqlen_k=96,
                                          vision_block_ids=vis)
    out.float().sum().backward()
    torch.cuda.synchronize()
    for x in (out, lse, qi.grad, ki.grad, vi.grad):
        assert torch.isfinite(x.float()).all()
