"""Parity of the benchmark configurations 2-5 at their full sizes, through the adapters.

Each configuration runs the route ``bench.py`` times: the packed adapter
(``fa4_global_varlen_forward`` / ``fa4_local_varlen_forward`` with the
workload's cu_seqlens, vision and document IDs) and ``torch.autograd.backward``
of O with dO, at the stated size (configuration 2: 8192 tokens; 3: 8192 tokens
with four 256-1120-token vision blocks; 4: 32768 packed tokens in segments of
1-2048; 5: 131072 packed tokens in 8 documents with vision blocks).  Values
are drawn on the GPU from the workload's seed (the distributions of the
benchmark; drawing the 3.2e9 values of configuration 5 on the CPU takes
half a minute).  Two checks:

* sampled heads: two KV groups in full (all of their query heads, every row,
  so rows crossing vision blocks, window edges and segment boundaries are all
  included) against the fp64 oracle computed on the GPU for those heads, with
  the reference's M1 forward envelopes and upstream-relative gradient rule plus
  rel-Frobenius bounds (tests/g4_testutil.py);
* Q = 0 closed forms over every head and row: all scores are 0, so P is uniform
  over each row's allowed interval [lo, hi] (``workloads.allowed_intervals``):
  LSE = ln(hi - lo + 1), O = mean of V over the interval, dV[k] = sum over the
  rows whose interval holds k of dO / (hi - lo + 1), and dK = dS^T Q = 0
  exactly (the analytic probe of
  scripts/probe_h100_global_varlen_backward.py:186-265, 581-700 at these sizes).
"""

import math

import pytest
import torch

from g4_testutil import check_forward, check_gradients
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL_UNIFORM = 2.0 ** -8  # bf16 rounding of P = 1/n and of the outputs, with margin


def _adapter(w, q, k, v, cu, vis, docs):
    import gemma4_fa4_amd as g

    m = max(w.seg_lengths)
    if w.kind == "local":
        return g.fa4_local_varlen_forward(q, k, v, cu, cu, max_seqlen_q=m, max_seqlen_k=m,
                                          vision_block_ids=vis, document_ids=docs)
    return g.fa4_global_varlen_forward(q, k, v, cu, cu, max_seqlen_q=m, max_seqlen_k=m)


def _fwd_bwd(w, q, k, v, do, cu, vis, docs):
    qd, kd, vd = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o, lse = _adapter(w, qd, kd, vd, cu, vis, docs)
    torch.autograd.backward(o, do)
    torch.cuda.synchronize()
    return o.detach(), lse.detach(), qd.grad, kd.grad, vd.grad


def _sampled_groups(w):
    return (0, w.hkv - 1)


def _check_sampled_heads(w, tensors, outs):
    q, k, v, do, cu, vis, docs = tensors
    o, lse, dq, dk, dv = outs
    rep = w.hq // w.hkv
    cc = w.cu()
    for g in _sampled_groups(w):
        heads = list(range(g * rep, (g + 1) * rep))
        print(f"  oracle: KV group {g}, query heads {heads[0]}-{heads[-1]}", flush=True)
        args = dict(sliding_window=w.window, vision_block_ids=vis, document_ids=docs,
                    allow_vision_bidirectional=w.kind == "local" and vis is not None,
                    heads=heads)
        o_r, l_r, dq_r, dk_r, dv_r = attention_fwd_bwd(
            q, k, v, cc, cc, do=do, compute_dtype=torch.float64, q_chunk=512, **args)
        _, bq, bk, bv = bf16_baseline_fwd_bwd(q, k, v, cc, cc, do=do, q_chunk=256, **args)
        h = slice(heads[0], heads[-1] + 1)
        gs = slice(g, g + 1)
        label = f"{w.name} group {g}"
        fro, lse_err = check_forward(o[:, h], lse[h], o_r[:, h].cpu(), l_r[h].cpu(),
                                     local=w.kind == "local", label=label)
        report = check_gradients([dq[:, h], dk[:, gs], dv[:, gs]],
                                 [dq_r[:, h].cpu(), dk_r[:, gs].cpu(), dv_r[:, gs].cpu()],
                                 [bq[:, h].cpu(), bk[:, gs].cpu(), bv[:, gs].cpu()],
                                 label=label)
        print(f"  O rel-fro {fro:.2e}, LSE max-abs {lse_err:.2e}, " + ", ".join(
            f"{n} max-abs {e:.2e} (limit {lim:.2e}) rel-fro {f:.2e}"
            for n, (e, lim, f) in report.items()), flush=True)
        del o_r, l_r, dq_r, dk_r, dv_r, bq, bk, bv
        torch.cuda.empty_cache()


def _interval_sum(x, lo, hi):
    """Rows of ``x`` (T, D) summed over [lo[i], hi[i]] for every i, via a prefix sum."""
    c = torch.zeros(x.shape[0] + 1, x.shape[1], dtype=torch.float64, device=x.device)
    torch.cumsum(x.double(), dim=0, out=c[1:])
    return c[hi + 1] - c[lo]


def _scatter_intervals(x, lo, hi, t):
    """out[k] = sum of x[i] over the rows i whose interval [lo[i], hi[i]] holds k."""
    acc = torch.zeros(t + 1, x.shape[1], dtype=torch.float64, device=x.device)
    acc.index_add_(0, lo, x)
    acc.index_add_(0, hi + 1, -x)
    return torch.cumsum(acc, dim=0)[:t]


def _check_uniform_scores(w, tensors):
    from gemma4_fa4_amd import workloads as wl

    _q, k, v, do, cu, vis, docs = tensors
    q0 = torch.zeros_like(_q)
    o, lse, dq, dk, dv = _fwd_bwd(w, q0, k, v, do, cu, vis, docs)
    lo_np, hi_np = wl.allowed_intervals(w)
    lo = torch.from_numpy(lo_np).to(DEV)
    hi = torch.from_numpy(hi_np).to(DEV)
    n = (hi - lo + 1).double()
    t = w.tokens
    rep = w.hq // w.hkv
    # LSE = ln(count) on every head
    lse_ref = torch.log(n).float()
    lse_err = (lse - lse_ref[None]).abs().max().item()
    assert lse_err < 1e-4, f"{w.name} Q=0: LSE max error {lse_err:.2e}"
    # dK = dS^T Q is exactly zero
    assert torch.count_nonzero(dk).item() == 0, f"{w.name} Q=0: dK is not exactly zero"
    for g in range(w.hkv):
        vg = v[:, g].double()
        mean_v = _interval_sum(vg, lo, hi) / n[:, None]
        bound_o = _interval_sum(vg.abs(), lo, hi) / n[:, None]
        dv_ref = torch.zeros(t, v.shape[-1], dtype=torch.float64, device=DEV)
        bound_dv = torch.zeros_like(dv_ref)
        for h in range(g * rep, (g + 1) * rep):
            err = (o[:, h].double() - mean_v).abs()
            lim = RTOL_UNIFORM * (bound_o + mean_v.abs()) + 1e-6
            bad = (err > lim).sum().item()
            assert bad == 0, f"{w.name} Q=0 head {h}: O off the mean of V at {bad} elements"
            contrib = do[:, h].double() / n[:, None]
            dv_ref += _scatter_intervals(contrib, lo, hi, t)
            bound_dv += _scatter_intervals(contrib.abs(), lo, hi, t)
        err = (dv[:, g].double() - dv_ref).abs()
        lim = RTOL_UNIFORM * (bound_dv + dv_ref.abs()) + 1e-6
        bad = (err > lim).sum().item()
        assert bad == 0, f"{w.name} Q=0 KV head {g}: dV off the closed form at {bad} elements"
    assert torch.isfinite(dq).all()


CONFIGS = ["config2", "config3", "config4", "config5"]


@pytest.mark.parametrize("name", CONFIGS)
def test_benchmark_configuration_at_full_size(name):
    from gemma4_fa4_amd import workloads as wl

    w = getattr(wl, name)()
    print(f"{w.name}: {w.tokens} tokens, {len(w.seg_lengths)} segments", flush=True)
    tensors = wl.tensors(w, DEV, device_rng=True)
    q, k, v, do, cu, vis, docs = tensors
    outs = _fwd_bwd(w, q, k, v, do, cu, vis, docs)
    for t in outs:
        assert torch.isfinite(t).all()
    _check_sampled_heads(w, tensors, outs)
    del outs
    torch.cuda.empty_cache()
    print(f"  Q=0 closed forms over all {w.hq} heads", flush=True)
    _check_uniform_scores(w, tensors)
    del tensors, q, k, v, do
    torch.cuda.empty_cache()


def test_closed_form_helpers_match_direct_sums():
    # The prefix-sum helpers of the Q=0 check against direct per-row sums.
    gen = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(50, 3, generator=gen, device=DEV, dtype=torch.float64)
    lo = torch.randint(0, 50, (50,), generator=gen, device=DEV)
    hi = torch.minimum(lo + torch.randint(0, 10, (50,), generator=gen, device=DEV),
                       torch.tensor(49, device=DEV))
    got = _interval_sum(x, lo, hi)
    want = torch.stack([x[a:b + 1].sum(0) for a, b in zip(lo.tolist(), hi.tolist())])
    torch.testing.assert_close(got, want)
    got = _scatter_intervals(x, lo, hi, 50)
    want = torch.zeros(50, 3, dtype=torch.float64, device=DEV)
    for i, (a, b) in enumerate(zip(lo.tolist(), hi.tolist())):
        want[a:b + 1] += x[i]
    torch.testing.assert_close(got, want)
    assert math.isclose(math.log(3), torch.log(torch.tensor(3.0, dtype=torch.float64)).item())
