"""C-ABI parity of the striped stored-dS backward (head dim 512, causal).

When the dense dS tiles of a single global sequence exceed the problem's
``ds_budget``, ``g4_attn_bwd`` cuts its 32-query rows into stripes that fit the
budget next to fp32 dK / dV sums: per stripe, the dK/dV launch stores that
stripe's dS and adds its dK / dV to the sums (the last stripe writes the bf16
gradients), then the dQ launch reads the stripe's tiles.  Nothing is
recomputed, so the route's dQ is the dense stored-dS route's dQ (same dS
values, same key order per query tile) and its dK / dV differ from the dense
route's only by the fp32 additions between stripes.  Each case is checked
against the dense route and against the fp64 oracle with the reference's M1
envelopes: several stripes (ragged last stripe, keys before the first query,
documents, the work-queue launch) and the smallest budget that still stripes.
Several sequences past the budget are striped by whole sequences instead (no
sums), and their gradients must equal the dense route's to the bit.
"""

import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q, k, v, do, dlse, lq, lk, *, docs=None, ds_budget=0, packed=True):
    from gemma4_fa4_amd import ops

    cq, ck = cu(lq), cu(lk)
    plan = ops.make_plan(
        num_seqs=1, seqlen_q=lq[0], seqlen_k=lk[0], num_q_heads=q.shape[1],
        num_kv_heads=k.shape[1], head_dim=512, window=None,
        documents=None if docs is None else docs.to(DEV),
        cu_q=cq.to(DEV) if packed else None, cu_k=ck.to(DEV) if packed else None,
        total_q=q.shape[0], total_k=k.shape[0], ds_budget=ds_budget)
    if not packed:
        q, k, v, do = (t[None] for t in (q, k, v, do))
        dlse = dlse[None]
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.backward()
    torch.cuda.synchronize()
    squeeze = (lambda t: t) if packed else (lambda t: t[0])
    return [squeeze(t).cpu() for t in (st.o, st.lse, st.dq, st.dk, st.dv)], plan


def _stored_bytes(plan):
    """Workspace bytes of the stored-dS route (dS buffer plus fp32 sums when striped)."""
    budget = plan.ds_budget
    stored = plan.workspace_bytes(1)
    plan.ds_budget = -1
    lean = plan.workspace_bytes(1)
    plan.ds_budget = budget
    return stored - lean


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


# (lq, lk, hq, hkv, packed, docs, units): units = (row, key tile) dS tiles the
# budget leaves for the largest stripe after the fp32 sums
CASES = [
    ([4096], [4096], 32, 4, True, False, 2048),   # three stripes
    ([4000], [4000], 16, 2, False, False, 4 * 63),  # many stripes, the last one ragged
    ([3000], [3500], 8, 1, True, True, 900),  # keys before the first query, documents
    ([8192], [8192], 32, 32, True, False, 3000),  # 2048 pair items: the work-queue launch
]


@pytest.mark.parametrize("lq,lk,hq,hkv,packed,with_docs,units", CASES)
def test_striped_backward_matches_the_dense_route_and_the_oracle(lq, lk, hq, hkv, packed,
                                                                  with_docs, units):
    label = f"striped lq={lq} lk={lk} hq={hq} hkv={hkv} packed={packed} docs={with_docs}"
    print(label, flush=True)
    q, k, v, do, dlse = qkv(9700 + lq[0] + hkv, lq[0], lk[0], hq, hkv, 512)
    docs = None
    if with_docs:
        docs = torch.zeros(lk[0], dtype=torch.int32)
        docs[1200:] = 1
        docs[2600:] = 2
    sums = 2 * lk[0] * hkv * 512 * 4
    unit = hq * 4096
    # dense rows: packed problems give each sequence total_q / 32 + 1 rows
    rows = lq[0] // 32 + 1 if packed else (lq[0] + 31) // 32
    dense_bytes = rows * ((lk[0] + 63) // 64) * unit
    budget = sums + units * unit
    assert budget < dense_bytes
    got, plan = _run(q, k, v, do, dlse, lq, lk, docs=docs, ds_budget=budget, packed=packed)
    stored = _stored_bytes(plan)
    assert sums < stored <= budget, "the problem is not striped"
    dense, dplan = _run(q, k, v, do, dlse, lq, lk, docs=docs, packed=packed)
    assert _stored_bytes(dplan) == dense_bytes
    assert torch.equal(got[0], dense[0]) and torch.equal(got[1], dense[1])
    # same dS, same key order per query tile: dQ to the bit
    assert torch.equal(got[2], dense[2]), "dQ differs from the dense stored-dS route"
    # dK / dV: fp32 partial sums per stripe instead of one accumulator
    for i, name in ((3, "dK"), (4, "dV")):
        assert _rel(got[i], dense[i]) < 2e-3, (name, _rel(got[i], dense[i]))
    # sampled heads: whole KV groups, so the sampled KV heads' dK / dV are complete
    grp = hq // hkv
    heads = list(range(hq)) if hq * lq[0] <= 16 * 4096 else list(range(grp * max(1, 3 // grp)))
    kvs = sorted({h // grp for h in heads})
    cq, ck = cu(lq), cu(lk)
    args = dict(document_ids=None if docs is None else docs.to(DEV), heads=heads)
    o_ref, l_ref, *refs = attention_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(),
                                          ck.tolist(), do=do.to(DEV), dlse=dlse.to(DEV), **args)
    check_forward(got[0][:, heads], got[1][heads], o_ref[:, heads].cpu(), l_ref[heads].cpu(),
                  local=False, label=label)
    check_gradients([got[2][:, heads], got[3][:, kvs], got[4][:, kvs]],
                    [refs[0][:, heads].cpu(), refs[1][:, kvs].cpu(), refs[2][:, kvs].cpu()],
                    [bq[:, heads].cpu(), bk[:, kvs].cpu(), bv[:, kvs].cpu()], label=label)


def test_smallest_striping_budget_and_repeat_calls():
    # 4 x 64 units: the last four rows reach all 64 key tiles, so every stripe
    # is at most 256 units (the first ones taller, the last ones four rows).
    # Two calls on one workspace give the same bits (the fp32 sums start over).
    lq = lk = [4096]
    q, k, v, do, dlse = qkv(9790, 4096, 4096, 8, 2, 512)
    budget = 2 * 4096 * 2 * 512 * 4 + 4 * 64 * 8 * 4096
    print("striped S=4096 at the smallest striping budget", flush=True)
    got, plan = _run(q, k, v, do, dlse, lq, lk, ds_budget=budget)
    assert _stored_bytes(plan) == budget
    from gemma4_fa4_amd import ops

    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.backward()
    st.dk.fill_(float("nan"))
    st.backward()
    torch.cuda.synchronize()
    for a, b in zip((st.dq, st.dk, st.dv), got[2:]):
        assert torch.equal(a.cpu(), b)
    dense, _ = _run(q, k, v, do, dlse, lq, lk)
    assert torch.equal(got[2], dense[2])
    for i in (3, 4):
        assert _rel(got[i], dense[i]) < 2e-3


def test_stage_entry_points_recompute_a_striped_problem():
    # g4_attn_bwd_dkdv / g4_attn_bwd_dq on their own cannot interleave stripes:
    # they take the recompute route (dK/dV as the dense route's, to the bit).
    from gemma4_fa4_amd import ops

    q, k, v, do, dlse = qkv(9791, 2048, 2048, 8, 2, 512)
    budget = 2 * 2048 * 2 * 512 * 4 + 4 * 32 * 8 * 4096
    print("stage entry points on a striped S=2048 problem", flush=True)
    got, plan = _run(q, k, v, do, dlse, [2048], [2048], ds_budget=budget)
    dense, _ = _run(q, k, v, do, dlse, [2048], [2048])
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.delta()
    st.dkdv()
    st.dq_stage()
    torch.cuda.synchronize()
    assert torch.equal(st.dk.cpu(), dense[3]) and torch.equal(st.dv.cpu(), dense[4])
    torch.testing.assert_close(st.dq.cpu().float(), dense[2].float(), atol=2e-2, rtol=1e-2)
    assert torch.equal(got[2], dense[2])


def test_global_sequence_past_the_default_ds_budget():
    # 514 rows x 257 key tiles x 32 heads x 4 KB > 16 GiB: with the default
    # budget the packed adapter's backward is striped; pinned budgets give the
    # recompute route (-1) and the dense stored-dS route (20 GiB) on the same
    # inputs.  All three against the fp64 oracle on one full KV group; dQ of
    # the striped and dense routes to the bit, dK / dV of the recompute and
    # dense routes to the bit.
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd.attention import _packed_plan

    s = 16448
    gen = torch.Generator(device=DEV).manual_seed(16448)
    sd = 512 ** -0.25
    q = (torch.randn(s, 32, 512, generator=gen, device=DEV) * sd).to(torch.bfloat16)
    k = (torch.randn(s, 4, 512, generator=gen, device=DEV) * sd).to(torch.bfloat16)
    v = torch.randn(s, 4, 512, generator=gen, device=DEV).to(torch.bfloat16)
    do = torch.randn(s, 32, 512, generator=gen, device=DEV).to(torch.bfloat16)
    c = torch.tensor([0, s], dtype=torch.int32, device=DEV)
    plan = _packed_plan(q, k, c, c, s, s, g.GLOBAL_ATTENTION)
    sums = 2 * s * 4 * 512 * 4
    assert sums < _stored_bytes(plan) <= 16 << 30  # striped at the default budget
    h = slice(8, 16)  # KV group 1 in full, so its dK/dV are complete
    routes = {}
    for name, pin in (("striped", None), ("recompute", -1), ("dense", 20 << 30)):
        print(f"global S={s} through fa4_global_varlen_forward: {name}", flush=True)
        previous = g.pin_backward_ds_budget(pin)
        try:
            qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
            o, lse = g.fa4_global_varlen_forward(qd, kd, vd, c, c, max_seqlen_q=s,
                                                 max_seqlen_k=s)
            torch.autograd.backward(o, do)
            torch.cuda.synchronize()
        finally:
            g.pin_backward_ds_budget(previous)
        routes[name] = [t.detach()[:, h].cpu() for t in (o, qd.grad)] + [
            lse.detach()[h].cpu(), kd.grad[:, 1:2].cpu(), vd.grad[:, 1:2].cpu()]
        del qd, kd, vd, o, lse
    heads = list(range(8, 16))
    cc = [0, s]
    o_ref, l_ref, dq_ref, dk_ref, dv_ref = attention_fwd_bwd(
        q, k, v, cc, cc, do=do, compute_dtype=torch.float64, heads=heads, q_chunk=1024)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(q, k, v, cc, cc, do=do, heads=heads, q_chunk=512)
    for name, (o, dq, lse, dk, dv) in routes.items():
        label = f"S16448 {name}"
        check_forward(o, lse, o_ref[:, h].cpu(), l_ref[h].cpu(), local=False, label=label)
        check_gradients([dq, dk, dv], [dq_ref[:, h].cpu(), dk_ref[:, 1:2].cpu(),
                                       dv_ref[:, 1:2].cpu()],
                        [bq[:, h].cpu(), bk[:, 1:2].cpu(), bv[:, 1:2].cpu()], label=label)
    assert torch.equal(routes["striped"][1], routes["dense"][1])
    assert torch.equal(routes["recompute"][3], routes["dense"][3])
    assert torch.equal(routes["recompute"][4], routes["dense"][4])
    for i in (3, 4):
        assert _rel(routes["striped"][i], routes["dense"][i]) < 2e-3


# ---------------------------------------------------------------------------
# Sequence stripes: several sequences (packed or fixed) past the budget.
# ---------------------------------------------------------------------------


def _run_multi(q, k, v, do, dlse, lq, lk, *, docs=None, ds_budget=0, packed=True):
    """g4_attn_fwd + g4_attn_bwd on a packed (T, H, D) or fixed (B, S, H, D) batch."""
    from gemma4_fa4_amd import ops

    cq, ck = cu(lq), cu(lk)
    plan = ops.make_plan(
        num_seqs=len(lq), seqlen_q=max(lq), seqlen_k=max(lk), num_q_heads=q.shape[1],
        num_kv_heads=k.shape[1], head_dim=512, window=None,
        documents=None if docs is None else docs.to(DEV),
        cu_q=cq.to(DEV) if packed else None, cu_k=ck.to(DEV) if packed else None,
        total_q=q.shape[0], total_k=k.shape[0], ds_budget=ds_budget)
    if not packed:  # B equal sequences: (B, S, H, D) views of the packed buffers
        b = len(lq)
        q, k, v, do = (t.view(b, t.shape[0] // b, *t.shape[1:]) for t in (q, k, v, do))
        dlse = dlse.view(dlse.shape[0], b, -1).permute(1, 0, 2).contiguous()
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.backward()
    torch.cuda.synchronize()
    flat = (lambda t: t) if packed else (lambda t: t.reshape(-1, *t.shape[2:]))
    return [flat(t).cpu() for t in (st.dq, st.dk, st.dv)], plan


def _seq_budget(lq, lk, hq, packed, extra):
    """Budget (bytes) whose stripes hold H = longest rows + extra first rows each."""
    rows_max = (max(lq) + 31) // 32
    per_row = (max(lk) + 63) // 64 * hq * 4096
    dense_rows = sum(lq) // 32 + len(lq) if packed else len(lq) * rows_max
    fit = 2 * rows_max - 1 + extra
    assert fit < dense_rows, "the batch must not fit the budget"
    return fit * per_row, dense_rows * per_row


SEQ_CASES = [
    # (lq, lk, hq, hkv, packed, docs, extra rows)
    ([300, 0, 517, 96, 1000, 64, 700], [300, 40, 600, 96, 1000, 64, 700], 8, 1, True, False, 0),
    ([1024] * 3, [1024] * 3, 16, 2, False, False, 7),  # fixed layout, an empty last stripe
    ([800, 1200, 30, 900], [900, 1200, 30, 1000], 8, 2, True, True, 5),  # documents
    ([400] * 70, [400] * 70, 8, 8, True, False, 3),  # > 64 sequences, work-queue launch
    ([1024] * 40, [1024] * 40, 8, 4, True, False, 20),  # by-length work-queue launch
]


@pytest.mark.parametrize("lq,lk,hq,hkv,packed,with_docs,extra", SEQ_CASES)
def test_sequence_stripes_match_the_dense_route(lq, lk, hq, hkv, packed, with_docs, extra):
    # Each sequence is handled whole by one stripe's launches of the same
    # kernels: dQ, dK and dV equal the dense stored-dS route's to the bit.
    label = f"sequence stripes n={len(lq)} hq={hq} hkv={hkv} packed={packed} docs={with_docs}"
    print(label, flush=True)
    q, k, v, do, dlse = qkv(9800 + len(lq) + hkv, sum(lq), sum(lk), hq, hkv, 512)
    docs = None
    if with_docs:
        docs = torch.zeros(sum(lk), dtype=torch.int32)
        docs[500:] = 1
        docs[1700:] = 2
    budget, dense_bytes = _seq_budget(lq, lk, hq, packed, extra)
    got, plan = _run_multi(q, k, v, do, dlse, lq, lk, docs=docs, ds_budget=budget,
                           packed=packed)
    assert 0 < _stored_bytes(plan) <= budget, "the batch is not striped"
    dense, dplan = _run_multi(q, k, v, do, dlse, lq, lk, docs=docs, packed=packed)
    assert _stored_bytes(dplan) == dense_bytes
    for i, name in enumerate(("dQ", "dK", "dV")):
        assert torch.equal(got[i], dense[i]), f"{name} differs from the dense route"
    if len(lq) <= 8:
        cq, ck = cu(lq), cu(lk)
        args = dict(document_ids=None if docs is None else docs.to(DEV))
        _o, _l, *refs = attention_fwd_bwd(
            q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
            dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
        _, bq, bk, bv = bf16_baseline_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(),
                                              ck.tolist(), do=do.to(DEV), dlse=dlse.to(DEV),
                                              **args)
        check_gradients(got, [t.cpu() for t in refs], [t.cpu() for t in (bq, bk, bv)],
                        label=label)


def test_packed_adapter_backward_takes_sequence_stripes():
    # Through fa4_global_varlen_forward: a pinned budget below the batch's dense
    # tiles but above two longest sequences' rows gives the striped route, with
    # gradients equal to the dense route's.
    import gemma4_fa4_amd as g

    lq = [700, 1500, 300, 1100]
    q, k, v, do, _dl = qkv(9850, sum(lq), sum(lq), 32, 4, 512)
    q, k, v, do = (t.to(DEV) for t in (q, k, v, do))
    c = cu(lq).to(DEV)
    budget, _dense = _seq_budget(lq, lq, 32, True, 2)
    grads = {}
    for name, pin in (("striped", budget), ("dense", 1 << 34)):
        print(f"packed adapter backward: {name}", flush=True)
        previous = g.pin_backward_ds_budget(pin)
        try:
            qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
            o, _lse = g.fa4_global_varlen_forward(qd, kd, vd, c, c, max_seqlen_q=max(lq),
                                                  max_seqlen_k=max(lq))
            torch.autograd.backward(o, do)
            torch.cuda.synchronize()
        finally:
            g.pin_backward_ds_budget(previous)
        grads[name] = [t.grad.cpu() for t in (qd, kd, vd)]
    for a, b in zip(grads["striped"], grads["dense"]):
        assert torch.equal(a, b)
