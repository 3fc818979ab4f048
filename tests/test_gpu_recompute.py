"""C-ABI parity of the backward without stored dS tiles (the dQ stage recomputes S and dP).

The dK/dV stage stores bf16 dS tiles for the dQ stage while they fit the
problem's ``ds_budget`` (16 GiB by default).  Past it -- packed global batches
whose rows times longest segment pass the budget, local bands that do not fit,
and the separate stage entry points of a single global sequence that
``g4_attn_bwd`` would stripe -- the dK/dV kernels run their store-less branch
and dQ comes from the recomputing role kernels (``dq_roles_kernel`` at head
dim 512, ``dq_roles256_kernel`` at 256).  A negative budget forces that route
at small sizes; every case is checked against the fp64 oracle with the
reference's M1 envelopes, and against the stored-dS route.  (A single global
sequence past the budget takes the striped stored-dS route of g4_attn_bwd,
tested on its own.)
"""

import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv, vision_blocks
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stages(q, k, v, do, dlse, cq, ck, window, *, vis=None, docs=None, ds_budget=0,
            packed=True):
    from gemma4_fa4_amd import ops

    lq = (cq[1:] - cq[:-1])
    lk = (ck[1:] - ck[:-1])
    plan = ops.make_plan(
        num_seqs=len(cq) - 1, seqlen_q=int(lq.max()), seqlen_k=int(lk.max()),
        num_q_heads=q.shape[1], num_kv_heads=k.shape[1], head_dim=q.shape[2], window=window,
        vision=None if vis is None else vis.to(DEV),
        documents=None if docs is None else docs.to(DEV),
        cu_q=cq.to(DEV) if packed else None, cu_k=ck.to(DEV) if packed else None,
        total_q=q.shape[0], total_k=k.shape[0], ds_budget=ds_budget)
    if not packed:  # one fixed sequence: (1, S, H, D) views of the same buffers
        q, k, v, do = (t[None] for t in (q, k, v, do))
        dlse = dlse[None]
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.delta()
    st.dkdv()
    st.dq_stage()
    torch.cuda.synchronize()
    squeeze = (lambda t: t) if packed else (lambda t: t[0])
    return [squeeze(t).cpu() for t in (st.o, st.lse, st.dq, st.dk, st.dv)], plan


def _oracle(q, k, v, do, dlse, cq, ck, window, vis=None, docs=None, heads=None):
    args = dict(sliding_window=window, vision_block_ids=None if vis is None else vis.to(DEV),
                document_ids=None if docs is None else docs.to(DEV),
                allow_vision_bidirectional=window is not None and vis is not None, heads=heads)
    ref = attention_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(),
                            do=do.to(DEV), dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(),
                                          ck.tolist(), do=do.to(DEV), dlse=dlse.to(DEV), **args)
    return [t.cpu() for t in ref], [t.cpu() for t in (bq, bk, bv)]


def _workspace_has_no_ds(plan):
    stored = plan.workspace_bytes(1)
    plan.ds_budget = -1
    none = plan.workspace_bytes(1)
    return stored == none


@pytest.mark.parametrize("hq,hkv,packed,with_docs", [
    (32, 4, True, False),
    (32, 4, False, False),
    (8, 8, True, True),
    (16, 2, True, False),
    (8, 1, False, False),
])
def test_d512_dq_recomputed_without_stored_ds(hq, hkv, packed, with_docs):
    lq, lk = ([300, 0, 517, 96], [300, 40, 600, 96]) if packed else ([700], [700])
    label = f"d512 recompute hq={hq} hkv={hkv} packed={packed} docs={with_docs}"
    print(label, flush=True)
    q, k, v, do, dlse = qkv(9100 + hq + hkv, sum(lq), sum(lk), hq, hkv, 512)
    cq, ck = cu(lq), cu(lk)
    docs = None
    if with_docs:
        docs = torch.zeros(sum(lk), dtype=torch.int32)
        docs[sum(lk) // 3:] = 1
    got, plan = _stages(q, k, v, do, dlse, cq, ck, None, docs=docs, ds_budget=-1, packed=packed)
    assert _workspace_has_no_ds(plan)
    (o_ref, l_ref, *refs), bf = _oracle(q, k, v, do, dlse, cq, ck, None, docs=docs)
    check_forward(got[0], got[1], o_ref, l_ref, local=False, label=label)
    check_gradients(got[2:], refs, bf, label=label)
    if packed:  # keys of the Q-empty segment get exact-zero gradients
        k0, k1 = lk[0], lk[0] + lk[1]
        assert torch.all(got[3][k0:k1] == 0) and torch.all(got[4][k0:k1] == 0)
    # the stored-dS route agrees: dK/dV to the bit (same kernel, same order),
    # dQ to fp32 summation order
    stored, _ = _stages(q, k, v, do, dlse, cq, ck, None, docs=docs, packed=packed)
    assert torch.equal(stored[3], got[3]) and torch.equal(stored[4], got[4])
    torch.testing.assert_close(stored[2].float(), got[2].float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("with_vision,with_docs", [(False, False), (True, False), (True, True)])
def test_d256_dq_recomputed_without_stored_ds(with_vision, with_docs):
    lq, lk = [1500, 0, 900, 1300], [1500, 50, 1100, 1300]
    label = f"d256 recompute vision={with_vision} docs={with_docs}"
    print(label, flush=True)
    q, k, v, do, dlse = qkv(9200 + 2 * with_vision + with_docs, sum(lq), sum(lk), 32, 16, 256)
    cq, ck = cu(lq), cu(lk)
    vis = vision_blocks(77, sum(lk), 5, 100, 700) if with_vision else None
    docs = None
    if with_docs:
        docs = torch.zeros(sum(lk), dtype=torch.int32)
        docs[1000:] = 1
        docs[3000:] = 2
    got, plan = _stages(q, k, v, do, dlse, cq, ck, 1024, vis=vis, docs=docs, ds_budget=-1)
    assert _workspace_has_no_ds(plan)
    (o_ref, l_ref, *refs), bf = _oracle(q, k, v, do, dlse, cq, ck, 1024, vis, docs)
    check_forward(got[0], got[1], o_ref, l_ref, local=True, label=label)
    check_gradients(got[2:], refs, bf, label=label)
    stored, _ = _stages(q, k, v, do, dlse, cq, ck, 1024, vis=vis, docs=docs)
    assert torch.equal(stored[3], got[3]) and torch.equal(stored[4], got[4])
    torch.testing.assert_close(stored[2].float(), got[2].float(), atol=2e-2, rtol=1e-2)


def test_d256_budget_between_the_band_and_its_vision_extension():
    # A budget that holds the window band (18 key tiles per row) but not the
    # 18 extra tiles for vision spans past a row's causal end: query tiles whose
    # vision spans reach past the band are recomputed in the second dQ launch.
    lq = lk = [2600]
    q, k, v, do, dlse = qkv(9300, 2600, 2600, 32, 16, 256)
    cq, ck = cu(lq), cu(lk)
    vis = torch.full((2600,), -1, dtype=torch.int32)
    vis[400:1500] = 0  # a 1100-token block: its early rows reach far past the band
    vis[1800:2100] = 1
    rows = 2600 // 32 + 1
    band = rows * 18 * 32 * 4096
    got, plan = _stages(q, k, v, do, dlse, cq, ck, 1024, vis=vis, ds_budget=band + 4096)
    full = plan.workspace_bytes(1)
    plan.ds_budget = -1
    # only the band is stored, plus the list of query tiles the stored-dS dQ
    # pass leaves for recomputation (16 bytes per 128-query tile and head)
    listed = -(-(((2600 + 127) // 128) * 32 * 16) // 256) * 256
    assert full - plan.workspace_bytes(1) == band + listed
    (o_ref, l_ref, *refs), bf = _oracle(q, k, v, do, dlse, cq, ck, 1024, vis)
    check_forward(got[0], got[1], o_ref, l_ref, local=True, label="partial band")
    check_gradients(got[2:], refs, bf, label="partial band")


def test_d256_listed_recompute_past_255_query_heads():
    # The recompute list keeps the query head in a field of its own, so heads
    # past 255 are recomputed as themselves (an 8-bit head field would wrap
    # 256.. onto 0..).  288 query heads, GQA 2, the partial-band budget of the
    # test above; checked on heads either side of 256.
    lq = lk = [2600]
    hq, hkv = 288, 144
    q, k, v, do, dlse = qkv(9400, 2600, 2600, hq, hkv, 256)
    cq, ck = cu(lq), cu(lk)
    vis = torch.full((2600,), -1, dtype=torch.int32)
    vis[400:1500] = 0
    vis[1800:2100] = 1
    band = (2600 // 32 + 1) * 18 * hq * 4096
    got, plan = _stages(q, k, v, do, dlse, cq, ck, 1024, vis=vis, ds_budget=band + 4096)
    heads = [0, 1, 254, 255, 256, 257, 286, 287]
    kvs = sorted({h // 2 for h in heads})
    (o_ref, l_ref, dq_ref, dk_ref, dv_ref), (bq, bk, bv) = _oracle(
        q, k, v, do, dlse, cq, ck, 1024, vis, heads=heads)
    label = "288 query heads, listed recompute"
    check_forward(got[0][:, heads], got[1][heads], o_ref[:, heads], l_ref[heads], local=True,
                  label=label)
    check_gradients([got[2][:, heads], got[3][:, kvs], got[4][:, kvs]],
                    [dq_ref[:, heads], dk_ref[:, kvs], dv_ref[:, kvs]],
                    [bq[:, heads], bk[:, kvs], bv[:, kvs]], label=label)
