"""Head-dim 256 backward with stored dS: the band and its recompute routing.

The local dK/dV kernel stores dS tiles in a band of key tiles per 32-query
row (window and causal part plus up to 18 tiles of vision spans); the dQ
stage takes the product over stored tiles for query tiles that stay inside
their band and recomputes the others.  A 1500-token vision block starting
past the first window reaches beyond the band of its first rows (those query
tiles are recomputed) but not of its later rows; documents are added on a
second segment.  Compared with the fp64 oracle through the C ABI stages, and the
stages repeated on one workspace against their first results.
"""

import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_long_vision_block_reaches_past_the_band():
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd import ops
    from gemma4_fa4_amd.attention import _packed_plan

    lens = [3000, 700]
    t = sum(lens)
    q, k, v, do, dlse = qkv(777, t, t, 32, 16, 256)
    vis = torch.full((t,), -1, dtype=torch.int32)
    vis[1100:2600] = 0          # 1500 tokens: rows near 1100 reach past their band
    vis[3000 + 100:3000 + 180] = 1
    docs = torch.zeros(t, dtype=torch.int32)
    docs[3000 + 400:] = 1       # second segment: two documents, the block in the first
    c = cu(lens)
    plan = _packed_plan(q.to(DEV), k.to(DEV), c.to(DEV), c.to(DEV), max(lens), max(lens),
                        g.SLIDING_ATTENTION, vision=vis.to(DEV), documents=docs.to(DEV))
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.delta()
    st.dkdv()
    st.dq_stage()
    torch.cuda.synchronize()
    args = dict(sliding_window=1024, vision_block_ids=vis.to(DEV), document_ids=docs.to(DEV),
                allow_vision_bidirectional=True)
    o, lse, dq, dk, dv = attention_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), c.tolist(), c.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), c.tolist(), c.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), **args)
    check_forward(st.o, st.lse, o.cpu(), lse.cpu(), local=True, label="band")
    check_gradients([st.dq, st.dk, st.dv], [x.cpu() for x in (dq, dk, dv)],
                    [x.cpu() for x in (bq, bk, bv)], label="band")
    # Stages repeated on one workspace (no delta pass between them, which is
    # what zeroes the queue counters): each launch leaves its work-queue
    # counters at zero, so the repeats visit every item again, bit for bit.
    first = [t.clone() for t in (st.dq, st.dk, st.dv)]
    st.dq.fill_(float("nan"))
    st.dq_stage()
    st.dq_stage()
    st.dk.fill_(float("nan"))
    st.dkdv()
    torch.cuda.synchronize()
    for a, b in zip((st.dq, st.dk, st.dv), first):
        assert torch.equal(a, b)


def test_work_queue_stages_repeat_on_one_workspace():
    # 71 query tiles x 16 head pairs = 1136 items: the persistent work-queue
    # launches (per-XCD runs for the stored-dS dQ).  Repeated without the delta
    # pass, each launch must find its counters at zero and redo every item.
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd import ops
    from gemma4_fa4_amd.attention import _packed_plan

    lens = [6000, 3000]
    t = sum(lens)
    q, k, v, do, dlse = qkv(778, t, t, 32, 16, 256)
    c = cu(lens)
    plan = _packed_plan(q.to(DEV), k.to(DEV), c.to(DEV), c.to(DEV), max(lens), max(lens),
                        g.SLIDING_ATTENTION)
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    print("work-queue stages repeated, local T=9000", flush=True)
    st.forward()
    st.delta()
    st.dkdv()
    st.dq_stage()
    torch.cuda.synchronize()
    first = [x.clone() for x in (st.dq, st.dk, st.dv)]
    for _ in range(2):
        st.dq.fill_(float("nan"))
        st.dk.fill_(float("nan"))
        st.dv.fill_(float("nan"))
        st.dkdv()
        st.dq_stage()
        torch.cuda.synchronize()
        for a, b in zip((st.dq, st.dk, st.dv), first):
            assert torch.equal(a, b)


@pytest.mark.parametrize("poison", [0xFF, 0x7F])
def test_repeated_vision_id_with_a_gap_and_a_poisoned_workspace(poison):
    """A vision ID in two runs with another block between them (queries shorter
    than keys, three packed sequences).  Queries of the first run attend the
    second, so the stored-dS dQ pass reads every band tile up to the second
    run's end for their rows, including the tiles of the block between the
    runs, which those queries do not attend: the dK/dV pass must write them
    (zeros).  The workspace is filled with NaN (0xFF) or large finite (0x7F)
    bytes first, so a tile read without being written shows in dQ."""
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd import ops
    from gemma4_fa4_amd.attention import _packed_plan

    lq, lk = [354, 7, 333], [549, 407, 727]
    q, k, v, do, dlse = qkv(5291, sum(lq), sum(lk), 4, 2, 256)
    vis = torch.full((sum(lk),), -1, dtype=torch.int32)
    s2 = lk[0] + lk[1]            # third sequence: queries at key positions 394..726
    vis[s2 + 399:s2 + 440] = 0
    vis[s2 + 440:s2 + 501] = 1    # first run of ID 1
    vis[s2 + 501:s2 + 642] = 2    # the block between the runs
    vis[s2 + 642:s2 + 716] = 1    # second run of ID 1
    vis[100:180] = 3              # and one ordinary block in the first sequence
    cq, ck = cu(lq), cu(lk)
    plan = _packed_plan(q.to(DEV), k.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                        g.SLIDING_ATTENTION, vision=vis.to(DEV))
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    print(f"repeated vision ID, workspace filled with {poison:#x}", flush=True)
    st.ws.fill_(poison)
    st.forward()
    st.backward()
    torch.cuda.synchronize()
    args = dict(sliding_window=1024, vision_block_ids=vis.to(DEV), allow_vision_bidirectional=True)
    o, lse, dq, dk, dv = attention_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), **args)
    check_forward(st.o, st.lse, o.cpu(), lse.cpu(), local=True, label="repeated id")
    check_gradients([st.dq, st.dk, st.dv], [x.cpu() for x in (dq, dk, dv)],
                    [x.cpu() for x in (bq, bk, bv)], label="repeated id")
