"""C-ABI parity of the work-queue variants of the backward tile kernels.

The dK/dV and dQ launchers switch to a persistent launch (each workgroup takes
further tiles from a ticket counter in the workspace) when there are more
than four work items per resident workgroup.  These packed problems of many
short segments have enough items for that (the assertions below check the
item counts against the device's CU count), so the queue variants run here:
d256 local with document IDs and vision blocks (dK/dV and dQ queues), d512
global (paired-key-tile dK/dV queue and the dQ-from-dS queue).  Every stage
runs twice on one workspace, so the second run starts from the counters the
first one left, and must repeat the first bitwise.
"""

import numpy as np
import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lengths(seed, n, lo, hi, n_empty_q):
    rng = np.random.default_rng(seed)
    lk = rng.integers(lo, hi + 1, size=n).tolist()
    lq = list(lk)
    for i in rng.choice(n, size=n_empty_q, replace=False):
        lq[int(i)] = 0  # Q-empty segments: their keys get exact-zero dK / dV
    return lq, lk


def _run(plan, q, k, v, do, dlse):
    from gemma4_fa4_amd import ops

    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    outs = []
    for _ in range(2):
        st.delta()
        st.dkdv()
        st.dq_stage()
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (st.dq, st.dk, st.dv)])
    for a, b in zip(*outs):
        assert torch.equal(a, b), "queue launches are not repeatable"
    return st


def _check(st, q, k, v, do, dlse, cq, ck, lq, lk, *, window, vis=None, docs=None):
    args = dict(sliding_window=window, vision_block_ids=None if vis is None else vis.to(DEV),
                document_ids=None if docs is None else docs.to(DEV),
                allow_vision_bidirectional=window is not None and vis is not None)
    o, lse, dq, dk, dv = attention_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), **args)
    local = window is not None
    check_forward(st.o, st.lse, o.cpu(), lse.cpu(), local=local, label="queue")
    check_gradients([st.dq, st.dk, st.dv], [t.cpu() for t in (dq, dk, dv)],
                    [t.cpu() for t in (bq, bk, bv)], label="queue")
    k_off = np.cumsum([0, *lk])
    for i, n in enumerate(lq):
        if n == 0:
            a, b = int(k_off[i]), int(k_off[i + 1])
            assert torch.all(st.dk[a:b] == 0) and torch.all(st.dv[a:b] == 0)


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def test_local_d256_queue_variants():
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd.attention import _packed_plan

    lq, lk = _lengths(21, 140, 96, 128, 3)
    # one 128-key dK/dV tile and one 128-query dQ tile per segment
    assert len(lk) * 16 > 4 * 2 * _cus() and len(lk) * 32 > 4 * 2 * _cus()
    tq, tk = sum(lq), sum(lk)
    q, k, v, do, dlse = qkv(4242, tq, tk, 32, 16, 256)
    rng = np.random.default_rng(5)
    docs = np.zeros(tk, dtype=np.int32)
    vis = np.full(tk, -1, dtype=np.int32)
    start, nid = 0, 0
    for s, n in enumerate(lk):
        cut = int(rng.integers(0, n + 1))
        docs[start:start + cut] = 2 * s
        docs[start + cut:start + n] = 2 * s + 1
        if s % 3 == 0 and cut >= 40:  # a vision block inside the first document
            b0 = int(rng.integers(0, cut - 30))
            vis[start + b0:start + b0 + 30] = nid
            nid += 1
        start += n
    docs_t, vis_t = torch.from_numpy(docs), torch.from_numpy(vis)
    cq, ck = cu(lq), cu(lk)
    plan = _packed_plan(q.to(DEV), k.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                        g.SLIDING_ATTENTION, vision=vis_t.to(DEV), documents=docs_t.to(DEV))
    st = _run(plan, q, k, v, do, dlse)
    _check(st, q, k, v, do, dlse, cq, ck, lq, lk, window=1024, vis=vis_t, docs=docs_t)


def test_global_d512_queue_variants():
    import gemma4_fa4_amd as g
    from gemma4_fa4_amd.attention import _packed_plan

    lq, lk = _lengths(22, 280, 96, 128, 4)
    # one pair of 64-key dK/dV tiles and one 128-query dQ tile per segment
    assert len(lk) * 4 > 4 * _cus() and len(lk) * 32 > 4 * _cus()
    tq, tk = sum(lq), sum(lk)
    q, k, v, do, dlse = qkv(4343, tq, tk, 32, 4, 512)
    cq, ck = cu(lq), cu(lk)
    plan = _packed_plan(q.to(DEV), k.to(DEV), cq.to(DEV), ck.to(DEV), max(lq), max(lk),
                        g.GLOBAL_ATTENTION)
    st = _run(plan, q, k, v, do, dlse)
    _check(st, q, k, v, do, dlse, cq, ck, lq, lk, window=None)
