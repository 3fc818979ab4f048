"""Split-key forward (decode): few query rows per KV head over a long key range.

A problem without key metadata whose query rows of one KV head (query heads of
the group x queries) fit one 32-row tile, over at least 256 keys, runs one
workgroup per (sequence, KV head, chunk of keys) and a merge of the chunks by
their running maxima and sums (the StaticCache decode operators' case:
one query against the cache).  Fixed and packed layouts, head dims 512 (global,
causal) and 256 (window 1024), rows from 1 to 32, sequences of one key and
sequences that reach past the window, each against the fp64 oracle.
"""

import pytest
import torch

from g4_testutil import check_forward, cu, qkv
from oracle.attention import attention_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # (d, hq, hkv, window, lq, lk, packed)
    (512, 32, 4, None, [1], [300], False),
    (512, 32, 4, None, [1, 1, 1], [5000, 300, 2000], True),
    (512, 32, 4, None, [4], [9000], False),  # 32 rows
    (512, 32, 4, None, [3, 1, 4], [3000, 1, 700], True),  # a one-key sequence
    (512, 8, 8, None, [2], [4096], False),  # GQA 1
    (256, 32, 16, 1024, [1], [5000], False),
    (256, 32, 16, 1024, [16, 5], [1500, 1100], True),  # 32 rows, past the window
    (256, 32, 16, 1024, [1, 1], [300, 40000], True),
]


@pytest.mark.parametrize("d,hq,hkv,window,lq,lk,packed", CASES)
def test_split_forward_matches_the_oracle(d, hq, hkv, window, lq, lk, packed):
    from gemma4_fa4_amd import _lib, ops

    label = f"split d{d} hq={hq} hkv={hkv} lq={lq} lk={lk} packed={packed}"
    print(label, flush=True)
    q, k, v, _do, _dl = qkv(9900 + d + sum(lk), sum(lq), sum(lk), hq, hkv, d)
    cq, ck = cu(lq), cu(lk)
    plan = ops.make_plan(
        num_seqs=len(lq), seqlen_q=max(lq), seqlen_k=max(lk), num_q_heads=hq,
        num_kv_heads=hkv, head_dim=d, window=window,
        cu_q=cq.to(DEV) if packed else None, cu_k=ck.to(DEV) if packed else None,
        total_q=q.shape[0], total_k=k.shape[0])
    # the workspace holds at least one chunk of partial rows: the split path
    rows = hq // hkv * max(lq)
    assert plan.workspace_bytes(0) >= len(lq) * hkv * rows * (d + 2) * 4
    if packed:
        args = [t.to(DEV) for t in (q, k, v)]
    else:
        assert len(lq) == 1
        args = [t.to(DEV)[None] for t in (q, k, v)]
    st = ops.Stages(plan, *args, args[0], forward_only=True)
    st.forward()
    torch.cuda.synchronize()
    o = st.o.cpu() if packed else st.o[0].cpu()
    lse = st.lse.cpu() if packed else st.lse[0].cpu()
    o_ref, l_ref, *_ = attention_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(),
                                         ck.tolist(), sliding_window=window,
                                         compute_dtype=torch.float64)
    check_forward(o, lse, o_ref.cpu(), l_ref.cpu(), local=window is not None, label=label)
    _lib.load()
