"""C-ABI parity over head layouts beyond the Gemma 4 31B ones.

The adapters lock the model's head counts (32 Q / 16 KV at d256, 32 Q / 4 KV at
d512), but the library takes any GQA ratio in {1, 2, 4, 8} and any head count.
The backward kernels walk (query tile, query head) steps with the GQA group's
heads innermost and reduce the group on chip, so each ratio is a different
step order; these cases run the forward and the three backward stages through
``ops.Stages`` (straight C-ABI calls) against the fp64 oracle, packed with
ragged and empty segments, with document IDs on every case and vision
blocks on the local ones.
"""

import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv, vision_blocks
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stages(q, k, v, do, dlse, cq, ck, window, vis=None, docs=None):
    from gemma4_fa4_amd import ops

    plan = ops.make_plan(
        num_seqs=len(cq) - 1, seqlen_q=int((cq[1:] - cq[:-1]).max()),
        seqlen_k=int((ck[1:] - ck[:-1]).max()), num_q_heads=q.shape[1],
        num_kv_heads=k.shape[1], head_dim=q.shape[2], window=window,
        vision=None if vis is None else vis.to(DEV),
        documents=None if docs is None else docs.to(DEV), cu_q=cq.to(DEV), cu_k=ck.to(DEV),
        total_q=q.shape[0], total_k=k.shape[0])
    st = ops.Stages(plan, q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV), dlse.to(DEV))
    st.forward()
    st.delta()
    st.dkdv()
    st.dq_stage()
    torch.cuda.synchronize()
    return st


def _oracle(q, k, v, do, dlse, cq, ck, window, vis=None, docs=None):
    big = q.shape[0] * q.shape[1] * k.shape[0] > 16 * 600 * 600
    dev = DEV if big else "cpu"
    args = dict(sliding_window=window, vision_block_ids=None if vis is None else vis.to(dev),
                document_ids=None if docs is None else docs.to(dev),
                allow_vision_bidirectional=window is not None and vis is not None)
    o, lse, dq, dk, dv = attention_fwd_bwd(
        q.to(dev), k.to(dev), v.to(dev), cq.tolist(), ck.tolist(), do=do.to(dev),
        dlse=dlse.to(dev), compute_dtype=torch.float64, **args)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(
        q.to(dev), k.to(dev), v.to(dev), cq.tolist(), ck.tolist(), do=do.to(dev),
        dlse=dlse.to(dev), **args)
    return [t.cpu() for t in (o, lse, dq, dk, dv)], [t.cpu() for t in (bq, bk, bv)]


@pytest.mark.parametrize("hq,hkv,d", [
    (8, 8, 256), (16, 4, 256), (8, 1, 256),
    (4, 4, 512), (16, 8, 512), (8, 2, 512),
])
def test_gqa_ratios_through_the_c_abi(hq, hkv, d):
    local = d == 256
    window = 1024 if local else None
    lq, lk = [200, 0, 1100, 33], [260, 7, 1100, 33]
    q, k, v, do, dlse = qkv(8000 + hq * 10 + hkv, sum(lq), sum(lk), hq, hkv, d)
    vis = None
    docs = torch.zeros(sum(lk), dtype=torch.int32)  # document IDs on every case
    docs[sum(lk) // 2:] = 1
    if local:
        vis = vision_blocks(31, sum(lk), 3, 40, 300)
    cq, ck = cu(lq), cu(lk)
    st = _stages(q, k, v, do, dlse, cq, ck, window, vis, docs)
    (o_ref, l_ref, *refs), bf = _oracle(q, k, v, do, dlse, cq, ck, window, vis, docs)
    label = f"hq={hq} hkv={hkv} d={d}"
    check_forward(st.o, st.lse, o_ref, l_ref, local=local, label=label)
    check_gradients([st.dq, st.dk, st.dv], refs, bf, label=label)
    # keys of the Q-empty segment get exact-zero gradients
    k0, k1 = lk[0], lk[0] + lk[1]
    assert torch.all(st.dk[k0:k1] == 0) and torch.all(st.dv[k0:k1] == 0)
