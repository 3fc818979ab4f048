"""Seeded sweep of random problems through the C ABI against the fp64 oracle.

Each case draws (from its seed) a head dimension, a GQA ratio, fixed or packed
layout, 1-5 sequences of random query and key lengths (queries the lower-right
suffix of their keys, including empty and one-token sequences), and for head
dim 256 random vision blocks and documents, sometimes a decode shape (a few
queries over many keys: the split-key forward) and sometimes a small dS
budget (striped or recompute backward).  The workspace and the outputs start
filled with NaN or large finite bytes.  The forward and the whole backward
(g4_attn_bwd) are checked against the fp64 oracle with the M1 envelopes.  The
cases are fixed by their seeds; the sweep exists to reach combinations the
targeted tests do not list one by one.
"""

import numpy as np
import pytest
import torch

from g4_testutil import check_forward, check_gradients, cu, qkv
from oracle.attention import attention_fwd_bwd, bf16_baseline_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _draw(seed):
    rng = np.random.default_rng(seed)
    d = int(rng.choice([256, 512]))
    grp = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 4])) if d == 512 else int(rng.choice([2, 4, 8]))
    hq = hkv * grp
    packed = bool(rng.integers(0, 4) > 0)
    nseq = int(rng.integers(1, 6)) if packed else int(rng.integers(1, 3))
    decode = bool(rng.integers(0, 4) == 0)
    if packed:
        lk = [int(x) for x in rng.integers(1, 900, size=nseq)]
        if decode:
            lk = [int(x) for x in rng.integers(256, 3000, size=nseq)]
            lq = [int(rng.integers(1, max(2, 32 // grp + 1))) for _ in lk]
        else:
            lq = [int(rng.integers(0, x + 1)) for x in lk]
        if sum(lq) == 0:
            lq[0] = 1
        lq = [min(a, b) for a, b in zip(lq, lk)]
    else:
        s_k = int(rng.integers(256, 3000)) if decode else int(rng.integers(1, 900))
        s_q = int(rng.integers(1, max(2, 32 // grp + 1))) if decode else int(rng.integers(1, s_k + 1))
        lq, lk = [min(s_q, s_k)] * nseq, [s_k] * nseq
    window = 1024 if d == 256 else None
    vis = docs = None
    tk = sum(lk)
    if d == 256 and not decode and rng.integers(0, 2):
        vis = np.full(tk, -1, dtype=np.int32)
        for b in range(int(rng.integers(1, 4))):
            a = int(rng.integers(0, tk))
            n = int(rng.integers(1, 300))
            vis[a:a + n] = b
        vis = torch.from_numpy(vis)
    if packed and not decode and rng.integers(0, 3) == 0:
        docs = torch.from_numpy(np.sort(rng.integers(0, 3, size=tk)).astype(np.int32))
    budget = 0
    if d == 512 and not decode and rng.integers(0, 3) == 0:
        budget = int(rng.choice([-1, 4 << 20, 16 << 20]))
    elif d == 256 and not decode and rng.integers(0, 4) == 0:
        budget = -1  # no stored dS band: the dQ stage recomputes S and dP
    return dict(d=d, hq=hq, hkv=hkv, packed=packed, lq=lq, lk=lk, window=window, vis=vis,
                docs=docs, budget=budget)


@pytest.mark.parametrize("seed", list(range(96)))
def test_random_problem_matches_the_oracle(seed):
    from gemma4_fa4_amd import ops

    c = _draw(1000 + seed)
    d, hq, hkv, lq, lk = c["d"], c["hq"], c["hkv"], c["lq"], c["lk"]
    label = (f"seed {seed}: d{d} hq={hq} hkv={hkv} packed={c['packed']} lq={lq} lk={lk} "
             f"vision={c['vis'] is not None} docs={c['docs'] is not None} budget={c['budget']}")
    print(label, flush=True)
    q, k, v, do, dlse = qkv(5000 + seed, sum(lq), sum(lk), hq, hkv, d)
    cq, ck = cu(lq), cu(lk)
    packed = c["packed"]
    plan = ops.make_plan(
        num_seqs=len(lq), seqlen_q=max(max(lq), 1), seqlen_k=max(lk), num_q_heads=hq,
        num_kv_heads=hkv, head_dim=d, window=c["window"],
        vision=None if c["vis"] is None else c["vis"].to(DEV),
        documents=None if c["docs"] is None else c["docs"].to(DEV),
        cu_q=cq.to(DEV) if packed else None, cu_k=ck.to(DEV) if packed else None,
        total_q=q.shape[0], total_k=k.shape[0], ds_budget=c["budget"])
    if packed:
        args = [t.to(DEV) for t in (q, k, v, do)]
        dl = dlse.to(DEV)
    else:
        b = len(lq)
        args = [t.view(b, t.shape[0] // b, *t.shape[1:]).to(DEV) for t in (q, k, v, do)]
        dl = dlse.view(hq, b, -1).permute(1, 0, 2).contiguous().to(DEV)
    st = ops.Stages(plan, *args, dl)
    # The workspace and the outputs are uninitialised memory for the library:
    # fill them with NaN (0xFF) or large finite (0x7F) bytes, so a value read
    # before it is written, or an output element never written, shows.
    for t in (st.ws, st.o, st.lse, st.dq, st.dk, st.dv):
        t.view(torch.uint8).fill_(0xFF if seed % 2 else 0x7F)
    st.forward()
    st.backward()
    torch.cuda.synchronize()
    flat = (lambda t: t.cpu()) if packed else (lambda t: t.reshape(-1, *t.shape[2:]).cpu())
    o, dq, dk, dv = (flat(t) for t in (st.o, st.dq, st.dk, st.dv))
    lse = st.lse.cpu() if packed else st.lse.permute(1, 0, 2).reshape(hq, -1).cpu()
    kw = dict(sliding_window=c["window"],
              vision_block_ids=None if c["vis"] is None else c["vis"].to(DEV),
              document_ids=None if c["docs"] is None else c["docs"].to(DEV),
              allow_vision_bidirectional=c["window"] is not None and c["vis"] is not None)
    o_ref, l_ref, *refs = attention_fwd_bwd(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(), ck.tolist(), do=do.to(DEV),
        dlse=dlse.to(DEV), compute_dtype=torch.float64, **kw)
    _, bq, bk, bv = bf16_baseline_fwd_bwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.tolist(),
                                          ck.tolist(), do=do.to(DEV), dlse=dlse.to(DEV), **kw)
    check_forward(o, lse, o_ref.cpu(), l_ref.cpu(), local=c["window"] is not None, label=label)
    check_gradients([dq, dk, dv], [t.cpu() for t in refs], [t.cpu() for t in (bq, bk, bv)],
                    label=label)
