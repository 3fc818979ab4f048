"""Forward parity of the gfx950 kernels against the fp64 oracle (O, LSE)."""

import pytest
import torch

from g4_testutil import GLOBAL, LOCAL, check_forward, cu, oracle_fwd_bwd, qkv, vision_blocks

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g():
    import gemma4_fa4_amd as g
    return g


@pytest.mark.parametrize("s", [1, 2, 31, 63, 64, 65, 127, 128, 129, 255, 1023, 1024, 1025])
def test_local_text_fixed(s):
    g = _g()
    q, k, v, _, _ = qkv(100 + s, s, s, **{k_: LOCAL[k_] for k_ in ("hq", "hkv", "d")})
    o, lse = g.fa4_local_text_forward(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV))
    torch.cuda.synchronize()
    assert o.shape == (1, s, 32, 256) and lse.shape == (1, 32, s) and lse.dtype == torch.float32
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cu([s]), cu([s]), window=1024)
    check_forward(o[0], lse[0], o_ref, l_ref, local=True, label=f"local S={s}")


@pytest.mark.parametrize("s", [1, 31, 64, 129, 511, 1025])
def test_local_text_fixed_unit_normal_inputs(s):
    # the reference's own calibration draws Q and K from N(0, 1) (large logits)
    g = _g()
    q, k, v, _, _ = qkv(7 + s, s, s, 32, 16, 256, unit_logits=False)
    o, lse = g.fa4_local_text_forward(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cu([s]), cu([s]), window=1024)
    check_forward(o[0], lse[0], o_ref, l_ref, local=True, label=f"local N(0,1) S={s}")


@pytest.mark.parametrize("s,nblk", [(129, 2), (700, 3), (1025, 4)])
def test_local_vision_fixed(s, nblk):
    g = _g()
    q, k, v, _, _ = qkv(200 + s, s, s, 32, 16, 256)
    vis = vision_blocks(s, s, nblk, 16, 300)
    o, lse = g.fa4_local_forward(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV),
                                 vision_block_ids=vis[None].to(torch.int64).to(DEV))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cu([s]), cu([s]), window=1024, vision=vis)
    check_forward(o[0], lse[0], o_ref, l_ref, local=True, label=f"local vision S={s}")


@pytest.mark.parametrize("lq,lk,meta", [
    ([5, 0, 130, 64], [5, 3, 200, 64], False),
    ([2048], [2048], False),
    ([700, 1, 1500], [1000, 1, 1500], True),
    ([1200, 900], [1300, 900], True),
])
def test_local_varlen(lq, lk, meta):
    g = _g()
    q, k, v, _, _ = qkv(sum(lk), sum(lq), sum(lk), 32, 16, 256)
    vis = docs = None
    if meta:
        vis = vision_blocks(3, sum(lk), 4, 64, 600)
        docs = torch.zeros(sum(lk), dtype=torch.int32)
        docs[sum(lk) // 3:] = 1
    cq, ck = cu(lq), cu(lk)
    o, lse = g.fa4_local_varlen_forward(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV),
        max_seqlen_q=max(lq), max_seqlen_k=max(lk),
        vision_block_ids=None if vis is None else vis.to(DEV),
        document_ids=None if docs is None else docs.to(DEV))
    assert o.shape == q.shape and lse.shape == (32, sum(lq))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cq, ck, window=1024, vision=vis, docs=docs)
    check_forward(o, lse, o_ref, l_ref, local=True, label=f"local varlen {lq}/{lk}")


def _many_lengths(nseq, seed, hi, extra):
    gen = torch.Generator().manual_seed(seed)
    lq = [int(x) for x in torch.randint(0, hi, (nseq,), generator=gen)]
    lq[:6] = [0, 1, 127, 128, 129, 700]
    lk = [n + int(x) for n, x in zip(lq, torch.randint(0, extra + 1, (nseq,), generator=gen))]
    return lq, lk


@pytest.mark.parametrize("nseq,meta", [(64, True), (65, True), (40, False)])
def test_local_varlen_many_sequences(nseq, meta):
    # A packed batch of 2..64 sequences runs a grid over the query tiles that
    # exist, sequence by sequence (65 takes the grid sized by the longest
    # sequence); with vision and document IDs the first launch lists the tiles
    # it leaves to the second by their index in the full grid.
    g = _g()
    lq, lk = _many_lengths(nseq, 600 + nseq, 300, 40)
    label = f"local varlen {nseq} sequences meta={meta}"
    print(label, flush=True)
    q, k, v, _, _ = qkv(nseq, sum(lq), sum(lk), 32, 16, 256)
    vis = docs = None
    if meta:
        vis = vision_blocks(nseq, sum(lk), 12, 16, 400)
        docs = torch.zeros(sum(lk), dtype=torch.int32)
        docs[sum(lk) // 4:] = 1
        docs[sum(lk) // 2:] = 2
    cq, ck = cu(lq), cu(lk)
    o, lse = g.fa4_local_varlen_forward(
        q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV),
        max_seqlen_q=max(lq), max_seqlen_k=max(lk),
        vision_block_ids=None if vis is None else vis.to(DEV),
        document_ids=None if docs is None else docs.to(DEV))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cq, ck, window=1024, vision=vis, docs=docs)
    check_forward(o, lse, o_ref, l_ref, local=True, label=label)


@pytest.mark.parametrize("s", [1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 511, 512, 513, 1000,
                               1024, 2048])
def test_global_text_fixed(s):
    g = _g()
    q, k, v, _, _ = qkv(300 + s, s, s, 32, 4, 512)
    o, lse = g.fa4_global_text_forward(q[None].to(DEV), k[None].to(DEV), v[None].to(DEV))
    assert o.shape == (1, s, 32, 512) and lse.shape == (1, 32, s)
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cu([s]), cu([s]), window=None)
    check_forward(o[0], lse[0], o_ref, l_ref, local=False, label=f"global S={s}")


def test_global_forward_only_rectangular_batched():
    g = _g()
    b, sq, sk = 2, 100, 333
    qs, ks, vs, refs = [], [], [], []
    for i in range(b):
        q, k, v, _, _ = qkv(400 + i, sq, sk, 32, 4, 512)
        qs.append(q); ks.append(k); vs.append(v)
    q, k, v = (torch.stack(x).to(DEV) for x in (qs, ks, vs))
    with torch.no_grad():
        o, lse = g.fa4_global_forward_only(q, k, v)
    for i in range(b):
        o_ref, l_ref, *_ = oracle_fwd_bwd(qs[i], ks[i], vs[i], cu([sq]), cu([sk]), window=None)
        check_forward(o[i], lse[i], o_ref, l_ref, local=False, label=f"global rect b={i}")


@pytest.mark.parametrize("lq,lk", [([17, 0, 300, 64, 1], [40, 5, 300, 64, 1]), ([2048, 77], [2048, 77])])
def test_global_varlen(lq, lk):
    g = _g()
    q, k, v, _, _ = qkv(500 + sum(lq), sum(lq), sum(lk), 32, 4, 512)
    cq, ck = cu(lq), cu(lk)
    with torch.no_grad():
        o, lse = g.fa4_global_varlen_forward_only(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV),
                                                  ck.to(DEV), max_seqlen_q=max(lq),
                                                  max_seqlen_k=max(lk))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cq, ck, window=None)
    check_forward(o, lse, o_ref, l_ref, local=False, label=f"global varlen {lq}")


@pytest.mark.parametrize("nseq", [64, 65])
def test_global_varlen_many_sequences(nseq):
    # the head-dim 512 fast pass over the tiles that exist (64 sequences) or
    # the full grid (65), then the rescaling pass over the flagged groups
    g = _g()
    lq, lk = _many_lengths(nseq, 700 + nseq, 200, 30)
    print(f"global varlen {nseq} sequences", flush=True)
    q, k, v, _, _ = qkv(800 + nseq, sum(lq), sum(lk), 32, 4, 512, unit_logits=False)
    cq, ck = cu(lq), cu(lk)
    with torch.no_grad():
        o, lse = g.fa4_global_varlen_forward_only(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV),
                                                  ck.to(DEV), max_seqlen_q=max(lq),
                                                  max_seqlen_k=max(lk))
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cq, ck, window=None)
    check_forward(o, lse, o_ref, l_ref, local=False, label=f"global varlen {nseq} sequences")


def test_forward_is_bitwise_repeatable_on_a_side_stream():
    g = _g()
    q, k, v, _, _ = qkv(9, 1025, 1025, 32, 16, 256)
    q, k, v = (t[None].to(DEV) for t in (q, k, v))
    o1, l1 = g.fa4_local_text_forward(q, k, v)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        o2, l2 = g.fa4_local_text_forward(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def _raise_flags(st, nseg, max_q, lq=None):
    """The d512 forward's per-(segment, 32-query group, head) raise flags (workspace head).

    Only the groups inside each segment (lengths lq) are written by the kernels;
    the slots past a shorter segment's end are never read and hold whatever the
    workspace held before.
    """
    nq32 = (max_q + 31) // 32
    flags = st.ws[: 4 * nseg * nq32 * 32].view(torch.int32).cpu().view(nseg, nq32, 32)
    if lq is None:
        return flags.flatten()
    return torch.cat([flags[s, : (n + 31) // 32].flatten() for s, n in enumerate(lq)])


@pytest.mark.parametrize("lq,lk", [([300, 450], [300, 450]), ([130], [700])])
def test_global_rescaling_pass_for_large_score_jumps(lq, lk):
    # Tiny first keys, then N(0, 1) keys against N(0, 1) queries: later tiles'
    # row maxima exceed the first tile's by far more than 2^48 in exp2 terms,
    # so the fast pass flags those rows and the rescaling pass recomputes them.
    from gemma4_fa4_amd import ops
    from gemma4_fa4_amd.attention import _packed_plan

    g = _g()
    q, k, v, _, _ = qkv(900 + sum(lq), sum(lq), sum(lk), 32, 4, 512, unit_logits=False)
    starts = cu(lk)[:-1].tolist()
    for s0 in starts:
        k[s0:s0 + 40] = (k[s0:s0 + 40].float() / 64).to(torch.bfloat16)
    cq, ck = cu(lq), cu(lk)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    plan = _packed_plan(qd, kd, cq.to(DEV), ck.to(DEV), max(lq), max(lk), g.GLOBAL_ATTENTION)
    st = ops.Stages(plan, qd, kd, vd, torch.zeros_like(qd))
    st.forward()
    torch.cuda.synchronize()
    assert int(_raise_flags(st, len(lq), max(lq), lq).sum()) > 0, "no row took the rescaling pass"
    o_ref, l_ref, *_ = oracle_fwd_bwd(q, k, v, cq, ck, window=None)
    check_forward(st.o, st.lse, o_ref, l_ref, local=False, label=f"global rescale {lq}/{lk}")
    o2, lse2 = g.fa4_global_varlen_forward_only(qd, kd, vd, cq.to(DEV), ck.to(DEV),
                                                max_seqlen_q=max(lq), max_seqlen_k=max(lk))
    assert torch.equal(o2, st.o) and torch.equal(lse2, st.lse)


def test_global_unit_logits_need_no_rescaling_pass():
    from gemma4_fa4_amd import ops
    from gemma4_fa4_amd.attention import _packed_plan

    g = _g()
    s = 1000
    q, k, v, _, _ = qkv(77, s, s, 32, 4, 512)
    c = cu([s]).to(DEV)
    st = ops.Stages(_packed_plan(q.to(DEV), k.to(DEV), c, c, s, s, g.GLOBAL_ATTENTION),
                    q.to(DEV), k.to(DEV), v.to(DEV), torch.zeros_like(q).to(DEV))
    st.forward()
    torch.cuda.synchronize()
    assert int(_raise_flags(st, 1, s).sum()) == 0
