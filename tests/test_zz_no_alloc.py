"""g4_attn_fwd_static: the forward with the library's own static workspace.

The entry point runs the kernels of g4_attn_fwd with the workspace in a
file-scope device array instead of a caller buffer, so it must return exactly
what g4_attn_fwd returns.  Each case makes two calls in a row through the C ABI,
the second on a smaller problem, so the second call starts from the array the
first one left (span tables of a longer K stream, flags of more query groups)
and must still match bit for bit.  Both uses of the workspace are covered: the
vision-span tables (head dim 256 with vision IDs and documents) and the
head-dim 512 pass flags (the wide forward plus its flagged-group pass, forced
here by score jumps above 2^8).
"""

import ctypes

import pytest
import torch

from g4_testutil import cu, qkv, vision_blocks

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _plan(q, k, lq, lk, window, vis=None, docs=None):
    from gemma4_fa4_amd import ops

    cq, ck = cu(lq), cu(lk)
    return ops.make_plan(
        num_seqs=len(lq), seqlen_q=max(lq), seqlen_k=max(lk), num_q_heads=q.shape[1],
        num_kv_heads=k.shape[1], head_dim=q.shape[2], window=window,
        vision=None if vis is None else vis.to(DEV),
        documents=None if docs is None else docs.to(DEV), cu_q=cq.to(DEV), cu_k=ck.to(DEV),
        total_q=q.shape[0], total_k=k.shape[0])


def _both(plan, q, k, v):
    """(O, LSE) from g4_attn_fwd with a caller workspace and from g4_attn_fwd_static."""
    from gemma4_fa4_amd import _lib
    from gemma4_fa4_amd.attention import _layout

    lib = _lib.load()
    prob = plan.problem()
    need = plan.workspace_bytes(0)
    assert 0 < need <= _lib.STATIC_WORKSPACE_BYTES
    outs = []
    for static in (False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full(plan.lse_shape(), float("nan"), dtype=torch.float32, device=DEV)
        stream = torch.cuda.current_stream().cuda_stream
        args = [ctypes.byref(prob), q.data_ptr(), _layout(q, True), k.data_ptr(), _layout(k, True),
                v.data_ptr(), _layout(v, True), o.data_ptr(), _layout(o, True), lse.data_ptr()]
        if static:
            rc = lib.g4_attn_fwd_static(*args, stream)
        else:
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=DEV)
            rc = lib.g4_attn_fwd(*args, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc)
        torch.cuda.synchronize()
        outs.append((o, lse))
    return outs


def _local_case(seed, lq, lk):
    q, k, v, _do, _dl = qkv(seed, sum(lq), sum(lk), 32, 16, 256)
    vis = vision_blocks(seed, sum(lk), 4, 50, 400)
    docs = torch.zeros(sum(lk), dtype=torch.int32)
    docs[sum(lk) // 2:] = 1
    plan = _plan(q, k, lq, lk, 1024, vis, docs)
    return plan, q.to(DEV), k.to(DEV), v.to(DEV)


def _global_case(seed, lq, lk):
    jumps = seed == 11
    q, k, v, _do, _dl = qkv(seed, sum(lq), sum(lk), 32, 4, 512, unit_logits=not jumps)
    if jumps:
        # Tiny first keys, then N(0, 1) keys against N(0, 1) queries: later
        # tiles' row maxima exceed the first tile's by far more than 2^48 in
        # exp2 terms, so the wide pass flags groups for the rescaling pass.
        for s0 in cu(lk)[:-1].tolist():
            k[s0:s0 + 40] = (k[s0:s0 + 40].float() / 64).to(torch.bfloat16)
    plan = _plan(q, k, lq, lk, None)
    return plan, q.to(DEV), k.to(DEV), v.to(DEV)


@pytest.mark.parametrize("make,first,second", [
    (_local_case, ([1500, 700], [1800, 700]), ([300], [450])),
    (_global_case, ([1200, 333], [1200, 400]), ([200, 64], [260, 64])),
])
def test_static_workspace_forward_matches_the_workspace_forward(make, first, second):
    for seed, (lq, lk) in ((11, first), (12, second)):
        plan, q, k, v = make(seed, lq, lk)
        print(f"{make.__name__} lq={lq} lk={lk}: g4_attn_fwd vs g4_attn_fwd_static", flush=True)
        (o_ws, l_ws), (o_st, l_st) = _both(plan, q, k, v)
        assert torch.isfinite(o_ws.float()).all() and torch.isfinite(l_ws).all()
        assert torch.equal(o_ws, o_st), "O differs between the two entry points"
        assert torch.equal(l_ws, l_st), "LSE differs between the two entry points"


def test_static_workspace_forward_replays_under_graph_capture():
    # After one call outside capture (which looks up the array's address on
    # this GPU and sets the kernels' launch attributes), g4_attn_fwd_static
    # records into a HIP graph; every replay, with eager work and a
    # synchronisation between replays, matches the eager g4_attn_fwd bit for bit.
    from gemma4_fa4_amd import _lib
    from gemma4_fa4_amd.attention import _layout

    plan, q, k, v = _local_case(13, [900], [1100])  # vision spans live in the array
    print("graph capture of g4_attn_fwd_static (local d256, vision + documents)", flush=True)
    (o_ws, l_ws), _ = _both(plan, q, k, v)  # includes the static entry point's first call
    lib = _lib.load()
    prob = plan.problem()
    o = torch.empty_like(q)
    lse = torch.empty(plan.lse_shape(), dtype=torch.float32, device=DEV)
    args = [ctypes.byref(prob), q.data_ptr(), _layout(q, True), k.data_ptr(), _layout(k, True),
            v.data_ptr(), _layout(v, True), o.data_ptr(), _layout(o, True), lse.data_ptr()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.g4_attn_fwd_static(*args, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    for _ in range(3):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ws) and torch.equal(lse, l_ws)
