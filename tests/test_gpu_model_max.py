"""The device predicate and scheduler at the model's maximum length, and a long local sequence.

The reference pins its local schedule on K = 262,144 sentinels
(tests/test_sparse_schedule.py:121-172): one text query at the end of the
stream (window-bounded work), and 2049 queries whose first one shares a vision
block with the very last key (a far-future key it must see), with a past key of
that block outside the window and a future key of that block in another
document (neither may be seen).  Here the same streams go through the device
mask (``g4_mask_materialize``, bit-exact against the oracle over the whole
grid) and the device scheduler (``g4_tile_ranges``: every allowed pair inside
its tile's range).  The device scheduler bounds each tile by one interval, not
by an exact tile list, so the reference's "tile not listed" assertions become
the mask's exact zeros.  A 65,536-token local sequence with vision blocks then
runs through ``fa4_local_varlen_forward`` against the fp64 oracle on sampled
heads.
"""

import numpy as np
import pytest
import torch

from g4_testutil import check_forward, cu, vision_blocks
from oracle.attention import attention_fwd_bwd
from oracle.masks import gemma4_attention_mask

pytestmark = pytest.mark.gpu

DEV = "cuda"
K_MAX = 262_144


def _plan(lq, lk, vision, docs):
    from gemma4_fa4_amd import ops

    return ops.make_plan(num_seqs=1, seqlen_q=lq, seqlen_k=lk, num_q_heads=32, num_kv_heads=16,
                         head_dim=256, window=1024,
                         vision=None if vision is None else vision.to(DEV),
                         documents=None if docs is None else docs.to(DEV))


def _oracle(lq, lk, vision, docs):
    return gemma4_attention_mask(
        batch_size=1, q_len=lq, kv_len=lk, sliding_window=1024,
        vision_block_ids=None if vision is None else vision[None],
        document_ids=None if docs is None else docs[None],
        allow_vision_bidirectional=vision is not None)[0, 0].numpy()


def _ranges_cover(allowed, rq, rk, row_q=128, row_k=64):
    lq, lk = allowed.shape
    for t in range((lq + row_q - 1) // row_q):
        cols = np.flatnonzero(allowed[t * row_q:(t + 1) * row_q].any(axis=0))
        lo, hi = rq[t]
        assert cols.size == 0 or (lo <= cols.min() and cols.max() < hi), (t, lo, hi)
    keys_seen = allowed.any(axis=0)
    for t in np.flatnonzero(keys_seen.reshape(-1, row_k).any(axis=1)):
        qs = np.flatnonzero(allowed[:, t * row_k:(t + 1) * row_k].any(axis=1))
        lo, hi = rk[t]
        assert lo <= qs.min() and qs.max() < hi, (t, lo, hi)


def test_model_maximum_text_query_is_window_bounded():
    from gemma4_fa4_amd import ops

    print(f"text Q1 K={K_MAX}", flush=True)
    docs = torch.zeros(K_MAX, dtype=torch.int32)
    vision = torch.full((K_MAX,), -1, dtype=torch.int32)
    plan = _plan(1, K_MAX, vision, docs)
    got = ops.mask_materialize(plan, DEV).cpu()[0].numpy().astype(bool)
    want = _oracle(1, K_MAX, vision, docs)
    assert np.array_equal(got, want)
    assert np.flatnonzero(want[0]).tolist() == list(range(K_MAX - 1024, K_MAX))
    rq = ops.tile_ranges(plan, 0, 128, DEV).cpu()[0].tolist()
    rk = ops.tile_ranges(plan, 1, 64, DEV).cpu()[0].tolist()
    assert rq == [[K_MAX - 1024, K_MAX]]  # exactly the window: 1024 keys
    busy = [t for t, (lo, hi) in enumerate(rk) if hi > lo]
    assert busy == list(range((K_MAX - 1024) // 64, K_MAX // 64))  # 16 key tiles, <= 17
    _ranges_cover(want, rq, rk)


def test_model_maximum_future_vision_and_document_isolation():
    from gemma4_fa4_amd import ops

    lq = 2049
    qa = K_MAX - lq  # K position of the first query
    vision = torch.full((K_MAX,), -1, dtype=torch.int32)
    docs = torch.zeros(K_MAX, dtype=torch.int32)
    vision[qa] = 7
    vision[-1] = 7  # far-future key of the first query's block
    mismatched = K_MAX - 161
    vision[mismatched] = 7  # same block, another document
    docs[mismatched] = 1
    vision[0] = 7  # same block, far outside the window
    print(f"vision/document sentinels Q{lq} K={K_MAX}", flush=True)
    plan = _plan(lq, K_MAX, vision, docs)
    got = ops.mask_materialize(plan, DEV).cpu()[0].numpy().astype(bool)
    want = _oracle(lq, K_MAX, vision, docs)
    assert np.array_equal(got, want)
    # the reference's sentinels, on the exact mask
    assert want[0, K_MAX - 1] and not want[0, mismatched] and not want[0, 0]
    assert not want[:, 0].any()
    rq = ops.tile_ranges(plan, 0, 128, DEV).cpu()[0].tolist()
    rk = ops.tile_ranges(plan, 1, 64, DEV).cpu()[0].tolist()
    assert rq[0][1] == K_MAX  # the first query tile reaches the far-future key
    assert rq[0][0] > 0  # but not the block's key at 0
    assert rk[(K_MAX - 1) // 64][0] <= 0  # the last key tile is seen from query 0
    _ranges_cover(want, rq, rk)


def test_long_local_sequence_with_vision_blocks_matches_the_oracle():
    import gemma4_fa4_amd as g

    s = 65_536
    print(f"local S={s} with vision blocks through fa4_local_varlen_forward", flush=True)
    gen = torch.Generator().manual_seed(65536)
    sd = 256 ** -0.25
    q = (torch.randn(s, 32, 256, generator=gen) * sd).to(torch.bfloat16)
    k = (torch.randn(s, 16, 256, generator=gen) * sd).to(torch.bfloat16)
    v = torch.randn(s, 16, 256, generator=gen).to(torch.bfloat16)
    vision = vision_blocks(65, s, 12, 256, 1120)
    assert int((vision >= 0).sum()) > 0
    c = cu([s])
    qd, kd, vd, cd, visd = (t.to(DEV) for t in (q, k, v, c, vision))
    with torch.no_grad():
        o, lse = g.fa4_local_varlen_forward(qd, kd, vd, cd, cd, max_seqlen_q=s, max_seqlen_k=s,
                                            vision_block_ids=visd)
    torch.cuda.synchronize()
    heads = [0, 17, 31]
    o_ref, l_ref, *_ = attention_fwd_bwd(qd, kd, vd, [0, s], [0, s], sliding_window=1024,
                                         vision_block_ids=visd, allow_vision_bidirectional=True,
                                         compute_dtype=torch.float64, heads=heads, q_chunk=1024)
    check_forward(o[:, heads].cpu(), lse[heads].cpu(), o_ref[:, heads].cpu(),
                  l_ref[heads].cpu(), local=True, label=f"local S={s}")
