"""Device mask predicate (bit-exact) and device tile-scheduler coverage on the GPU."""

import numpy as np
import pytest
import torch

from g4_testutil import cu, vision_blocks
from oracle.masks import gemma4_attention_mask

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    from gemma4_fa4_amd import ops
    return ops


def _oracle_mask(lq, lk, window, vision, docs, bidir=True):
    return gemma4_attention_mask(
        batch_size=1, q_len=lq, kv_len=lk, sliding_window=window,
        vision_block_ids=None if vision is None else vision[None],
        document_ids=None if docs is None else docs[None],
        allow_vision_bidirectional=bidir and vision is not None)[0, 0]


CASES = [
    # (q lengths, k lengths, window, with vision, with docs, seed)
    ([67], [67], 5, False, False, 0),
    ([67], [67], 5, True, False, 1),
    ([40], [67], 7, True, True, 2),
    ([130], [130], 1024, True, False, 3),
    ([3, 0, 17, 9], [5, 4, 17, 30], 6, True, True, 4),
    ([33, 64, 1], [33, 100, 2], None, False, True, 5),
    ([200], [200], None, False, False, 6),
]


@pytest.mark.parametrize("lq,lk,window,with_vid,with_doc,seed", CASES)
def test_device_mask_is_bit_exact(lq, lk, window, with_vid, with_doc, seed):
    ops = _ops()
    rng = np.random.default_rng(seed)
    tk = sum(lk)
    vision = torch.from_numpy(rng.integers(-1, 3, size=tk).astype(np.int32)) if with_vid else None
    docs = torch.from_numpy(rng.integers(0, 2, size=tk).astype(np.int32)) if with_doc else None
    packed = len(lq) > 1
    plan = ops.make_plan(
        num_seqs=len(lq), seqlen_q=max(lq), seqlen_k=max(lk), num_q_heads=32, num_kv_heads=16,
        head_dim=256, window=window,
        vision=None if vision is None else vision.to(DEV),
        documents=None if docs is None else docs.to(DEV),
        cu_q=cu(lq).to(DEV) if packed else None, cu_k=cu(lk).to(DEV) if packed else None,
        total_q=sum(lq), total_k=tk)
    got = ops.mask_materialize(plan, DEV).cpu()
    ks = 0
    for s, (a, b) in enumerate(zip(lq, lk)):
        seg_v = None if vision is None else vision[ks:ks + b]
        seg_d = None if docs is None else docs[ks:ks + b]
        if a:
            want = _oracle_mask(a, b, window, seg_v, seg_d)
            assert torch.equal(got[s, :a, :b], want), f"segment {s}"
        assert not got[s, a:, :].any() and not got[s, :, b:].any()
        ks += b


def _check_ranges(ranges_q, ranges_k, allowed, row_tile_q, row_tile_k, tight):
    lq, lk = allowed.shape
    for t in range((lq + row_tile_q - 1) // row_tile_q):
        rows = allowed[t * row_tile_q:(t + 1) * row_tile_q]
        cols = np.flatnonzero(rows.any(axis=0))
        lo, hi = ranges_q[t]
        assert lo <= cols.min() and cols.max() < hi, (t, lo, hi, cols.min(), cols.max())
        if tight:
            assert rows[:, lo].any() and rows[:, hi - 1].any()
    for t in range((lk + row_tile_k - 1) // row_tile_k):
        cols = allowed[:, t * row_tile_k:(t + 1) * row_tile_k]
        qs = np.flatnonzero(cols.any(axis=1))
        lo, hi = ranges_k[t]
        if qs.size:
            assert lo <= qs.min() and qs.max() < hi, (t, lo, hi, qs.min(), qs.max())


def _reach(vision, docs, n):
    """Each position's furthest key: its own position, or the last position of
    its (document, vision ID) pair."""
    reach = np.arange(n)
    if vision is not None:
        v = vision.numpy()
        d = docs.numpy() if docs is not None else np.zeros(n, dtype=np.int64)
        last = {}
        for a in range(n):
            if v[a] >= 0:
                last[(int(d[a]), int(v[a]))] = a
        for a in range(n):
            if v[a] >= 0:
                reach[a] = max(a, last[(int(d[a]), int(v[a]))])
    return reach


def _check_key_ranges_hold_band_rows(ranges_k, reach, window, row_tile_k):
    """A query row's stored-dS band runs over the key tiles from its window
    start to its reach, and the dQ pass reads all of them, so each of those key
    tiles must hold the row in its query range (the dK/dV pass then writes the
    tile, zeros where the row attends none of its keys)."""
    for a in range(len(reach)):
        t0 = max(0, a - window + 1) // row_tile_k if window else 0
        for t in range(t0, reach[a] // row_tile_k + 1):
            lo, hi = ranges_k[t]
            assert lo <= a < hi, (a, t, lo, hi)


@pytest.mark.parametrize("seed,length,nblk,window,with_doc", [
    (0, 1500, 3, 1024, False), (1, 3000, 4, 1024, False), (2, 777, 2, 100, True),
    (3, 2600, 5, 1024, False), (4, 4096, 0, 1024, False), (5, 4096, 0, None, False),
])
def test_device_scheduler_ranges_cover_the_mask(seed, length, nblk, window, with_doc):
    ops = _ops()
    vision = vision_blocks(seed, length, nblk, 256, 1120) if nblk else None
    docs = None
    if with_doc:
        docs = torch.zeros(length, dtype=torch.int32)
        docs[length // 2:] = 1
    plan = ops.make_plan(num_seqs=1, seqlen_q=length, seqlen_k=length, num_q_heads=32,
                         num_kv_heads=16, head_dim=256, window=window,
                         vision=None if vision is None else vision.to(DEV),
                         documents=None if docs is None else docs.to(DEV))
    rq = ops.tile_ranges(plan, 0, 128, DEV).cpu()[0].tolist()
    rk = ops.tile_ranges(plan, 1, 64, DEV).cpu()[0].tolist()
    allowed = _oracle_mask(length, length, window, vision, docs).numpy()
    _check_ranges(rq, rk, allowed, 128, 64, tight=docs is None)
    _check_key_ranges_hold_band_rows(rk, _reach(vision, docs, length), window, 64)


def test_device_scheduler_handles_repeated_noncontiguous_ids():
    ops = _ops()
    length = 700
    vision = torch.full((length,), -1, dtype=torch.int32)
    vision[10:20] = 4
    vision[500:510] = 4   # same block ID again, far in the future
    vision[300:305] = 2
    plan = ops.make_plan(num_seqs=1, seqlen_q=length, seqlen_k=length, num_q_heads=32,
                         num_kv_heads=16, head_dim=256, window=1024, vision=vision.to(DEV))
    rq = ops.tile_ranges(plan, 0, 128, DEV).cpu()[0].tolist()
    rk = ops.tile_ranges(plan, 1, 64, DEV).cpu()[0].tolist()
    allowed = _oracle_mask(length, length, 1024, vision, None).numpy()
    _check_ranges(rq, rk, allowed, 128, 64, tight=True)
    assert rq[0][1] == 510  # query 10 reaches key 509
    # Key tiles between the two runs of ID 4 hold the first run's rows.
    _check_key_ranges_hold_band_rows(rk, _reach(vision, None, length), 1024, 64)
    assert rk[5][0] <= 10
