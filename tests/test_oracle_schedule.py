"""Pins oracle.schedule against brute-force incidence of the exact mask.

Restates the reference's schedule tests (tests/test_sparse_schedule.py).
"""

from itertools import product

import pytest
import torch

from oracle.masks import gemma4_attention_mask
from oracle.schedule import (
    SparseScheduleWorkLimitExceeded,
    SparseTileRows,
    brute_force_tile_rows,
    build_gemma4_local_sparse_schedule,
    gemma4_local_sparse_storage_upper_bound,
    transpose_rows,
)


def _allowed(vision, docs, q_len):
    return gemma4_attention_mask(
        batch_size=1, q_len=q_len, kv_len=len(vision), sliding_window=1024,
        vision_block_ids=torch.tensor([vision]), document_ids=torch.tensor([docs]),
        allow_vision_bidirectional=True)[0, 0].numpy()


def _check(vision, docs, q_len, fwd=(2, 3), bwd=(3, 2)):
    sched = build_gemma4_local_sparse_schedule(vision, docs, q_length=q_len, k_length=len(vision),
                                               forward_block_size=fwd, backward_block_size=bwd)
    allowed = _allowed(vision, docs, q_len)
    assert sched.forward.rows == brute_force_tile_rows(allowed, fwd)
    bq2k = SparseTileRows(brute_force_tile_rows(allowed, bwd), bwd[0], bwd[1],
                          (len(vision) + bwd[1] - 1) // bwd[1])
    assert sched.backward.rows == transpose_rows(bq2k).rows
    return sched


# tests/test_sparse_schedule.py:72-83
@pytest.mark.parametrize(("vision", "docs", "q_len"), [
    ([-1] * 9, [0] * 9, 9),
    ([-1, 7, 7, -1, 7, 7, -1, -1, 7], [0] * 9, 5),
    ([3] * 8, [0, 0, 0, 0, 1, 1, 1, 1], 4),
    ([0, 0, -1, 0, 0, -1, 0], [2] * 7, 3),
    ([5, -1, 5, -1, 5, -1, 5, -1, 5, -1], [1, 2] * 5, 7),
])
def test_adversarial_metadata(vision, docs, q_len):
    _check(vision, docs, q_len)


# tests/test_sparse_schedule.py:86-91
def test_exhaustive_small_metadata():
    for vision in product((-1, 0, 1), repeat=4):
        for docs in product((0, 1), repeat=4):
            _check(list(vision), list(docs), 3)


# tests/test_sparse_schedule.py:93-118
def test_far_future_vision_but_not_far_past():
    k_len = 2050
    vision = [-1] * k_len
    docs = [0] * k_len
    vision[k_len - 1] = 9
    vision[0] = 9
    s = _check(vision, docs, 1, fwd=(128, 80), bwd=(64, 64))
    assert 0 not in s.forward.rows[0]
    assert (k_len - 1 - 1023) // 80 in s.forward.rows[0]
    s = _check(vision, docs, k_len, fwd=(128, 80), bwd=(64, 64))
    assert (k_len - 1) // 80 in s.forward.rows[0]


# tests/test_sparse_schedule.py:121-131
def test_model_maximum_text_is_window_bounded():
    k_len = 262_144
    s = build_gemma4_local_sparse_schedule([-1] * k_len, [0] * k_len, q_length=1, k_length=k_len)
    assert s.forward.candidate_pairs <= 14
    assert s.backward.candidate_pairs <= 17
    assert s.storage_bytes < 128 * 1024


# tests/test_sparse_schedule.py:134-146
def test_document_mismatch_filtered_from_causal_band():
    s = _check([-1] * 2049, [0] * 2048 + [1], 1, fwd=(128, 80), bwd=(64, 64))
    assert s.forward.rows == ((2048 // 80,),)
    assert all(not r for r in s.backward.rows[:-1])
    assert s.backward.rows[-1] == (0,)


# tests/test_sparse_schedule.py:149-171
def test_model_maximum_future_vision_and_document_isolation():
    k_len, q_len = 262_144, 2049
    qa = k_len - q_len
    vision = [-1] * k_len
    docs = [0] * k_len
    vision[qa] = 7
    vision[-1] = 7
    mismatched = k_len - 161
    vision[mismatched] = 7
    docs[mismatched] = 1
    vision[0] = 7
    s = build_gemma4_local_sparse_schedule(vision, docs, q_length=q_len, k_length=k_len)
    assert (k_len - 1) // 80 in s.forward.rows[0]
    assert mismatched // 80 not in s.forward.rows[0]
    assert 0 not in s.forward.rows[0]
    assert 0 in s.backward.rows[(k_len - 1) // 64]
    assert 0 not in s.backward.rows[mismatched // 64]


# tests/test_sparse_schedule.py:174-175
def test_storage_upper_bound_is_pinned():
    assert gemma4_local_sparse_storage_upper_bound(262_144, 262_144) == 94_027_776


# tests/test_sparse_schedule.py:178-188
def test_work_budget_stops_construction():
    with pytest.raises(SparseScheduleWorkLimitExceeded, match="construction budget"):
        build_gemma4_local_sparse_schedule([0] * 64, [0] * 64, q_length=64, k_length=64,
                                           forward_block_size=(8, 8), backward_block_size=(4, 4),
                                           max_scheduled_score_slots=32 * 8 * 8)


# tests/test_sparse_schedule.py:191-211
def test_rejects_invalid_contract():
    with pytest.raises(ValueError, match="Sq <= Sk"):
        build_gemma4_local_sparse_schedule([-1], [0], q_length=2, k_length=1)
    with pytest.raises(ValueError, match="match Sk"):
        build_gemma4_local_sparse_schedule([-1], [], q_length=1, k_length=1)
    s = build_gemma4_local_sparse_schedule([-1], [0], q_length=1, k_length=1,
                                           forward_block_size=(2, 2), backward_block_size=(3, 2))
    assert s.forward.rows == s.backward.rows == ((0,),)
    with pytest.raises(ValueError, match="sorted and unique"):
        SparseTileRows(((1, 1),), 2, 2, 2)
    with pytest.raises(ValueError, match="out of range"):
        SparseTileRows(((2,),), 2, 2, 2)
