"""Pins oracle.masks against the reference's truth tables and a per-pair brute force."""

from itertools import product

import numpy as np
import pytest
import torch

from oracle.masks import gemma4_attention_mask, mask_predicate_scalar


def _m(**kw):
    return gemma4_attention_mask(batch_size=1, device="cpu", **kw)[0, 0]


# tests/test_masks.py:11-17
def test_sliding_window_exact_lower_bound():
    mask = _m(q_len=6, kv_len=6, sliding_window=4)
    assert mask[5].tolist() == [False, False, True, True, True, True]


# tests/test_masks.py:19-22
def test_text_local_is_causal():
    mask = _m(q_len=4, kv_len=4, sliding_window=4)
    assert not mask[1, 2]
    assert mask[1, 1]


# tests/test_masks.py:25-35
def test_local_vision_span_is_bidirectional_inside_window():
    blocks = torch.tensor([[-1, 7, 7, 7, -1]], dtype=torch.int32)
    mask = _m(q_len=5, kv_len=5, sliding_window=5, vision_block_ids=blocks,
              allow_vision_bidirectional=True)
    assert mask[1, 3]
    assert not mask[0, 1]


# tests/test_masks.py:38-47
def test_global_ignores_vision_bidirectionality():
    blocks = torch.tensor([[-1, 7, 7, 7, -1]], dtype=torch.int32)
    mask = _m(q_len=5, kv_len=5, sliding_window=None, vision_block_ids=blocks,
              allow_vision_bidirectional=False)
    assert not mask[1, 3]


# tests/test_masks.py:50-54
def test_document_boundary_blocks_cross_document_attention():
    docs = torch.tensor([[1, 1, 2, 2]], dtype=torch.int32)
    mask = _m(q_len=4, kv_len=4, sliding_window=None, document_ids=docs)
    assert not mask[3, 1]
    assert mask[3, 2]


# tests/test_masks.py:57-60
def test_key_padding_mask():
    valid = torch.tensor([[True, True, False, False]])
    mask = _m(q_len=4, kv_len=4, sliding_window=None, key_padding_mask=valid)
    assert not mask[:, 2:].any()


# tests/test_masks.py:63-72
def test_invalid_query_offset_is_rejected():
    with pytest.raises(ValueError, match="query positions"):
        gemma4_attention_mask(batch_size=1, q_len=4, kv_len=4, q_start=2, sliding_window=None)


# tests/test_masks.py:75-79
def test_default_query_alignment_is_lower_right():
    mask = _m(q_len=2, kv_len=5, sliding_window=None)
    assert mask[0].tolist() == [True, True, True, True, False]
    assert mask[1].tolist() == [True, True, True, True, True]


# tests/test_masks.py:82-96
def test_vision_future_exception_has_no_right_window_cap():
    blocks = torch.tensor([[5, 5, 5, 5, 5, 5]], dtype=torch.int32)
    mask = _m(q_len=6, kv_len=6, sliding_window=3, vision_block_ids=blocks,
              allow_vision_bidirectional=True)
    assert mask[2, 4]
    assert mask[2, 5]
    assert not mask[5, 0]


def _brute(q_len, kv_len, window, vision, docs, bidir):
    start = kv_len - q_len
    out = np.zeros((q_len, kv_len), dtype=bool)
    for i in range(q_len):
        for j in range(kv_len):
            out[i, j] = mask_predicate_scalar(start + i, j, window=window, vision=vision,
                                              documents=docs, bidirectional=bidir)
    return out


@pytest.mark.parametrize("window", [None, 1, 2, 3])
@pytest.mark.parametrize("q_len", [1, 3, 4])
def test_vectorised_mask_equals_per_pair_predicate_exhaustively(window, q_len):
    kv_len = 4
    for vision in product((-1, 0, 1), repeat=kv_len):
        for docs in product((0, 1), repeat=kv_len):
            got = _m(q_len=q_len, kv_len=kv_len, sliding_window=window,
                     vision_block_ids=torch.tensor([vision]),
                     document_ids=torch.tensor([docs]),
                     allow_vision_bidirectional=True).numpy()
            want = _brute(q_len, kv_len, window, vision, docs, True)
            assert (got == want).all(), (vision, docs)


def test_window_1024_strict_edge_by_predicate():
    # q_abs = 1024 sees k = 1 .. 1024 but not k = 0 (k > q - 1024)
    assert not mask_predicate_scalar(1024, 0, window=1024)
    assert mask_predicate_scalar(1024, 1, window=1024)
