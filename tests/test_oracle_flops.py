"""Pins oracle.flops: closed forms against the popcount of the exact mask."""

import numpy as np
import pytest
import torch

from oracle.flops import attention_flops, exact_pair_count, valid_pair_count
from oracle.masks import gemma4_attention_mask


@pytest.mark.parametrize("s", [1, 2, 7, 64, 129, 1025, 2048])
@pytest.mark.parametrize("window", [None, 1024, 3])
def test_valid_pair_count_equals_mask_popcount(s, window):
    mask = gemma4_attention_mask(batch_size=1, q_len=s, kv_len=s, sliding_window=window)
    assert int(mask.sum()) == valid_pair_count(s, window)
    assert exact_pair_count([0, s], [0, s], sliding_window=window) == valid_pair_count(s, window)


def test_baseline_pair_counts():
    # BASELINE c1 (local S=2048) and c2 (global S=8192) pair counts
    assert valid_pair_count(2048, 1024) == 1_573_376
    assert valid_pair_count(8192, None) == 33_558_528
    assert attention_flops(33_558_528, num_q_heads=32, head_dim_qk=512, head_dim_v=512,
                           mode="fwd_bwd") == pytest.approx(7.698e12, rel=1e-3)


# tests/test_reference.py:410-414
def test_flop_mode_ratios():
    f = attention_flops(100, num_q_heads=4, head_dim_qk=8, head_dim_v=8, mode="fwd")
    assert attention_flops(100, num_q_heads=4, head_dim_qk=8, head_dim_v=8, mode="bwd") == 2.5 * f
    assert attention_flops(100, num_q_heads=4, head_dim_qk=8, head_dim_v=8,
                           mode="fwd_bwd") == 3.5 * f


def test_exact_pair_count_with_metadata_matches_mask():
    rng = np.random.default_rng(0)
    for trial in range(40):
        lengths_k = rng.integers(1, 40, size=rng.integers(1, 4)).tolist()
        lengths_q = [int(rng.integers(0, lk + 1)) for lk in lengths_k]
        tk = sum(lengths_k)
        vision = rng.integers(-1, 3, size=tk)
        docs = rng.integers(0, 2, size=tk)
        window = [None, 3, 8][trial % 3]
        bidir = trial % 2 == 0
        want = 0
        ks = 0
        for lq, lk in zip(lengths_q, lengths_k):
            if lq:
                m = gemma4_attention_mask(
                    batch_size=1, q_len=lq, kv_len=lk, sliding_window=window,
                    vision_block_ids=torch.tensor(vision[ks:ks + lk])[None],
                    document_ids=torch.tensor(docs[ks:ks + lk])[None],
                    allow_vision_bidirectional=bidir)
                want += int(m.sum())
            ks += lk
        cq = np.concatenate([[0], np.cumsum(lengths_q)])
        ck = np.concatenate([[0], np.cumsum(lengths_k)])
        got = exact_pair_count(cq, ck, sliding_window=window, vision_block_ids=vision,
                               document_ids=docs, allow_vision_bidirectional=bidir)
        assert got == want
