"""The benchmark workload definitions: shapes per configuration and exact pair counts.

The interval-arithmetic pair counter is pinned against the oracle's mask-based
count (oracle/flops.py exact_pair_count) on small random packed workloads
with vision blocks and documents, and against the closed forms of the
reference's text-only count (reference.py:331-343).
"""

import numpy as np
import pytest

from gemma4_fa4_amd import workloads as wl
from oracle.flops import exact_pair_count, valid_pair_count


def _small(seed, kind, lengths, vision_frac, with_docs):
    rng = np.random.default_rng(seed)
    t = sum(lengths)
    vision = np.full(t, -1, dtype=np.int32)
    docs = np.zeros(t, dtype=np.int32) if with_docs else None
    start, nid = 0, 0
    for si, n in enumerate(lengths):
        if with_docs:
            cut = int(rng.integers(0, n + 1))  # two documents per segment
            docs[start: start + cut] = 2 * si
            docs[start + cut: start + n] = 2 * si + 1
        if vision_frac:
            nid += wl._place_blocks(rng, n, 3, 3, 20, nid, vision, start)
        start += n
    if with_docs:
        # vision blocks must not straddle a document boundary
        for b in np.unique(vision[vision >= 0]):
            idx = np.nonzero(vision == b)[0]
            if len(np.unique(docs[idx])) > 1:
                vision[idx] = -1
    w = wl.Workload("small", kind, lengths, ("fwd",), vision=vision if vision_frac else None,
                    documents=docs)
    return w


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("with_docs", [False, True])
def test_pair_count_matches_the_oracle_mask_count(seed, with_docs, monkeypatch):
    lengths = [37, 1, 90, 64]
    w = _small(seed, "local", lengths, vision_frac=True, with_docs=with_docs)
    monkeypatch.setattr(wl, "LOCAL_WINDOW", 16)
    monkeypatch.setattr(wl.Workload, "window", property(lambda self: 16))
    cu = w.cu()
    expected = exact_pair_count(cu, cu, sliding_window=16, vision_block_ids=w.vision,
                                document_ids=w.documents, allow_vision_bidirectional=True)
    assert wl.allowed_pairs(w) == expected


def test_text_counts_match_the_reference_closed_forms():
    for cfg in (wl.config1, wl.config2, wl.config4):
        w = cfg()
        assert wl.allowed_pairs(w) == wl.text_pairs(w)
        assert wl.text_pairs(w) == sum(valid_pair_count(n, w.window) for n in w.seg_lengths)
    assert wl.allowed_pairs(wl.config1()) == 1_573_376
    assert wl.allowed_pairs(wl.config2()) == 33_558_528


def test_workload_shapes_follow_the_configurations():
    c3 = wl.config3()
    assert c3.tokens == 8192 and c3.kind == "local"
    ids = c3.vision[c3.vision >= 0]
    assert len(np.unique(ids)) == 4
    for b in np.unique(ids):
        n = int((c3.vision == b).sum())
        assert 256 <= n <= 1120
    assert wl.allowed_pairs(c3) > wl.text_pairs(c3)

    c4 = wl.config4()
    assert c4.tokens == 32768 and all(1 <= n <= 2048 for n in c4.seg_lengths)
    assert c4.modes == ("bwd",) and (c4.hkv, c4.d) == (4, 512)

    c5 = wl.config5()
    assert c5.tokens == 131072 and len(c5.seg_lengths) == 8
    assert max(c5.seg_lengths) <= 65536
    frac = float((c5.vision >= 0).mean())
    assert 0.08 <= frac <= 0.25
    cu = c5.cu()
    for s in range(8):
        assert len(np.unique(c5.documents[cu[s]: cu[s + 1]])) == 1
    for b in np.unique(c5.vision[c5.vision >= 0]):
        idx = np.nonzero(c5.vision == b)[0]
        assert idx[-1] - idx[0] + 1 == len(idx) and 256 <= len(idx) <= 1120
        assert len(np.unique(c5.documents[idx])) == 1


def test_workloads_are_seed_deterministic():
    a, b = wl.config5(), wl.config5()
    assert a.seg_lengths == b.seg_lengths and np.array_equal(a.vision, b.vision)
    t1 = wl.tensors(wl.config1(), "cpu")
    t2 = wl.tensors(wl.config1(), "cpu")
    assert all((x is None and y is None) or bool((x == y).all()) for x, y in zip(t1, t2))


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("with_docs", [False, True])
def test_allowed_intervals_are_the_mask_rows(seed, with_docs, monkeypatch):
    # Every row of the oracle's mask is one interval [lo, hi] of the packed
    # key stream (the Q=0 closed forms of the full-size GPU tests rely on it).
    import torch

    from oracle.masks import gemma4_attention_mask

    lengths = [37, 1, 90, 64]
    w = _small(seed, "local", lengths, vision_frac=True, with_docs=with_docs)
    monkeypatch.setattr(wl.Workload, "window", property(lambda self: 16))
    lo, hi = wl.allowed_intervals(w)
    cu = w.cu()
    for s in range(len(lengths)):
        a, b = cu[s], cu[s + 1]
        mask = gemma4_attention_mask(
            batch_size=1, q_len=b - a, kv_len=b - a, sliding_window=16,
            vision_block_ids=torch.from_numpy(w.vision[a:b])[None],
            document_ids=None if w.documents is None else torch.from_numpy(w.documents[a:b])[None],
            allow_vision_bidirectional=True)[0, 0].numpy()
        for i in range(b - a):
            row = np.nonzero(mask[i])[0]
            assert row[0] == lo[a + i] - a and row[-1] == hi[a + i] - a
            assert len(row) == row[-1] - row[0] + 1


def test_allowed_intervals_of_a_global_workload_are_causal_prefixes():
    w = wl.config4()
    lo, hi = wl.allowed_intervals(w)
    cu = w.cu()
    for s in range(len(w.seg_lengths)):
        assert np.all(lo[cu[s]: cu[s + 1]] == cu[s])
        assert np.array_equal(hi[cu[s]: cu[s + 1]], np.arange(cu[s], cu[s + 1]))
