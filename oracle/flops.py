"""Pair counts and the mask-aware FLOP model -- TEST INFRASTRUCTURE ONLY.

``valid_pair_count`` / ``attention_flops`` follow ``src/gemma4_fa4/reference.py:331-356``:
global pairs ``S(S+1)/2``; local pairs ``S*w - w(w-1)/2`` with ``w = min(W, S)``;
fwd FLOPs ``2*B*Hq*pairs*(Dqk+Dv)``; bwd ``2*B*Hq*pairs*(3*Dqk+2*Dv)``.  These count
text-only pairs ("no multimodal expansion", reference.py:345).

``exact_pair_count`` counts the allowed pairs of the full mask (vision, documents,
packed lower-right segments) by interval arithmetic per query; it is the pair
count the benchmark uses for the multimodal and packed configurations.

Pinned by ``tests/test_oracle_flops.py``: the closed forms against the popcount
of the exact boolean mask, and the 2.5x / 3.5x mode ratios of the reference
(tests/test_reference.py:410-414).
"""

from __future__ import annotations

import numpy as np


def valid_pair_count(seqlen: int, sliding_window: int | None) -> int:
    if sliding_window is None:
        return seqlen * (seqlen + 1) // 2
    w = min(sliding_window, seqlen)
    return seqlen * w - w * (w - 1) // 2


def attention_flops(
    pairs: int,
    *,
    num_q_heads: int,
    head_dim_qk: int,
    head_dim_v: int,
    batch: int = 1,
    mode: str = "fwd",
) -> float:
    fwd = 2.0 * batch * num_q_heads * pairs * (head_dim_qk + head_dim_v)
    bwd = 2.0 * batch * num_q_heads * pairs * (3 * head_dim_qk + 2 * head_dim_v)
    if mode == "fwd":
        return fwd
    if mode == "bwd":
        return bwd
    if mode == "fwd_bwd":
        return fwd + bwd
    raise ValueError(mode)


def _segment_pairs(
    lq: int,
    lk: int,
    window: int | None,
    vision: np.ndarray | None,
    docs: np.ndarray | None,
    bidirectional: bool,
) -> int:
    qpos = np.arange(lk - lq, lk, dtype=np.int64)
    docs = np.zeros(lk, dtype=np.int64) if docs is None else docs.astype(np.int64)
    total = 0
    # causal (and windowed) part, restricted to the query's document
    for doc in np.unique(docs[qpos]):
        keys = np.flatnonzero(docs == doc)
        qs = qpos[docs[qpos] == doc]
        hi = np.searchsorted(keys, qs, side="right")
        if window is None:
            lo = np.zeros_like(hi)
        else:
            lo = np.searchsorted(keys, qs - window, side="right")
        total += int((hi - lo).sum())
    # future keys of the same (document, vision block); no right cap
    if bidirectional and vision is not None:
        vision = vision.astype(np.int64)
        vq = vision[qpos]
        sel = vq >= 0
        if sel.any():
            pairs = np.stack([docs[qpos][sel], vq[sel]], axis=1)
            qsel = qpos[sel]
            for doc, vid in np.unique(pairs, axis=0):
                keys = np.flatnonzero((docs == doc) & (vision == vid))
                qs = qsel[(pairs[:, 0] == doc) & (pairs[:, 1] == vid)]
                total += int((len(keys) - np.searchsorted(keys, qs, side="right")).sum())
    return total


def exact_pair_count(
    cu_seqlens_q,
    cu_seqlens_k,
    *,
    sliding_window: int | None,
    vision_block_ids=None,
    document_ids=None,
    allow_vision_bidirectional: bool = False,
) -> int:
    """Allowed (q, k) pairs of one head summed over packed segments."""
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    vision = None if vision_block_ids is None else np.asarray(vision_block_ids)
    docs = None if document_ids is None else np.asarray(document_ids)
    total = 0
    for qs, qe, ks, ke in zip(cq[:-1], cq[1:], ck[:-1], ck[1:]):
        lq, lk = qe - qs, ke - ks
        if lq == 0:
            continue
        total += _segment_pairs(
            lq,
            lk,
            sliding_window,
            None if vision is None else vision[ks:ke],
            None if docs is None else docs[ks:ke],
            allow_vision_bidirectional,
        )
    return total
