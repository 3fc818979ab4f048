"""The five benchmark workloads of the Gemma 4 attention path, as synthetic packed inputs.

Each workload is the configuration the reference's headline benchmark and its
notes describe (bench_attention.py:80-133, 331-367 run configs 1 and 2; the
multimodal and packed configs follow the same value distributions):

1. local d256 sliding forward, S=2048, text only;
2. global d512 causal forward+backward, S=8192;
3. local d256 multimodal forward+backward, S=8192, 4 vision blocks of
   256-1120 tokens at seeded, non-overlapping offsets;
4. packed global d512 backward, 32768 tokens in segments of U[1, 2048]
   tokens (the last one truncated), Sq = Sk per segment;
5. packed local d256 forward+backward, 131072 tokens in 8 segments of at most
   65536 tokens, one document ID per segment, about 15% of tokens in vision
   blocks of 256-1120 tokens inside segments.

Values: Q, K ~ N(0, 1/sqrt(d)) (unit-variance logits), V, dO ~ N(0, 1),
drawn on the CPU from a seeded generator so every device sees the same data.

``allowed_pairs`` counts the mask's allowed (query, key) pairs per head
exactly, by interval arithmetic per row (the mask-aware FLOP model of
reference.py:331-356 counts pairs; for vision masks the future keys of a
row's own vision block are added).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

LOCAL_WINDOW = 1024


@dataclass
class Workload:
    name: str
    kind: str  # "local" (d256, window 1024) or "global" (d512 causal)
    seg_lengths: list[int]
    modes: tuple[str, ...]  # timed: "fwd", "bwd", "fwd_bwd"
    vision: np.ndarray | None = None  # int32 per token, -1 text
    documents: np.ndarray | None = None  # int32 per token
    seed: int = 0
    notes: dict = field(default_factory=dict)
    device_rng: bool = False  # draw the operands on the device (very large workloads)

    @property
    def hq(self) -> int:
        return 32

    @property
    def hkv(self) -> int:
        return 16 if self.kind == "local" else 4

    @property
    def d(self) -> int:
        return 256 if self.kind == "local" else 512

    @property
    def window(self) -> int | None:
        return LOCAL_WINDOW if self.kind == "local" else None

    @property
    def tokens(self) -> int:
        return int(sum(self.seg_lengths))

    def cu(self) -> list[int]:
        return [0, *np.cumsum(self.seg_lengths).tolist()]


def _place_blocks(rng: np.random.Generator, length: int, count: int, lo: int, hi: int,
                  start_id: int, out: np.ndarray, offset: int) -> int:
    """Place up to `count` non-overlapping blocks of U[lo, hi] tokens in [0, length)."""
    placed = 0
    taken = np.zeros(length, dtype=bool)
    tries = 0
    while placed < count and tries < 1000:
        tries += 1
        n = int(rng.integers(lo, hi + 1))
        if n > length:
            continue
        s = int(rng.integers(0, length - n + 1))
        if taken[max(0, s - 1): s + n + 1].any():  # keep blocks apart
            continue
        taken[s: s + n] = True
        out[offset + s: offset + s + n] = start_id + placed
        placed += 1
    return placed


def config1(seed: int = 1) -> Workload:
    return Workload("config1_local_d256_S2048_fwd", "local", [2048], ("fwd",), seed=seed)


def config2(seed: int = 0) -> Workload:
    return Workload("config2_global_d512_S8192_fwd_bwd", "global", [8192],
                    ("fwd", "bwd", "fwd_bwd"), seed=seed)


def config3(seed: int = 3) -> Workload:
    s = 8192
    rng = np.random.default_rng(seed)
    vision = np.full(s, -1, dtype=np.int32)
    n = _place_blocks(rng, s, 4, 256, 1120, 0, vision, 0)
    assert n == 4
    return Workload("config3_local_d256_S8192_vision_fwd_bwd", "local", [s],
                    ("fwd", "bwd", "fwd_bwd"), vision=vision, seed=seed)


def config4(seed: int = 4) -> Workload:
    rng = np.random.default_rng(seed)
    lengths, total = [], 32768
    while sum(lengths) < total:
        lengths.append(int(rng.integers(1, 2049)))
    lengths[-1] -= sum(lengths) - total
    return Workload("config4_packed_global_d512_T32768_bwd", "global", lengths, ("bwd",),
                    seed=seed)


def config5(seed: int = 5) -> Workload:
    rng = np.random.default_rng(seed)
    total, nseg, cap = 131072, 8, 65536
    while True:
        cuts = np.sort(rng.choice(np.arange(1, total), size=nseg - 1, replace=False))
        lengths = np.diff(np.concatenate([[0], cuts, [total]])).tolist()
        if max(lengths) <= cap and min(lengths) >= 1024:
            break
    vision = np.full(total, -1, dtype=np.int32)
    documents = np.zeros(total, dtype=np.int32)
    next_id, start = 0, 0
    for doc, n in enumerate(lengths):
        documents[start: start + n] = doc
        want = int(round(0.15 * n / 688))  # 688 = mean block length
        next_id += _place_blocks(rng, n, max(want, 1), 256, 1120, next_id, vision, start)
        start += n
    return Workload("config5_packed_local_d256_T131072_vision_docs_fwd_bwd", "local",
                    [int(x) for x in lengths], ("fwd", "bwd", "fwd_bwd"), vision=vision,
                    documents=documents, seed=seed)


def config6(seed: int = 6) -> Workload:
    """Long context (not a BASELINE configuration): one global d512 causal sequence of
    65536 tokens, the reference's S64K row (EXP-0035:69-70).  Its dense stored-dS
    buffer (256 GiB) exceeds the default budget, so the backward stores dS stripe by
    stripe (ten stripes of query rows within the 16 GiB default)."""
    return Workload("config6_global_d512_S65536_fwd_bwd", "global", [65536],
                    ("fwd", "bwd", "fwd_bwd"), seed=seed, device_rng=True)


ALL_CONFIGS = (config1, config2, config3, config4, config5)


def _runs_last_index(ids: np.ndarray) -> np.ndarray:
    """For each position, the last index of its maximal run of equal values."""
    n = ids.shape[0]
    change = np.ones(n, dtype=bool)
    change[:-1] = ids[1:] != ids[:-1]
    idx = np.where(change, np.arange(n), n)
    return np.minimum.accumulate(idx[::-1])[::-1]


def _runs_first_index(ids: np.ndarray) -> np.ndarray:
    n = ids.shape[0]
    start = np.ones(n, dtype=bool)
    start[1:] = ids[1:] != ids[:-1]
    idx = np.where(start, np.arange(n), -1)
    return np.maximum.accumulate(idx)


def allowed_intervals(w: Workload) -> tuple[np.ndarray, np.ndarray]:
    """Per token of the packed stream, the allowed keys [lo, hi] (absolute indices).

    Sq = Sk per segment.  Row a (position in its segment) admits keys
    [max(first of its document run, a - W + 1), a] and, for a vision token, the
    later keys of its own vision block up to the block's end (blocks are
    contiguous runs inside one document, by construction), so every row's
    allowed set is one interval.
    """
    lo_all = np.empty(w.tokens, dtype=np.int64)
    hi_all = np.empty(w.tokens, dtype=np.int64)
    start = 0
    for n in w.seg_lengths:
        a = np.arange(n, dtype=np.int64)
        lo = np.zeros(n, dtype=np.int64)
        if w.documents is not None:
            lo = _runs_first_index(w.documents[start: start + n]).astype(np.int64)
        if w.window is not None:
            lo = np.maximum(lo, a - w.window + 1)
        hi = a.copy()
        if w.vision is not None:
            vis = w.vision[start: start + n]
            key = vis.astype(np.int64)
            if w.documents is not None:
                key = key * (1 << 20) + w.documents[start: start + n]
            last = _runs_last_index(key)
            hi = np.where(vis >= 0, np.maximum(a, last), a)
        lo_all[start: start + n] = start + lo
        hi_all[start: start + n] = start + hi
        start += n
    return lo_all, hi_all


def allowed_pairs(w: Workload) -> int:
    """Exact allowed (q, k) pairs per head (the sum of the rows' interval lengths)."""
    lo, hi = allowed_intervals(w)
    return int((hi - lo + 1).sum())


def text_pairs(w: Workload) -> int:
    """The reference's text-only count (valid_pair_count summed over segments)."""
    total = 0
    for n in w.seg_lengths:
        if w.window is None:
            total += n * (n + 1) // 2
        else:
            m = min(w.window, n)
            total += n * m - m * (m - 1) // 2
    return total


def tensors(w: Workload, device, *, device_rng: bool = False):
    """Packed THD bf16 q, k, v, dO and int32 cu / vision / documents on `device`.

    Values are drawn on the CPU from a generator seeded with the workload's
    seed (so every device sees the same data), or, with ``device_rng``, on
    `device` from a device generator with the same seed (same distributions,
    different values; seconds faster for the large configurations).
    """
    where = torch.device(device) if device_rng else torch.device("cpu")
    g = torch.Generator(device=where).manual_seed(w.seed)
    t, sd = w.tokens, w.d ** -0.25

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=where)

    q = (randn(t, w.hq, w.d) * sd).to(torch.bfloat16)
    k = (randn(t, w.hkv, w.d) * sd).to(torch.bfloat16)
    v = randn(t, w.hkv, w.d).to(torch.bfloat16)
    do = randn(t, w.hq, w.d).to(torch.bfloat16)
    cu = torch.tensor(w.cu(), dtype=torch.int32)
    vis = None if w.vision is None else torch.from_numpy(w.vision)
    docs = None if w.documents is None else torch.from_numpy(w.documents)
    move = lambda x: None if x is None else x.to(device)  # noqa: E731
    return [move(x) for x in (q, k, v, do, cu, vis, docs)]
