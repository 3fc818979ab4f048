"""Exact tile incidence of the local Gemma mask -- TEST INFRASTRUCTURE ONLY.

Restates ``src/gemma4_fa4/sparse_schedule.py``:

* ``SparseTileRows`` (18-56): ordered row-tile -> column-tile adjacency, compact
  width ``max(1, longest row)``, storage ``4 * rows * (3 + width)`` bytes.
* ``build_gemma4_local_sparse_schedule`` (291-374): forward rows are exact
  Q-tile -> K-tile incidence at the forward block size; backward rows are exact
  incidence at the backward block size, transposed to K-tile -> Q-tile (350-362).
  Incidence per Q tile is the union, per document, of the strict-window intervals
  ``[q - W + 1, q]`` of the tile's queries (225-252), plus every K tile holding a
  key of the same (document, vision) pair after the earliest query of that pair in
  the tile (254-260).  A work budget stops construction early (264-268).
* ``gemma4_local_sparse_storage_upper_bound`` (94-135).

Pinned by ``tests/test_oracle_schedule.py``: equality with the brute-force
incidence of the exact boolean mask (``brute_force_tile_rows``) on the
reference's adversarial cases and exhaustively over 3-valued vision x 2-valued
document metadata (tests/test_sparse_schedule.py:72-91), the model-maximum
bounds (121-131, 149-175) and the pinned storage bound 94,027,776.

The HIP path replaces this host schedule with a device tile scheduler; the
tests use this module to check that scheduler's coverage.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


class SparseScheduleWorkLimitExceeded(RuntimeError):
    """Raised before an exact sparse schedule exceeds its work budget."""


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


@dataclass(frozen=True)
class SparseTileRows:
    rows: tuple
    row_block_size: int
    column_block_size: int
    column_blocks: int

    def __post_init__(self) -> None:
        if self.row_block_size <= 0 or self.column_block_size <= 0:
            raise ValueError("sparse tile sizes must be positive")
        if self.column_blocks <= 0:
            raise ValueError("a sparse schedule requires at least one column block")
        for row in self.rows:
            if tuple(sorted(set(row))) != tuple(row):
                raise ValueError("sparse row indices must be sorted and unique")
            if any(i < 0 or i >= self.column_blocks for i in row):
                raise ValueError("sparse row index is out of range")

    @property
    def compact_width(self) -> int:
        return max([1] + [len(r) for r in self.rows])

    @property
    def candidate_pairs(self) -> int:
        return sum(len(r) for r in self.rows)

    @property
    def storage_bytes(self) -> int:
        return 4 * len(self.rows) * (3 + self.compact_width)


@dataclass(frozen=True)
class Gemma4LocalSparseSchedule:
    q_length: int
    k_length: int
    forward: SparseTileRows
    backward: SparseTileRows

    @property
    def candidate_pairs(self) -> int:
        return self.forward.candidate_pairs + self.backward.candidate_pairs

    @property
    def storage_bytes(self) -> int:
        return self.forward.storage_bytes + self.backward.storage_bytes

    def scheduled_score_slots(self, num_q_heads: int) -> int:
        if num_q_heads <= 0:
            raise ValueError("num_q_heads must be positive")
        f, b = self.forward, self.backward
        return num_q_heads * (
            f.candidate_pairs * f.row_block_size * f.column_block_size
            + b.candidate_pairs * b.row_block_size * b.column_block_size
        )


def sparse_tile_rows_storage_upper_bound(
    row_length: int, column_length: int, *, row_block_size: int, column_block_size: int
) -> int:
    if row_length <= 0 or column_length <= 0:
        raise ValueError("sparse row and column lengths must be positive")
    if row_block_size <= 0 or column_block_size <= 0:
        raise ValueError("sparse block sizes must be positive")
    return 4 * _cdiv(row_length, row_block_size) * (3 + _cdiv(column_length, column_block_size))


def gemma4_local_sparse_storage_upper_bound(
    q_length: int,
    k_length: int,
    *,
    forward_block_size=(128, 80),
    backward_block_size=(64, 64),
) -> int:
    if q_length <= 0 or k_length <= 0 or q_length > k_length:
        raise ValueError("sparse scheduling requires 1 <= Sq <= Sk")
    fwd = sparse_tile_rows_storage_upper_bound(
        q_length,
        k_length,
        row_block_size=forward_block_size[0],
        column_block_size=forward_block_size[1],
    )
    bwd = sparse_tile_rows_storage_upper_bound(
        k_length,
        q_length,
        row_block_size=backward_block_size[1],
        column_block_size=backward_block_size[0],
    )
    return fwd + bwd


def _incidence_rows(
    vision: np.ndarray,
    docs: np.ndarray,
    *,
    q_length: int,
    k_length: int,
    q_block: int,
    k_block: int,
    window: int,
    max_pairs: int | None,
    direction: str,
) -> SparseTileRows:
    offset = k_length - q_length
    doc_keys = {int(d): np.flatnonzero(docs == d) for d in np.unique(docs)}
    pair_keys: dict[tuple[int, int], np.ndarray] = {}
    vis_pos = np.flatnonzero(vision >= 0)
    if vis_pos.size:
        keys = np.stack([docs[vis_pos], vision[vis_pos]], axis=1)
        for d, v in np.unique(keys, axis=0):
            pair_keys[(int(d), int(v))] = vis_pos[(keys[:, 0] == d) & (keys[:, 1] == v)]

    rows = []
    total = 0
    for t in range(_cdiv(q_length, q_block)):
        qa = np.arange(offset + t * q_block, offset + min(q_length, (t + 1) * q_block))
        tiles: set[int] = set()
        tile_docs = docs[qa]
        for d in np.unique(tile_docs):
            qs = qa[tile_docs == d]  # ascending
            keys = doc_keys[int(d)]
            starts = np.maximum(0, qs - window + 1)
            # merge [start, q] intervals of consecutive queries of this document
            seg_start, seg_end = int(starts[0]), int(qs[0])
            intervals = []
            for s, e in zip(starts[1:].tolist(), qs[1:].tolist()):
                if s <= seg_end + 1:
                    seg_end = e
                else:
                    intervals.append((seg_start, seg_end))
                    seg_start, seg_end = s, e
            intervals.append((seg_start, seg_end))
            for s, e in intervals:
                i0 = np.searchsorted(keys, s, side="left")
                i1 = np.searchsorted(keys, e, side="right")
                tiles.update((keys[i0:i1] // k_block).tolist())
        vq = vision[qa]
        sel = vq >= 0
        if sel.any():
            seen: dict[tuple[int, int], int] = {}
            for q, d, v in zip(qa[sel].tolist(), tile_docs[sel].tolist(), vq[sel].tolist()):
                seen.setdefault((d, v), q)  # earliest query of the pair in this tile
            for pair, first_q in seen.items():
                keys = pair_keys.get(pair)
                if keys is None:
                    continue
                after = keys[np.searchsorted(keys, first_q, side="right") :]
                tiles.update((after // k_block).tolist())
        row = tuple(sorted(tiles))
        rows.append(row)
        total += len(row)
        if max_pairs is not None and total > max_pairs:
            raise SparseScheduleWorkLimitExceeded(
                f"exact {direction} sparse schedule exceeds its "
                f"{max_pairs}-tile construction budget"
            )
    return SparseTileRows(tuple(rows), q_block, k_block, _cdiv(k_length, k_block))


def transpose_rows(rows: SparseTileRows) -> SparseTileRows:
    out: list[list[int]] = [[] for _ in range(rows.column_blocks)]
    for r, cols in enumerate(rows.rows):
        for c in cols:
            out[c].append(r)
    return SparseTileRows(
        tuple(tuple(x) for x in out),
        rows.column_block_size,
        rows.row_block_size,
        len(rows.rows),
    )


def build_gemma4_local_sparse_schedule(
    vision_block_ids,
    document_ids,
    *,
    q_length: int,
    k_length: int,
    sliding_window: int = 1024,
    forward_block_size=(128, 80),
    backward_block_size=(64, 64),
    num_q_heads: int = 32,
    max_scheduled_score_slots: int | None = None,
) -> Gemma4LocalSparseSchedule:
    if q_length <= 0 or k_length <= 0 or q_length > k_length:
        raise ValueError("sparse scheduling requires 1 <= Sq <= Sk")
    if len(vision_block_ids) != k_length or len(document_ids) != k_length:
        raise ValueError("vision/document metadata must match Sk")
    if sliding_window <= 0:
        raise ValueError("sliding_window must be positive")
    if any(s <= 0 for s in (*forward_block_size, *backward_block_size)):
        raise ValueError("sparse block sizes must be positive")
    if num_q_heads <= 0:
        raise ValueError("num_q_heads must be positive")
    if max_scheduled_score_slots is not None and max_scheduled_score_slots <= 0:
        raise ValueError("max_scheduled_score_slots must be positive")
    vision = np.asarray(vision_block_ids, dtype=np.int64)
    docs = np.asarray(document_ids, dtype=np.int64)
    fwd_slots = num_q_heads * forward_block_size[0] * forward_block_size[1]
    max_fwd = None if max_scheduled_score_slots is None else max_scheduled_score_slots // fwd_slots
    forward = _incidence_rows(
        vision,
        docs,
        q_length=q_length,
        k_length=k_length,
        q_block=forward_block_size[0],
        k_block=forward_block_size[1],
        window=sliding_window,
        max_pairs=max_fwd,
        direction="forward",
    )
    remaining = (
        None
        if max_scheduled_score_slots is None
        else max_scheduled_score_slots - forward.candidate_pairs * fwd_slots
    )
    bwd_slots = num_q_heads * backward_block_size[0] * backward_block_size[1]
    max_bwd = None if remaining is None else remaining // bwd_slots
    backward = transpose_rows(
        _incidence_rows(
            vision,
            docs,
            q_length=q_length,
            k_length=k_length,
            q_block=backward_block_size[0],
            k_block=backward_block_size[1],
            window=sliding_window,
            max_pairs=max_bwd,
            direction="backward",
        )
    )
    return Gemma4LocalSparseSchedule(q_length, k_length, forward, backward)


def brute_force_tile_rows(allowed, block_size) -> tuple:
    """Q-tile -> sorted K-tiles holding at least one allowed pair of ``allowed (Q, K)``."""
    allowed = np.asarray(allowed, dtype=bool)
    qb, kb = block_size
    rows = [set() for _ in range(_cdiv(allowed.shape[0], qb))]
    for qi, ki in zip(*np.nonzero(allowed)):
        rows[qi // qb].add(int(ki) // kb)
    return tuple(tuple(sorted(r)) for r in rows)
