"""Exact Gemma 4 allow-mask, restated -- TEST INFRASTRUCTURE ONLY.

Follows the reference mask builder ``src/gemma4_fa4/masks.py:8-80``:

* causal ``k <= q`` (masks.py:46);
* vision overlay ``allowed |= vid[q] == vid[k] and vid[q] >= 0`` only when
  ``allow_vision_bidirectional`` (masks.py:49-59);
* strict sliding window ``allowed &= k > q - W`` (masks.py:61-63);
* documents ``allowed &= doc[q] == doc[k]`` (masks.py:65-71);
* key padding (masks.py:73-78);
* query positions default to the lower-right suffix ``q_start = kv - q``
  (masks.py:41).

Pinned by: the reference's boolean truth tables (tests/test_masks.py:11-96),
restated in ``tests/test_oracle_masks.py``, and an exhaustive comparison of the
vectorised builder against ``mask_predicate_scalar`` (a per-element pure-Python
statement of the predicate) over every small metadata assignment.
"""

from __future__ import annotations

import numpy as np
import torch


def _as_numpy(x):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy()
    return np.asarray(x)


def gemma4_attention_mask(
    *,
    batch_size: int,
    q_len: int,
    kv_len: int,
    device="cpu",
    sliding_window: int | None,
    vision_block_ids=None,
    document_ids=None,
    key_padding_mask=None,
    q_start: int | None = None,
    allow_vision_bidirectional: bool = False,
) -> torch.Tensor:
    """Return a bool tensor ``(B, 1, Q, K)`` where True means the pair is allowed."""
    if batch_size < 1 or q_len < 0 or kv_len < 0:
        raise ValueError("invalid attention shape")
    if q_len > kv_len and q_start is None:
        raise ValueError("q_len cannot exceed kv_len when q_start is omitted")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError("sliding_window must be positive")
    start = kv_len - q_len if q_start is None else q_start
    if start < 0 or start + q_len > kv_len:
        raise ValueError("query positions must lie inside the KV stream")

    qpos = np.arange(start, start + q_len, dtype=np.int64)[:, None]
    kpos = np.arange(kv_len, dtype=np.int64)[None, :]
    allowed = np.broadcast_to(kpos <= qpos, (batch_size, q_len, kv_len)).copy()

    vids = _as_numpy(vision_block_ids)
    if vids is not None:
        if vids.shape != (batch_size, kv_len):
            raise ValueError(
                f"vision_block_ids must be {(batch_size, kv_len)}, got {tuple(vids.shape)}"
            )
        if allow_vision_bidirectional:
            vq = vids[:, start : start + q_len]
            same = (vq[:, :, None] == vids[:, None, :]) & (vq[:, :, None] >= 0)
            allowed |= same
    if sliding_window is not None:
        allowed &= (kpos > qpos - sliding_window)[None]
    docs = _as_numpy(document_ids)
    if docs is not None:
        if docs.shape != (batch_size, kv_len):
            raise ValueError(
                f"document_ids must be {(batch_size, kv_len)}, got {tuple(docs.shape)}"
            )
        dq = docs[:, start : start + q_len]
        allowed &= dq[:, :, None] == docs[:, None, :]
    pad = _as_numpy(key_padding_mask)
    if pad is not None:
        if pad.shape != (batch_size, kv_len):
            raise ValueError(
                f"key_padding_mask must be {(batch_size, kv_len)}, got {tuple(pad.shape)}"
            )
        allowed &= pad.astype(bool)[:, None, :]
    return torch.from_numpy(np.ascontiguousarray(allowed[:, None])).to(device)


def mask_predicate_scalar(
    q_abs: int,
    k_abs: int,
    *,
    window: int | None,
    vision=None,
    documents=None,
    bidirectional: bool = False,
) -> bool:
    """Per-pair statement of the Gemma predicate, used as a brute-force check.

    ``window AND (causal OR same non-negative vision block) AND same document``
    (h100_masks.py:26-84 states the same predicate per element).
    """
    keep = k_abs <= q_abs
    if bidirectional and vision is not None:
        vq, vk = int(vision[q_abs]), int(vision[k_abs])
        if vq >= 0 and vq == vk:
            keep = True
    if window is not None and not (k_abs > q_abs - window):
        keep = False
    if documents is not None and int(documents[q_abs]) != int(documents[k_abs]):
        keep = False
    return keep
