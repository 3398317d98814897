"""numpy restatement of the slot-indexed state-pool copies -- test infrastructure.

Semantics (reference csrc/state_io.cu:16-26; slot <= 0 is padding):
  gather   out[r] = pool[slot_r] if slot_r > 0 and valid[r] else 0
  scatter  pool[slot_r] = packed[r] for slot_r > 0; other rows skipped
  copy     pool[dst_p] = pool[src_p] when src_p > 0 and dst_p > 0 (all reads before writes),
           except for pairs that overlap another live pair: a source that is another live
           pair's destination, or a destination that is another live pair's source or
           destination.  Such pairs are rejected (nothing written), the rule of this build's
           ld_state_copy (no reference counterpart: the reference has no slot-to-slot copy)
  zero     pool[slot_i] = 0 for slot_i > 0 (no reference counterpart: the in-place form of
           gather's zero fill of rows that are not valid, csrc/state_io.cu:17-25)
Arrays may have any dtype; comparisons against the HIP kernels are bit-exact.
"""

from __future__ import annotations

import numpy as np


def gather(pool: np.ndarray, slots: np.ndarray, valid: np.ndarray | None) -> np.ndarray:
    out = np.zeros((len(slots), *pool.shape[1:]), dtype=pool.dtype)
    for r, slot in enumerate(slots):
        if slot > 0 and (valid is None or bool(valid[r])):
            out[r] = pool[slot]
    return out


def scatter(packed: np.ndarray, slots: np.ndarray, pool: np.ndarray) -> np.ndarray:
    result = pool.copy()
    for r, slot in enumerate(slots):
        if slot > 0:
            result[slot] = packed[r]
    return result


def copy_rejected(src: np.ndarray, dst: np.ndarray) -> np.ndarray:
    """Per pair: True when the pair is live (both slots > 0) and overlaps another live pair
    (its source is another's destination, or its destination is another's source or
    destination)."""
    live = [(int(s), int(d)) if s > 0 and d > 0 else None for s, d in zip(src, dst)]
    rejected = np.zeros(len(live), dtype=bool)
    for p, pair in enumerate(live):
        if pair is None:
            continue
        for q, other in enumerate(live):
            if q != p and other is not None and (
                    other[1] == pair[0] or other[0] == pair[1] or other[1] == pair[1]):
                rejected[p] = True
                break
    return rejected


def copy(pool: np.ndarray, src: np.ndarray, dst: np.ndarray) -> np.ndarray:
    result = pool.copy()
    rejected = copy_rejected(src, dst)
    for p, (s, d) in enumerate(zip(src, dst)):
        if s > 0 and d > 0 and not rejected[p]:
            result[d] = pool[s]  # reads the pool as it was before the call
    return result


def zero(pool: np.ndarray, slots: np.ndarray) -> np.ndarray:
    result = pool.copy()
    for slot in slots:
        if slot > 0:
            result[slot] = 0
    return result
