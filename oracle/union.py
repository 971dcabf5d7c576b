"""The batch union cap of the reference (``cap_union``), restated on the CPU.

Test infrastructure: only the tests, ``__graft_entry__.smoke`` and the
benchmark's CPU baseline use this module, to compare against.

Reference: ``src/deepseeker/mlx_forward.py:213-254`` (``cap_union``), called by
``moe_layer`` for lock-step batches of more than one row (``:294-305``) with
the router's un-biased scores for ranking.  Steps, in the reference's
arithmetic (numpy float32):

1. If the batch's expert union already fits (``unique(idx).size <= budget``),
   nothing changes (coverage 1).
2. ``score[e] = sum of scores[t, e]`` over the rows t routed to e, accumulated
   in row order (``np.add.at`` over ``idx.ravel()``).
3. The ``budget`` experts with the largest ``score`` are kept.  The reference
   takes them with ``np.argpartition``, whose choice among exactly equal
   scores at the boundary is unspecified; this restatement (and the GPU
   kernel) order by score descending, then expert id ascending.  For
   distinct scores the kept set is the reference's.
4. A row with no kept expert keeps its largest-weight expert (``argmax``:
   the first maximum in the reference's slot order) unless ``strict``.
5. ``scale = rowsum(w) / (rowsum(kept_w) + 1e-20)``, ``w' = kept_w * scale``,
   dropped slots get index -1.  Row sums are numpy's float32 pairwise sums
   (``pairwise_sum``): fewer than 8 terms added one by one from 0, otherwise 8
   running sums (terms i, i+8, ...) combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))
   and the remaining tail added one by one.
6. ``coverage = rowsum-total(kept_w) / total(w)`` before rescaling.

The reference's slot order is ascending key (``argsort`` tail); the build's
router returns descending key order.  ``cap_union`` takes and returns the
build's order and applies the steps above in the reference's order (slots
reversed), so the row sums and the argmax rescue see the same sequence as
the reference.

Pinned by the reference's own cases (``tests/test_batch.py:203-249``: union
that fits is unchanged; the union shrinks to at most budget + rows and every
row keeps its weight sum and its within-row weight ratios; a row that would
lose everything keeps one expert), by a brute-force check of the kept set on
small inputs, and by the closed form of numpy's float32 row sum (against
``ndarray.sum`` itself).
"""

from __future__ import annotations

import numpy as np


def pairwise_sum_f32(a: np.ndarray) -> np.ndarray:
    """numpy's float32 pairwise row sum of a [rows, n] array, n <= 128, restated."""
    a = np.asarray(a, dtype=np.float32)
    n = a.shape[1]
    if n < 8:
        res = np.zeros(a.shape[0], dtype=np.float32)
        for i in range(n):
            res = (res + a[:, i]).astype(np.float32)
        return res
    if n > 128:
        raise ValueError("rows longer than 128 use numpy's recursive blocking")
    r = [a[:, j].copy() for j in range(8)]
    i = 8
    while i < n - (n % 8):
        for j in range(8):
            r[j] = (r[j] + a[:, i + j]).astype(np.float32)
        i += 8
    res = (((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))).astype(np.float32)
    for j in range(i, n):
        res = (res + a[:, j]).astype(np.float32)
    return res


def keep_set(score: np.ndarray, budget: int) -> np.ndarray:
    """Boolean mask of the ``budget`` experts with the largest score (ties: lower id)."""
    order = np.lexsort((np.arange(score.size), -score.astype(np.float64)))
    keep = np.zeros(score.size, dtype=bool)
    keep[order[:budget]] = True
    return keep


def cap_union_reference_order(idx: np.ndarray, w: np.ndarray, n_experts: int, budget: int,
                              scores: np.ndarray | None = None, strict: bool = False):
    """Steps 1-6 on (idx, w) in the reference's slot order (ascending key).
    Returns (idx' int64, w' float32, coverage)."""
    idx = np.asarray(idx, dtype=np.int64)
    w = np.asarray(w, dtype=np.float32)
    if np.unique(idx).size <= budget:
        return idx, w, 1.0
    score = np.zeros(n_experts, dtype=np.float32)
    if scores is not None:
        raw = np.asarray(scores, dtype=np.float32)[np.arange(idx.shape[0])[:, None], idx]
        np.add.at(score, idx.ravel(), raw.ravel())
    else:
        np.add.at(score, idx.ravel(), w.ravel())
    kept = keep_set(score, budget)[idx]
    empty = ~kept.any(axis=1)
    if empty.any() and not strict:
        kept[np.where(empty)[0], w[empty].argmax(axis=1)] = True
    kept_w = np.where(kept, w, np.float32(0.0)).astype(np.float32)
    total = float(w.sum())
    kept_sum = float(kept_w.sum())
    scale = (pairwise_sum_f32(w) / (pairwise_sum_f32(kept_w) + np.float32(1e-20))).astype(np.float32)
    out_w = (kept_w * scale[:, None]).astype(np.float32)
    out_idx = np.where(kept, idx, -1).astype(np.int64)
    return out_idx, out_w, (kept_sum / total if total > 0 else 1.0)


def cap_union(idx: np.ndarray, w: np.ndarray, n_experts: int, budget: int,
              scores: np.ndarray | None = None, strict: bool = False):
    """``cap_union`` on the build's routing (descending key order per row):
    (idx' int32 with -1 for dropped slots, w' float32, coverage)."""
    ri, rw, cov = cap_union_reference_order(np.asarray(idx)[:, ::-1], np.asarray(w)[:, ::-1], n_experts,
                                            budget, scores, strict)
    return (np.ascontiguousarray(ri[:, ::-1]).astype(np.int32),
            np.ascontiguousarray(rw[:, ::-1]).astype(np.float32), cov)
