"""Token -> expert dispatch, restated on the CPU (integer work, numpy).

Reference: ``src/deepseeker/mlx_forward.py:294-312, 388-396`` groups the
routed (token, slot) pairs per unique expert in ascending expert id, rows in
ascending token order, and skips negative ids; ``src/deepseeker/moe_align.py:21-46``
(``align_block_size``) states the same grouping as a stable argsort of the
flattened ``topk_ids`` with block padding; ``src/deepseeker/grouped.py:19-31``
(``plan_groups``) keeps duplicates in row order.

Definition used by the build (flat position ``p = t*k + j``):
``counts[e]`` = number of p with ``idx[p] == e``; ``offsets`` = exclusive
prefix sum of ``counts`` (length E+1); ``perm`` = positions sorted by
``(idx[p], p)``; ``rank[p]`` = the dispatch row of p (inverse of ``perm``),
-1 for dropped positions.  Positions with ``idx < 0`` (the reference's
dropped slots) or ``idx >= E`` are dropped.

Pinned by the reference's known-answer tests (``tests/test_audit.py:37-44``,
``tests/test_grouped.py:29-39``) and its random property test
(``tests/test_audit.py:47-60``), restated in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import numpy as np


def dispatch(idx: np.ndarray, n_experts: int):
    """idx [T, k] -> (counts [E], offsets [E+1], perm [n_valid], rank [T*k]) all int32."""
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    valid = (flat >= 0) & (flat < n_experts)
    key = np.where(valid, flat, n_experts)           # dropped entries sort last
    order = np.argsort(key, kind="stable")
    n_valid = int(valid.sum())
    perm = order[:n_valid].astype(np.int32)
    counts = np.bincount(flat[valid], minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    rank = np.full(flat.size, -1, dtype=np.int32)
    rank[perm] = np.arange(n_valid, dtype=np.int32)
    return counts, offsets, perm, rank


def active_experts(counts: np.ndarray) -> np.ndarray:
    """Experts with at least one routed position, ascending (the reference's ``np.unique``)."""
    return np.nonzero(np.asarray(counts) > 0)[0].astype(np.int32)


def align_block_size(topk_ids: np.ndarray, block_size: int, num_experts: int):
    """Padded-block form of the dispatch (the ``moe_align_block_size`` contract).

    Returns (sorted_ids, expert_ids per block, num_tokens_post_pad); each
    expert's run of flat positions is padded to a multiple of ``block_size``
    with the sentinel ``M*K``.  Same contract as
    ``src/deepseeker/moe_align.py:21-46``.
    """
    ids = np.asarray(topk_ids)
    if ids.ndim != 2:
        raise ValueError(f"topk_ids must be 2-D, got shape {ids.shape}")
    if block_size < 1 or num_experts < 1:
        raise ValueError("block_size and num_experts must be >= 1")
    flat = ids.reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= num_experts):
        raise ValueError("expert ids out of range")
    counts, offsets, perm, _ = dispatch(ids, num_experts)
    sentinel = flat.size
    sorted_ids, expert_ids = [], []
    for e in range(num_experts):
        run = perm[offsets[e]:offsets[e + 1]].tolist()
        run += [sentinel] * ((-len(run)) % block_size)
        sorted_ids.extend(run)
        expert_ids.extend([e] * (len(run) // block_size))
    return (np.asarray(sorted_ids, dtype=np.int64),
            np.asarray(expert_ids, dtype=np.int64), len(sorted_ids))


def plan_groups(topk_ids, n_experts: int) -> dict[int, list[tuple[int, int]]]:
    """expert -> [(row, slot)] in ascending row order (``grouped.py:19-31`` contract)."""
    groups: dict[int, list[tuple[int, int]]] = {}
    for row, experts in enumerate(topk_ids):
        for pos, expert in enumerate(experts):
            if not 0 <= expert < n_experts:
                raise ValueError(f"expert {expert} out of range [0, {n_experts})")
            groups.setdefault(int(expert), []).append((row, pos))
    return groups
