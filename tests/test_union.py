"""The oracle's cap_union (reference src/deepseeker/mlx_forward.py:213-254) pinned
by the reference's own cases (tests/test_batch.py:203-249), a brute-force check of
the kept expert set, and numpy's float32 row sum restated."""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import union as U


def test_pairwise_row_sum_is_numpys():
    rng = np.random.default_rng(3)
    for n in range(1, 33):
        a = (rng.random((400, n)) * 10.0 ** rng.integers(-3, 3, size=(400, n))).astype(np.float32)
        np.testing.assert_array_equal(U.pairwise_sum_f32(a), a.sum(axis=1))


def test_union_that_fits_is_unchanged():                       # tests/test_batch.py:203-210
    idx = np.array([[1, 2, 3], [3, 4, 5]], dtype=np.int64)
    w = np.array([[0.7, 0.5, 0.3], [0.6, 0.5, 0.4]], dtype=np.float32)
    out_i, out_w, coverage = U.cap_union_reference_order(idx, w, 8, 5)
    np.testing.assert_array_equal(out_i, idx)
    np.testing.assert_array_equal(out_w, w)
    assert coverage == 1.0


def test_union_shrinks_and_rows_keep_their_sums():            # tests/test_batch.py:213-234
    rng = np.random.default_rng(0)
    idx = np.array([[0, 1, 2], [0, 3, 4], [0, 5, 6], [1, 3, 5], [2, 4, 6], [7, 8, 9]], dtype=np.int64)
    w = rng.random((6, 3)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    w *= 1.5
    out_i, out_w, coverage = U.cap_union_reference_order(idx, w, 12, 4)
    live = out_i[out_i >= 0]
    assert np.unique(live).size <= 4 + idx.shape[0]
    np.testing.assert_allclose(out_w.sum(axis=1), w.sum(axis=1), rtol=1e-5)
    kept = out_i >= 0
    for r in range(idx.shape[0]):
        vals = out_w[r][kept[r]] / w[r][kept[r]]
        np.testing.assert_allclose(vals, vals[0], rtol=1e-5)
        assert vals[0] >= 1.0 - 1e-6
    assert 0.0 < coverage <= 1.0
    assert np.all(out_w[~kept] == 0.0)


def test_row_never_loses_every_expert_unless_strict():       # tests/test_batch.py:237-249
    idx = np.array([[90, 91, 92], [1, 2, 3], [1, 2, 4]], dtype=np.int64)
    w = np.array([[0.5, 0.5, 0.5], [5.0, 4.0, 3.0], [5.0, 4.0, 3.0]], dtype=np.float32)
    out_i, out_w, coverage = U.cap_union_reference_order(idx, w, 93, 3)
    assert (out_i[0] >= 0).sum() == 1 and out_i[0, 0] == 90       # first maximum kept
    np.testing.assert_allclose(out_w[0].sum(), w[0].sum(), rtol=1e-5)
    assert coverage < 1.0
    s_i, s_w, _ = U.cap_union_reference_order(idx, w, 93, 3, strict=True)
    assert (s_i[0] >= 0).sum() == 0 and np.all(s_w[0] == 0.0)
    assert np.unique(s_i[s_i >= 0]).size == 3


def test_kept_set_maximises_the_summed_score_brute_force():
    rng = np.random.default_rng(11)
    for trial in range(60):
        T, k, E, budget = int(rng.integers(2, 6)), int(rng.integers(1, 4)), 9, int(rng.integers(1, 5))
        idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int64)
        scores = rng.random((T, E)).astype(np.float32) + 0.01
        w = np.take_along_axis(scores, idx, 1)
        out_i, _, _ = U.cap_union_reference_order(idx, w, E, budget, scores=scores, strict=True)
        if np.unique(idx).size <= budget:
            continue
        score = np.zeros(E)
        for t in range(T):
            for e in idx[t]:
                score[e] += scores[t, e]
        best = max(sum(score[list(c)]) for c in itertools.combinations(range(E), budget))
        kept = set(np.unique(out_i[out_i >= 0]).tolist())
        # the union of the rows' surviving experts is the kept set restricted to routed experts
        routed_kept = sorted(kept)
        assert len(routed_kept) <= budget
        assert abs(sum(score[routed_kept]) - best) < 1e-4, (trial, kept)


def test_build_order_wrapper_flips_slots():
    rng = np.random.default_rng(5)
    T, k, E = 7, 6, 20
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    scores = rng.random((T, E)).astype(np.float32)
    w = np.take_along_axis(scores, idx, 1)
    bi, bw, bc = U.cap_union(idx, w, E, 5, scores=scores)
    ri, rw, rc = U.cap_union_reference_order(idx[:, ::-1], w[:, ::-1], E, 5, scores=scores)
    np.testing.assert_array_equal(bi, ri[:, ::-1])
    np.testing.assert_array_equal(bw, rw[:, ::-1])
    assert bc == rc
    with pytest.raises(ValueError):
        U.pairwise_sum_f32(np.zeros((1, 200), np.float32))
