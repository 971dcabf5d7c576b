"""GPU dispatch parity: counts, offsets, permutation, inverse and active list
bit-identical to the oracle (stable counting sort by expert), for the
one-workgroup form (``dsk_dispatch``) and, from 8192 positions, the
multi-workgroup form the forward call runs (``dsk_dispatch_ws``): position
counts that are and are not multiples of a workgroup's 2048, a single expert
taking every position, dropped entries and E up to 1024."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from oracle import dispatch as D

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check(idx: np.ndarray, n_experts: int, multi_block: bool = False):
    print(f"dispatch shape={idx.shape} E={n_experts} multi_block={multi_block}", flush=True)
    got = dsk_moe.dispatch(torch.from_numpy(idx.astype(np.int32)).to(DEV), n_experts, multi_block=multi_block)
    counts, offsets, perm, rank = D.dispatch(idx, n_experts)
    act = D.active_experts(counts)
    np.testing.assert_array_equal(got["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(got["offsets"].cpu().numpy(), offsets)
    n_valid = int(offsets[-1])
    np.testing.assert_array_equal(got["perm"].cpu().numpy()[:n_valid], perm)
    np.testing.assert_array_equal(got["rank"].cpu().numpy(), rank)
    a = got["active"].cpu().numpy()
    assert a[0] == len(act)
    np.testing.assert_array_equal(a[1:1 + len(act)], act)


def test_dispatch_reference_known_answer():
    # reference tests/test_audit.py:37-44
    check(np.array([[1, 2, 3], [0, 1, 3], [0, 2, 3], [0, 1, 2]]), 4)


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (8, 8, 256), (64, 8, 256), (256, 6, 384),
                                   (4096, 8, 256), (3, 2, 8), (1000, 6, 1024), (50, 16, 16)])
def test_dispatch_random(T, k, E):
    rng = np.random.default_rng(T + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]) if k <= E else None
    check(idx, E)


def test_dispatch_skewed_duplicates_and_drops():
    rng = np.random.default_rng(3)
    idx = rng.zipf(1.3, size=(4096, 8)) - 1
    idx[idx >= 256] = -1                     # dropped slots
    idx[::17, 0] = -1
    check(idx, 256)


@pytest.mark.parametrize("T,k,E", [(1024, 8, 256), (4096, 8, 256), (1100, 8, 256), (2049, 6, 384),
                                   (1366, 6, 1024), (600, 16, 64), (64, 8, 256)])
def test_dispatch_multi_block(T, k, E):
    rng = np.random.default_rng(7 * T + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    check(idx, E, multi_block=True)


def test_dispatch_multi_block_skewed_and_drops():
    rng = np.random.default_rng(5)
    idx = rng.zipf(1.2, size=(4096, 8)) - 1
    idx[idx >= 256] = -1
    idx[::13, 3] = -1
    check(idx, 256, multi_block=True)
    one = np.zeros((1500, 8), dtype=np.int64)      # every position on expert 0
    one[::7, 1] = 255
    check(one, 256, multi_block=True)


def test_dispatch_real_trace_replay(golden):
    # real DeepSeek routing recorded by the reference (E = 384, k = 6)
    ex = golden("trace_routes.npz")["experts"]
    check(ex[:2048], 384)


def test_align_block_size_matches_oracle():
    rng = np.random.default_rng(0)
    topk = rng.integers(0, 384, size=(256, 6))
    s_got, e_got, n_got = dsk_moe.align_block_size(torch.from_numpy(topk).to(DEV), 16, 384)
    s_want, e_want, n_want = D.align_block_size(topk, 16, 384)
    assert n_got == n_want
    np.testing.assert_array_equal(s_got.cpu().numpy(), s_want)
    np.testing.assert_array_equal(e_got.cpu().numpy(), e_want)
