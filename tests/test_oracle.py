"""Pins the CPU oracle before the GPU results are compared against it.

Each test names what it pins: the reference's own known-answer tests and
seeded vectors (restated here, the reference cannot be imported), closed
forms, brute force on small inputs, and invariants.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dispatch as D
from oracle import formats as F
from oracle import layer as L
from oracle import router as R
from oracle import synth


# ------------------------------------------------------------------ FP4 decode
def test_fp4_table_spot_values():
    # reference tests/test_metal_fp4.py:35-41
    assert F.FP4_TABLE[0x7] == 6.0
    assert F.FP4_TABLE[0xF] == -6.0
    assert F.FP4_TABLE[0x8] == 0.0
    s = F.e8m0_to_f32(np.array([127, 128, 0xFF], dtype=np.uint8))
    assert s[0] == 1.0 and s[1] == 2.0 and np.isnan(s[2])


def test_fp4_table_is_e2m1():
    # closed form of e2m1: sign | 2 exponent bits (bias 1) | 1 mantissa bit
    for code in range(16):
        sign = -1.0 if code & 8 else 1.0
        e, m = (code >> 1) & 3, code & 1
        mag = (m * 0.5) if e == 0 else (1 + m / 2) * 2.0 ** (e - 1)
        assert F.FP4_TABLE[code] == (sign * mag if mag else 0.0)


def test_fp4_nibble_order_low_first():
    # reference tests/test_q3.py:132-140: byte 0x13 -> [T[3], T[1]] * 2
    vals = F.fp4_dequant(np.array([[0x13] * 16], dtype=np.uint8), np.array([[128]], dtype=np.uint8))
    assert vals[0, 0] == F.FP4_TABLE[3] * 2.0 and vals[0, 1] == F.FP4_TABLE[1] * 2.0


def test_fp4_dequant_reference_random_vectors():
    # reference tests/test_metal_fp4.py:44-54 (numpy default_rng(3), 512 bytes,
    # scales 2^U{-3..2}); its expected values are the table times the scale.
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 256, size=512, dtype=np.uint8)
    scales_f = np.exp2(rng.integers(-3, 3, size=32).astype(np.float32))
    sbytes = (np.log2(scales_f).astype(np.int32) + 127).astype(np.uint8)
    got = F.fp4_dequant(packed[None, :], sbytes[None, :])[0]
    raw = packed.astype(np.int64)
    want = np.empty(1024, dtype=np.float32)
    want[0::2] = F.FP4_TABLE[raw & 15]
    want[1::2] = F.FP4_TABLE[raw >> 4]
    want *= np.repeat(scales_f, 32)
    np.testing.assert_array_equal(got, want)


def test_fp4_dequant_torch_crosscheck():
    # reference tests/test_mlx_weights.py:77-87 recipe (default_rng(2), scale bytes 120..134)
    rng = np.random.default_rng(2)
    packed = rng.integers(0, 256, size=(4, 64), dtype=np.uint8)
    sbytes = rng.integers(120, 135, size=(4, 4), dtype=np.uint8)
    got = F.fp4_dequant(packed, sbytes)
    tbl = torch.tensor(F.FP4_TABLE)
    raw = torch.from_numpy(packed.astype(np.int64))
    vals = torch.stack([tbl[raw & 15], tbl[raw >> 4]], dim=-1).reshape(4, 128)
    scale = torch.pow(2.0, torch.from_numpy(sbytes.astype(np.float32)) - 127).repeat_interleave(32, 1)
    np.testing.assert_array_equal(got, (vals * scale).numpy())


# ------------------------------------------------------------------ FP4 quantiser
def test_fp4_scale_exponent_is_ceil_log2():
    rng = np.random.default_rng(5)
    amax = np.concatenate([rng.random(2000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 2000),
                           np.float32([6.0, 3.0, 1.5, 0.75, 6 * 2.0 ** -40, 12.0])]).astype(np.float32)
    e = F.fp4_scale_exponent(amax)
    for a, ee in zip(amax.astype(np.float64), e):
        # smallest integer e with 6 * 2^e >= amax, checked exactly
        assert 6.0 * 2.0 ** ee >= a and 6.0 * 2.0 ** (ee - 1) < a


def test_fp4_quantize_nearest_even_brute_force():
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    w[0, :32] = np.linspace(-6, 6, 32, dtype=np.float32)        # exact grid hits and ties
    w[1, :32] = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4) * np.float32(
        [1, -1] * 16)
    packed, scales = F.fp4_quantize(w)
    deq = F.fp4_dequant(packed, scales)
    codes = F.fp4_codes(packed)
    grid = np.array(sorted(set(np.abs(F.FP4_TABLE).tolist())))
    sc = np.repeat(F.e8m0_to_f32(scales), 32, axis=1)
    for r in range(w.shape[0]):
        for c in range(w.shape[1]):
            q = abs(float(w[r, c])) / float(sc[r, c])
            d = np.abs(grid - min(q, 6.0))
            best = np.flatnonzero(d == d.min())
            mags = [float(F.FP4_TABLE[i]) for i in range(8)]
            cand = [mags.index(grid[b]) for b in best]
            want = min(cand, key=lambda i: (i % 2, i))      # tie: even code index
            assert codes[r, c] & 7 == want, (r, c, q)
            assert not (codes[r, c] == 8)                    # never negative zero
    assert np.all(np.abs(deq) <= np.abs(w).max() * 1.5 + 1e-9)


# ------------------------------------------------------------------ Q3
def test_q3_pack_roundtrip_and_geometry():
    rng = np.random.default_rng(11)
    for k in (384, 1024, 1152):
        q = rng.integers(0, 8, size=(5, k), dtype=np.uint8)
        packed = F.q3_pack(q)
        assert packed.shape == (5, k * 3 // 8)
        np.testing.assert_array_equal(F.q3_unpack(packed, k), q)


def test_q3_pack_known_answer():
    # one code at a time: code 32*g + 8*m + j = 5 lands in lane group g's words
    for m, g, j in [(0, 0, 0), (0, 0, 1), (2, 1, 4), (3, 3, 6), (3, 3, 7), (1, 2, 3)]:
        q = np.zeros((1, 128), dtype=np.uint8)
        q[0, 32 * g + 8 * m + j] = 5
        words = F.q3_pack(q).view("<u4").reshape(4, 3)
        p = 4 * m + j // 2
        expect = np.zeros((4, 3), dtype=np.uint32)
        if p < 15:
            expect[g, p // 5] = 5 << (3 * (p % 5) + (16 if j % 2 else 0))
        else:
            for t in range(3):
                expect[g, t] = ((5 >> t) & 1) << (31 if j % 2 else 15)
        np.testing.assert_array_equal(words, expect)


def test_q3_pack_superblock_placement():
    # K = 640: one 512-code superblock (lane group g's chunks of blocks 0..3 at
    # bytes 48g + 12b) and one plain 48-byte tail block at byte 192
    for b, g, m, j in [(0, 0, 0, 0), (1, 2, 1, 3), (3, 3, 3, 7), (2, 1, 0, 2), (4, 0, 0, 1), (4, 3, 2, 5)]:
        q = np.zeros((1, 640), dtype=np.uint8)
        q[0, 128 * b + 32 * g + 8 * m + j] = 6
        packed = F.q3_pack(q)
        off = 48 * g + 12 * b if b < 4 else 192 + 12 * g
        nz = np.flatnonzero(packed[0])
        assert nz.size and nz.min() >= off and nz.max() < off + 12, (b, g, nz)
        words = packed[0, off:off + 12].copy().view("<u4")
        p = 4 * m + j // 2
        expect = np.zeros(3, dtype=np.uint32)
        if p < 15:
            expect[p // 5] = 6 << (3 * (p % 5) + (16 if j % 2 else 0))
        else:
            for t in range(3):
                expect[t] = ((6 >> t) & 1) << (31 if j % 2 else 15)
        np.testing.assert_array_equal(words, expect)
        np.testing.assert_array_equal(F.q3_unpack(packed, 640), q)


def test_q3_quantize_error_bound():
    # reference tests/test_q3.py:89-105 geometry: 8 x 256 at O(0.05) scale -> rms < 0.08
    rng = np.random.default_rng(7)
    vals = (rng.standard_normal((8, 256)) * 0.05).astype(np.float32)
    packed, s, b = F.q3_quantize(vals)
    assert packed.nbytes == 8 * 24 * 4 and s.shape == (8, 4) and b.shape == (8, 4)
    rt = F.q3_dequant(packed, s, b)
    rms = np.sqrt(np.mean((vals.astype(np.float64) - rt) ** 2)) / np.abs(vals).max()
    assert 0.0 < rms < 0.08
    # every value within half a step (plus fp16 rounding of s, b) of its group
    step = np.repeat(s.astype(np.float32), 64, axis=1)
    assert np.all(np.abs(rt - vals) <= 0.5 * step + 2e-3)


def test_q3_rowmajor_known_answer_and_bitstream():
    """Checkpoint q3 layout: codes 0..7 of a pack make the 24-bit integer
    0o76543210 (bytes 88 C6 FA, little-endian); a whole row is a little-endian
    bit stream with code c at bits 3c..3c+2, restated here with numpy.packbits."""
    q = np.arange(8, dtype=np.uint8)[None]
    np.testing.assert_array_equal(F.q3_pack_rowmajor(q), [[0x88, 0xC6, 0xFA]])
    assert 0o76543210 == 0xFAC688
    q = np.array([[7, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 5, 0, 0, 0, 0]], dtype=np.uint8)
    # code 0 = 7 -> bits 0..2 of byte 0; code 11 = 5 (101b) -> bits 33..35 -> byte 4 bits 1 and 3
    np.testing.assert_array_equal(F.q3_pack_rowmajor(q), [[0x07, 0, 0, 0, 0x0A, 0]])
    rng = np.random.default_rng(17)
    for n, k in ((3, 128), (8, 256), (2, 2304), (1, 5120)):
        q = rng.integers(0, 8, size=(n, k), dtype=np.uint8)
        bits = ((q[..., None] >> np.arange(3)) & 1).astype(np.uint8).reshape(n, 3 * k)
        stream = np.packbits(bits, axis=1, bitorder="little")
        got = F.q3_pack_rowmajor(q)
        np.testing.assert_array_equal(got, stream)
        np.testing.assert_array_equal(F.q3_unpack_rowmajor(got, k), q)
        # reference geometry (tests/test_q3.py:89-105): 3K/32 u32 words per row
        assert got.view("<u4").shape == (n, 3 * k // 32)
        np.testing.assert_array_equal(F.q3_unpack(F.q3_rowmajor_to_canonical(got, k), k), q)


# ------------------------------------------------------------------ router
def test_exp_log1p_sqrt_against_math():
    xs = np.linspace(-700, 700, 20001)
    got = R.exp_d(xs)
    want = np.array([math.exp(v) for v in xs])
    assert np.max(np.abs(got - want) / want) < 4e-16
    u = np.linspace(0, 1, 5001)
    assert np.max(np.abs(R.log1p_d(u) - np.array([math.log1p(v) for v in u]))) < 4e-16
    v = np.concatenate([np.random.default_rng(0).random(20000) * 50, [0.0, 1.0, 4.0, 2.25]])
    r = R.sqrt_round_f32(v)
    # correctly rounded: |r - sqrt(v)| <= half an ulp, with exact rationals
    from fractions import Fraction
    for vv, rr in zip(v[:3000], r[:3000]):
        rr = float(rr)
        ulp = float(np.spacing(np.float32(rr)))
        assert abs(Fraction(rr) ** 2 - Fraction(vv)) <= (Fraction(rr) + Fraction(ulp) / 2) * Fraction(ulp) + Fraction(ulp) ** 2


def test_ln2_split_exact():
    from fractions import Fraction
    hi = Fraction(R.LN2_HI)
    assert hi.denominator & (hi.denominator - 1) == 0
    # k * LN2_HI exact for |k| < 2^20
    assert float(Fraction(R.LN2_HI) * (2 ** 20 - 1)) == R.LN2_HI * (2 ** 20 - 1)
    assert abs(float(hi + Fraction(R.LN2_LO)) - math.log(2)) == 0.0


def _round_f32(v):
    """The float32 nearest to the rational v, ties to even (v finite, in range)."""
    from fractions import Fraction
    if v == 0:
        return np.float32(0.0)
    f = np.float32(float(v))
    cands = [f, np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))]
    err = [abs(Fraction(float(c)) - v) for c in cands]
    best = min(err)
    ties = [c for c, e in zip(cands, err) if e == best]
    return min(ties, key=lambda c: int(np.float32(c).view(np.uint32)) & 1)


def _fma_exact(a, b, c):
    """fma(a, b, c) in float32: the exact value a*b + c rounded once."""
    from fractions import Fraction
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _gate_scalar(x, w, fused=True):
    # the fixed order, one scalar at a time: fused steps from exact rationals,
    # the butterfly and segment sums as float32 adds of numpy scalars
    h = x.shape[0]
    steps = -(-h // 256)
    seg = -(-steps // 4)
    z = None
    for sw in range(4):
        p = [np.float32(0.0)] * 64
        for m in range(sw * seg, min((sw + 1) * seg, steps)):
            for v in range(4):
                for lane in range(64):
                    c = 256 * m + 4 * lane + v
                    if c < h:
                        if fused:
                            p[lane] = _fma_exact(x[c], w[c], p[lane])
                        else:
                            p[lane] = np.float32(p[lane] + np.float32(np.float32(x[c]) * np.float32(w[c])))
        for s in (32, 16, 8, 4, 2, 1):
            p = [np.float32(p[i] + p[i ^ s]) for i in range(64)]
        z = p[0] if z is None else np.float32(z + p[0])
    return z


def test_gate_logits_vectorised_equals_scalar_order():
    rng = np.random.default_rng(1)
    for h in (64, 260, 512, 1300):
        x = rng.standard_normal((2, h)).astype(np.float32)
        w = rng.standard_normal((3, h)).astype(np.float32)
        z = R.gate_logits(x, w)
        for t in range(2):
            for e in range(3):
                assert z[t, e] == _gate_scalar(x[t], w[e])


def test_gate_logits_fused_not_unfused():
    """Lane 0 takes x0*w0 = -(1 + 2^-11) and then (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24:
    fused, the chain keeps 2^-24; with the product rounded first (1 + 2^-11) it is 0."""
    x = np.zeros((1, 256), dtype=np.float32)
    w = np.zeros((1, 256), dtype=np.float32)
    x[0, 0], w[0, 0] = 1.0, -(1.0 + 2.0 ** -11)
    x[0, 1] = w[0, 1] = 1.0 + 2.0 ** -12
    assert R.gate_logits(x, w)[0, 0] == np.float32(2.0 ** -24)
    assert _gate_scalar(x[0], w[0]) == np.float32(2.0 ** -24)
    assert _gate_scalar(x[0], w[0], fused=False) == 0.0


def test_gate_logits_instruction_and_libm_forms_agree():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((5, 1000)) * np.exp(rng.standard_normal((5, 1000)) * 4)).astype(np.float32)
    w = rng.standard_normal((7, 1000)).astype(np.float32)
    np.testing.assert_array_equal(R.gate_logits(x, w).view(np.uint32),
                                  R.gate_logits(x, w, force_libm=True).view(np.uint32))


def test_gate_logits_close_to_float64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    w = (rng.standard_normal((16, 4096)) / 64).astype(np.float32)
    z = R.gate_logits(x, w).astype(np.float64)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 4096 * 2.0 ** -23 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(z - ref) <= bound)


def test_router_matches_reference_torch_recipe():
    # reference tests/test_mlx_numerics.py:69-89 (torch.manual_seed(2), n=3, dim=16, E=8, k=2)
    torch.manual_seed(2)
    n, dim, n_exp, top_k = 3, 16, 8, 2
    x = torch.randn(n, dim)
    w = torch.randn(n_exp, dim) * 0.1
    b = torch.randn(n_exp)
    scores = torch.sqrt(torch.nn.functional.softplus(x.float() @ w.float().T))
    indices = (scores + b).topk(top_k, dim=-1)[1]
    weights = scores.gather(1, indices)
    weights = weights / (weights.sum(-1, keepdim=True) + 1e-20) * 1.5
    idx, wt, s, _ = R.route(x.numpy(), w.numpy(), b.numpy(), top_k, R.SCORE_SQRTSOFTPLUS, 1.5)
    got = sorted(zip(idx.ravel().tolist(), wt.ravel().tolist()))
    want = sorted(zip(indices.numpy().ravel().tolist(), weights.numpy().ravel().tolist()))
    assert [p[0] for p in got] == [p[0] for p in want]
    np.testing.assert_allclose([p[1] for p in got], [p[1] for p in want], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(s, scores.numpy(), rtol=1e-6, atol=1e-6)


def test_sigmoid_scores_match_torch():
    rng = np.random.default_rng(4)
    z = np.concatenate([rng.standard_normal(5000) * 8, [0.0, -0.0, 250.0, -250.0, 1e-8]]).astype(np.float32)
    s = R.scores_from_logits(z[None, :], R.SCORE_SIGMOID)[0]
    ref = torch.sigmoid(torch.from_numpy(z).double()).float().numpy()
    assert np.max(np.abs(s.astype(np.float64) - ref)) <= 6e-8


@pytest.mark.parametrize("k", [2, 3, 4, 6])
def test_route_weights_sum_to_scale(k):
    # reference tests/test_batch.py:321-337
    rng = np.random.default_rng(1)
    s = (rng.standard_normal((5, 384)) * 0.05 + 0.4).astype(np.float32)
    idx, w = R.topk_weights(s, np.zeros(384, np.float32), k, 1.5)
    assert idx.shape == (5, k) and idx.min() >= 0 and idx.max() < 384
    for row in range(5):
        assert len(set(idx[row].tolist())) == k
        assert abs(float(w[row].sum()) - 1.5) < 1e-4


def test_route_bias_steers_selection_only():
    # reference tests/test_mlx_forward.py:161-169
    rng = np.random.default_rng(0)
    s = (rng.standard_normal((2, 8)) * 0.01 + 0.5).astype(np.float32)
    bias = np.array([0, 0, 0, 0, 0, 0, 0, 10.0], np.float32)
    idx, w = R.topk_weights(s, bias, 2, 1.5)
    assert 7 in idx[0]
    j = list(idx[0]).index(7)
    other = idx[0][1 - j]
    assert abs(w[0][j] / w[0][1 - j] - s[0, 7] / s[0, other]) < 1e-6


def test_sqrtsoftplus_nonnegative():
    # reference tests/test_mlx_forward.py:172-177
    s = R.scores_from_logits(np.array([[-100.0, 0.0, 100.0, -1e30, 1e30]], np.float32),
                             R.SCORE_SQRTSOFTPLUS)
    assert np.all(s >= 0) and s[0, 1] == np.float32(math.sqrt(math.log(2)))


def test_topk_ties_go_to_lower_index_descending():
    s = np.array([[0.5, 0.7, 0.7, 0.2, 0.7, -0.0, 0.0]], np.float32)
    idx, _ = R.topk_weights(s, np.zeros(7, np.float32), 5, 1.0)
    assert idx[0].tolist() == [1, 2, 4, 0, 3]
    idx, _ = R.topk_weights(s, np.zeros(7, np.float32), 7, 1.0)
    assert idx[0].tolist()[-2:] == [5, 6]        # -0 and +0 tie: lower id first


def test_real_trace_weights_sum_to_reference_route_scale(golden):
    # reference profiles/traces/mlx-*.jsonl: every record's weights sum to 1.5
    d = golden("trace_routes.npz")
    assert d["experts"].shape[1] == 6
    np.testing.assert_allclose(d["weights"].sum(axis=1), 1.5, atol=5e-7)
    assert d["experts"].min() >= 0 and d["experts"].max() < 384


# ------------------------------------------------------------------ dispatch
def test_dispatch_align_docstring_example():
    # reference tests/test_audit.py:37-44
    topk = np.array([[1, 2, 3], [0, 1, 3], [0, 2, 3], [0, 1, 2]])
    sorted_ids, expert_ids, n_pad = D.align_block_size(topk, 4, 4)
    assert n_pad == 16
    assert list(expert_ids) == [0, 1, 2, 3]
    assert sorted(int(i) for i in sorted_ids if i != 12) == list(range(12))
    assert all(int(sorted_ids[i]) == 12 for i in (3, 7, 11, 15))
    counts, offsets, perm, rank = D.dispatch(topk, 4)
    assert perm.tolist() == [3, 6, 9, 0, 4, 10, 1, 7, 11, 2, 5, 8]
    assert counts.tolist() == [3, 3, 3, 3] and offsets.tolist() == [0, 3, 6, 9, 12]
    assert np.array_equal(perm[rank], np.arange(12))


def test_dispatch_properties_random():
    # reference tests/test_audit.py:47-60 (default_rng(0), 256 x 6, E = 384, block 16)
    rng = np.random.default_rng(0)
    topk = rng.integers(0, 384, size=(256, 6))
    sorted_ids, expert_ids, n_pad = D.align_block_size(topk, 16, 384)
    assert n_pad % 16 == 0 and len(expert_ids) == n_pad // 16
    flat = topk.reshape(-1)
    for expert in range(384):
        run = [int(i) for i in sorted_ids if i != len(flat) and flat[i] == expert]
        assert len(run) == int((flat == expert).sum())
        assert run == sorted(run)                      # stable
    counts, offsets, perm, rank = D.dispatch(topk, 384)
    np.testing.assert_array_equal(perm, np.argsort(flat, kind="stable"))


def test_dispatch_drops_negative_ids():
    idx = np.array([[3, -1], [-1, 0], [3, 7]])
    counts, offsets, perm, rank = D.dispatch(idx, 8)
    assert perm.tolist() == [3, 0, 4, 5]
    assert rank.tolist() == [1, -1, -1, 0, 2, 3]
    assert D.active_experts(counts).tolist() == [0, 3, 7]


def test_plan_groups_known_answer():
    # reference tests/test_grouped.py:29-39
    topk = [[2, 0], [1, 2], [0, 0]]
    assert D.plan_groups(topk, 3) == {2: [(0, 0), (1, 1)], 0: [(0, 1), (2, 0), (2, 1)], 1: [(1, 0)]}
    assert D.plan_groups([[], []], 3) == {}
    with pytest.raises(ValueError):
        D.plan_groups([[9]], 3)


def test_align_rejects_bad_input():
    with pytest.raises(ValueError):
        D.align_block_size(np.array([1, 2, 3]), 4, 4)
    with pytest.raises(ValueError):
        D.align_block_size(np.array([[0, 99]]), 4, 4)


# ------------------------------------------------------------------ layer
@pytest.fixture(scope="module")
def tiny():
    spec = synth.tiny_spec()
    d = synth.make_layer(spec, 1, 3)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    return spec, d, r


def test_layer_fp32_matches_fp64_brute_force(tiny):
    spec, d, r = tiny
    y64 = L.moe_forward_f64(d["x"], r["idx"], r["w"], d["bank"], d["shared"], spec)
    np.testing.assert_allclose(r["y_ref"].numpy(), y64, rtol=1e-4, atol=1e-5 * np.abs(y64).max())


def test_layer_grouped_equals_per_token(tiny):
    # reference tests/test_grouped.py:42-59: grouped evaluation == per-(token, slot) loop
    spec, d, r = tiny
    x32 = d["x"].float()
    acc = torch.zeros_like(x32)
    for t in range(x32.shape[0]):
        for e in sorted(r["idx"][t].tolist()):
            j = r["idx"][t].tolist().index(e)
            w1, w3, w2 = (torch.from_numpy(d["bank"].dequant(e, n)) for n in ("w1", "w3", "w2"))
            h = L.swiglu(x32[t:t + 1] @ w1.T, x32[t:t + 1] @ w3.T, spec.limit) * float(r["w"][t, j])
            acc[t] += (h @ w2.T)[0]
    routed = r["y_ref"] - L.shared_forward(x32, *d["shared"], spec.limit).to(torch.bfloat16).float()
    np.testing.assert_allclose(routed.numpy(), acc.numpy(), rtol=1e-5, atol=1e-6)


def _expert_contrib(spec, d, r, e):
    """Rows routed to expert e and their weighted w2 outputs, one (token, slot) at a time."""
    x32 = d["x"].float()
    rows, outs = [], []
    for t in range(x32.shape[0]):
        js = [j for j in range(r["idx"].shape[1]) if int(r["idx"][t, j]) == e]
        for j in js:
            w1, w3, w2 = (torch.from_numpy(d["bank"].dequant(e, n)) for n in ("w1", "w3", "w2"))
            h = L.swiglu(x32[t:t + 1] @ w1.T, x32[t:t + 1] @ w3.T, spec.limit) * float(r["w"][t, j])
            rows.append(t)
            outs.append((h @ w2.T)[0])
    return np.asarray(rows, dtype=np.int32), torch.stack(outs)


def test_layer_pinned_contributions(tiny):
    # reference mlx_forward.py:313-321, 388-393: a pinned expert's rows and weighted
    # outputs are added in its place instead of computing it
    spec, d, r = tiny
    sel = sorted({int(v) for v in r["idx"].ravel()})
    e0, e1 = sel[0], sel[-1]
    own = {e: _expert_contrib(spec, d, r, e) for e in (e0, e1)}
    same = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec, pinned=own)
    np.testing.assert_allclose(same["y_ref"].numpy(), r["y_ref"].numpy(), rtol=1e-5, atol=1e-6)
    rows, contrib = own[e1]
    zero = {e1: (rows, torch.zeros_like(contrib))}
    dropped = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec, pinned=zero)
    want = r["y_ref"].clone().index_add_(0, torch.from_numpy(rows.astype(np.int64)), -contrib)
    np.testing.assert_allclose(dropped["y_ref"].numpy(), want.numpy(), rtol=1e-5, atol=1e-6)
    unused = [e for e in range(spec.E) if e not in sel][0]
    ignored = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec,
                            pinned={unused: (np.array([0], dtype=np.int32), torch.ones((1, spec.H)))})
    np.testing.assert_array_equal(ignored["y_ref"].numpy(), r["y_ref"].numpy())


def test_layer_shared_changes_output(tiny):
    # reference tests/test_mlx_forward.py:324-353
    spec, d, r = tiny
    r0 = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)
    assert float((r["y_ref"] - r0["y_ref"]).abs().max()) > 1e-4
    np.testing.assert_array_equal(r0["idx"], r["idx"])


def test_layer_route_weight_before_w2_is_linear():
    # scaling the route scale scales the routed part exactly (weights multiply h before w2)
    spec = synth.tiny_spec()
    spec.I_shared = 0
    d = synth.make_layer(spec, 3, 2)
    a = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)["y_ref"]
    spec.route_scale = 5.0
    b = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)["y_ref"]
    np.testing.assert_allclose(b.numpy(), 2 * a.numpy(), rtol=1e-5, atol=1e-7)


def _digest(a) -> str:
    import hashlib
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu()
        a = (a.view(torch.int16) if a.dtype == torch.bfloat16 else a).numpy()
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_golden_cfg0_matches_oracle(golden):
    """Generator and oracle have not drifted from the committed cfg0 fixture."""
    import json
    g = golden("cfg0.npz")
    spec = synth.config0_spec()
    d = synth.make_layer(spec, 0, 4)
    want = json.loads(str(g["digests"]))
    assert _digest(d["x"]) == want["x"] and _digest(d["gate_w"]) == want["gate_w"]
    for role, parts in d["bank"].roles.items():
        for i, p in enumerate(parts):
            assert _digest(p) == want[f"{role}.{i}"], role
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    np.testing.assert_array_equal(r["idx"], g["idx"])
    np.testing.assert_array_equal(r["w"], g["w"])
    np.testing.assert_array_equal(r["perm"], g["perm"])
    np.testing.assert_array_equal(r["counts"], g["counts"])
    np.testing.assert_allclose(r["y_ref"].numpy(), g["y_ref"], rtol=1e-5, atol=1e-6)
    assert abs(float(r["w"].sum(axis=1).mean()) - 2.5) < 1e-6
