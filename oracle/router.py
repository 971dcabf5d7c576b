"""Router of the MoE layer, restated on the CPU with a fixed arithmetic order.

Reference: ``src/deepseeker/mlx_forward.py:62-65`` (``sqrtsoftplus_scores``:
``z = f32(x) @ f32(W).T``, ``s = sqrt(logaddexp(z, 0))``) and ``:68-81``
(``route_topk``: select the top-k of ``s + bias``, weights are the un-biased
scores of the selected experts divided by ``(sum + 1e-20)`` and multiplied by
the route scale).  The workload spec uses sigmoid scores and route scale 2.5;
the reference default is sqrt-softplus with 1.5.  Both are supported.

Routing indices must be bit-identical between this oracle and the GPU, so
every floating-point step has one defined order that the HIP kernel mirrors:

1. Gate logit ``z[t, e]``: H is cut into 256-element steps ``m`` (positions
   >= H contribute nothing) and the steps into 4 segments of ``S = ceil(steps/4)``
   consecutive steps (segment w holds steps [w*S, (w+1)*S)).  In each segment,
   64 partial sums: partial ``l`` starts at +0 and takes, for its steps ``m`` in
   order and then ``v = 0..3``, ``p = fma(x[256*m + 4*l + v], W[256*m + 4*l + v], p)``
   (the IEEE fused multiply-add: one rounding).  The 64 partials are combined
   by an XOR butterfly (for s = 32, 16, 8, 4, 2, 1: ``p[l] = p[l] + p[l ^ s]``)
   into the segment sum ``s_w = p[0]``, and ``z = ((s_0 + s_1) + s_2) + s_3``.
   The chains are evaluated by ``oracle/gate_fma.c`` (C ``fmaf``), built on
   first use by ``oracle/build_c.py``.
2. Scores are computed in float64 from ``z`` with this module's own ``exp``
   (Cody-Waite reduction by ln2 split in a 32-bit-exact high part and a low
   part, degree-14 Taylor polynomial in Horner form, ``ldexp``) and
   ``log1p(u) = 2 * atanh(u / (2 + u))`` (odd series to degree 37), then
   rounded once to float32.  sqrt-softplus takes the correctly rounded
   float32 square root of the float64 softplus, found with exact float64
   midpoint tests (independent of any library ``sqrt``).
3. ``key = f32(s + bias) + 0`` (turns -0 into +0).  The k largest keys are
   taken in descending key order, ties to the lower expert index.  (The
   reference returns the same set in ascending order, ``argsort`` tail.)
4. ``w_j = (s_j / (((s_0 + s_1) + ...) + 1e-20)) * route_scale`` in float32,
   the sum taken in selection order.

Parity: the fused chain is pinned in the tests by an exact-rational scalar
restatement (every fma rounded once from the exact value, ties to even) and by
inputs where an unfused product would differ; the closed forms are pinned by the reference's own
torch router recipe (``tests/test_mlx_numerics.py:69-89``), the invariants
of ``tests/test_batch.py:321-337`` and ``tests/test_mlx_forward.py:161-177``,
and by comparing ``exp``/``log1p``/``sqrt`` with ``math`` on many points.
"""

from __future__ import annotations

import concurrent.futures as cf
import ctypes
import math
import os
import threading
from fractions import Fraction

import numpy as np

SCORE_SIGMOID = 0
SCORE_SQRTSOFTPLUS = 1

GATE_LANES = 64
GATE_VEC = 4
GATE_STEP = GATE_LANES * GATE_VEC   # 256 elements of H per step

_LN2 = Fraction(
    "0.693147180559945309417232121458176568075500134360255254120680009493393621969694715605863326996418687")


def _ln2_split() -> tuple[float, float]:
    """ln2 = HI + LO with HI holding 32 significant bits (k*HI exact for |k| < 2**21)."""
    hi = float(_LN2)
    m, e = math.frexp(hi)
    hi = math.ldexp(math.floor(m * 2**32) / 2**32, e)
    lo = float(_LN2 - Fraction(hi))
    return hi, lo


LN2_HI, LN2_LO = _ln2_split()
LOG2E = float(1 / _LN2)
EXP_COEF = [float(Fraction(1, math.factorial(n))) for n in range(15)]    # 1/n!, n = 0..14
ATANH_COEF = [float(Fraction(1, 2 * n + 1)) for n in range(19)]          # 1/(2n+1), n = 0..18
SIGMOID_CLAMP = 200.0      # sigmoid(+-200) already rounds to 1 / 0 in float32
SOFTPLUS_TAIL = 1000.0     # exp(-1000) underflows float64: the log1p term is 0


def exp_d(x: np.ndarray) -> np.ndarray:
    """float64 exp for |x| <= 1000 (Cody-Waite + Taylor), order fixed for the GPU."""
    x = np.asarray(x, dtype=np.float64)
    k = np.rint(x * LOG2E)
    r = (x - k * LN2_HI) - k * LN2_LO
    p = np.full_like(r, EXP_COEF[14])
    for n in range(13, -1, -1):
        p = p * r + EXP_COEF[n]
    return np.ldexp(p, k.astype(np.int64))


def log1p_d(u: np.ndarray) -> np.ndarray:
    """float64 log(1 + u) for u in [0, 1]: 2 * atanh(u / (2 + u))."""
    u = np.asarray(u, dtype=np.float64)
    s = u / (2.0 + u)
    s2 = s * s
    p = np.full_like(s, ATANH_COEF[18])
    for n in range(17, -1, -1):
        p = p * s2 + ATANH_COEF[n]
    return 2.0 * (s * p)


def sqrt_round_f32(v: np.ndarray) -> np.ndarray:
    """Correctly rounded float32 sqrt of float64 v >= 0 (round half to even).

    Start from any estimate within one float32 ulp, then compare v with the
    squares of the two neighbouring float32 midpoints; both squares are exact
    in float64 (25-bit midpoints), so the correction is exact.
    """
    v = np.asarray(v, dtype=np.float64)
    r = np.sqrt(v).astype(np.float32)
    rd = r.astype(np.float64)
    dn = np.nextafter(r, np.float32(0.0))
    up = np.nextafter(r, np.float32(np.inf))
    lo = (rd + dn.astype(np.float64)) * 0.5
    hi = (rd + up.astype(np.float64)) * 0.5
    lo2 = lo * lo
    hi2 = hi * hi
    r_even = (r.view(np.uint32) & 1) == 0
    go_dn = (r > 0) & ((v < lo2) | ((v == lo2) & ~r_even))
    go_up = (v > hi2) | ((v == hi2) & ~r_even)
    out = np.where(go_dn, dn, np.where(go_up, up, r))
    return out.astype(np.float32)


GATE_SEGMENTS = 4

_LIB = None
_LIB_LOCK = threading.Lock()


def _gate_lib() -> ctypes.CDLL:
    """The oracle's C gate chains (``oracle/gate_fma.c``), built on first use."""
    global _LIB
    with _LIB_LOCK:
        if _LIB is None:
            from . import build_c
            if not build_c.LIB.exists():
                build_c.build()
            lib = ctypes.CDLL(str(build_c.LIB))
            fn = lib.dsk_oracle_gate_fma
            fn.restype = None
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                           ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32]
            _LIB = lib
    return _LIB


def _by_step(a: np.ndarray, steps: int) -> np.ndarray:
    """[N, H] float32 -> [N, steps, 4, 64]: element (m, v, l) is position 256 m + 4 l + v (zero past H)."""
    n, h = a.shape
    hp = steps * GATE_STEP
    if hp != h:
        a = np.pad(a, ((0, 0), (0, hp - h)))
    return np.ascontiguousarray(a.reshape(n, steps, GATE_LANES, GATE_VEC).transpose(0, 1, 3, 2))


def gate_logits(x: np.ndarray, gate_w: np.ndarray, workers: int | None = None,
                force_libm: bool = False) -> np.ndarray:
    """z = f32(x) @ f32(W).T in the fixed segment/lane order of the module docstring.

    x: [T, H] (any float dtype, converted exactly to float32), gate_w: [E, H].
    Token chunks are independent, so they are spread over ``workers`` threads
    (the C chains run without the GIL); every logit's arithmetic is the same
    whatever the chunking.  ``force_libm`` evaluates every fma through the C
    library's ``fmaf`` instead of the CPU's FMA instruction (same results).
    """
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(gate_w, dtype=np.float32)
    t, h = x.shape
    e = w.shape[0]
    steps = -(-h // GATE_STEP)
    xt, wt = _by_step(x, steps), _by_step(w, steps)
    out = np.empty((t, e), dtype=np.float32)
    lib = _gate_lib()
    n = max(1, min(t, workers or min(16, os.cpu_count() or 1)))
    bounds = [(t * i) // n for i in range(n + 1)]

    def chunk(i: int) -> None:
        lib.dsk_oracle_gate_fma(xt.ctypes.data, wt.ctypes.data, e, steps, bounds[i], bounds[i + 1],
                                out.ctypes.data, 1 if force_libm else 0)

    if n == 1:
        chunk(0)
    else:
        with cf.ThreadPoolExecutor(max_workers=n) as ex:
            list(ex.map(chunk, range(n)))
    return out


def scores_from_logits(z: np.ndarray, score_func: int) -> np.ndarray:
    """float32 logits -> float32 scores (sigmoid or sqrt(softplus))."""
    zd = np.asarray(z, dtype=np.float32).astype(np.float64)
    if score_func == SCORE_SIGMOID:
        zc = np.clip(zd, -SIGMOID_CLAMP, SIGMOID_CLAMP)
        return (1.0 / (1.0 + exp_d(-zc))).astype(np.float32)
    if score_func == SCORE_SQRTSOFTPLUS:
        a = np.abs(zd)
        u = np.where(a > SOFTPLUS_TAIL, 0.0, exp_d(-np.minimum(a, SOFTPLUS_TAIL)))
        sp = np.maximum(zd, 0.0) + log1p_d(u)
        return sqrt_round_f32(sp)
    raise ValueError(f"unknown score_func {score_func}")


def topk_weights(scores: np.ndarray, bias: np.ndarray, k: int,
                 route_scale: float) -> tuple[np.ndarray, np.ndarray]:
    """(idx [T, k] int32, w [T, k] float32) from float32 scores and bias."""
    s = np.asarray(scores, dtype=np.float32)
    t, e = s.shape
    if not 1 <= k <= e:
        raise ValueError(f"top_k={k} must be in [1, {e}]")
    key = (s + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32) + np.float32(0.0)
    order = np.argsort(-key, axis=1, kind="stable")
    idx = order[:, :k].astype(np.int32)
    sel = np.take_along_axis(s, idx, axis=1)
    acc = np.zeros(t, dtype=np.float32)
    for j in range(k):
        acc = (acc + sel[:, j]).astype(np.float32)
    denom = (acc + np.float32(1e-20)).astype(np.float32)
    w = ((sel / denom[:, None]).astype(np.float32) * np.float32(route_scale)).astype(np.float32)
    return idx, w


def route(x: np.ndarray, gate_w: np.ndarray, gate_b: np.ndarray, k: int,
          score_func: int = SCORE_SIGMOID, route_scale: float = 2.5):
    """Full router: returns (idx, w, scores, logits)."""
    z = gate_logits(x, gate_w)
    s = scores_from_logits(z, score_func)
    idx, w = topk_weights(s, gate_b, k, route_scale)
    return idx, w, s, z
