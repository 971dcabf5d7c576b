"""RMSNorm of a residual stream and the layer-stack composition, restated on the CPU.

Test infrastructure only (what the stack runner is compared against).

Reference: ``rmsnorm`` (``src/deepseeker/mlx_forward.py:45-59``): for
lower-precision inputs ``xf = f32(x)``, ``rstd = rsqrt(mean(xf * xf) + eps)``,
``y = (xf * rstd * f32(weight)).astype(x.dtype)``; the runner's layer loop
(``src/deepseeker/mlx_runner.py:2138-2145``) carries the residual stream
between layers.  The stack composition is

    h_0 = x;  y_l = rmsnorm(h_l);  h_{l+1} = round(h_l + layer_l(y_l))

with the sum rounded to the stream's dtype.

The mean of squares has one defined order, so that the normalised rows (which
feed the next layer's router) are bit-identical to the device kernel: the row
is cut into 4-element chunks; accumulator t (t = 0..255) adds, for its chunks
c = t, t + 256, ... in order and then the 4 elements of each chunk, the
rounded square (product rounded, then sum rounded, no fused multiply-add);
each group of 64 accumulators is combined by an XOR tree (for s = 32..1:
p[l] = p[l] + p[l ^ s]; the tree value is p[0]), and the 4 group values are
added in order.  Then rstd = 1 / sqrt(sum / H + eps) with correctly rounded
float32 division and square root, and y = (h * rstd) * gamma, each product
rounded to float32, then one rounding to the output dtype.

Pinned by the tests against torch's ``rms_norm`` (float64 closeness), closed
forms (constant rows, scaling by powers of two) and a scalar loop of the same
order.
"""

from __future__ import annotations

import numpy as np

THREADS = 256


def _round_bf16(v: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 -> float32."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(v)
    out[nan] = np.float32(np.nan)
    return out


def round_to(v: np.ndarray, dtype: str) -> np.ndarray:
    return _round_bf16(v) if dtype == "bf16" else np.asarray(v, dtype=np.float32)


def sum_of_squares(h: np.ndarray) -> np.ndarray:
    """Per-row sum of squares in the defined order; h [rows, H] float32, H % 4 == 0."""
    h = np.asarray(h, dtype=np.float32)
    rows, hd = h.shape
    nch = hd // 4
    hc = h.reshape(rows, nch, 4)
    acc = np.zeros((rows, THREADS), dtype=np.float32)
    for j in range(-(-nch // THREADS)):
        lo, hi = j * THREADS, min((j + 1) * THREADS, nch)
        n = hi - lo
        for q in range(4):
            v = hc[:, lo:hi, q]
            acc[:, :n] = acc[:, :n] + (v * v).astype(np.float32)
    waves = acc.reshape(rows, THREADS // 64, 64)
    lanes = np.arange(64)
    for s in (32, 16, 8, 4, 2, 1):
        waves = (waves + waves[:, :, lanes ^ s]).astype(np.float32)
    tot = np.zeros(rows, dtype=np.float32)
    for w in range(THREADS // 64):
        tot = (tot + waves[:, w, 0]).astype(np.float32)
    return tot


def rmsnorm(x: np.ndarray, eps: float = 1e-6, gamma: np.ndarray | None = None,
            residual: np.ndarray | None = None, dtype: str = "bf16"):
    """(h, y): h = round(x + residual) (or x), y = round((h * rstd) * gamma).

    x, residual: float32 arrays holding values of ``dtype`` ("bf16" or "f32")."""
    h = np.asarray(x, dtype=np.float32)
    if residual is not None:
        h = round_to((h + np.asarray(residual, dtype=np.float32)).astype(np.float32), dtype)
    tot = sum_of_squares(h)
    hd = np.float32(h.shape[1])
    rstd = (np.float32(1.0) / np.sqrt((tot / hd + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = (h * rstd[:, None]).astype(np.float32)
    if gamma is not None:
        y = (y * np.asarray(gamma, dtype=np.float32)[None, :]).astype(np.float32)
    return h, round_to(y, dtype)


def rmsnorm_scalar(row: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """One row, pure-Python loops in the defined order (small rows only): the
    independent restatement that pins ``sum_of_squares``."""
    row = [np.float32(v) for v in row]
    nch = len(row) // 4
    acc = [np.float32(0.0)] * THREADS
    for t in range(THREADS):
        c = t
        while c < nch:
            for q in range(4):
                v = row[4 * c + q]
                acc[t] = np.float32(acc[t] + np.float32(v * v))
            c += THREADS
    tot = np.float32(0.0)
    for w in range(THREADS // 64):
        p = acc[64 * w: 64 * w + 64]
        for s in (32, 16, 8, 4, 2, 1):
            p = [np.float32(p[l] + p[l ^ s]) for l in range(64)]
        tot = np.float32(tot + p[0])
    rstd = np.float32(np.float32(1.0) / np.float32(np.sqrt(np.float32(tot / np.float32(len(row)) + np.float32(eps)))))
    return np.array([np.float32(v * rstd) for v in row], dtype=np.float32)


def stack_forward(x: np.ndarray, layer_fns, eps: float = 1e-6, dtype: str = "bf16"):
    """h_L of the stack; layer_fns[l](y) returns layer l's output as float32 values of ``dtype``."""
    h = np.asarray(x, dtype=np.float32)
    for fn in layer_fns:
        _, y = rmsnorm(h, eps, dtype=dtype)
        h = round_to((h + np.asarray(fn(y), dtype=np.float32)).astype(np.float32), dtype)
    return h
