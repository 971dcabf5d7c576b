"""Weight formats of the routed experts, restated on the CPU with numpy.

FP4 (mxfp4)
    Two e2m1 codes per byte, low nibble first, one E8M0 scale byte per 32
    codes along K.  A role of shape [N, K] is stored as ``packed [N, K/2] u8``
    and ``scales [N, K/32] u8``.  Decode:
    ``v[n, c] = FP4_TABLE[(packed[n, c>>1] >> 4*(c&1)) & 15] * 2**(scales[n, c>>5] - 127)``
    with scale byte 0xFF decoding to NaN.  Follows the reference's
    ``src/deepseeker/metal_fp4.py:21-26`` (table), ``:96-103`` (E8M0 LUT),
    ``:122-131`` (``reference_dequant``) and
    ``src/deepseeker/mlx_weights.py:66-79, 148-166``.
    Pinned by the reference's known-answer tests (``tests/test_metal_fp4.py:35-41``,
    ``tests/test_q3.py:132-140``) and its seeded random vectors
    (``tests/test_metal_fp4.py:44-54``, regenerated with numpy).

FP4 quantiser
    The reference quantises with MLX (``mx.quantize(mode="mxfp4")``), whose
    rounding is not visible here.  The workload spec fixes the rule instead:
    per 32-group, ``scale = 2**ceil(log2(amax/6))`` (computed exactly from
    ``frexp``), each value rounded to nearest-even on the e2m1 grid,
    saturating at +-6, never emitting the negative-zero code 0x8.
    Pinned by brute force: every code's decode is the grid point nearest to
    the input (checked against an exhaustive search in the tests).

Q3 affine (group 64, fp16 scale and bias)
    ``W = s * q + b`` with ``q`` in [0, 7]; ``scales``/``biases`` are
    ``[N, K/64] f16`` as in the reference (``src/deepseeker/mlx_weights.py:119-145``;
    ``scripts/requant_experts_3bit.py:69-83``).  The reference's code packing is
    MLX-internal and not visible, so the codes use this build's canonical
    layout (3 bits per code, 48 bytes per 128 codes, lane-group chunks of 4
    blocks interleaved per 512 codes): see ``q3_pack``.
    Parity with MLX's packing and its quantiser rounding is unpinned; the
    layout is pinned by a pack/unpack round trip and a hand-built
    known-answer vector in the tests.

FP8 E4M3 with 32 x 32 block scales (the checkpoint's dense weights, e.g. the
shared expert)
    OCP e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 15
    with mantissa 7 is NaN (no infinities, the rest of that row is
    256 * (1 + m/8)); exponent 0 is subnormal, m/8 * 2**-6.  One E8M0 scale
    per 32 x 32 block: ``w[i, j] = E4M3[codes[i, j]] * 2**(scales[i//32, j//32] - 127)``.
    Follows ``src/deepseeker/mlx_weights.py:29-41`` (table) and ``:82-89``
    (``dequant_fp8_block``).  Pinned by torch's ``float8_e4m3fn`` decode of all
    256 bytes, the reference's spot values (``tests/test_mlx_weights.py:47-57``)
    and its seeded block test (``:64-74``, regenerated with numpy).
"""

from __future__ import annotations

import numpy as np

# e2m1 value of each nibble; code 8 (negative zero) decodes to +0, as in the
# reference table.
FP4_TABLE = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
     0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
FP4_GROUP = 32
Q3_GROUP = 64
Q3_BITS = 3
Q3_BLOCK = 128               # codes per 48-byte block (four 12-byte lane-group chunks)
Q3_BLOCK_BYTES = 48
Q3_SUPERBLOCK = 512          # four blocks whose lane-group chunks are interleaved
Q3_SUPERBLOCK_BYTES = 192


def e8m0_to_f32(scales: np.ndarray) -> np.ndarray:
    """E8M0 bytes -> float32 powers of two; 0xFF -> NaN.

    Follows ``src/deepseeker/metal_fp4.py:96-103`` and
    ``src/deepseeker/mlx_weights.py:66-79``.  Byte 0 is 2**-127, a float32
    subnormal, which is exact.
    """
    b = np.asarray(scales, dtype=np.uint8).astype(np.int32)
    out = np.ldexp(np.float32(1.0), np.minimum(b, 254) - 127).astype(np.float32)
    out[b == 0xFF] = np.nan
    return out


def fp4_codes(packed: np.ndarray) -> np.ndarray:
    """[..., K/2] u8 -> [..., K] u8 nibble codes, low nibble first."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


# value pair of every packed byte: (low nibble, high nibble)
_FP4_PAIRS = np.stack([FP4_TABLE[np.arange(256) & 15], FP4_TABLE[np.arange(256) >> 4]], axis=-1)


def fp4_dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """FP4 role [..., K/2] u8 + [..., K/32] u8 -> float32 [..., K].

    Same arithmetic as the reference's ``reference_dequant``
    (``src/deepseeker/metal_fp4.py:122-131``): table value times the decoded
    scale, one float32 multiply per element (exact: both factors are short).
    The table is looked up per byte (both nibbles at once, low first).
    """
    p = np.asarray(packed, dtype=np.uint8)
    k = p.shape[-1] * 2
    s = np.asarray(scales, dtype=np.uint8)
    if s.shape[-1] * FP4_GROUP != k:
        raise ValueError(f"scales {s.shape} do not cover K={k} in groups of 32")
    vals = np.take(_FP4_PAIRS, p, axis=0).reshape(p.shape[:-1] + (k // FP4_GROUP, FP4_GROUP))
    return (vals * e8m0_to_f32(s)[..., None]).reshape(p.shape[:-1] + (k,))


def fp4_scale_exponent(amax: np.ndarray) -> np.ndarray:
    """Smallest integer e with 6 * 2**e >= amax, i.e. ceil(log2(amax / 6)).

    Exact: with ``amax = m * 2**x`` (``frexp``, m in [0.5, 1)),
    ``6 * 2**(x-3) = 0.75 * 2**x``, so e = x-3 when m <= 0.75, else x-2.
    amax == 0 maps to e = 0 (scale byte 127; every code is then 0).
    """
    a = np.asarray(amax, dtype=np.float32)
    m, x = np.frexp(a)
    e = np.where(m <= 0.75, x - 3, x - 2).astype(np.int32)
    return np.where(a == 0, 0, e).astype(np.int32)


# Magnitude thresholds (in units of the group scale) between successive
# e2m1 grid points 0, .5, 1, 1.5, 2, 3, 4, 6.  At a tie the code with an even
# index wins (round-half-even on the code index): <= keeps the lower code,
# < moves to the upper one.
_FP4_EDGES = ((0.25, True), (0.75, False), (1.25, True), (1.75, False),
              (2.5, True), (3.5, False), (5.0, True))


def fp4_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float32 [..., K] -> (packed [..., K/2] u8, scales [..., K/32] u8).

    The workload-spec quantiser described in the module docstring.  NaN and
    infinite inputs are outside its contract.
    """
    w = np.asarray(w, dtype=np.float32)
    k = w.shape[-1]
    if k % FP4_GROUP:
        raise ValueError(f"K={k} is not a multiple of {FP4_GROUP}")
    g = w.reshape(w.shape[:-1] + (k // FP4_GROUP, FP4_GROUP))
    amax = np.abs(g).max(axis=-1)
    e = fp4_scale_exponent(amax)
    sbyte = np.clip(e + 127, 0, 254).astype(np.int32)
    e_eff = sbyte - 127
    q = np.ldexp(np.abs(g), -e_eff[..., None]).astype(np.float32)
    mag = np.zeros(q.shape, dtype=np.uint8)
    for edge, inclusive in _FP4_EDGES:
        mag += (q > edge) if inclusive else (q >= edge)
    code = np.where((mag != 0) & (g < 0), mag | 8, mag).astype(np.uint8)
    code = code.reshape(w.shape)
    packed = (code[..., 0::2] | (code[..., 1::2] << 4)).astype(np.uint8)
    return packed, sbyte.astype(np.uint8)


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def q3_quantize_codes(w: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """float32 [N, K] -> (q [N, K] u8 in 0..7, scales f16 [N, K/64], biases f16 [N, K/64]).

    Per 64-group: ``s = f16((max - min) / 7)``, ``b = f16(min)``,
    ``q = clip(rint((w - b) / s), 0, 7)`` in float32 (q = 0 where s == 0).
    This rule is this build's own ("MLX-style" affine, group 64, bits 3);
    MLX's exact rounding is parity unpinned.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % Q3_GROUP:
        raise ValueError(f"K={k} is not a multiple of {Q3_GROUP}")
    g = w.reshape(n, k // Q3_GROUP, Q3_GROUP)
    wmin = g.min(axis=-1)
    wmax = g.max(axis=-1)
    scale32 = ((wmax - wmin) / np.float32(7.0)).astype(np.float32)
    s16 = scale32.astype(np.float16)
    b16 = wmin.astype(np.float16)
    s = s16.astype(np.float32)[..., None]
    b = b16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        t = ((g - b) / np.where(s == 0, np.float32(1.0), s)).astype(np.float32)
    q = np.clip(np.rint(t), 0, 7)
    q = np.where(s == 0, 0, q).astype(np.uint8)
    return q.reshape(n, k), s16, b16


def _q3_pair_table():
    """For each of the 16 code pairs of a lane word group: (m, i)."""
    return [(p // 4, p % 4) for p in range(16)]


def q3_chunk_offset(k: int, kb: int, g: int) -> int:
    """Byte offset, within a row of K codes, of lane group g's 12 bytes of
    128-code block kb: in a full 512-code superblock the chunks of one lane
    group are contiguous (``192 * (kb // 4) + 48 * g + 12 * (kb % 4)``); blocks
    after the last full superblock are plain 48-byte blocks (``48 * kb + 12 * g``)."""
    if kb // 4 < k // Q3_SUPERBLOCK:
        return (kb // 4) * Q3_SUPERBLOCK_BYTES + 48 * g + 12 * (kb % 4)
    return kb * Q3_BLOCK_BYTES + 12 * g


def _q3_byte_index(k: int) -> np.ndarray:
    """[K/128, 4, 12] row byte index of each block's lane-group chunks."""
    nb = k // Q3_BLOCK
    off = np.array([[q3_chunk_offset(k, kb, g) for g in range(4)] for kb in range(nb)], dtype=np.int64)
    return off[:, :, None] + np.arange(12)


def q3_pack(q: np.ndarray) -> np.ndarray:
    """Codes [N, K] (0..7) -> canonical packed bytes [N, 3K/8] u8.

    Canonical layout (this build's; K must be a multiple of 128): a row is a
    sequence of 128-code blocks.  Lane group g (0..3) of a block owns 12
    bytes, read as three little-endian u32 words d0, d1, d2, holding the 32
    consecutive codes ``32*g + 8*m + j`` (m = 0..3, j = 0..7) of the block as
    16 pairs P = 4*m + j//2, the even-j code in the low half and the odd-j
    code in the high half.  Pair P < 15 sits in word P // 5: low code at bit
    3*(P % 5), high code at bit 16 + 3*(P % 5).  Pair 15 uses the spare bits:
    bit t of its low code is bit 15 of word t, bit t of its high code is bit
    31 of word t.  The chunks are placed by ``q3_chunk_offset``: within each
    full 512-code superblock (192 bytes) lane group g's chunks of the four
    blocks are the 48 contiguous bytes at 48*g, so a lane reads four blocks
    as three aligned 16-byte words; a tail of fewer than four blocks keeps
    plain 48-byte blocks.
    A lane group's 32 codes are the same K range an FP4 lane group reads
    (one 16-byte word of 32 codes), all in one 64-group (g < 2: the block's
    first group), and every pair is one shift-and-mask away from a packed
    16-bit pair.
    """
    q = np.asarray(q, dtype=np.uint32)
    n, k = q.shape
    if k % Q3_BLOCK:
        raise ValueError(f"K={k} is not a multiple of {Q3_BLOCK}")
    if q.size and q.max() > 7:
        raise ValueError("q3 codes must be in 0..7")
    nb = k // Q3_BLOCK
    # code index within block = 32*g + 8*m + j  -> axes [N, nb, g, m, j]
    c = q.reshape(n, nb, 4, 4, 8)
    words = np.zeros((n, nb, 4, 3), dtype=np.uint32)   # [.., g, d]
    for p, (m, i) in enumerate(_q3_pair_table()):
        lo = c[:, :, :, m, 2 * i]
        hi = c[:, :, :, m, 2 * i + 1]
        if p < 15:
            d, s = p // 5, 3 * (p % 5)
            words[:, :, :, d] |= (lo << s) | (hi << (16 + s))
        else:
            for t in range(3):
                words[:, :, :, t] |= (((lo >> t) & 1) << 15) | (((hi >> t) & 1) << 31)
    chunks = words.astype("<u4").view(np.uint8).reshape(n, nb, 4, 12)
    out = np.zeros((n, k * 3 // 8), dtype=np.uint8)
    out[:, _q3_byte_index(k)] = chunks
    return out


def q3_unpack(packed: np.ndarray, k: int) -> np.ndarray:
    """Canonical packed bytes [N, 3K/8] -> codes [N, K] u8 (inverse of ``q3_pack``)."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n = p.shape[0]
    if k % Q3_BLOCK or p.shape[1] != k * 3 // 8:
        raise ValueError(f"packed {p.shape} does not hold K={k} q3 codes")
    nb = k // Q3_BLOCK
    chunks = np.ascontiguousarray(p[:, _q3_byte_index(k)])           # [N, nb, 4, 12]
    words = chunks.view("<u4").reshape(n, nb, 4, 3).astype(np.uint32)
    c = np.zeros((n, nb, 4, 4, 8), dtype=np.uint32)    # [.., g, m, j]
    for pidx, (m, i) in enumerate(_q3_pair_table()):
        if pidx < 15:
            d, s = pidx // 5, 3 * (pidx % 5)
            lo = (words[:, :, :, d] >> s) & 7
            hi = (words[:, :, :, d] >> (16 + s)) & 7
        else:
            lo = np.zeros((n, nb, 4), dtype=np.uint32)
            hi = np.zeros((n, nb, 4), dtype=np.uint32)
            for t in range(3):
                lo |= ((words[:, :, :, t] >> 15) & 1) << t
                hi |= ((words[:, :, :, t] >> 31) & 1) << t
        c[:, :, :, m, 2 * i] = lo
        c[:, :, :, m, 2 * i + 1] = hi
    return c.reshape(n, k).astype(np.uint8)


def q3_pack_rowmajor(q: np.ndarray) -> np.ndarray:
    """Codes [N, K] (0..7) -> row-major 3-byte packs [N, 3K/8] u8 (the checkpoint layout).

    Bytes ``3m..3m+2`` of a row hold codes ``8m..8m+7`` as one 24-bit
    little-endian integer, code ``i`` of the pack at bits ``3i..3i+2``; equally,
    a row is a little-endian bit stream with code ``c`` at bits ``3c..3c+2``.
    Viewed as little-endian u32 words this is the ``[N, ceil(3K/32)]`` ``U32_Q3_AFFINE``
    tensor of the reference's q3 checkpoints (``src/deepseeker/mlx_weights.py:119-141``;
    written by ``scripts/requant_experts_3bit.py:69-83, 135-148``), whose word order
    the reference calls MLX-internal: this build fixes it as stated here.
    K must be a multiple of 8.  Pinned in the tests by the known answer
    codes 0..7 -> 0o76543210 (bytes 88 C6 FA), by the bit-stream restatement
    (``numpy.packbits`` in little-endian bit order) and by round trips.
    """
    q = np.asarray(q, dtype=np.uint32)
    n, k = q.shape
    if k % 8:
        raise ValueError(f"K={k} is not a multiple of 8")
    if q.size and q.max() > 7:
        raise ValueError("q3 codes must be in 0..7")
    packs = np.zeros((n, k // 8), dtype=np.uint32)
    for i in range(8):
        packs |= q[:, i::8] << (3 * i)
    out = np.empty((n, k // 8, 3), dtype=np.uint8)
    for byte in range(3):
        out[:, :, byte] = (packs >> (8 * byte)) & 0xFF
    return out.reshape(n, k * 3 // 8)


def q3_unpack_rowmajor(packed: np.ndarray, k: int) -> np.ndarray:
    """Row-major 3-byte packs [N, 3K/8] u8 -> codes [N, K] u8 (inverse of ``q3_pack_rowmajor``)."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n = p.shape[0]
    if k % 8 or p.shape[1] != k * 3 // 8:
        raise ValueError(f"packed {p.shape} does not hold K={k} q3 codes")
    b = p.reshape(n, k // 8, 3).astype(np.uint32)
    packs = b[:, :, 0] | (b[:, :, 1] << 8) | (b[:, :, 2] << 16)
    q = np.empty((n, k), dtype=np.uint8)
    for i in range(8):
        q[:, i::8] = (packs >> (3 * i)) & 7
    return q


def q3_rowmajor_to_canonical(packed: np.ndarray, k: int) -> np.ndarray:
    """Checkpoint (row-major 3-byte packs) -> this build's canonical kernel layout."""
    return q3_pack(q3_unpack_rowmajor(packed, k))


def q3_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """float32 [N, K] -> (packed [N, 3K/8] u8, scales f16 [N, K/64], biases f16 [N, K/64])."""
    q, s, b = q3_quantize_codes(w)
    return q3_pack(q), s, b


def q3_dequant(packed: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """Canonical q3 role -> float32 [N, K]: ``f32(s) * q + f32(b)``, two roundings.

    Same closed form as the reference's affine dequant (``W = s*q + b`` per
    64-group, ``src/deepseeker/mlx_weights.py:119-141``).
    """
    s = np.asarray(scales).astype(np.float32)
    b = np.asarray(biases).astype(np.float32)
    n, groups = s.shape
    k = groups * Q3_GROUP
    q = q3_unpack(packed, k).astype(np.float32).reshape(n, groups, Q3_GROUP)
    return ((s[..., None] * q) + b[..., None]).astype(np.float32).reshape(n, k)


def _e4m3_table() -> np.ndarray:
    b = np.arange(256)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = (b & 7).astype(np.float64)
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    t = (sign * mag).astype(np.float32)
    t[(e == 15) & ((b & 7) == 7)] = np.nan
    return t


E4M3_TABLE = _e4m3_table()


def fp8_block_dequant(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[R, C] E4M3 bytes + [R/32, C/32] E8M0 block scales -> float32 [R, C]."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, cols = codes.shape
    if rows % 32 or cols % 32 or scales.shape != (rows // 32, cols // 32):
        raise ValueError(f"codes {codes.shape} / scales {scales.shape} do not tile in 32 x 32 blocks")
    gain = np.repeat(np.repeat(e8m0_to_f32(np.asarray(scales, dtype=np.uint8)), 32, axis=0), 32, axis=1)
    return (E4M3_TABLE[codes] * gain).astype(np.float32)
