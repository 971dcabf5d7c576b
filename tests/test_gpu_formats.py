"""GPU parity of the weight-format kernels against the oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from oracle import formats as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_fp4_dequant_exhaustive_codes_and_scales():
    # every (code byte, scale byte) pair: 256 scale bytes x 16 bytes x 32 codes
    packed = np.tile(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 1))  # [4096, 16]
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)[:, None]             # [4096, 1]
    want = F.fp4_dequant(packed, scales)
    got = dsk_moe.fp4_dequant(torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV))
    got = got.cpu().numpy()
    both_nan = np.isnan(got) & np.isnan(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # bit patterns, so the sign of zero counts too
    assert np.array_equal(got[~both_nan].view(np.uint32), want[~both_nan].view(np.uint32))


def test_fp4_dequant_bf16_is_exact():
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 256, size=(64, 512), dtype=np.uint8)
    scales = rng.integers(100, 150, size=(64, 32), dtype=np.uint8)
    want = torch.from_numpy(F.fp4_dequant(packed, scales)).to(torch.bfloat16)
    got = dsk_moe.fp4_dequant(torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV),
                              out_dtype=torch.bfloat16).cpu()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got.float(), want.float())


def test_fp4_reference_random_vectors():
    # reference tests/test_metal_fp4.py:44-54 recipe
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 256, size=512, dtype=np.uint8)
    sbytes = (rng.integers(-3, 3, size=32) + 127).astype(np.uint8)
    want = F.fp4_dequant(packed[None, :], sbytes[None, :])
    got = dsk_moe.fp4_dequant(torch.from_numpy(packed[None, :]).to(DEV),
                              torch.from_numpy(sbytes[None, :]).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("scale", [0.02, 1.0, 1e-30, 1e30])
def test_fp4_quantize_bit_exact(scale):
    g = torch.Generator().manual_seed(17)
    w = (torch.randn((96, 1024), generator=g) * scale).float()
    w[0, :32] = torch.linspace(-6, 6, 32)
    w[1, :32] = 0.0
    w[2, :32] = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4)
    p_want, s_want = F.fp4_quantize(w.numpy())
    p_got, s_got = dsk_moe.fp4_quantize(w.to(DEV))
    np.testing.assert_array_equal(s_got.cpu().numpy(), s_want)
    np.testing.assert_array_equal(p_got.cpu().numpy(), p_want)


@pytest.mark.parametrize("cols", [512, 640, 1408])
def test_q3_quantize_and_dequant_bit_exact(cols):
    """Full 512-code superblocks and a tail of plain 128-code blocks."""
    g = torch.Generator().manual_seed(5)
    w = (torch.randn((64, cols), generator=g) * 0.02).float()
    w[3, :64] = 0.0          # zero range group
    p_want, s_want, b_want = F.q3_quantize(w.numpy())
    p_got, s_got, b_got = dsk_moe.q3_quantize(w.to(DEV))
    np.testing.assert_array_equal(s_got.cpu().numpy().view(np.uint16), s_want.view(np.uint16))
    np.testing.assert_array_equal(b_got.cpu().numpy().view(np.uint16), b_want.view(np.uint16))
    np.testing.assert_array_equal(p_got.cpu().numpy(), p_want)
    d_want = F.q3_dequant(p_want, s_want, b_want)
    d_got = dsk_moe.q3_dequant(p_got, s_got, b_got).cpu().numpy()
    np.testing.assert_array_equal(d_got, d_want)
    d16 = dsk_moe.q3_dequant(p_got, s_got, b_got, out_dtype=torch.bfloat16).cpu()
    assert torch.equal(d16.view(torch.int16), torch.from_numpy(d_want).to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(5, 128), (64, 512), (33, 2304), (4, 5120), (7, 1408)])
def test_q3_repack_checkpoint_layout_bit_exact(rows, cols):
    """dsk_q3_repack: checkpoint row-major 3-byte packs -> canonical layout, against
    the oracle's q3_pack of the same codes (superblocks and tails), from u8 bytes and
    from the [rows, 3K/32] u32 word view the checkpoint stores."""
    print(f"q3 repack {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows * cols)
    q = rng.integers(0, 8, size=(rows, cols), dtype=np.uint8)
    src = F.q3_pack_rowmajor(q)
    want = F.q3_pack(q)
    got = dsk_moe.q3_repack(torch.from_numpy(src).to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, want)
    words = torch.from_numpy(src.view("<i4").copy()).to(DEV)
    np.testing.assert_array_equal(dsk_moe.q3_repack(words).cpu().numpy(), want)
