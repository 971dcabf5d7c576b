"""CPU pinning of the oracle's RMSNorm (fixed summation order) and stack composition."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import stack as S


@pytest.mark.parametrize("hidden", [4, 64, 1028, 4096])
def test_rmsnorm_vectorised_equals_scalar_order(hidden):
    rng = np.random.default_rng(hidden)
    x = rng.standard_normal((3, hidden)).astype(np.float32)
    _, y = S.rmsnorm(x, 1e-6, dtype="f32")
    for r in range(3):
        np.testing.assert_array_equal(y[r], S.rmsnorm_scalar(x[r], 1e-6))


def test_rmsnorm_close_to_torch_rms_norm():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 4096)).astype(np.float32) * 3
    g = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    _, y = S.rmsnorm(x, 1e-6, gamma=g, dtype="f32")
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (4096,), torch.from_numpy(g).double(), 1e-6)
    np.testing.assert_allclose(y, ref.numpy(), rtol=2e-6, atol=1e-7)


def test_rmsnorm_power_of_two_scaling_and_constant_rows():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    _, y = S.rmsnorm(x, 0.0, dtype="f32")
    for k in (-3, 5):
        _, yk = S.rmsnorm((x * np.float32(2.0 ** k)).astype(np.float32), 0.0, dtype="f32")
        np.testing.assert_array_equal(yk, y)
    c = np.full((1, 256), 2.0, dtype=np.float32)
    _, yc = S.rmsnorm(c, 0.0, dtype="f32")
    np.testing.assert_array_equal(yc, np.ones_like(c))


def test_bf16_rounding_and_residual():
    rng = np.random.default_rng(3)
    a = torch.randn(2, 64, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    b = torch.randn(2, 64, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    h, y = S.rmsnorm(a.float().numpy(), 1e-6, residual=b.float().numpy(), dtype="bf16")
    np.testing.assert_array_equal(h, (a.float() + b.float()).to(torch.bfloat16).float().numpy())
    _, y32 = S.rmsnorm(h, 1e-6, dtype="f32")
    np.testing.assert_array_equal(y, torch.from_numpy(y32).to(torch.bfloat16).float().numpy())
    v = rng.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(S.round_to(v, "bf16"), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


def test_stack_composition():
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal((2, 64)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    fns = [lambda y: S.round_to(y * np.float32(0.5), "bf16"), lambda y: S.round_to(-y, "bf16")]
    h = S.stack_forward(x, fns, 1e-6)
    want = x
    for fn in fns:
        _, y = S.rmsnorm(want, 1e-6)
        want = S.round_to(want + fn(y), "bf16")
    np.testing.assert_array_equal(h, want)
