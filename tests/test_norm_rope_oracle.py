"""CPU checks that pin the norm + rotary oracle (``oracle/norm_rope_oracle.py``).
No GPU is needed."""

import numpy as np
import pytest
import torch

from oracle import norm_rope_oracle as NR

DTYPES = [torch.float16, torch.bfloat16]


def _ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two 16-bit tensors of one
    type (same-sign values; the checks below only compare such)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_agrees_with_the_reference_formula(dtype):
    """The fixed-order sum and 1/sqrt differ from torch's mean and rsqrt at
    most in the last place, and only on a small fraction of elements."""
    gen = torch.Generator().manual_seed(1)
    x = (torch.randn(4096, 8, 128, generator=gen) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(128, generator=gen)).to(dtype)
    ones = torch.ones(128, dtype=dtype)
    for weight, max_ulps in ((ones, 1), (w, 2)):
        # a one-ulp difference in the normalized value can become two after
        # the weight's rounding
        got = NR.rms_norm(x, weight, 1e-6)
        ref = NR.rms_norm_reference_formula(x, weight, 1e-6)
        same_sign = (got.float() * ref.float()) > 0
        d = _ulps(got, ref)[same_sign]
        assert d.max().item() <= max_ulps
        assert (d > 0).float().mean().item() < 5e-3
        assert torch.equal(got.float().sign(), ref.float().sign())


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_of_equal_magnitude_rows_is_exactly_signed_weight(dtype):
    """|x_i| = 2^k for every i gives var = 4^k, r = 2^-k and n = +-1 exactly."""
    gen = torch.Generator().manual_seed(2)
    signs = torch.randint(0, 2, (64, 128), generator=gen) * 2 - 1
    mag = 2.0 ** torch.randint(-6, 6, (64, 1), generator=gen)
    x = (signs * mag).to(dtype)
    w = torch.randn(128, generator=gen).to(dtype)
    got = NR.rms_norm(x, w, 0.0)
    assert torch.equal(got, (signs.to(dtype) * w))


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_at_position_zero_is_identity(dtype):
    cos, sin = NR.rope_tables(16, 1e6, dtype)
    assert torch.equal(cos[0], torch.ones(128, dtype=dtype))
    assert torch.equal(sin[0], torch.zeros(128, dtype=dtype))
    x = torch.randn(5, 4, 128).to(dtype)
    out = NR.rope(x, cos, sin, torch.zeros(5, dtype=torch.int64))
    assert torch.equal(out, x)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_rotates_pairs_d_and_d_plus_64(dtype):
    """Against float64 trigonometry: (a, b) at (d, d+64) becomes
    (a cos - b sin, b cos + a sin) with the angle p * base^(-2d/128)."""
    gen = torch.Generator().manual_seed(3)
    base, maxp = 1e6, 40960
    cos, sin = NR.rope_tables(maxp, base, dtype)
    pos = torch.randint(0, maxp, (256,), generator=gen)
    x = torch.randn(256, 2, 128, generator=gen).to(dtype)
    out = NR.rope(x, cos, sin, pos).double()
    inv = 1.0 / (base ** (np.arange(0, 128, 2) / 128.0))
    ang = torch.from_numpy(pos.numpy()[:, None] * inv[None, :])[:, None, :]
    a, b = x.double()[..., :64], x.double()[..., 64:]
    exp = torch.cat((a * ang.cos() - b * ang.sin(), b * ang.cos() + a * ang.sin()), -1)
    # fp32 angles of large positions are off by up to ~4e-3 rad (the
    # reference computes t * inv_freq in fp32), plus three 16-bit roundings
    tol = 4e-2 if dtype == torch.bfloat16 else 1.5e-2
    assert (out - exp).abs().max().item() < tol * max(1.0, exp.abs().max().item())


def test_lane_order_covers_every_element_once():
    o = NR._lane_order()
    assert sorted(o.tolist()) == list(range(128))
    assert o[:16].tolist() == list(range(8)) + list(range(64, 72))


def test_fixed_order_sum_is_close_to_the_exact_sum():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(512, 128, generator=gen).to(torch.float16)
    w = torch.ones(128, dtype=torch.float16)
    got = NR.rms_norm(x, w, 1e-6).double()
    xd = x.double()
    exact = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6)
    assert (got - exact).abs().max().item() < 2 * 2.0 ** -10 * exact.abs().max().item()
