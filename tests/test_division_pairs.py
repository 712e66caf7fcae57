"""CPU checks of the division-sensitive row sets the store's GPU tests use
(``tests/division_pairs.py``): they cover what they claim, the torch formula
they are checked against agrees with the oracle's quantizer on their hardest
elements, and a kernel that multiplied by the reciprocal instead of
dividing would fail on them."""

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from tests import division_pairs as DP


@pytest.fixture(scope="module")
def bf16_rows():
    return DP.bf16_all_pairs()


@pytest.fixture(scope="module")
def fp16_rows():
    return DP.fp16_midpoint_pairs()


def test_bf16_pairs_are_the_whole_space(bf16_rows):
    x = bf16_rows.float()
    amax = x.abs().amax(-1)
    assert torch.equal(amax, x[:, 0])                    # element 0 is the row amax
    scales = (amax.clamp_min(1e-8) / 448).unique()
    assert scales.min().item() == pytest.approx(1e-8 / 448, rel=1e-6)
    assert scales.max().item() == pytest.approx(3.3895e38 / 448, rel=1e-3)
    # every amax >= 1e-8 is present, plus one row group at the floor scale
    bits = np.arange(1, 0x7F80, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    assert scales.numel() == int((vals >= np.float32(1e-8)).sum()) + 1
    # for one amax, every smaller bf16 whose quotient is >= 2^-11 is present
    a = torch.tensor(1.3984375, dtype=torch.bfloat16)     # 0x3FB3
    sel = bf16_rows[bf16_rows[:, 0] == a][:, 1:].float().reshape(-1)
    sel = sel[sel != 0].unique()
    s = float(torch.tensor(a.float().item()).clamp_min(1e-8) / 448)
    want = torch.from_numpy(vals[(vals <= a.float().item()) & (vals >= s * 2.0 ** -11)])
    assert torch.equal(sel.sort().values, want.sort().values)


def test_fp16_pairs_surround_every_midpoint(fp16_rows):
    x = fp16_rows.float()
    assert torch.equal(x.abs().amax(-1), x[:, 0])
    assert (x[:, 0] > 0).all() and x[:, 0].unique().numel() == 0x7C00 - 1
    assert int((x[:, 1:] != 0).sum()) > 10_000_000


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_formula_matches_oracle_on_the_hardest_elements(kind, bf16_rows, fp16_rows):
    rows = bf16_rows if kind == "bf16" else fp16_rows
    rows = torch.cat([rows, DP.negate(rows)])
    hard = DP.near_midpoint(rows)
    pick = hard.any(1).nonzero().view(-1)
    pick = pick[torch.randperm(pick.numel(), generator=torch.Generator().manual_seed(1))[:40000]]
    sub = rows[pick]
    q, s = DP.torch_formula(sub)
    oq, os_ = O.quantize_rows(sub.float().numpy())
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.numpy().view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_reciprocal_multiply_fails_on_these_rows(kind, bf16_rows, fp16_rows):
    """x * (1 / s) in place of x / s changes bytes on these rows, so the GPU
    tests would catch a kernel that made that substitution."""
    rows = bf16_rows if kind == "bf16" else fp16_rows
    x = rows.float()
    s = x.abs().amax(-1).clamp_min(1e-8) / 448
    recip = (x * (1.0 / s)[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    q, _ = DP.torch_formula(rows)
    assert int((recip != q).sum()) > 1000
