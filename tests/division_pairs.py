"""Rows that exercise the store's per-element division ``x / scale`` where a
wrong last bit would change the e4m3 byte.

A row's bytes depend on each element ``x`` and the row scale
``s = max(amax, 1e-8) / 448`` only (``fp8_kv_cache.py:24-27``), and ``s``
depends only on the row's largest magnitude ``A``.  So the (x, A) pairs with
``|x| <= A`` are the whole input space of the division, and a row ``[A,
x_0 .. x_126]`` tests 127 of them at once.

* ``bf16_all_pairs`` lists every such pair of positive finite bfloat16
  values whose quotient is at least 2^-11 (smaller quotients encode to zero
  whatever their last bits) -- about 84 million pairs, every scale from
  1e-8 / 448 = 2.2e-11 to 3.4e38 / 448 = 7.6e35.  Rows with ``A < 1e-8``
  share the floor scale, so only the largest such ``A`` is kept.
* ``fp16_midpoint_pairs`` takes every positive finite float16 ``A`` and, for
  every e4m3 rounding midpoint ``m`` (the point halfway between two adjacent
  e4m3 values), the float16 values nearest to ``m * s`` (round to nearest
  and one ulp either side): the pairs whose quotient lands closest to a
  point where the byte changes -- about 12 million pairs.

``torch_formula`` is the reference's quantizer written with torch CPU ops
(``tests/test_fp8.py:25-26``); ``near_midpoint`` marks the elements whose
fp32 quotient lies within two ulps of an e4m3 rounding boundary.
"""

from __future__ import annotations

import numpy as np
import torch

E4M3_POS = None


def _e4m3_positive_values() -> np.ndarray:
    global E4M3_POS
    if E4M3_POS is None:
        b = torch.arange(0, 0x7F, dtype=torch.int32).to(torch.uint8)
        E4M3_POS = b.view(torch.float8_e4m3fn).double().numpy()
    return E4M3_POS


def _scale_f32(a: np.ndarray) -> np.ndarray:
    """fp32 ``max(a, 1e-8) / 448`` exactly as the reference computes it."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return (t.clamp_min(1e-8) / 448).numpy()


def _pack(a_bits: np.ndarray, counts: np.ndarray, x_bits: np.ndarray) -> np.ndarray:
    """Rows ``[A, x...]`` of 128 int16 bit patterns: group i holds ``counts[i]``
    consecutive entries of ``x_bits`` with amax bits ``a_bits[i]``, padded
    with +0."""
    per = 127
    nrows = (counts + per - 1) // per
    total = int(nrows.sum())
    grp = np.repeat(np.arange(len(counts)), nrows)
    first_row = np.concatenate([[0], np.cumsum(nrows)[:-1]])
    r_in = np.arange(total) - first_row[grp]
    x_start = np.concatenate([[0], np.cumsum(counts)[:-1]])
    j = np.arange(per)[None, :]
    idx = r_in[:, None] * per + j                      # index within the group
    ok = idx < counts[grp][:, None]
    flat = np.where(ok, x_start[grp][:, None] + idx, 0)
    xs = np.where(ok, x_bits[flat], 0)
    rows = np.empty((total, 128), np.int16)
    rows[:, 0] = a_bits[grp]
    rows[:, 1:] = xs
    return rows


def bf16_all_pairs() -> torch.Tensor:
    """Every (x, A) pair of positive finite bf16 with x <= A and x / s >=
    2^-11, as bf16 rows ``[num_rows, 128]``."""
    bits = np.arange(1, 0x7F80, dtype=np.int64)
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    s = _scale_f32(vals)
    floor = vals < np.float32(1e-8)
    keep = ~floor
    keep[np.nonzero(floor)[0][-1]] = True               # one row group at the floor scale
    a_bits = bits[keep]
    lo_val = s[keep].astype(np.float64) * 2.0 ** -11
    lo = np.searchsorted(vals.astype(np.float64), lo_val)  # first x >= lo_val
    counts = (np.nonzero(keep)[0] - lo + 1).astype(np.int64)
    x_bits = np.concatenate([bits[l:a + 1] for l, a in zip(lo, np.nonzero(keep)[0])])
    rows = _pack(a_bits, counts, x_bits)
    return torch.from_numpy(rows).view(torch.bfloat16)


def fp16_midpoint_pairs() -> torch.Tensor:
    """For every positive finite fp16 amax A and every e4m3 midpoint m, the
    fp16 values nearest to m * s (and one ulp either side) that are <= A,
    as fp16 rows ``[num_rows, 128]``."""
    a_bits = np.arange(1, 0x7C00, dtype=np.int64)
    a_vals = a_bits.astype(np.uint16).view(np.float16).astype(np.float32)
    s = _scale_f32(a_vals).astype(np.float64)
    v = _e4m3_positive_values()
    mids = (v[:-1] + v[1:]) / 2                          # 126 midpoints, exact in f64
    target = s[:, None] * mids[None, :]                  # [A, midpoint]
    near = torch.from_numpy(target).to(torch.float16).view(torch.int16).numpy().astype(np.int64)
    cand = near[:, :, None] + np.array([-1, 0, 1])[None, None, :]
    cand = cand.reshape(len(a_bits), -1)
    ok = (cand >= 1) & (cand <= a_bits[:, None])
    counts = ok.sum(1).astype(np.int64)
    x_bits = cand[ok]
    rows = _pack(a_bits, counts, x_bits)
    return torch.from_numpy(rows).view(torch.float16)


def negate(rows: torch.Tensor) -> torch.Tensor:
    """The same rows with every element's sign flipped (-A is the amax)."""
    return (rows.view(torch.int16) ^ torch.tensor(-32768, dtype=torch.int16)).view(rows.dtype)


def torch_formula(rows: torch.Tensor):
    """``tests/test_fp8.py:25-26``: scale = max(amax, 1e-8) / 448 and
    e4m3fn(clamp(x / scale, -448, 448)) with torch CPU ops.  Returns
    (uint8 bytes, float32 scales)."""
    x = rows.float()
    s = x.abs().amax(-1).clamp_min(1e-8) / 448
    q = (x / s[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), s


def near_midpoint(rows: torch.Tensor) -> torch.Tensor:
    """Bool mask of elements whose fp32 quotient x / s lies within two ulps
    of an e4m3 rounding boundary (moving it two ulps either way changes the
    byte)."""
    x = rows.float()
    s = x.abs().amax(-1).clamp_min(1e-8) / 448
    q = (x / s[..., None]).clamp(-448, 448)
    up = torch.nextafter(torch.nextafter(q, torch.tensor(np.inf)), torch.tensor(np.inf))
    dn = torch.nextafter(torch.nextafter(q, torch.tensor(-np.inf)), torch.tensor(-np.inf))
    enc = lambda t: t.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    mask = enc(up) != enc(dn)
    mask[:, 0] = False                                   # the amax element itself
    return mask
