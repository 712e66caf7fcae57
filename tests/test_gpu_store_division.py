"""GPU parity of the store's division ``x / scale`` on the inputs where a
wrong last bit of the quotient changes the stored byte.

The kernels divide through a per-row reciprocal with two FMA corrections
(``RowDivider`` in ``csrc/fp8_row.h``) instead of one IEEE division per
element.  These tests hold every store path to the reference's formula
(``fp8_kv_cache.py:24-27``; ``tests/test_fp8.py:25-26``), evaluated with
torch CPU ops, on:

* every (element, row amax) pair of positive finite bfloat16 values whose
  quotient does not encode to zero -- the whole input space of the bf16
  division, 50 million pairs per sign, every scale from 2.2e-11 to 7.6e35;
* for every float16 amax, the float16 elements closest to each e4m3
  rounding midpoint times the scale -- 11.6 million pairs per sign.

Both signs run.  ``store_fp8_kvcache`` and the fused prologue
``qk_norm_rope_store`` (whose v rows take the same quantizer) must give
the formula's bytes and scales exactly.
"""

import pytest
import torch

from microserve_amd import qk_norm_rope_store, store_fp8_kvcache
from tests import division_pairs as DP
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

_ROWS = {}


def _rows(kind):
    if kind not in _ROWS:
        base = DP.bf16_all_pairs() if kind == "bf16" else DP.fp16_midpoint_pairs()
        _ROWS[kind] = torch.cat([base, DP.negate(base)])
    return _ROWS[kind]


def _as_tokens(rows, hk=8):
    pad = (-rows.shape[0]) % hk
    if pad:
        rows = torch.cat([rows, torch.zeros(pad, rows.shape[1], dtype=rows.dtype)])
    return rows.view(-1, hk, H.D)


def _check(kc, ks, want_q, want_s, nrows, what):
    got = kc.view(torch.uint8).view(-1, H.D)[:nrows].cpu()
    got_s = ks.view(-1)[:nrows].cpu()
    bad = (got != want_q).nonzero()
    assert bad.numel() == 0, f"{what}: {bad.shape[0]} bytes differ, first (row, col) {bad[:3].tolist()}"
    assert torch.equal(got_s.view(torch.int32), want_s.view(torch.int32)), f"{what}: scales differ"


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_store_division_every_sensitive_pair(kind):
    rows = _rows(kind)
    near = int(DP.near_midpoint(rows).sum())
    print(f"{kind}: {rows.shape[0]} rows, {int((rows.float()[:, 1:] != 0).sum())} pairs, "
          f"{near} within two ulps of an e4m3 rounding boundary", flush=True)
    assert near > 1_000_000
    want_q, want_s = DP.torch_formula(rows)
    tok = _as_tokens(rows)
    n = tok.shape[0]
    nb = (n + H.BLOCK - 1) // H.BLOCK
    kc, vc, ks, vs = H.alloc_cache(nb)
    slots = torch.arange(n, dtype=torch.int64, device=H.DEV)
    td = tok.to(H.DEV)
    store_fp8_kvcache(td, td, kc, vc, ks, vs, slots)
    torch.cuda.synchronize()
    _check(kc, ks, want_q, want_s, rows.shape[0], "store k")
    _check(vc, vs, want_q, want_s, rows.shape[0], "store v")


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_fused_prologue_division_every_sensitive_pair(kind):
    """The same rows as the v of the fused prologue, which stores v with the
    store's quantizer (no norm, no rotation on v)."""
    rows = _rows(kind)
    want_q, want_s = DP.torch_formula(rows)
    tok = _as_tokens(rows).to(H.DEV)
    n, hk = tok.shape[0], tok.shape[1]
    nb = (n + H.BLOCK - 1) // H.BLOCK
    kc, vc, ks, vs = H.alloc_cache(nb)
    zeros = torch.zeros(n, hk, H.D, dtype=tok.dtype, device=H.DEV)
    cos = torch.ones(1, H.D, dtype=tok.dtype, device=H.DEV)
    sin = torch.zeros(1, H.D, dtype=tok.dtype, device=H.DEV)
    pos = torch.zeros(n, dtype=torch.int64, device=H.DEV)
    slots = torch.arange(n, dtype=torch.int64, device=H.DEV)
    qk_norm_rope_store(pos, zeros, zeros, tok, None, None, 1e-6, cos, sin, kc, vc, ks, vs,
                       slots, return_k=False)
    torch.cuda.synchronize()
    _check(vc, vs, want_q, want_s, rows.shape[0], "fused prologue v")
