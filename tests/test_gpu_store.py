"""GPU parity of store_fp8_kvcache: cache bytes, scales and slot placement
bit-exact against the oracle (``fp8_kv_cache.py:11-61``)."""

import hashlib
import json
import os
import sys

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import cases  # noqa: E402

from microserve_amd import store_fp8_kvcache  # noqa: E402


def _edge_rows(dtype, gen, n):
    x = H.randn(gen, (n, 8, H.D), dtype)
    x[0, 0] = 0                                  # all-zero row
    x[0, 1] = -0.0                               # all -0.0 row -> bytes 0x80
    x[1, 0, ::7] *= 20                           # outliers
    x[1, 1] = torch.linspace(-448, 448, H.D).to(dtype)   # amax 448 -> scale 1
    x[2, 0] = x[2, 0] * 1e-3
    x[2, 1, 5] = 1e4                             # one dominant element
    if dtype == torch.bfloat16:
        x[3, 0] = (torch.randn(H.D, generator=gen) * 1e-39).to(dtype)  # subnormal inputs
        x[3, 1] = (torch.randn(H.D, generator=gen) * 1e30).to(dtype)
    else:
        x[3, 0] = (torch.randn(H.D, generator=gen) * 1e-6).to(dtype)   # fp16 subnormals
        # large but finite: randn * 3e4 would overflow fp16 to inf, and
        # inf/NaN inputs are unspecified by the reference
        x[3, 1] = (torch.randn(H.D, generator=gen) * 1e4).clamp(-6e4, 6e4).to(dtype)
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_store_matches_oracle_bytes(dtype, slot_dtype):
    gen = torch.Generator().manual_seed(11)
    nb, n = 16, 1500
    key = _edge_rows(dtype, gen, n)
    value = _edge_rows(dtype, gen, n).flip(0).contiguous()
    slots = torch.randperm(nb * H.BLOCK, generator=gen)[:n]
    slots[7] = -1                                # skipped
    slots[8] = nb * H.BLOCK                      # past the pool: skipped
    kc, vc, ks, vs = H.alloc_cache(nb)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), kc, vc, ks, vs,
                      slots.to(slot_dtype).to(H.DEV))
    got = H.cache_to_numpy(kc, vc, ks, vs)
    want = H.oracle_store_numpy(key, value, slots, nb)
    for g, w, name in zip(got, want, ("k_cache", "v_cache", "k_scale", "v_scale")):
        if g.dtype == np.float32:
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), name
        else:
            bad = np.argwhere(g != w)
            assert bad.size == 0, f"{name}: {len(bad)} mismatched bytes, first {bad[:3]}"


def test_store_fp32_rows_match_oracle_bytes():
    """fp32 K/V rows (the reference upcasts any float input,
    ``fp8_kv_cache.py:22-23``): full 24-bit mantissas exercise the division
    far beyond the 8 and 11 bits of bf16 and fp16 rows, plus the edge rows
    (zeros, -0, outliers, amax 448, fp32 subnormals, 1e30)."""
    gen = torch.Generator().manual_seed(17)
    nb, n = 32, 7000
    key = torch.randn(n, 8, H.D, generator=gen) * torch.exp(
        torch.randn(n, 8, 1, generator=gen) * 4)
    key[:4] = _edge_rows(torch.float32, gen, 4)
    value = torch.randn(n, 8, H.D, generator=gen)
    value[-4:] = _edge_rows(torch.float32, gen, 4)
    slots = torch.randperm(nb * H.BLOCK, generator=gen)[:n]
    kc, vc, ks, vs = H.alloc_cache(nb)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), kc, vc, ks, vs, slots.to(H.DEV))
    got = H.cache_to_numpy(kc, vc, ks, vs)
    want = H.oracle_store_numpy(key, value, slots, nb)
    for g, w, name in zip(got, want, ("k_cache", "v_cache", "k_scale", "v_scale")):
        if g.dtype == np.float32:
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), name
        else:
            bad = np.argwhere(g != w)
            assert bad.size == 0, f"{name}: {len(bad)} mismatched bytes, first {bad[:3]}"


def test_store_division_sensitive_rows():
    with open(os.path.join(GOLDEN, "division_rows.json")) as f:
        rows = json.load(f)
    for dtype_name in ("bfloat16", "float16"):
        sel = [r for r in rows if r["dtype"] == dtype_name]
        dt = getattr(torch, dtype_name)
        x = torch.stack([torch.tensor(r["bits"], dtype=torch.int16).view(dt) for r in sel])
        key = x[:, None, :].repeat(1, 8, 1).contiguous()
        slots = torch.arange(len(sel), dtype=torch.int64)
        kc, vc, ks, vs = H.alloc_cache(1)
        store_fp8_kvcache(key.to(H.DEV), key.to(H.DEV), kc, vc, ks, vs, slots.to(H.DEV))
        got = kc.view(torch.uint8).cpu()
        for i, r in enumerate(sel):
            assert got[0, i, 0].tolist() == r["bytes"]
            assert got[0, i, 0, 1].item() != r["reciprocal_byte"]
            assert ks[0, i, 0].cpu().view(torch.int32).item() == r["scale_bits"]


def test_store_exhaustive_16bit_patterns_at_unit_scale():
    """Rows whose amax is exactly 448 have scale 1, so every byte equals the
    plain e4m3fn cast: this sweeps every bf16 and fp16 value in [-448, 448]."""
    for dt in (torch.bfloat16, torch.float16):
        bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
        vals = bits.view(dt).float()
        keep = torch.isfinite(vals) & (vals.abs() <= 448)
        vals = vals[keep]
        per_row = H.D - 1
        nrows = (vals.numel() + per_row - 1) // per_row
        pad = torch.zeros(nrows * per_row)
        pad[:vals.numel()] = vals
        rows = torch.cat([torch.full((nrows, 1), 448.0), pad.view(nrows, per_row)], 1).to(dt)
        ntok = (nrows + 7) // 8
        x = torch.zeros(ntok * 8, H.D, dtype=dt)
        x[:nrows] = rows
        x[nrows:, 0] = 448
        key = x.view(ntok, 8, H.D)
        nb = (ntok + H.BLOCK - 1) // H.BLOCK
        kc, vc, ks, vs = H.alloc_cache(nb)
        slots = torch.arange(ntok, dtype=torch.int64)
        store_fp8_kvcache(key.to(H.DEV), key.to(H.DEV), kc, vc, ks, vs, slots.to(H.DEV))
        got = kc.view(torch.uint8).view(-1, H.D)[: ntok * 8].cpu().numpy()
        assert (ks.view(-1)[: ntok * 8].cpu() == 1.0).all()
        want = O.e4m3fn_encode(x.float().numpy())
        assert np.array_equal(got, want)


def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("which", ["decode", "chunk"])
def test_store_reference_case_cache_digest(which):
    g = np.load(os.path.join(GOLDEN, "ref_shapes.npz"))
    c = cases.decode_case() if which == "decode" else cases.chunk_case()
    kc, vc, ks, vs = H.alloc_cache(c["num_blocks"])
    store_fp8_kvcache(c["key"].to(H.DEV), c["value"].to(H.DEV), kc, vc, ks, vs,
                      c["slots"].to(H.DEV))
    key = "dec_cache" if which == "decode" else "pre_cache"
    assert _digest(*H.cache_to_numpy(kc, vc, ks, vs)) == str(g[key])


def test_store_fill_qwen3_8b_pool_sampled_and_roundtrip():
    """The Qwen3-8B fill (64 x 4096 tokens into a permuted 2048-block pool):
    sampled rows bit-exact against the oracle, every row within the
    quantization bound, and untouched blocks still at their initial state."""
    gen = torch.Generator().manual_seed(21)
    lens = [4096] * 64
    tables, slots = H.paged_layout(gen, lens, 2048)
    n = slots.numel()
    key = H.randn(gen, (n, 8, H.D), torch.bfloat16)
    value = H.randn(gen, (n, 8, H.D), torch.bfloat16)
    kc, vc, ks, vs = H.alloc_cache(2048)
    kd, vd = key.to(H.DEV), value.to(H.DEV)
    sd = slots.to(H.DEV)
    store_fp8_kvcache(kd, vd, kc, vc, ks, vs, sd)
    # sampled bit-exact parity
    pick = torch.randperm(n, generator=gen)[:4096]
    kq, kscale = O.quantize_rows(key[pick].float().numpy())
    rows = slots[pick].to(H.DEV)
    got_k = kc.view(torch.uint8).view(-1, 8, H.D)[rows].cpu().numpy()
    got_s = ks.view(-1, 8)[rows].cpu().numpy()
    assert np.array_equal(got_k, kq)
    assert np.array_equal(got_s.view(np.uint32), kscale.view(np.uint32))
    vq, vscale = O.quantize_rows(value[pick].float().numpy())
    assert np.array_equal(vc.view(torch.uint8).view(-1, 8, H.D)[rows].cpu().numpy(), vq)
    # round trip on every row: |x - deq| <= scale * 2^-4 * |x/scale| + subnormal step
    deq = kc.view(-1, 8, H.D)[sd].float() * ks.view(-1, 8)[sd][..., None]
    x = kd.float()
    bound = x.abs() * 2.0 ** -4 + ks.view(-1, 8)[sd][..., None] * 2.0 ** -9
    assert ((deq - x).abs() <= bound).all()
    # blocks outside the tables keep their initial bytes and unit scales
    used = torch.zeros(2048, dtype=torch.bool)
    used[tables[tables >= 0].long()] = True
    assert used.sum() == 1024
    free = (~used).nonzero().view(-1).to(H.DEV)
    assert (kc.view(torch.uint8)[free] == 0).all() and (ks[free] == 1).all()
