"""CPU checks that pin the oracle before it is trusted as the checker.

Each check is chosen so that a plausible slip in the oracle (a wrong rounding
direction, a dropped sign, a transposed head map, an off-by-one causal bound)
fails it.  Nothing here needs a GPU.
"""

import hashlib
import json
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import cases  # noqa: E402


def _division_rows():
    with open(os.path.join(GOLDEN, "division_rows.json")) as f:
        return json.load(f)


def _row_values(row) -> np.ndarray:
    dt = torch.bfloat16 if row["dtype"] == "bfloat16" else torch.float16
    return torch.tensor(row["bits"], dtype=torch.int16).view(dt).float().numpy()


# ---------------------------------------------------------------- e4m3fn ----

def _torch_cast(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def _in_range(x):
    return np.isfinite(x) & (np.abs(x) <= 448.0)


def test_e4m3_known_answers():
    # Hand-derived from the OCP definition (bias 7, 3 mantissa bits).
    cases = [
        (0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (1.0625, 0x38),  # tie -> even (1.0)
        (1.1875, 0x3A),                                          # tie -> even (1.25)
        (17.0, 0x58),                                            # tie 16|18 -> 16
        (448.0, 0x7E), (-448.0, 0xFE), (2.0 ** -6, 0x08),        # min normal
        (2.0 ** -9, 0x01), (0.001, 0x01), (2.0 ** -10, 0x00),    # tie 0|2^-9 -> 0
        (-(2.0 ** -10), 0x80), (3 * 2.0 ** -10, 0x02),           # tie 1|2 -> 2
        (240.0, 0x77), (256.0, 0x78), (0.5, 0x30),
    ]
    xs = np.array([c[0] for c in cases], dtype=np.float32)
    got = O.e4m3fn_encode(xs)
    want = np.array([c[1] for c in cases], dtype=np.uint8)
    assert (got == want).all(), list(zip(xs, got, want))


def test_e4m3_matches_torch_all_bf16_and_fp16_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    bf = (bits << 16).view(np.float32)
    fp = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    for x in (bf, fp):
        x = x[_in_range(x)]
        assert (O.e4m3fn_encode(x) == _torch_cast(x)).all()


def test_e4m3_matches_torch_structured_fp32():
    # every sign x exponent x leading-7-mantissa-bit combination, with low
    # bits at the tie point, just either side of it, and a few others
    s = np.arange(2, dtype=np.uint32)[:, None, None, None]
    e = np.arange(256, dtype=np.uint32)[None, :, None, None]
    m = np.arange(128, dtype=np.uint32)[None, None, :, None]
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234, 0xC3A1,
                     0x4000, 0xBFFF], dtype=np.uint32)[None, None, None, :]
    u = (s << 31) | (e << 23) | (m << 16) | lows
    x = u.reshape(-1).view(np.float32)
    x = x[_in_range(x)]
    assert x.size > 300_000
    assert (O.e4m3fn_encode(x) == _torch_cast(x)).all()


def test_e4m3_random_fp32_and_roundtrip():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(2_000_000) * np.exp(rng.uniform(-12, 6, 2_000_000))).astype(np.float32)
    x = np.clip(x, -448, 448).astype(np.float32)
    b = O.e4m3fn_encode(x)
    assert (b == _torch_cast(x)).all()
    # decode is exact and encode(decode(b)) == b for every non-NaN byte
    allb = np.arange(256, dtype=np.uint8)
    vals = O.e4m3fn_decode(allb)
    fin = ~np.isnan(vals)
    assert (O.e4m3fn_encode(vals[fin]) == allb[fin]).all()
    tv = torch.from_numpy(allb.copy()).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals[fin], tv[fin])


# -------------------------------------------------------------- quantize ----

def test_quantize_rows_matches_torch_formula():
    torch.manual_seed(0)
    for dt in (torch.bfloat16, torch.float16):
        x = torch.randn(257, 8, 128).to(dt)
        x[0, 0] = 0
        x[1, 1, 5] = -0.0
        x[3] *= 20
        ref_s = x.float().abs().amax(-1).clamp_min(1e-8) / 448
        ref_q = (x.float() / ref_s[..., None]).clamp(-448, 448).to(
            torch.float8_e4m3fn).view(torch.uint8)
        q, s = O.quantize_rows(x.float().numpy())
        assert np.array_equal(s, ref_s.numpy())
        assert np.array_equal(q, ref_q.numpy())


def test_quantize_rows_closed_forms():
    # a row containing 448 has scale exactly 1, so bytes == plain cast
    rng = np.random.default_rng(1)
    row = rng.uniform(-448, 448, 128).astype(np.float32)
    row[7] = 448.0
    q, s = O.quantize_rows(row[None])
    assert s[0] == np.float32(1.0)
    assert np.array_equal(q[0], O.e4m3fn_encode(row))
    # all-zero rows: scale 1e-8/448; bytes 0x00, and 0x80 for -0.0
    z = np.zeros((2, 128), dtype=np.float32)
    z[1, ::2] = -0.0
    q, s = O.quantize_rows(z)
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(448))
    assert (q[0] == 0).all() and (q[1, ::2] == 0x80).all() and (q[1, 1::2] == 0).all()
    # the amax element always maps to +-448 exactly
    x = rng.standard_normal((64, 128)).astype(np.float32)
    q, s = O.quantize_rows(x)
    idx = np.abs(x).argmax(-1)
    top = q[np.arange(64), idx] & 0x7F
    assert (top == 0x7E).all()


def test_store_placement_brute_force():
    rng = np.random.default_rng(2)
    nb, bs, h, d = 5, 16, 2, 8
    n = 40
    k = rng.standard_normal((n, h, d)).astype(np.float32)
    v = rng.standard_normal((n, h, d)).astype(np.float32)
    slots = rng.permutation(nb * bs)[:n]
    slots[3] = -1                                   # skipped
    kc = np.zeros((nb, bs, h, d), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((nb, bs, h), np.float32)
    vs = np.ones_like(ks)
    O.store_fp8_kvcache(k, v, kc, vc, ks, vs, slots)
    kq, kscale = O.quantize_rows(k)
    vq, vscale = O.quantize_rows(v)
    for t in range(n):
        if slots[t] < 0:
            continue
        blk, off = slots[t] // bs, slots[t] % bs
        for hh in range(h):
            assert ks[blk, off, hh] == kscale[t, hh] and vs[blk, off, hh] == vscale[t, hh]
            for dd in range(d):
                assert kc[blk, off, hh, dd] == kq[t, hh, dd]
                assert vc[blk, off, hh, dd] == vq[t, hh, dd]
    written = np.zeros(nb * bs, bool)
    written[slots[slots >= 0]] = True
    assert (kc.reshape(nb * bs, -1)[~written] == 0).all()
    assert (ks.reshape(nb * bs, -1)[~written] == 1).all()


def test_store_torch_matches_store_oracle():
    """The vectorized torch store (the bench's multi-core CPU baseline) writes
    the same bytes and scales as the loop oracle: random rows over a wide
    range of magnitudes, edge rows (zeros, -0, amax 448, tiny and huge),
    skipped slots, and the reference-style int64 slot tensor."""
    rng = np.random.default_rng(5)
    nb, bs, h, d = 6, 32, 4, 128
    n = 150
    k = (rng.standard_normal((n, h, d)) * np.exp(rng.standard_normal((n, h, 1)) * 3)).astype(np.float32)
    v = rng.standard_normal((n, h, d)).astype(np.float32)
    k[0, 0] = 0.0
    k[0, 1] = -0.0
    k[1, 0] = np.linspace(-448, 448, d, dtype=np.float32)
    k[1, 1] = rng.standard_normal(d).astype(np.float32) * 1e-39
    v[2, 2] = rng.standard_normal(d).astype(np.float32) * 1e30
    slots = rng.permutation(nb * bs)[:n]
    slots[5] = -1
    slots[6] = nb * bs
    want = [np.zeros((nb, bs, h, d), np.uint8), np.zeros((nb, bs, h, d), np.uint8),
            np.ones((nb, bs, h), np.float32), np.ones((nb, bs, h), np.float32)]
    O.store_fp8_kvcache(k, v, *want, slots)
    got = [torch.zeros(nb, bs, h, d, dtype=torch.uint8), torch.zeros(nb, bs, h, d, dtype=torch.uint8),
           torch.ones(nb, bs, h), torch.ones(nb, bs, h)]
    O.store_fp8_kvcache_torch(torch.from_numpy(k), torch.from_numpy(v), *got,
                              torch.from_numpy(slots))
    for g, w in zip(got, want):
        g = g.numpy()
        if g.dtype == np.float32:
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
        else:
            assert np.array_equal(g, w)


# ------------------------------------------------------------- attention ----

def _filled_cache(rng, nb, bs, hk, d, tables, lens, scale_k=1.0, scale_v=1.0):
    kc = np.zeros((nb, bs, hk, d), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((nb, bs, hk), np.float32)
    vs = np.ones_like(ks)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        k = (rng.standard_normal((n, hk, d)) * scale_k).astype(np.float32)
        v = (rng.standard_normal((n, hk, d)) * scale_v).astype(np.float32)
        pos = np.arange(n)
        slots = tables[b][pos // bs] * bs + pos % bs
        O.store_fp8_kvcache(k, v, kc, vc, ks, vs, slots)
    return kc, vc, ks, vs


def test_decode_vectorized_vs_loop():
    rng = np.random.default_rng(3)
    bs, hq, hk, d = 16, 4, 2, 32
    lens = [1, 5, 37, 0]
    tables = np.array([[3, 0, 1], [2, 5, 4], [6, 8, 7], [-1, -1, -1]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 9, bs, hk, d, tables, lens)
    q = rng.standard_normal((4, hq, d)).astype(np.float32)
    sc = d ** -0.5
    a = O.decode_attention(q, kc, vc, ks, vs, np.array(lens, np.int32), tables, sc).numpy()
    b = O.decode_attention_loop(torch.from_numpy(q), kc, vc, ks, vs, np.array(lens), tables, sc)
    assert np.abs(a - b).max() < 1e-5
    assert (a[3] == 0).all()


def test_decode_matches_sdpa_and_invariants():
    rng = np.random.default_rng(4)
    bs, hq, hk, d = 32, 8, 2, 64
    lens = [70, 1]
    tables = np.array([[2, 0, 3], [1, -1, -1]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 4, bs, hk, d, tables, lens)
    q = rng.standard_normal((2, hq, d)).astype(np.float32)
    sc = d ** -0.5
    out = O.decode_attention(q, kc, vc, ks, vs, np.array(lens), tables, sc)
    # SDPA on the dequantized rows, GQA expanded by repeat_interleave
    k = O.dequant_gather(kc, ks, tables[0], 70)          # [L, hk, d]
    v = O.dequant_gather(vc, vs, tables[0], 70)
    kk = k.permute(1, 0, 2).repeat_interleave(hq // hk, 0)[None]
    vv = v.permute(1, 0, 2).repeat_interleave(hq // hk, 0)[None]
    qq = torch.from_numpy(q[0])[None, :, None, :]
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, scale=sc)[0, :, 0]
    assert (out[0] - ref).abs().max() < 1e-5
    # one-token context returns that token's dequantized V (per q head's kv head)
    v1 = O.dequant_gather(vc, vs, tables[1], 1)[0]
    assert torch.allclose(out[1], v1[torch.arange(hq) // (hq // hk)], atol=1e-6)
    # relabelling physical blocks leaves the output unchanged
    perm = np.array([3, 2, 1, 0])
    kc2, vc2, ks2, vs2 = (np.empty_like(a) for a in (kc, vc, ks, vs))
    for src, dst in enumerate(perm):
        kc2[dst], vc2[dst], ks2[dst], vs2[dst] = kc[src], vc[src], ks[src], vs[src]
    tables2 = np.where(tables >= 0, perm[np.maximum(tables, 0)], -1).astype(np.int32)
    out2 = O.decode_attention(q, kc2, vc2, ks2, vs2, np.array(lens), tables2, sc)
    assert torch.equal(out, out2)


def test_decode_equal_scores_give_mean_v():
    rng = np.random.default_rng(5)
    bs, hq, hk, d = 16, 2, 1, 16
    lens = [20]
    tables = np.array([[1, 0]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 2, bs, hk, d, tables, lens)
    q = np.zeros((1, hq, d), np.float32)                 # all scores 0
    out = O.decode_attention(q, kc, vc, ks, vs, np.array(lens), tables, 1.0)
    v = O.dequant_gather(vc, vs, tables[0], 20)
    assert torch.allclose(out[0, 0], v[:, 0].mean(0), atol=1e-6)


def test_varlen_prefill_vs_loop_and_sdpa():
    rng = np.random.default_rng(6)
    bs, hq, hk, d = 16, 4, 2, 32
    lk = [21, 9]
    lq = [5, 9]                                          # seq 1 is fresh (prefix 0)
    tables = np.array([[4, 1], [0, 3]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 5, bs, hk, d, tables, lk)
    cu_q = np.array([0, 5, 14], np.int32)
    cu_k = np.array([0, 21, 30], np.int32)
    q = rng.standard_normal((14, hq, d)).astype(np.float32)
    sc = d ** -0.5
    a = O.varlen_prefill_attention(q, kc, vc, ks, vs, tables, cu_q, cu_k, sc).numpy()
    b = O.varlen_prefill_attention_loop(torch.from_numpy(q), kc, vc, ks, vs, tables, cu_q, cu_k, sc)
    assert np.abs(a - b).max() < 1e-5
    # SDPA with is_causal on the fresh sequence (prefix 0 -> square causal)
    k = O.dequant_gather(kc, ks, tables[1], 9).permute(1, 0, 2).repeat_interleave(2, 0)[None]
    v = O.dequant_gather(vc, vs, tables[1], 9).permute(1, 0, 2).repeat_interleave(2, 0)[None]
    qq = torch.from_numpy(q[5:14]).permute(1, 0, 2)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qq, k, v, is_causal=True, scale=sc)
    assert np.abs(a[5:14] - ref[0].permute(1, 0, 2).numpy()).max() < 1e-5
    # the last query row of a chunk sees the whole context == decode
    dec = O.decode_attention(q[4:5], kc, vc, ks, vs, np.array([21]), tables[:1], sc)
    assert np.abs(a[4] - dec[0].numpy()).max() < 1e-5
    # the first query row of the chunk sees prefix + 1 positions
    dec = O.decode_attention(q[0:1], kc, vc, ks, vs, np.array([17]), tables[:1], sc)
    assert np.abs(a[0] - dec[0].numpy()).max() < 1e-5


def test_varlen_prefill_selected_rows():
    """``rows=`` computes only the listed query rows: they equal the same rows
    of the full result and the float64 loop, in every sequence, and a row
    moved by one position (a wrong causal bound for the subset) does not."""
    rng = np.random.default_rng(61)
    bs, hq, hk, d = 16, 4, 2, 32
    lk = [30, 12, 40]
    lq = [9, 12, 0]
    tables = np.array([[4, 1, -1], [0, -1, -1], [2, 3, 5]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 6, bs, hk, d, tables, lk)
    cu_q = np.array([0, 9, 21, 21], np.int32)
    cu_k = np.array([0, 30, 42, 82], np.int32)
    q = rng.standard_normal((21, hq, d)).astype(np.float32)
    sc = d ** -0.5
    full = O.varlen_prefill_attention(q, kc, vc, ks, vs, tables, cu_q, cu_k, sc)
    rows = np.array([0, 3, 8, 9, 15, 20])
    sub = O.varlen_prefill_attention(q, kc, vc, ks, vs, tables, cu_q, cu_k, sc, rows=rows)
    assert sub.shape == (6, hq, d)
    assert torch.allclose(sub, full[rows], atol=1e-6)
    loop = O.varlen_prefill_attention_loop(torch.from_numpy(q), kc, vc, ks, vs, tables, cu_q,
                                           cu_k, sc)
    assert np.abs(sub.numpy() - loop[rows]).max() < 1e-5
    # every row differs from its neighbour's result (the check can fail)
    assert (sub[1:] - full[rows[1:] - 1]).abs().max(-1).values.min() > 1e-4


def test_dense_varlen_vs_loop_sdpa_and_paged_oracle():
    """The fresh-PREFILL oracle: float64 loop, SDPA on the square causal
    case, and the paged oracle on a cache holding the same K/V exactly."""
    rng = np.random.default_rng(16)
    hq, hk, d = 4, 2, 32
    lq = [7, 5, 6]
    lk = [7, 12, 3]                       # fresh, cached prefix, Lq > Lk
    cu_q = np.array([0, 7, 12, 18], np.int32)
    cu_k = np.array([0, 7, 19, 22], np.int32)
    q = rng.standard_normal((18, hq, d)).astype(np.float32)
    k = rng.standard_normal((22, hk, d)).astype(np.float32)
    v = rng.standard_normal((22, hk, d)).astype(np.float32)
    sc = d ** -0.5
    a = O.dense_varlen_attention(q, k, v, cu_q, cu_k, sc).numpy()
    b = O.dense_varlen_attention_loop(q, k, v, cu_q, cu_k, sc)
    assert np.abs(a - b).max() < 1e-5
    # Lq > Lk: query i sees keys j <= i - 3; the first three rows see nothing
    assert np.all(a[12:15] == 0) and np.abs(a[15:18]).max() > 0
    # rows=: a subset in every sequence, empty rows included, against the loop
    rows = np.array([0, 3, 6, 8, 12, 14, 17])
    sub = O.dense_varlen_attention(q, k, v, cu_q, cu_k, sc, rows=rows).numpy()
    assert sub.shape == (rows.size, hq, d)
    assert np.abs(sub - b[rows]).max() < 1e-5
    # square causal == SDPA is_causal (GQA expanded)
    qq = torch.from_numpy(q[0:7]).permute(1, 0, 2)[None]
    kk = torch.from_numpy(k[0:7]).permute(1, 0, 2).repeat_interleave(2, 0)[None]
    vv = torch.from_numpy(v[0:7]).permute(1, 0, 2).repeat_interleave(2, 0)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True, scale=sc)
    assert np.abs(a[0:7] - ref[0].permute(1, 0, 2).numpy()).max() < 1e-5
    # the paged oracle on an exact cache: e4m3-representable rows whose amax is
    # 448 quantize with scale 1, so the cache holds K/V exactly
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    exact = O.e4m3fn_decode(np.concatenate([codes, codes | 0x80]))
    kx = rng.choice(exact, (22, hk, d)).astype(np.float32)
    vx = rng.choice(exact, (22, hk, d)).astype(np.float32)
    kx[:, :, 0] = 448.0
    vx[:, :, 0] = 448.0
    bs = 8
    tables = np.array([[0, -1], [1, 2], [3, -1]], np.int32)
    kc = np.zeros((4, bs, hk, d), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.zeros((4, bs, hk), np.float32)
    vs = np.zeros_like(ks)
    slots = np.concatenate([tables[s_][np.arange(n) // bs] * bs + np.arange(n) % bs
                            for s_, n in enumerate(lk)])
    O.store_fp8_kvcache(kx, vx, kc, vc, ks, vs, slots)
    used = np.zeros((4, bs), bool)
    used.reshape(-1)[slots] = True
    assert np.all(ks[used] == 1) and np.all(vs[used] == 1)
    qx = (q * 0.01).astype(np.float32)
    a = O.dense_varlen_attention(qx, kx, vx, cu_q, cu_k, sc)
    b = O.varlen_prefill_attention(qx, kc, vc, ks, vs, tables, cu_q, cu_k, sc)
    ok = [*range(0, 12), *range(15, 18)]           # rows that see at least one key
    assert torch.allclose(a[ok], b[ok], atol=1e-3, rtol=1e-5)


def test_chunk_prefill_wrapper_equals_varlen():
    rng = np.random.default_rng(7)
    bs, hq, hk, d = 16, 4, 2, 32
    tables = np.array([[1, 0, 2]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 3, bs, hk, d, tables, [40])
    q = rng.standard_normal((7, hq, d)).astype(np.float32)
    a = O.chunk_prefill_attention(q, kc, vc, ks, vs, tables[0], 33, 0.2)
    b = O.varlen_prefill_attention(q, kc, vc, ks, vs, tables,
                                   np.array([0, 7]), np.array([0, 40]), 0.2)
    assert torch.equal(a, b)


def test_oracle_catches_planted_mistakes():
    """A checker that cannot fail pins nothing: plant slips in copies."""
    x = np.array([1.0625, 17.0, -(2.0 ** -10)], np.float32)
    # round-half-away-from-zero would give 0x39, 0x59, 0x81
    away = np.array([0x39, 0x59, 0x81], np.uint8)
    assert not np.array_equal(O.e4m3fn_encode(x), away)
    # a reciprocal-multiply quantizer differs from the division one on the
    # committed division-sensitive rows
    for row in _division_rows():
        x = _row_values(row)
        q, s = O.quantize_rows(x[None])
        recip = (x * (np.float32(1) / s[0])).astype(np.float32)
        assert O.e4m3fn_encode(np.clip(recip[1:2], -448, 448))[0] == row["reciprocal_byte"]
        assert q[0, 1] != row["reciprocal_byte"]
    rng = np.random.default_rng(8)
    # an off-by-one causal bound changes the first chunk row
    bs, hq, hk, d = 16, 2, 1, 16
    tables = np.array([[0, 1]], np.int32)
    kc, vc, ks, vs = _filled_cache(rng, 2, bs, hk, d, tables, [20])
    qq = rng.standard_normal((4, hq, d)).astype(np.float32)
    good = O.varlen_prefill_attention(qq, kc, vc, ks, vs, tables, [0, 4], [0, 20], 0.25)
    right = O.decode_attention(qq[0:1], kc, vc, ks, vs, np.array([17]), tables, 0.25)
    assert torch.allclose(good[0], right[0], atol=1e-5)
    for off_by_one in (16, 18):   # visible = prefix + i, prefix + i + 2
        bad = O.decode_attention(qq[0:1], kc, vc, ks, vs, np.array([off_by_one]), tables, 0.25)
        assert not torch.allclose(good[0], bad[0], atol=1e-4)


# ---------------------------------------------------------------- golden ----

def test_oracle_matches_division_rows():
    rows = _division_rows()
    assert len(rows) == 12
    for row in rows:
        q, s = O.quantize_rows(_row_values(row)[None])
        assert q[0].tolist() == row["bytes"]
        assert int(s.view(np.int32)[0]) == row["scale_bits"]


def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _oracle_fill(c, num_blocks):
    kc = np.zeros((num_blocks, cases.BLOCK, cases.KVH, cases.D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((num_blocks, cases.BLOCK, cases.KVH), np.float32)
    vs = np.ones_like(ks)
    O.store_fp8_kvcache(c["key"].float().numpy(), c["value"].float().numpy(),
                        kc, vc, ks, vs, c["slots"].numpy())
    return kc, vc, ks, vs


def test_oracle_matches_reference_shape_fixtures():
    g = np.load(os.path.join(GOLDEN, "ref_shapes.npz"))
    c = cases.decode_case()
    assert _digest(c["key"].view(torch.uint8).numpy(), c["value"].view(torch.uint8).numpy(),
                   c["query"].view(torch.uint8).numpy()) == str(g["dec_inputs"])
    kc, vc, ks, vs = _oracle_fill(c, c["num_blocks"])
    assert _digest(kc, vc, ks, vs) == str(g["dec_cache"])
    out = O.decode_attention(c["query"], kc, vc, ks, vs, np.array(c["lengths"]),
                             c["tables"], cases.D ** -0.5)
    assert np.abs(out.numpy() - g["dec_out"]).max() < 1e-5
    c = cases.chunk_case()
    assert _digest(c["key"].view(torch.uint8).numpy(), c["value"].view(torch.uint8).numpy(),
                   c["query"].view(torch.uint8).numpy()) == str(g["pre_inputs"])
    kc, vc, ks, vs = _oracle_fill(c, c["num_blocks"])
    assert _digest(kc, vc, ks, vs) == str(g["pre_cache"])
    out = O.chunk_prefill_attention(c["query"], kc, vc, ks, vs, c["table"][0],
                                    c["prefix"], cases.D ** -0.5)
    assert np.abs(out.numpy() - g["pre_out"]).max() < 1e-5
