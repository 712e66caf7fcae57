"""GPU parity of the FP8-MFMA chunk / varlen prefill against the oracle
(``fp8_chunk_prefill_attention.py:16-67``): outputs within 2e-2 max-abs and
1e-2 relative (Frobenius) error.  The kernel splits q into e4m3 parts for
the QK^T MFMAs and rounds the weights p * v_scale to fp16 for the PV MFMAs;
the oracle does neither, so these bounds measure those choices."""

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

from microserve_amd import (  # noqa: E402
    fp8_chunk_prefill_attention, fp8_varlen_prefill_attention, store_fp8_kvcache)


def test_chunk_prefill_reference_case():
    """tests/test_fp8_kv_attention.py::test_chunk_prefill's shape: prefix 273,
    31 queries, permuted table [[1, 0]], unscaled V."""
    g = np.load(os.path.join(GOLDEN, "ref_shapes.npz"))
    c = cases.chunk_case()
    caches = H.alloc_cache(c["num_blocks"])
    store_fp8_kvcache(c["key"].to(H.DEV), c["value"].to(H.DEV), *caches, c["slots"].to(H.DEV))
    out = fp8_chunk_prefill_attention(c["query"].to(H.DEV), *caches, c["table"].to(H.DEV),
                                      c["prefix"], cases.D ** -0.5)
    ref = torch.from_numpy(g["pre_out"])
    max_abs, rel = H.assert_attention_close(out, ref)
    print(f"chunk prefill reference case: max_abs {max_abs:.4e} rel {rel:.4e}")


def _varlen_setup(seed, lq, lk, hq, hk, dtype=torch.bfloat16, outliers=0.0,
                  extra_blocks=3, block_size=H.BLOCK):
    gen = torch.Generator().manual_seed(seed)
    pages = sum((n + block_size - 1) // block_size for n in lk)
    nb = pages + extra_blocks
    tables, slots = H.paged_layout(gen, lk, nb, block_size)
    n = slots.numel()
    key = torch.randn(n, hk, H.D, generator=gen)
    if outliers:
        mask = torch.rand(n, hk, H.D, generator=gen) < outliers
        key = torch.where(mask, key * 20, key)
    key = key.to(dtype)
    value = H.randn(gen, (n, hk, H.D), dtype)
    query = H.randn(gen, (sum(lq), hq, H.D), dtype)
    caches = H.alloc_cache(nb, block_size, hk)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    return query, tables, caches, cu_q, cu_k


def _varlen_check(query, tables, caches, cu_q, cu_k, lq):
    scale = H.D ** -0.5
    out = fp8_varlen_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV),
                                       cu_q.to(H.DEV), cu_k.to(H.DEV), max(lq), scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.varlen_prefill_attention(query, kc, vc, ks, vs, tables, cu_q, cu_k, scale)
    return H.assert_attention_close(out, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_prefill_mixed_batch(dtype):
    """Cached prefixes of several lengths, a fresh sequence (prefix 0) and
    ragged query lengths in one launch."""
    lq = [31, 200, 1, 77, 300]
    lk = [304, 200, 900, 77 + 513, 300 + 1024]
    query, tables, caches, cu_q, cu_k = _varlen_setup(201, lq, lk, 32, 8, dtype)
    _varlen_check(query, tables, caches, cu_q, cu_k, lq)


@pytest.mark.parametrize("hq,hk", [(16, 8), (8, 8), (64, 8), (32, 2), (16, 1), (24, 8), (40, 2),
                                   (20, 1), (48, 2)])
def test_varlen_prefill_gqa_groups(hq, hk):
    lq = [64, 130]
    lk = [64 + 300, 130 + 5]
    query, tables, caches, cu_q, cu_k = _varlen_setup(211 + hq, lq, lk, hq, hk)
    _varlen_check(query, tables, caches, cu_q, cu_k, lq)


@pytest.mark.parametrize("block_size", [512, 1024])
def test_varlen_prefill_larger_block_sizes(block_size):
    """Pages of 512 and 1024 tokens: 128-key tiles never straddle a page,
    and prefixes and chunks end mid-page."""
    lq = [100, 1, 300]
    lk = [100 + 700, 1 + 1023, 300 + 1100]
    query, tables, caches, cu_q, cu_k = _varlen_setup(251, lq, lk, 32, 8,
                                                      block_size=block_size)
    _varlen_check(query, tables, caches, cu_q, cu_k, lq)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_prefill_qwen3_8b_chunk_with_outliers(dtype):
    """A scaled Qwen3-8B chunked prefill: 2 sequences x (2048 cached + 512
    new), 1% of K entries x20."""
    lq = [512, 512]
    lk = [2048 + 512, 2048 + 512]
    query, tables, caches, cu_q, cu_k = _varlen_setup(221, lq, lk, 32, 8, dtype, outliers=0.01)
    max_abs, rel = _varlen_check(query, tables, caches, cu_q, cu_k, lq)
    print(f"outlier chunk prefill {dtype}: max_abs {max_abs:.4e} rel {rel:.4e}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("v_mult", [0.0, 1e-6])
def test_varlen_prefill_dominant_keys_with_vanishing_values(v_mult, dtype):
    """5% of the keys take ~95% of the attention, and their V rows are zero
    (stored with the 1e-8 / 448 floor scale) or 1e-6 of the others.  Their
    probability still counts in the softmax denominator, as in the
    reference, so the output stays near zero instead of becoming the
    average of the remaining keys."""
    gen = torch.Generator().manual_seed(241)
    hq, hk = 32, 8
    lq = [48, 96]
    lk = [700 + 48, 300 + 96]
    nb = sum((n + 255) // 256 for n in lk) + 2
    tables, slots = H.paged_layout(gen, lk, nb)
    n = slots.numel()
    key = torch.randn(n, hk, H.D, generator=gen)
    value = torch.randn(n, hk, H.D, generator=gen)
    u = torch.randn(hk, H.D, generator=gen)
    u = u / u.norm(dim=-1, keepdim=True)
    special = torch.rand(n, generator=gen) < 0.05
    key[special] = 19.0 * u  # logit ~5 above the others (softmax scale 1/sqrt(128))
    value[special] = value[special] * v_mult
    query = torch.randn(sum(lq), hq, H.D, generator=gen)
    query = query + 3.0 * u.repeat_interleave(hq // hk, dim=0)[None]
    key, value, query = key.to(dtype), value.to(dtype), query.to(dtype)
    caches = H.alloc_cache(nb, H.BLOCK, hk)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    max_abs, rel = _varlen_check(query, tables, caches, cu_q, cu_k, lq)
    print(f"vanishing-V dominant keys (x{v_mult}, {dtype}): max_abs {max_abs:.4e} rel {rel:.4e}")


def _v_ratio_case(r, dtype, seed=261, hq=32, hk=8):
    """One key in every 128-key tile (position 37) has V scaled by r and a
    score ~20 below the rest, so it carries almost no probability but sets
    the tile's largest v_scale; 5% of the keys (equal, dominant scores)
    carry ~all of it with ordinary V.  Outputs stay below 1 in magnitude,
    so the bf16 output rounding stays far under the gate and what is left
    is the precision of the dominant keys' weights next to a v_scale r
    times their own."""
    gen = torch.Generator().manual_seed(seed)
    lq = [128, 64]
    lk = [128 + 896, 64 + 448]
    nb = sum((n + 255) // 256 for n in lk) + 2
    tables, slots = H.paged_layout(gen, lk, nb)
    n = slots.numel()
    key = torch.randn(n, hk, H.D, generator=gen)
    value = torch.randn(n, hk, H.D, generator=gen)
    u = torch.randn(hk, H.D, generator=gen)
    u = u / u.norm(dim=-1, keepdim=True)
    pos = torch.cat([torch.arange(x) for x in lk])
    big = (pos % 128) == 37
    dom = (torch.rand(n, generator=gen) < 0.05) & ~big
    key[dom] = 19.0 * u
    key[big] = -19.0 * u
    value[big] *= r
    query = torch.randn(sum(lq), hq, H.D, generator=gen)
    query = query + 6.0 * u.repeat_interleave(hq // hk, dim=0)[None]
    key, value, query = key.to(dtype), value.to(dtype), query.to(dtype)
    caches = H.alloc_cache(nb, H.BLOCK, hk)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    return query, tables, caches, cu_q, cu_k, lq


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("r", [1, 100, 1000, 5000, 10000])
def test_varlen_prefill_v_scale_ratio_inside_a_tile(r, dtype):
    """The reference dequantizes V per element
    (fp8_chunk_prefill_attention.py:49-50,60), so a key with a huge V in the
    same tile costs the other keys nothing.  The PV product here weights
    each key by fp16(p) * fp16(v_scale * fw), fw set from the largest v_scale
    the wave has seen: a key whose v_scale lies within 2^21 of that largest
    one keeps a normal fp16 scale (11 significant bits), so at every ratio
    tested here the error must stay at its ratio-1 level (measured rel
    1.66e-3 bf16, 2.8e-4 fp16 at every ratio up to 10000; fp16 inputs
    overflow beyond that), far inside the usual gate.  Ratios past 2^21 give
    the smaller keys subnormal scales with fewer bits (not tested)."""
    query, tables, caches, cu_q, cu_k, lq = _v_ratio_case(r, dtype)
    max_abs, rel = _varlen_check(query, tables, caches, cu_q, cu_k, lq)
    print(f"V-scale ratio {r} {dtype}: max_abs {max_abs:.4e} rel {rel:.4e}")
    assert rel < (2.5e-3 if dtype == torch.bfloat16 else 5e-4), rel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_prefill_v_scale_growing_along_the_keys(dtype):
    """V magnitudes grow by 2^12 along each sequence's keys and 2% of the V
    rows are zeros.  Every 128-key tile brings a larger v_scale, so each
    wave's power-of-two weight scale shrinks tile after tile and its
    accumulator is rescaled; the zero rows' weights underflow while their
    probabilities still count.  Outputs stay O(1)."""
    gen = torch.Generator().manual_seed(271)
    hq, hk = 32, 8
    lq = [96, 200, 1]
    lk = [96 + 1500, 200, 1 + 700]
    nb = sum((n + H.BLOCK - 1) // H.BLOCK for n in lk) + 2
    tables, slots = H.paged_layout(gen, lk, nb)
    n = slots.numel()
    pos = torch.cat([torch.arange(x) for x in lk]).float()
    grow = torch.exp2(12.0 * pos / max(lk) - 12.0)
    key = torch.randn(n, hk, H.D, generator=gen)
    value = torch.randn(n, hk, H.D, generator=gen) * grow[:, None, None]
    value[torch.rand(n, generator=gen) < 0.02] = 0.0
    query = torch.randn(sum(lq), hq, H.D, generator=gen)
    key, value, query = key.to(dtype), value.to(dtype), query.to(dtype)
    caches = H.alloc_cache(nb, H.BLOCK, hk)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    max_abs, rel = _varlen_check(query, tables, caches, cu_q, cu_k, lq)
    print(f"growing V {dtype}: max_abs {max_abs:.4e} rel {rel:.4e}")


def test_varlen_prefill_empty_sequences_and_oversized_max_seqlen():
    """Sequences with no new tokens (one with a cached prefix, one empty) in
    the batch, and max_seqlen_q far above the longest query: the extra
    query blocks find nothing to do and every row matches the oracle."""
    lq = [0, 50, 0, 130]
    lk = [500, 50 + 300, 0, 130 + 77]
    query, tables, caches, cu_q, cu_k = _varlen_setup(271, lq, lk, 32, 8)
    scale = H.D ** -0.5
    out = fp8_varlen_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV),
                                       cu_q.to(H.DEV), cu_k.to(H.DEV), max(lq) + 1000, scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.varlen_prefill_attention(query, kc, vc, ks, vs, tables, cu_q, cu_k, scale)
    H.assert_attention_close(out, ref)


@pytest.mark.parametrize("scale", [0.0, -0.088, float("nan"), float("inf")])
def test_prefill_rejects_a_softmax_scale_that_is_not_positive(scale):
    """The row maxima are taken before the softmax scale, so a scale that is
    not positive and finite raises (MSKV_EUNSUPPORTED) instead of returning
    rows normalized against the wrong maximum."""
    lq, lk = [20], [20 + 100]
    query, tables, caches, cu_q, cu_k = _varlen_setup(233, lq, lk, 32, 8)
    with pytest.raises(RuntimeError, match="status -2"):
        fp8_varlen_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV),
                                     cu_q.to(H.DEV), cu_k.to(H.DEV), 20, scale)
    with pytest.raises(RuntimeError, match="status -2"):
        fp8_chunk_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV), 100, scale)


def test_chunk_prefill_single_equals_varlen():
    lq, lk = [100], [100 + 700]
    query, tables, caches, cu_q, cu_k = _varlen_setup(231, lq, lk, 32, 8)
    a = fp8_chunk_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV), 700, 0.088)
    b = fp8_varlen_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV),
                                     cu_q.to(H.DEV), cu_k.to(H.DEV), 100, 0.088)
    assert torch.equal(a, b)
