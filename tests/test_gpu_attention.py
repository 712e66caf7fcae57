"""The drop-in ``Attention`` layer + ``Context`` on the GPU: store-then-attend
in each mode (``attention.py:36-61``) against the oracle."""

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

from microserve_amd import (  # noqa: E402
    Attention, AttentionMode, Context, reset_context, set_context)


def _layer(hq=32, hk=8, nb=16):
    attn = Attention(hq, H.D, H.D ** -0.5, hk)
    attn.k_cache, attn.v_cache, attn.k_scale_cache, attn.v_scale_cache = H.alloc_cache(nb, H.BLOCK, hk)
    attn.kv_cache_dtype = "fp8_e4m3"
    return attn


def _np_caches(attn):
    return H.cache_to_numpy(attn.k_cache, attn.v_cache, attn.k_scale_cache, attn.v_scale_cache)


def test_attention_chunk_then_decode():
    gen = torch.Generator().manual_seed(301)
    attn = _layer()
    table = torch.tensor([[5, 2, 9]], dtype=torch.int32)
    # chunk prefill: 300 tokens already cached, 40 new
    pre_k = H.randn(gen, (300, 8, H.D), torch.bfloat16)
    pre_v = H.randn(gen, (300, 8, H.D), torch.bfloat16)
    pos = torch.arange(300)
    slots = table[0, pos // H.BLOCK].long() * H.BLOCK + pos % H.BLOCK
    from microserve_amd import store_fp8_kvcache
    store_fp8_kvcache(pre_k.to(H.DEV), pre_v.to(H.DEV), attn.k_cache, attn.v_cache,
                      attn.k_scale_cache, attn.v_scale_cache, slots.to(H.DEV))
    q = H.randn(gen, (40, 32, H.D), torch.bfloat16)
    k = H.randn(gen, (40, 8, H.D), torch.bfloat16)
    v = H.randn(gen, (40, 8, H.D), torch.bfloat16)
    pos = torch.arange(300, 340)
    slots = table[0, pos // H.BLOCK].long() * H.BLOCK + pos % H.BLOCK
    set_context(Context(mode=AttentionMode.CHUNK_PREFILL, slot_mapping=slots.to(H.DEV),
                        block_tables=table.to(H.DEV), prefix_len=300, query_len=40,
                        cache_seqlens=torch.tensor([340], dtype=torch.int32, device=H.DEV)))
    try:
        out = attn(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV))
    finally:
        reset_context()
    kc, vc, ks, vs = _np_caches(attn)
    ref = O.chunk_prefill_attention(q, kc, vc, ks, vs, table[0], 300, H.D ** -0.5)
    H.assert_attention_close(out, ref)
    # the chunk's own K/V were stored bit-exactly at their slots
    kq, _ = O.quantize_rows(k.float().numpy())
    assert np.array_equal(kc.reshape(-1, 8, H.D)[slots.numpy()], kq)
    # one decode step at position 340
    q = H.randn(gen, (1, 32, H.D), torch.bfloat16)
    k = H.randn(gen, (1, 8, H.D), torch.bfloat16)
    v = H.randn(gen, (1, 8, H.D), torch.bfloat16)
    slot = torch.tensor([int(table[0, 340 // H.BLOCK]) * H.BLOCK + 340 % H.BLOCK])
    set_context(Context(mode=AttentionMode.DECODE, slot_mapping=slot.to(H.DEV),
                        cache_seqlens=torch.tensor([341], dtype=torch.int32, device=H.DEV),
                        block_tables=table.to(H.DEV)))
    try:
        out = attn(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV))
    finally:
        reset_context()
    kc, vc, ks, vs = _np_caches(attn)
    ref = O.decode_attention(q, kc, vc, ks, vs, np.array([341]), table, H.D ** -0.5)
    H.assert_attention_close(out, ref)


def test_attention_fresh_prefill_attends_unquantized_and_stores():
    """PREFILL as the reference runner issues it (no block tables): the K/V
    are stored into the FP8 cache and attention runs over the unquantized
    new tokens (flash_attn_varlen_func, attention.py:49-55)."""
    gen = torch.Generator().manual_seed(311)
    attn = _layer(nb=8)
    lens = [100, 37]
    tables, slots = H.paged_layout(gen, lens, 8)
    q = H.randn(gen, (137, 32, H.D), torch.bfloat16)
    k = H.randn(gen, (137, 8, H.D), torch.bfloat16)
    v = H.randn(gen, (137, 8, H.D), torch.bfloat16)
    cu = torch.tensor([0, 100, 137], dtype=torch.int32)
    set_context(Context(mode=AttentionMode.PREFILL, cu_seqlens_q=cu.to(H.DEV),
                        cu_seqlens_k=cu.to(H.DEV), max_seqlen_q=100, max_seqlen_k=100,
                        slot_mapping=slots.to(H.DEV)))
    try:
        out = attn(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV))
    finally:
        reset_context()
    ref = O.dense_varlen_attention(q, k, v, cu, cu, H.D ** -0.5)
    H.assert_attention_close(out, ref)
    # the step's K/V were stored: chunk prefill over the cache agrees with
    # the FP8-dequantized oracle
    kc, vc, ks, vs = _np_caches(attn)
    ref_cache = O.varlen_prefill_attention(q, kc, vc, ks, vs, tables, cu, cu, H.D ** -0.5)
    from microserve_amd import fp8_varlen_prefill_attention
    got = fp8_varlen_prefill_attention(q.to(H.DEV), attn.k_cache, attn.v_cache, attn.k_scale_cache,
                                       attn.v_scale_cache, tables.to(H.DEV), cu.to(H.DEV),
                                       cu.to(H.DEV), 100, H.D ** -0.5)
    H.assert_attention_close(got, ref_cache)


def test_attention_unknown_mode_raises():
    attn = _layer(nb=2)
    set_context(Context(mode="bogus", slot_mapping=torch.zeros(1, dtype=torch.int64, device=H.DEV)))
    try:
        with pytest.raises(RuntimeError):
            attn(torch.zeros(1, 32, H.D, dtype=torch.bfloat16, device=H.DEV),
                 torch.zeros(1, 8, H.D, dtype=torch.bfloat16, device=H.DEV),
                 torch.zeros(1, 8, H.D, dtype=torch.bfloat16, device=H.DEV))
    finally:
        reset_context()


@pytest.mark.gpu
def test_wrappers_reject_host_tensors_among_gpu_arguments():
    """A host tensor among GPU arguments raises before any launch."""
    from microserve_amd import (fp8_decode_attention, qk_norm_rope_store, store_fp8_kvcache,
                                varlen_attention)
    from tests.gpu_helpers import alloc_cache
    kc, vc, ks, vs = alloc_cache(2)
    key = torch.zeros(3, 8, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="must be on"):
        store_fp8_kvcache(key, key, kc, vc, ks, vs, torch.zeros(3, dtype=torch.int64))
    q = torch.zeros(3, 32, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="must be on"):
        fp8_decode_attention(q, kc, vc, ks, vs, torch.ones(3, dtype=torch.int32, device="cuda"),
                             torch.zeros(3, 1, dtype=torch.int32), 0.1)
    cu = torch.tensor([0, 3], dtype=torch.int32)
    with pytest.raises(AssertionError, match="must be on"):
        varlen_attention(q, key, key, cu, cu.cuda(), 3, 3, 0.1)
    tab = torch.ones(16, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="must be on"):
        qk_norm_rope_store(torch.zeros(3, dtype=torch.int64), q, key, key, None, None, 1e-6, tab,
                           tab, kc, vc, ks, vs, torch.zeros(3, dtype=torch.int64, device="cuda"))


def test_empty_batches_are_no_ops():
    """Zero tokens to store, a decode batch of zero sequences and prefill
    calls with no query rows return empty results without launching."""
    from microserve_amd import (fp8_chunk_prefill_attention, fp8_decode_attention,
                                fp8_varlen_prefill_attention, store_fp8_kvcache,
                                varlen_attention)
    caches = H.alloc_cache(4)
    before = [c.clone() for c in caches]
    e = torch.zeros(0, 8, H.D, dtype=torch.bfloat16, device=H.DEV)
    store_fp8_kvcache(e, e, *caches, torch.zeros(0, dtype=torch.int64, device=H.DEV))
    q0 = torch.zeros(0, 32, H.D, dtype=torch.bfloat16, device=H.DEV)
    out = fp8_decode_attention(q0, *caches, torch.zeros(0, dtype=torch.int32, device=H.DEV),
                               torch.zeros(0, 2, dtype=torch.int32, device=H.DEV), 0.088)
    assert out.shape == (0, 32, H.D)
    table = torch.tensor([0, 1], dtype=torch.int32, device=H.DEV)
    out = fp8_chunk_prefill_attention(q0, *caches, table, 100, 0.088)
    assert out.shape == (0, 32, H.D)
    cu0 = torch.zeros(2, dtype=torch.int32, device=H.DEV)
    out = fp8_varlen_prefill_attention(q0, *caches, table.view(1, 2), cu0, cu0, 0, 0.088)
    assert out.shape == (0, 32, H.D)
    out = varlen_attention(q0, e, e, cu0, cu0, 0, 0, 0.088)
    assert out.shape == (0, 32, H.D)
    torch.cuda.synchronize()
    for a, b in zip(caches, before):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a,
                           b.view(torch.uint8) if b.dtype == torch.float8_e4m3fn else b)
