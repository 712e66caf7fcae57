"""GPU parity of the step-input builder (``step_inputs_kernel`` through
``mskv_build_step_inputs``) against the oracle restatement of the runner's
builders: every field bit-exact."""

import numpy as np
import pytest
import torch

from microserve_amd import step_inputs as SI
from microserve_amd.context import AttentionMode
from oracle import step_inputs_oracle as SO
from tests.seqs import Seq, random_batch

DEV = "cuda"


def _eq(t, ref, what):
    got = t.cpu().numpy()
    assert got.dtype == ref.dtype, (what, got.dtype, ref.dtype)
    assert np.array_equal(got, ref), f"{what} differs"


@pytest.mark.gpu
@pytest.mark.parametrize("n_seqs,bs,max_len", [(256, 256, 32768), (64, 256, 4096), (1, 16, 40),
                                                (37, 32, 1000)])
def test_decode_matches_oracle(n_seqs, bs, max_len):
    rng = np.random.default_rng(n_seqs)
    seqs = random_batch(rng, "decode", n_seqs, bs, 40000, max_len)
    print(f"decode batch {n_seqs} block {bs} max_len {max_len}", flush=True)
    ctx, ids, pos = SI.compile_decode(seqs, bs, DEV)
    torch.cuda.synchronize()
    ref = SO.compile_decode(seqs, bs)
    assert ctx.mode == AttentionMode.DECODE
    _eq(ids, ref["input_ids"], "input_ids")
    _eq(pos, ref["positions"], "positions")
    _eq(ctx.slot_mapping, ref["slot_mapping"], "slot_mapping")
    _eq(ctx.cache_seqlens, ref["cache_seqlens"], "cache_seqlens")
    _eq(ctx.block_tables, ref["block_tables"], "block_tables")


@pytest.mark.gpu
def test_decode_graph_padding_into_fixed_buffers():
    """The graph form writes the padded rows straight into the caller's
    buffers and leaves rows past pad_to alone."""
    rng = np.random.default_rng(7)
    bs, max_bs, width, garbage = 256, 64, 20, 2048 * 256
    seqs = random_batch(rng, "decode", 37, bs, 2048, 4096)
    gv = {"input_ids": torch.full((max_bs,), 77, dtype=torch.int64, device=DEV),
          "positions": torch.full((max_bs,), 77, dtype=torch.int64, device=DEV),
          "slot_mapping": torch.full((max_bs,), 77, dtype=torch.int64, device=DEV),
          "cache_seqlens": torch.full((max_bs,), 77, dtype=torch.int32, device=DEV),
          "block_tables": torch.full((max_bs, width), 77, dtype=torch.int32, device=DEV)}
    for pad_to in (48, 40):
        ctx, ids, pos = SI.compile_decode(seqs, bs, DEV, pad_to=pad_to, table_width=width,
                                          garbage_slot=garbage, out=gv)
        torch.cuda.synchronize()
        ref = SO.pad_decode(SO.compile_decode(seqs, bs), pad_to, width, garbage)
        assert ctx.slot_mapping.data_ptr() == gv["slot_mapping"].data_ptr()
        _eq(ids, ref["input_ids"], "input_ids")
        _eq(pos, ref["positions"], "positions")
        _eq(ctx.slot_mapping, ref["slot_mapping"], "slot_mapping")
        _eq(ctx.cache_seqlens, ref["cache_seqlens"], "cache_seqlens")
        _eq(ctx.block_tables, ref["block_tables"], "block_tables")
    assert (gv["slot_mapping"][48:] == 77).all() and (gv["block_tables"][48:] == 77).all()


@pytest.mark.gpu
@pytest.mark.parametrize("n_seqs,bs,max_len", [(8, 256, 8192), (3, 16, 300), (1, 256, 1)])
def test_prefill_matches_oracle(n_seqs, bs, max_len):
    rng = np.random.default_rng(100 + n_seqs)
    seqs = random_batch(rng, "prefill", n_seqs, bs, 4096, max(2, max_len))
    if max_len == 1:
        seqs = [Seq([5], 0, 1, [3], num_tokens_with_spec=2)]
    print(f"prefill batch {n_seqs} block {bs}", flush=True)
    ctx, cu_q, ids, pos = SI.compile_prefill(seqs, bs, DEV)
    torch.cuda.synchronize()
    ref = SO.compile_prefill(seqs, bs)
    assert ctx.mode == AttentionMode.PREFILL and ctx.block_tables is None
    assert ctx.max_seqlen_q == ref["max_seqlen_q"] == ctx.max_seqlen_k
    _eq(cu_q, ref["cu_seqlens_q"], "cu_seqlens_q")
    _eq(ctx.cu_seqlens_k, ref["cu_seqlens_k"], "cu_seqlens_k")
    _eq(ids, ref["input_ids"], "input_ids")
    _eq(pos, ref["positions"], "positions")
    _eq(ctx.slot_mapping, ref["slot_mapping"], "slot_mapping")


@pytest.mark.gpu
def test_chunk_prefill_matches_oracle():
    rng = np.random.default_rng(11)
    for seq in random_batch(rng, "chunk", 6, 256, 4096, 20000):
        ctx, ids, pos = SI.compile_chunk_prefill(seq, 256, DEV)
        torch.cuda.synchronize()
        ref = SO.compile_chunk_prefill(seq, 256)
        assert ctx.mode == AttentionMode.CHUNK_PREFILL
        for k in ("prefix_len", "query_len", "max_seqlen_q", "max_seqlen_k"):
            assert getattr(ctx, k) == ref[k], k
        _eq(ids, ref["input_ids"], "input_ids")
        _eq(pos, ref["positions"], "positions")
        _eq(ctx.slot_mapping, ref["slot_mapping"], "slot_mapping")
        _eq(ctx.block_tables, ref["block_tables"], "block_tables")
        _eq(ctx.cache_seqlens, ref["cache_seqlens"], "cache_seqlens")
        _eq(ctx.cu_seqlens_q, ref["cu_seqlens_q"], "cu_seqlens_q")
        _eq(ctx.cu_seqlens_k, ref["cu_seqlens_k"], "cu_seqlens_k")


@pytest.mark.gpu
def test_make_block_tables_with_empty_rows():
    seqs = [Seq([], 0, 0, []), Seq([], 0, 0, [5, 9, 2]), Seq([], 0, 0, [4])]
    bt = SI.make_block_tables(seqs, DEV)
    torch.cuda.synchronize()
    _eq(bt, SO.make_block_tables(seqs), "block_tables")


@pytest.mark.gpu
def test_built_context_drives_store_and_decode():
    """The builder's context feeds the FP8 Attention layer directly: the
    cache rows it writes are those the oracle's slots name."""
    from microserve_amd import Attention, set_context, reset_context
    from tests.gpu_helpers import alloc_cache
    rng = np.random.default_rng(5)
    bs, hq, hk, d = 256, 32, 8, 128
    seqs = random_batch(rng, "decode", 16, bs, 128, 1500)
    kc, vc, ks, vs = alloc_cache(128)
    attn = Attention(hq, d, d ** -0.5, hk)
    attn.k_cache, attn.v_cache, attn.k_scale_cache, attn.v_scale_cache = kc, vc, ks, vs
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(16, hq, d, generator=gen).bfloat16().to(DEV)
    k = torch.randn(16, hk, d, generator=gen).bfloat16().to(DEV)
    v = torch.randn(16, hk, d, generator=gen).bfloat16().to(DEV)
    ctx, _, _ = SI.compile_decode(seqs, bs, DEV)
    set_context(ctx)
    try:
        attn(q, k, v)
    finally:
        reset_context()
    torch.cuda.synchronize()
    slots = SO.compile_decode(seqs, bs)["slot_mapping"]
    rows = kc.view(-1, hk, d)[torch.from_numpy(slots).to(DEV)]
    assert rows.view(torch.uint8).any(dim=-1).all(), "a stored row is missing"
