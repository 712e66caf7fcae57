"""GPU parity of fp8_decode_attention against the oracle
(``fp8_decode_attention.py:16-58``): outputs within 2e-2 max-abs and
1e-2 relative (Frobenius) error, plus size-independent properties at the
Qwen3-8B / 32B shapes."""

import importlib
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
    decode_num_splits, fp8_decode_attention, store_fp8_kvcache)


def _setup(seed, lens, hq, hk, num_blocks, dtype=torch.bfloat16, kscale=1.0,
           vscale=1.0, qscale=1.0, block_size=H.BLOCK):
    gen = torch.Generator().manual_seed(seed)
    tables, slots = H.paged_layout(gen, lens, num_blocks, block_size)
    n = slots.numel()
    key = H.randn(gen, (n, hk, H.D), dtype, kscale)
    value = H.randn(gen, (n, hk, H.D), dtype, vscale)
    query = H.randn(gen, (len(lens), hq, H.D), dtype, qscale)
    caches = H.alloc_cache(num_blocks, block_size, hk)
    if n:
        store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    return query, tables, caches


def _run_and_check(query, lens, tables, caches, atol=2e-2, rtol=1e-2):
    scale = H.D ** -0.5
    seqlens = torch.tensor(lens, dtype=torch.int32)
    out = fp8_decode_attention(query.to(H.DEV), *caches, seqlens.to(H.DEV),
                               tables.to(H.DEV), scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.decode_attention(query, kc, vc, ks, vs, seqlens, tables, scale)
    return H.assert_attention_close(out, ref, atol, rtol), out


def test_decode_reference_case():
    """tests/test_fp8_kv_attention.py::test_decode's shape and tolerance."""
    g = np.load(os.path.join(GOLDEN, "ref_shapes.npz"))
    c = cases.decode_case()
    caches = H.alloc_cache(c["num_blocks"])
    store_fp8_kvcache(c["key"].to(H.DEV), c["value"].to(H.DEV), *caches, c["slots"].to(H.DEV))
    out = fp8_decode_attention(c["query"].to(H.DEV), *caches,
                               torch.tensor(c["lengths"], dtype=torch.int32, device=H.DEV),
                               c["tables"].to(H.DEV), cases.D ** -0.5)
    err = (out.float().cpu() - torch.from_numpy(g["dec_out"]).half().float()).abs().max().item()
    assert torch.isfinite(out).all()
    assert err < 0.004, err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_qwen3_06b_config(dtype):
    """Qwen3-0.6B layer: 16 q / 8 kv heads, batch 4, lengths U[1, 1024], a
    randomly permuted 64-block pool."""
    gen = torch.Generator().manual_seed(31)
    lens = torch.randint(1, 1025, (4,), generator=gen).tolist()
    query, tables, caches = _setup(32, lens, 16, 8, 64, dtype)
    _run_and_check(query, lens, tables, caches)


@pytest.mark.parametrize("hq,hk", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (32, 2), (64, 2),
                                   (24, 8), (40, 2), (20, 1), (96, 4)])
def test_decode_gqa_groups(hq, hk):
    lens = [1, 255, 256, 257, 700, 0, 1023, 33]
    query, tables, caches = _setup(41 + hq + hk, lens, hq, hk, 40)
    _run_and_check(query, lens, tables, caches)


def test_decode_zero_length_and_padded_rows():
    """Runner padding (``model_runner.py:268-273``): rows with seq_len 0 and an
    all -1 table give zeros; real rows are unaffected."""
    lens = [300, 0, 5, 0]
    query, tables, caches = _setup(51, lens, 32, 8, 8)
    (_, _), out = _run_and_check(query, lens, tables, caches)
    assert (out[1] == 0).all() and (out[3] == 0).all()


def test_decode_no_split_path():
    """A batch large enough that the kernel writes the output directly."""
    lens = [int(x) for x in torch.randint(1, 512, (512,), generator=torch.Generator().manual_seed(5))]
    assert decode_num_splits(512, 32, 8, 2, H.BLOCK) == 1
    query, tables, caches = _setup(61, lens, 32, 8, 1100)
    _run_and_check(query, lens, tables, caches)


def test_decode_invalid_block_ids_read_as_empty():
    """Block ids outside the pool are skipped instead of read (an extension:
    the reference never produces them)."""
    lens = [512, 512]
    query, tables, caches = _setup(71, lens, 32, 8, 4)
    bad = tables.clone()
    bad[0, 1] = 1 << 20          # second page of sequence 0 is out of the pool
    out = fp8_decode_attention(query.to(H.DEV), *caches,
                               torch.tensor(lens, dtype=torch.int32, device=H.DEV),
                               bad.to(H.DEV), H.D ** -0.5)
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref0 = O.decode_attention(query[:1], kc, vc, ks, vs, torch.tensor([256]), tables[:1], H.D ** -0.5)
    ref1 = O.decode_attention(query[1:], kc, vc, ks, vs, torch.tensor([512]), tables[1:], H.D ** -0.5)
    H.assert_attention_close(out[:1], ref0)
    H.assert_attention_close(out[1:], ref1)


def test_decode_invalid_first_page_keeps_weight_precision():
    """A split whose first page is an invalid block id sees no valid token
    in its first steps.  The PV weights' power-of-two scale is then chosen at
    the first step that has one, so V rows with small scales (V ~ 1e-4,
    v_scale ~ 1e-6) keep fp16's 11 significant bits instead of going
    subnormal.  At batch 64 x 4096 a split holds four pages, so sequence 0's
    first split still has three valid pages after its invalid first one; its
    result is attention over pages 1-15."""
    lens = [4096] * 64
    assert decode_num_splits(64, 32, 8, 16, H.BLOCK) == 4
    query, tables, caches = _setup(73, lens, 32, 8, 1100, vscale=1e-4)
    bad = tables.clone()
    bad[0, 0] = 1 << 20
    out = fp8_decode_attention(query.to(H.DEV), *caches,
                               torch.tensor(lens, dtype=torch.int32, device=H.DEV),
                               bad.to(H.DEV), H.D ** -0.5)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.decode_attention(query[:1], kc, vc, ks, vs, torch.tensor([4096 - H.BLOCK]),
                             tables[:1, 1:].contiguous(), H.D ** -0.5)
    max_abs, rel = H.attention_errors(out[:1], ref)
    assert rel < 2e-3, f"max_abs {max_abs:.3e} rel {rel:.3e}"


@pytest.mark.parametrize("block_size", [512, 1024])
def test_decode_larger_block_sizes(block_size):
    """Pages of 512 and 1024 tokens (any multiple of 256 is a valid
    block_size, Config.py:28): lengths around page boundaries."""
    lens = [1, 511, 512, 513, 1500, 3000, 4096]
    nb = sum((n + block_size - 1) // block_size for n in lens) + 2
    query, tables, caches = _setup(151, lens, 32, 8, nb, block_size=block_size)
    _run_and_check(query, lens, tables, caches)


def test_decode_qwen3_8b_full_shape():
    """Batch 64 x 4096 tokens, 32 q / 8 kv heads, 2048-block permuted pool."""
    lens = [4096] * 64
    query, tables, caches = _setup(81, lens, 32, 8, 2048)
    _run_and_check(query, lens, tables, caches)


def test_decode_block_relabel_and_split_invariance():
    """Relabelling physical blocks gives a bitwise identical result, and a
    sequence decoded inside the batch (split-KV) matches it decoded alone."""
    lens = [4096] * 64
    query, tables, caches = _setup(91, lens, 32, 8, 2048)
    kc, vc, ks, vs = caches
    seqlens = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
    out = fp8_decode_attention(query.to(H.DEV), kc, vc, ks, vs, seqlens, tables.to(H.DEV), 0.088)
    perm = torch.randperm(2048, generator=torch.Generator().manual_seed(3)).to(H.DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(2048, device=H.DEV)
    kc2, vc2, ks2, vs2 = (torch.empty_like(t) for t in (kc, vc, ks, vs))
    kc2.view(torch.uint8)[perm] = kc.view(torch.uint8)
    vc2.view(torch.uint8)[perm] = vc.view(torch.uint8)
    ks2[perm] = ks
    vs2[perm] = vs
    t2 = perm[tables.to(H.DEV).long()].to(torch.int32)
    out2 = fp8_decode_attention(query.to(H.DEV), kc2, vc2, ks2, vs2, seqlens, t2, 0.088)
    assert torch.equal(out, out2)
    # the first sequence alone uses a different split count
    solo = fp8_decode_attention(query[:1].to(H.DEV), kc, vc, ks, vs, seqlens[:1],
                                tables[:1].to(H.DEV), 0.088)
    assert decode_num_splits(1, 32, 8, 16, H.BLOCK) != decode_num_splits(64, 32, 8, 16, H.BLOCK)
    assert (solo.float() - out[:1].float()).abs().max().item() < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_ragged_fragmented(dtype):
    """Ragged lengths, log-uniform in [16, 32768], blocks sampled from a
    fragmented pool.  17 splits x 48 sequences is 816 eight-wave workgroups,
    over the launcher's limit for row order, so this runs the longest-first
    work items of the pre-pass (the Qwen3-8B full shape, 256 workgroups,
    runs in row order), in both activation types."""
    gen = torch.Generator().manual_seed(101)
    b = 48
    lens = torch.exp(torch.empty(b).uniform_(np.log(16), np.log(32768), generator=gen)).long().tolist()
    pages = sum((n + 255) // 256 for n in lens)
    query, tables, caches = _setup(102, lens, 32, 8, pages + 97, dtype)
    _run_and_check(query, lens, tables, caches)


def test_decode_work_items_cover_every_split_4096_sequences():
    """The pre-pass at its batch limit: 4096 sequences (the sort's LDS
    arrays full), mostly one split each plus a few of 16, with the workspace
    filled with NaN bytes first, so a split that no work item covered would
    merge a NaN partial.  Called through the C ABI with that workspace."""
    from microserve_amd import _lib
    gen = torch.Generator().manual_seed(107)
    b, w = 4096, 64
    lens = torch.randint(1, 65, (b,), generator=gen).tolist()
    for i in range(0, b, 512):
        lens[i] = w * H.BLOCK
        lens[i + 1] = 2000
    lens[3] = 0
    splits = decode_num_splits(b, 32, 8, w, H.BLOCK)
    assert splits == 16
    pages = sum((n + H.BLOCK - 1) // H.BLOCK for n in lens)
    query, tables, caches = _setup(108, lens, 32, 8, pages + 5)
    assert tables.shape[1] == w
    lib = _lib.load()
    need = lib.mskv_decode_workspace_bytes(b, 32, 8, H.D, splits)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=H.DEV)
    q = query.to(H.DEV)
    out = torch.empty_like(q)
    kc, vc, ks, vs = caches
    seqlens = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
    t = tables.to(H.DEV)
    status = lib.mskv_fp8_decode_attention(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(),
        seqlens.data_ptr(), t.data_ptr(), out.data_ptr(), b, 32, 8, H.D, H.BLOCK, kc.shape[0], w,
        H.D ** -0.5, _lib.act_dtype(q), splits, ws.data_ptr(), need, _lib.stream_of(q))
    assert status == 0
    torch.cuda.synchronize()
    kcn, vcn, ksn, vsn = H.cache_to_numpy(*caches)
    ref = O.decode_attention(query, kcn, vcn, ksn, vsn, torch.tensor(lens), tables, H.D ** -0.5)
    H.assert_attention_close(out, ref)
    assert (out[3] == 0).all()


def test_decode_narrow_workgroups_wide_gqa_group():
    """GQA 32 (64 q / 2 kv heads: two 16-head units per kv head, four in
    all) on the 4-wave workgroup shape over the work items: 96 sequences x
    16 splits of one 8-wave workgroup each is over the launcher's limit for
    row order, and eight waves would leave four idle."""
    gen = torch.Generator().manual_seed(105)
    b = 96
    lens = torch.exp(torch.empty(b).uniform_(np.log(16), np.log(16384), generator=gen)).long().tolist()
    lens[0] = 16384                      # the table is 64 pages wide
    assert decode_num_splits(b, 64, 2, 64, H.BLOCK) == 16
    pages = sum((n + 255) // 256 for n in lens)
    query, tables, caches = _setup(106, lens, 64, 2, pages + 5, torch.float16)
    _run_and_check(query, lens, tables, caches)


def test_decode_row_order_past_the_work_item_limit():
    """300 sequences x 256 splits (32-token pages, 1024 pages wide) is past
    the work items' limit of 65,536 (sequence, split) pairs: this runs the
    4-wave workgroups in row order, empty splits interleaved."""
    gen = torch.Generator().manual_seed(181)
    b, bs = 300, 32
    lens = torch.exp(torch.empty(b).uniform_(np.log(1), np.log(2048), generator=gen)).long().tolist()
    lens[7] = 1024 * bs                  # the table is 1024 pages wide
    lens[8] = 0
    splits = decode_num_splits(b, 8, 8, 1024, bs)
    assert b * splits > 65536
    pages = sum((n + bs - 1) // bs for n in lens)
    query, tables, caches = _setup(182, lens, 8, 8, pages + 3, block_size=bs)
    assert tables.shape[1] == 1024
    _, out = _run_and_check(query, lens, tables, caches)
    assert (out[8] == 0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_v_scale_growing_along_the_sequence(dtype):
    """V magnitudes grow by 2^12 along each sequence (log-linear in the
    position) and 2% of the rows are stored as zeros.  Each wave meets
    larger v_scales step after step, so the power of two that keeps its
    fp16 weights in range shrinks and the accumulator is rescaled many
    times; the zero rows' weights underflow while their probabilities still
    count.  Outputs stay O(1), so the usual gate applies."""
    gen = torch.Generator().manual_seed(121)
    lens = [5000, 777, 4096, 1, 300]
    hq, hk = 32, 8
    pages = sum((n + H.BLOCK - 1) // H.BLOCK for n in lens)
    tables, slots = H.paged_layout(gen, lens, pages + 3)
    n = slots.numel()
    pos = torch.cat([torch.arange(x) for x in lens]).float()
    grow = torch.exp2(12.0 * pos / max(lens) - 12.0)
    key = H.randn(gen, (n, hk, H.D), dtype)
    value = torch.randn(n, hk, H.D, generator=gen) * grow[:, None, None]
    value[torch.rand(n, generator=gen) < 0.02] = 0.0
    value = value.to(dtype)
    query = H.randn(gen, (len(lens), hq, H.D), dtype)
    caches = H.alloc_cache(pages + 3, H.BLOCK, hk)
    store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    (max_abs, rel), _ = _run_and_check(query, lens, tables, caches)
    print(f"growing V {dtype}: max_abs {max_abs:.3e} rel {rel:.3e}")


def test_decode_long_context_qwen3_32b():
    """131072 tokens at 64 q / 8 kv heads: split-KV across the whole GPU plus
    the log-sum-exp combine."""
    lens = [131072]
    query, tables, caches = _setup(111, lens, 64, 8, 512)
    assert decode_num_splits(1, 64, 8, 512, H.BLOCK) >= 128
    _run_and_check(query, lens, tables, caches)


def test_decode_graph_replay_matches_eager():
    """Capture store + decode in a HIP graph with runner-style padded inputs
    and replay it with new contents; every replay equals the eager result."""
    hq, hk, nb, max_bs, width = 32, 8, 64, 8, 8
    garbage_slot = (nb - 1) * H.BLOCK
    caches = H.alloc_cache(nb)
    gen = torch.Generator().manual_seed(121)
    static = dict(
        q=torch.zeros(max_bs, hq, H.D, dtype=torch.bfloat16, device=H.DEV),
        k=torch.zeros(max_bs, hk, H.D, dtype=torch.bfloat16, device=H.DEV),
        v=torch.zeros(max_bs, hk, H.D, dtype=torch.bfloat16, device=H.DEV),
        slot=torch.full((max_bs,), garbage_slot, dtype=torch.int64, device=H.DEV),
        lens=torch.zeros(max_bs, dtype=torch.int32, device=H.DEV),
        tables=torch.full((max_bs, width), -1, dtype=torch.int32, device=H.DEV),
        out=torch.zeros(max_bs, hq, H.D, dtype=torch.bfloat16, device=H.DEV))
    # prefill some history on the first 4 sequences
    lens0 = [700, 1, 256, 1500]
    tables, slots = H.paged_layout(gen, lens0, nb - 1)
    n = slots.numel()
    store_fp8_kvcache(H.randn(gen, (n, hk, H.D), torch.bfloat16).to(H.DEV),
                      H.randn(gen, (n, hk, H.D), torch.bfloat16).to(H.DEV),
                      *caches, slots.to(H.DEV))

    def step():
        store_fp8_kvcache(static["k"], static["v"], *caches, static["slot"])
        fp8_decode_attention(static["q"], *caches, static["lens"], static["tables"],
                             0.088, out=static["out"])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    lens = list(lens0)
    for it in range(3):
        bs = 4
        q = H.randn(gen, (bs, hq, H.D), torch.bfloat16)
        k = H.randn(gen, (bs, hk, H.D), torch.bfloat16)
        v = H.randn(gen, (bs, hk, H.D), torch.bfloat16)
        new_slots = []
        for b in range(bs):
            p = lens[b]
            new_slots.append(int(tables[b, p // H.BLOCK]) * H.BLOCK + p % H.BLOCK)
            lens[b] += 1
        static["q"].zero_(); static["q"][:bs] = q.to(H.DEV)
        static["k"].zero_(); static["k"][:bs] = k.to(H.DEV)
        static["v"].zero_(); static["v"][:bs] = v.to(H.DEV)
        static["slot"].fill_(garbage_slot)
        static["slot"][:bs] = torch.tensor(new_slots, device=H.DEV)
        static["lens"].zero_(); static["lens"][:bs] = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
        static["tables"].fill_(-1); static["tables"][:bs, :tables.shape[1]] = tables.to(H.DEV)
        snapshot = [c.clone() for c in caches]
        graph.replay()
        torch.cuda.synchronize()
        got = static["out"].clone()
        # eager on a copy of the pre-step caches
        eager_caches = snapshot
        store_fp8_kvcache(static["k"], static["v"], *eager_caches, static["slot"])
        want = fp8_decode_attention(static["q"], *eager_caches, static["lens"],
                                    static["tables"], 0.088)
        torch.cuda.synchronize()
        assert torch.equal(got[:bs], want[:bs]), f"replay {it}"
        assert (got[bs:] == 0).all()
        for a, b_ in zip(caches, eager_caches):
            if a.dtype == torch.float8_e4m3fn:
                same = torch.equal(a.view(torch.uint8)[: nb - 1], b_.view(torch.uint8)[: nb - 1])
            else:
                same = torch.equal(a[: nb - 1], b_[: nb - 1])
            assert same, f"cache differs after replay {it}"


def test_decode_graph_replay_longest_first_order():
    """The longest-first pre-pass (shapes of many workgroup rounds) inside a
    captured graph: each replay ranks the sequences by their new lengths,
    ties and empty rows included, and equals the eager result bit for bit;
    the first replay is also checked against the oracle."""
    hq, hk, b = 32, 8, 48
    gen = torch.Generator().manual_seed(171)
    lens = torch.exp(torch.empty(b).uniform_(np.log(16), np.log(16384), generator=gen)).long().tolist()
    lens[0] = 16384                      # the table is 64 pages wide: 16 splits
    pages = [(n + H.BLOCK - 1) // H.BLOCK for n in lens]
    query, tables, caches = _setup(172, lens, hq, hk, sum(pages) + 7)
    width = tables.shape[1]
    assert b * decode_num_splits(b, hq, hk, width, H.BLOCK) > 512
    scale = H.D ** -0.5
    q_d = query.to(H.DEV)
    tables_d = tables.to(H.DEV)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
    out = torch.zeros_like(q_d)

    def step():
        fp8_decode_attention(q_d, *caches, lens_d, tables_d, scale, out=out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for it in range(3):
        # new lengths inside each row's pages: a new ranking every replay,
        # with repeated lengths and empty rows
        new = [int(torch.randint(0, p * H.BLOCK + 1, (1,), generator=gen)) for p in pages]
        new[1] = new[2] = new[3]
        new[4] = 0
        lens_d.copy_(torch.tensor(new, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = fp8_decode_attention(q_d, *caches, lens_d, tables_d, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {it}"
        assert (got[4] == 0).all()
        if it == 0:
            kc, vc, ks, vs = H.cache_to_numpy(*caches)
            ref = O.decode_attention(query, kc, vc, ks, vs, torch.tensor(new, dtype=torch.int32),
                                     tables, scale)
            H.assert_attention_close(got, ref, 2e-2, 1e-2)


def test_decode_scratch_reuse_across_shapes():
    """Calls of different batch sizes share the per-device partials scratch;
    a large batch after a small one still merges its own partials."""
    lens = [4096] * 64
    query, tables, caches = _setup(131, lens, 32, 8, 2048)
    q = query.to(H.DEV)
    t = tables.to(H.DEV)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
    a = fp8_decode_attention(q, *caches, lens_d, t, 0.088)
    small = fp8_decode_attention(q[:8], *caches, lens_d[:8], t[:8], 0.088)
    c = fp8_decode_attention(q, *caches, lens_d, t, 0.088)
    torch.cuda.synchronize()
    assert torch.equal(a, c)
    assert (small.float() - a[:8].float()).abs().max().item() < 1e-2


def test_decode_graph_survives_scratch_growth(monkeypatch):
    """A graph captured before a larger batch grew its stream's partials
    scratch still replays correctly: the buffer it addresses is kept, not
    handed back to the allocator for other tensors (the runner captures its
    graphs from the smallest batch up, with an eager warm-up of each before
    capture).  The scratch is per (device, stream): here the warm-up, the
    capture and the growth all run on one capture stream."""
    M = importlib.import_module("microserve_amd.fp8_decode_attention")
    monkeypatch.setattr(M, "_SCRATCH", {})
    monkeypatch.setattr(M, "_RETIRED", [])
    lens = [4096] * 64
    query, tables, caches = _setup(141, lens, 32, 8, 1100)
    q = query.to(H.DEV)
    t = tables.to(H.DEV)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=H.DEV)
    small = dict(q=q[:1].clone(), lens=lens_d[:1].clone(), t=t[:1].clone(),
                 out=torch.zeros_like(q[:1]))

    def step():
        fp8_decode_attention(small["q"], *caches, small["lens"], small["t"], 0.088,
                             out=small["out"])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    key = (q.device, s.cuda_stream)
    captured = M._SCRATCH[key]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step()
    assert M._SCRATCH[key] is captured, "the capture must reuse the warmed-up scratch"
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        want = fp8_decode_attention(q, *caches, lens_d, t, 0.088)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert M._SCRATCH[key] is not captured, "the large batch must grow the scratch"
    assert any(r is captured for r in M._RETIRED)
    # tensors of the old buffer's size, filled with a pattern: a freed
    # buffer would be handed to one of them and the replay would overwrite it
    churn = [torch.full((captured.numel(),), 0x5A, dtype=torch.uint8, device=H.DEV)
             for _ in range(4)]
    graph.replay()
    torch.cuda.synchronize()
    got = small["out"].clone()
    eager = fp8_decode_attention(small["q"], *caches, small["lens"], small["t"], 0.088)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
    assert (got.float() - want[:1].float()).abs().max().item() < 1e-2
    for c in churn:
        assert bool((c == 0x5A).all()), "the replay wrote into another tensor"


def test_decode_concurrent_streams_match_the_oracle():
    """Two streams decode different batches at the same time: each stream has
    its own partials scratch, so neither overwrites the other's, as with the
    reference, whose call keeps no state between calls
    (``fp8_decode_attention.py:93``).  Both batches use several splits."""
    lens_a = [4096] * 16
    lens_b = [3000 + 37 * i for i in range(16)]
    qa, ta, caches = _setup(151, lens_a + lens_b, 32, 8, 1100)
    qb, tb = qa[16:].contiguous(), ta[16:].contiguous()
    qa, ta = qa[:16].contiguous(), ta[:16].contiguous()
    assert decode_num_splits(16, 32, 8, ta.shape[1], H.BLOCK) > 1
    args_a = (qa.to(H.DEV), ta.to(H.DEV), torch.tensor(lens_a, dtype=torch.int32, device=H.DEV))
    args_b = (qb.to(H.DEV), tb.to(H.DEV), torch.tensor(lens_b, dtype=torch.int32, device=H.DEV))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs_a, outs_b = [], []
    for _ in range(4):
        with torch.cuda.stream(s1):
            outs_a.append(fp8_decode_attention(args_a[0], *caches, args_a[2], args_a[1], 0.088))
        with torch.cuda.stream(s2):
            outs_b.append(fp8_decode_attention(args_b[0], *caches, args_b[2], args_b[1], 0.088))
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref_a = O.decode_attention(qa, kc, vc, ks, vs, torch.tensor(lens_a), ta, 0.088)
    ref_b = O.decode_attention(qb, kc, vc, ks, vs, torch.tensor(lens_b), tb, 0.088)
    for oa, ob in zip(outs_a, outs_b):
        H.assert_attention_close(oa, ref_a)
        H.assert_attention_close(ob, ref_b)
        assert torch.equal(oa, outs_a[0]) and torch.equal(ob, outs_b[0])
