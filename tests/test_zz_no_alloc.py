"""GPU checks of mskv_fp8_decode_attention_noalloc, the decode entry point
that allocates nothing (its split partials live in a library-owned device
array): called through the C ABI, its output equals mskv_fp8_decode_attention's
bit for bit on two calls in a row, the second with a smaller input (the array
then holds the first call's partials), then on a ragged batch whose grid runs
the longest-first work items (kept in the same array); captured in a HIP
graph after an eager warm-up, its replays with new lengths equal the
workspace entry point's eager output; a shape whose partials exceed the
array is rejected."""

import numpy as np

import ctypes

import pytest
import torch

from microserve_amd import _lib, decode_num_splits, fp8_decode_attention
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _noalloc(query, caches, seqlens, tables, out, scale):
    kc, vc, ks, vs = caches
    b, hq, d = query.shape
    hk, bs = kc.shape[2], kc.shape[1]
    w = tables.shape[1]
    splits = decode_num_splits(b, hq, hk, w, bs)
    lib = _lib.load()
    return lib.mskv_fp8_decode_attention_noalloc(
        query.data_ptr(), kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(),
        seqlens.data_ptr(), tables.data_ptr(), out.data_ptr(), b, hq, hk, d, bs,
        kc.shape[0], w, ctypes.c_float(scale).value, _lib.act_dtype(query), splits,
        _lib.stream_of(query))


def _setup(seed, lens, hq, hk, num_blocks, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    tables, slots = H.paged_layout(gen, lens, num_blocks)
    caches = H.alloc_cache(num_blocks, kv_heads=hk)
    from microserve_amd import store_fp8_kvcache
    n = slots.numel()
    store_fp8_kvcache(H.randn(gen, (n, hk, H.D), dtype).to(H.DEV),
                      H.randn(gen, (n, hk, H.D), dtype).to(H.DEV), *caches, slots.to(H.DEV))
    q = H.randn(gen, (len(lens), hq, H.D), dtype).to(H.DEV)
    return q, caches, torch.tensor(lens, dtype=torch.int32, device=H.DEV), tables.to(H.DEV)


def test_noalloc_decode_equals_workspace_decode_twice():
    scale = H.D ** -0.5
    # call 1: the Qwen3-8B batch 64 x 4096 step (4 splits, 4.2 MB of partials)
    q, caches, lens, tables = _setup(301, [4096] * 64, 32, 8, 1100)
    out = torch.empty_like(q)
    assert _noalloc(q, caches, lens, tables, out, scale) == 0
    want = fp8_decode_attention(q, *caches, lens, tables, scale)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    # call 2, smaller: ragged lengths, fp16, GQA 8; the array still holds
    # call 1's partials, and no part of it needs to start at zero
    q2, caches2, lens2, tables2 = _setup(302, [3000, 1, 0, 777, 2049], 64, 8, 40,
                                         torch.float16)
    assert decode_num_splits(5, 64, 8, tables2.shape[1], H.BLOCK) > 1
    out2 = torch.empty_like(q2)
    assert _noalloc(q2, caches2, lens2, tables2, out2, scale) == 0
    want2 = fp8_decode_attention(q2, *caches2, lens2, tables2, scale)
    torch.cuda.synchronize()
    assert torch.equal(out2, want2)
    assert (out2[2] == 0).all()


def test_noalloc_decode_work_items_in_the_array():
    """48 ragged sequences x 17 splits: over 512 eight-wave workgroups, so the
    pre-pass writes its work items after the partials in the array (14 MB in
    all); two calls, the second with new lengths."""
    scale = H.D ** -0.5
    gen = torch.Generator().manual_seed(303)
    b = 48
    lens = torch.exp(torch.empty(b).uniform_(np.log(16), np.log(32768), generator=gen)).long().tolist()
    lens[0] = 32768
    pages = sum((n + H.BLOCK - 1) // H.BLOCK for n in lens)
    q, caches, seqlens, tables = _setup(304, lens, 32, 8, pages + 9)
    lib = _lib.load()
    splits = decode_num_splits(b, 32, 8, tables.shape[1], H.BLOCK)
    assert b * splits > 512
    assert lib.mskv_decode_workspace_bytes(b, 32, 8, H.D, splits) <= SCRATCH_BYTES
    out = torch.empty_like(q)
    for it in range(2):
        if it:
            seqlens = torch.tensor([max(0, n - 3 * n // 4) for n in lens], dtype=torch.int32,
                                   device=H.DEV)
        assert _noalloc(q, caches, seqlens, tables, out, scale) == 0
        want = fp8_decode_attention(q, *caches, seqlens, tables, scale)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"call {it}"


def test_noalloc_decode_under_graph_capture():
    """After one eager call on the device (which looks up the array's address
    there), the call is captured into a HIP graph on the work-item shape (48
    ragged sequences, 17 splits) and replayed three times with new lengths,
    eager work and synchronizations between the replays: every replay equals
    the workspace entry point's eager output bit for bit."""
    scale = H.D ** -0.5
    gen = torch.Generator().manual_seed(305)
    b = 48
    lens = torch.exp(torch.empty(b).uniform_(np.log(16), np.log(32768), generator=gen)).long().tolist()
    lens[0] = 32768
    pages = sum((n + H.BLOCK - 1) // H.BLOCK for n in lens)
    q, caches, seqlens, tables = _setup(306, lens, 32, 8, pages + 9)
    assert b * decode_num_splits(b, 32, 8, tables.shape[1], H.BLOCK) > 512
    out = torch.empty_like(q)
    assert _noalloc(q, caches, seqlens, tables, out, scale) == 0
    torch.cuda.synchronize()
    static_lens = seqlens.clone()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=s):
        status = _noalloc(q, caches, static_lens, tables, out, scale)
    assert status == 0
    torch.cuda.synchronize()
    for it in range(3):
        new = [max(0, n - (it + 1) * n // 5) for n in lens]
        new[it] = 0
        static_lens.copy_(torch.tensor(new, dtype=torch.int32))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = fp8_decode_attention(q, *caches, static_lens, tables, scale)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {it}"


def test_noalloc_decode_rejects_partials_over_the_limit():
    """Batch 256 x 32 splits at 32 q heads needs 135 MB of partials."""
    lib = _lib.load()
    splits = decode_num_splits(256, 32, 8, 128, H.BLOCK)
    need = lib.mskv_decode_workspace_bytes(256, 32, 8, 128, splits)
    assert need > SCRATCH_BYTES
    status = lib.mskv_fp8_decode_attention_noalloc(
        None, None, None, None, None, None, None, None, 256, 32, 8, 128, H.BLOCK, 40000, 128,
        0.088, _lib.BFLOAT16, splits, None)
    assert status == -3
    assert "workspace" in lib.mskv_status_string(status).decode()
