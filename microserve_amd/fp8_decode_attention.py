"""Decode attention over a paged FP8 E4M3 KV cache (drop-in for
``microserve/layers/fp8_decode_attention.py``), backed by the gfx950 HIP
split-KV kernel."""

from __future__ import annotations

import torch

from microserve_amd import _lib


# Per (device, stream), the split-partials scratch, grown on demand and
# reused by every call on that stream: calls on one stream (graph replays
# included) run one after another, so they never hold it at the same time,
# and calls on different streams each have their own, like the reference's
# call, which keeps no state between calls (fp8_decode_attention.py:93).
# The buffer is allocated on the stream that uses it (the caching allocator
# ties a block to the stream it was allocated on).  A graph captured before
# the scratch grew still addresses the old buffer, so a grown-out buffer is
# retired, never freed; growth at least doubles, so few exist.
_SCRATCH: dict = {}
_RETIRED: list = []


def _scratch(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device, stream)
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 16)
        if buf is not None:
            _RETIRED.append(buf)
            size = max(size, 2 * buf.numel())
        buf = torch.empty(size, dtype=torch.uint8, device=device)
        _SCRATCH[key] = buf
    return buf


_PLAN: dict = {}


def _plan(batch_size, num_q_heads, num_kv_heads, head_dim, max_num_blocks,
          block_size):
    """(splits, scratch bytes) for a shape, computed once per shape."""
    key = (batch_size, num_q_heads, num_kv_heads, head_dim, max_num_blocks, block_size)
    plan = _PLAN.get(key)
    if plan is None:
        lib = _lib.load()
        splits = int(lib.mskv_decode_num_splits(batch_size, num_q_heads, num_kv_heads,
                                                max_num_blocks, block_size))
        ws = int(lib.mskv_decode_workspace_bytes(batch_size, num_q_heads, num_kv_heads,
                                                 head_dim, splits))
        plan = _PLAN[key] = (splits, ws)
    return plan


def decode_num_splits(batch_size: int, num_q_heads: int, num_kv_heads: int,
                      max_num_blocks: int, block_size: int) -> int:
    """Split-KV partition count for a decode shape (shapes only)."""
    return int(_lib.load().mskv_decode_num_splits(
        batch_size, num_q_heads, num_kv_heads, max_num_blocks, block_size))


def fp8_decode_attention(
    query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    k_scale_cache: torch.Tensor, v_scale_cache: torch.Tensor,
    cache_seqlens: torch.Tensor, block_tables: torch.Tensor,
    softmax_scale: float, block_n: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode step: ``query`` ``[B, H_q, D]`` against the paged cache.

    Same signature, assertions and result as the reference
    (``fp8_decode_attention.py:62-101``), except that ``query`` may be fp16 or
    bf16 and ``block_n`` is accepted and ignored (the tile size is the
    kernel's).  The split-KV partition count depends only on shapes and the
    partials scratch is a persistent buffer per (device, stream), so the call
    can be captured in a HIP graph, and calls on different streams may run
    concurrently.
    ``out``, when given, receives the result instead of a new tensor.
    """
    del block_n
    query = query.contiguous()
    cache_seqlens = cache_seqlens.contiguous()
    block_tables = block_tables.contiguous()
    batch_size, num_q_heads, head_dim = query.shape
    num_kv_heads = k_cache.shape[2]
    block_size = k_cache.shape[1]
    max_num_blocks = block_tables.shape[1]
    assert query.dtype in (torch.float16, torch.bfloat16)
    assert k_cache.dtype == v_cache.dtype == torch.float8_e4m3fn
    assert k_scale_cache.dtype == v_scale_cache.dtype == torch.float32
    assert cache_seqlens.dtype == torch.int32
    assert block_tables.dtype == torch.int32
    assert num_q_heads % num_kv_heads == 0
    assert head_dim == k_cache.shape[3]
    assert block_tables.shape[0] == batch_size == cache_seqlens.numel()
    for t in (k_cache, v_cache, k_scale_cache, v_scale_cache):
        assert t.is_contiguous(), "caches must be contiguous"
    _lib.on_device("fp8_decode_attention", query, k_cache, v_cache, k_scale_cache,
                   v_scale_cache, cache_seqlens, block_tables, out)
    if out is None:
        out = torch.empty_like(query)
    else:
        assert out.shape == query.shape and out.dtype == query.dtype and out.is_contiguous()
    lib = _lib.load()
    splits, ws_bytes = _plan(batch_size, num_q_heads, num_kv_heads, head_dim,
                             max_num_blocks, block_size)
    stream = _lib.stream_of(query)
    ws = _scratch(query.device, stream, ws_bytes) if ws_bytes else None
    status = lib.mskv_fp8_decode_attention(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        cache_seqlens.data_ptr(), block_tables.data_ptr(), out.data_ptr(),
        batch_size, num_q_heads, num_kv_heads, head_dim, block_size,
        k_cache.shape[0], max_num_blocks, float(softmax_scale),
        _lib.act_dtype(query), splits,
        ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    _lib.check(status, "fp8_decode_attention")
    return out
