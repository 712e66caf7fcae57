"""Causal chunk / varlen prefill over a paged FP8 E4M3 KV cache (drop-in for
``microserve/layers/fp8_chunk_prefill_attention.py``), backed by the gfx950
FP8-MFMA HIP kernel."""

from __future__ import annotations

import torch

from microserve_amd import _lib


def _check_common(query, k_cache, v_cache, k_scale_cache, v_scale_cache):
    _, num_q_heads, head_dim = query.shape
    num_kv_heads = k_cache.shape[2]
    assert query.dtype in (torch.float16, torch.bfloat16)
    assert k_cache.dtype == v_cache.dtype == torch.float8_e4m3fn
    assert k_scale_cache.dtype == v_scale_cache.dtype == torch.float32
    assert num_q_heads % num_kv_heads == 0
    assert head_dim == k_cache.shape[3]
    for t in (k_cache, v_cache, k_scale_cache, v_scale_cache):
        assert t.is_contiguous(), "caches must be contiguous"
    _lib.on_device("prefill attention", query, k_cache, v_cache, k_scale_cache,
                   v_scale_cache)


def fp8_chunk_prefill_attention(
    query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    k_scale_cache: torch.Tensor, v_scale_cache: torch.Tensor,
    block_table: torch.Tensor, prefix_len: int, softmax_scale: float,
    block_m: int | None = None, block_n: int | None = None,
) -> torch.Tensor:
    """Single-sequence causal chunk prefill, the reference's signature.

    ``query`` ``[Lq, H_q, D]`` attends over ``prefix_len + Lq`` cached
    positions read through the flattened ``block_table``
    (``fp8_chunk_prefill_attention.py:70-109``); query ``i`` sees positions
    ``< prefix_len + i + 1``.  ``block_m``/``block_n`` are accepted and
    ignored.  QK^T runs as FP8 MFMA contractions (the query split into exact
    e4m3 parts, the K bytes as stored); PV runs on the fp16 MFMA, with V's
    bytes converted to fp16 exactly and fp16 probability weights, which at
    the same matrix-core time as two FP8 parts of P keeps 11 significant
    bits for every weight.
    """
    del block_m, block_n
    query = query.contiguous()
    block_table = block_table.contiguous().view(-1)
    query_len, num_q_heads, head_dim = query.shape
    _check_common(query, k_cache, v_cache, k_scale_cache, v_scale_cache)
    assert block_table.dtype == torch.int32
    _lib.on_device("fp8_chunk_prefill_attention", query, block_table)
    prefix_len = int(prefix_len)
    assert prefix_len >= 0
    output = torch.empty_like(query)
    if query_len == 0:
        return output
    lib = _lib.load()
    status = lib.mskv_fp8_prefill_attention(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        block_table.data_ptr(), None, None, prefix_len, output.data_ptr(),
        1, query_len, query_len, num_q_heads, k_cache.shape[2], head_dim,
        k_cache.shape[1], k_cache.shape[0], block_table.numel(),
        float(softmax_scale), _lib.act_dtype(query), _lib.stream_of(query))
    _lib.check(status, "fp8_chunk_prefill_attention")
    return output


def fp8_varlen_prefill_attention(
    query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
    k_scale_cache: torch.Tensor, v_scale_cache: torch.Tensor,
    block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor, max_seqlen_q: int, softmax_scale: float,
) -> torch.Tensor:
    """Varlen causal prefill with cached prefixes, in one launch.

    The batch the runner describes with ``cu_seqlens_q``/``cu_seqlens_k``
    (``model_runner.py:184-192``): sequence ``s`` owns query rows
    ``cu_seqlens_q[s]:cu_seqlens_q[s+1]`` and ``Lk = cu_seqlens_k[s+1] -
    cu_seqlens_k[s]`` cached positions (its new tokens included, since they
    are stored first); query ``i`` sees positions ``< Lk - Lq + i + 1``.
    ``block_tables`` is int32 ``[num_seqs, max_blocks]``.  ``max_seqlen_q``
    is a host integer, as in the reference's ``Context``.
    """
    query = query.contiguous()
    block_tables = block_tables.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    cu_seqlens_k = cu_seqlens_k.contiguous()
    total_q, num_q_heads, head_dim = query.shape
    _check_common(query, k_cache, v_cache, k_scale_cache, v_scale_cache)
    assert block_tables.dtype == cu_seqlens_q.dtype == cu_seqlens_k.dtype == torch.int32
    num_seqs = cu_seqlens_q.numel() - 1
    assert cu_seqlens_k.numel() == num_seqs + 1
    assert block_tables.dim() == 2 and block_tables.shape[0] == num_seqs
    _lib.on_device("fp8_varlen_prefill_attention", query, block_tables, cu_seqlens_q,
                   cu_seqlens_k)
    output = torch.empty_like(query)
    if total_q == 0 or num_seqs == 0:
        return output
    lib = _lib.load()
    status = lib.mskv_fp8_prefill_attention(
        query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        block_tables.data_ptr(), cu_seqlens_q.data_ptr(),
        cu_seqlens_k.data_ptr(), 0, output.data_ptr(), num_seqs, total_q,
        int(max_seqlen_q), num_q_heads, k_cache.shape[2], head_dim,
        k_cache.shape[1], k_cache.shape[0], block_tables.shape[1],
        float(softmax_scale), _lib.act_dtype(query), _lib.stream_of(query))
    _lib.check(status, "fp8_varlen_prefill_attention")
    return output
