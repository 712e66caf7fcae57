"""Causal varlen attention over unquantized q/k/v: the fresh PREFILL of the
FP8-KV path (drop-in for the ``flash_attn_varlen_func`` call in
``microserve/layers/attention.py:49-55``), backed by the gfx950 HIP kernel
``mskv_prefill_attention``."""

from __future__ import annotations

import torch

from microserve_amd import _lib


def varlen_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int, max_seqlen_k: int | None = None,
    softmax_scale: float | None = None, causal: bool = True,
) -> torch.Tensor:
    """``flash_attn_varlen_func`` with ``causal=True`` on fp16/bf16 tensors.

    ``q`` is ``[total_q, H_q, D]``, ``k``/``v`` are ``[total_k, H_kv, D]``;
    sequence ``s`` owns rows ``cu_seqlens_q[s]:cu_seqlens_q[s+1]`` of ``q``
    and ``cu_seqlens_k[s]:cu_seqlens_k[s+1]`` of ``k``/``v``.  Query ``i``
    sees key ``j`` iff ``j <= i + Lk - Lq`` (the causal mask aligned to the
    bottom right, as flash-attn does); a row that sees no key is zero.
    ``max_seqlen_q`` is a host integer (the reference's ``Context`` field);
    ``max_seqlen_k`` is accepted for signature compatibility.  The
    probabilities are rounded to the input type for the PV product, with
    fp32 accumulation.
    """
    del max_seqlen_k
    assert causal, "only causal attention is provided (the path never calls it otherwise)"
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    cu_seqlens_k = cu_seqlens_k.contiguous()
    total_q, num_q_heads, head_dim = q.shape
    total_k, num_kv_heads = k.shape[0], k.shape[1]
    assert q.dtype in (torch.float16, torch.bfloat16)
    assert k.dtype == v.dtype == q.dtype
    assert k.shape == v.shape and k.shape[2] == head_dim
    assert num_q_heads % num_kv_heads == 0
    assert cu_seqlens_q.dtype == cu_seqlens_k.dtype == torch.int32
    num_seqs = cu_seqlens_q.numel() - 1
    assert cu_seqlens_k.numel() == num_seqs + 1
    _lib.on_device("varlen_attention", q, k, v, cu_seqlens_q, cu_seqlens_k)
    if softmax_scale is None:
        softmax_scale = head_dim ** -0.5
    out = torch.empty_like(q)
    if total_q == 0 or num_seqs == 0:
        return out
    lib = _lib.load()
    status = lib.mskv_prefill_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs,
        total_q, total_k, int(max_seqlen_q), num_q_heads, num_kv_heads,
        head_dim, float(softmax_scale), _lib.act_dtype(q), _lib.stream_of(q))
    _lib.check(status, "varlen_attention")
    return out


# the name the reference imports for this call (attention.py:4)
flash_attn_varlen_func = varlen_attention
