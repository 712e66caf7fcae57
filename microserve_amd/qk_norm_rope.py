"""Fused attention prologue: per-head q/k RMSNorm, rotary embedding and the
FP8 store of k and v in one kernel.

Replaces, in one launch, ``microserve/models/qwen3.py:49-53``::

    q = self.q_norm(q); k = self.k_norm(k)
    q, k = self.rotary_emb(positions, q, k)

and the ``store_fp8_kvcache`` call at the top of ``Attention.forward``
(``microserve/layers/attention.py:41-43``).  Arguments are the tensors those
modules hold: the norms' ``weight`` and ``eps`` (``layernorm.py:47-53``) and
the rotary ``cos_cache``/``sin_cache`` buffers (``rotary_embedding.py:21-22``),
in the activation type as the runner's ``.to(dtype)`` leaves them.
"""

from __future__ import annotations

import torch

from microserve_amd import _lib

__all__ = ["qk_norm_rope_store"]


def qk_norm_rope_store(positions, q, k, v, q_norm_weight, k_norm_weight, eps,
                       cos_cache, sin_cache, k_cache, v_cache, k_scale_cache,
                       v_scale_cache, slot_mapping, *, return_k: bool = True):
    """Returns ``(q_embed, k_embed)``: rotated (and, with weights, normalized)
    q and k as new contiguous ``[T, H, D]`` tensors; ``k_embed`` is None when
    ``return_k`` is false (decode and chunked prefill read k back from the
    cache).  k_embed and v are stored into the FP8 cache at
    ``slot_mapping``, byte-identical to ``store_fp8_kvcache(k_embed, v, ...)``.

    ``q``, ``k``, ``v`` may be strided views of the qkv projection (heads
    contiguous within a token).  ``q_norm_weight``/``k_norm_weight`` None
    skips the norm (models with a qkv bias).  A token whose position is
    outside the rotary tables gets zero outputs and is not stored (the
    reference's table lookup would raise there).
    """
    assert q.dim() == 3 and k.dim() == 3 and v.dim() == 3
    n, hq, d = q.shape
    hk = k.shape[1]
    assert k.shape == (n, hk, d) and v.shape == (n, hk, d), (q.shape, k.shape, v.shape)
    assert q.dtype == k.dtype == v.dtype, (q.dtype, k.dtype, v.dtype)
    dt = _lib.act_dtype(q)
    for name, t in (("q", q), ("k", k), ("v", v)):
        assert t.stride(2) == 1 and t.stride(1) == d, f"{name}: heads must be contiguous per token"
    assert (q_norm_weight is None) == (k_norm_weight is None)
    if q_norm_weight is not None:
        assert q_norm_weight.dtype == q.dtype and k_norm_weight.dtype == q.dtype
        q_norm_weight = q_norm_weight.contiguous()
        k_norm_weight = k_norm_weight.contiguous()
        assert q_norm_weight.numel() == d and k_norm_weight.numel() == d
    cos = cos_cache.reshape(-1, d)
    sin = sin_cache.reshape(-1, d)
    if cos.dtype != q.dtype:  # the reference's .to(dtype) at lookup time
        cos, sin = cos.to(q.dtype), sin.to(q.dtype)
    cos, sin = cos.contiguous(), sin.contiguous()
    assert cos.shape == sin.shape
    positions = positions.reshape(-1).to(torch.int64).contiguous()
    assert positions.numel() == n
    slot_mapping = slot_mapping.contiguous()
    assert slot_mapping.dtype in (torch.int32, torch.int64) and slot_mapping.numel() == n
    assert k_cache.dtype == torch.float8_e4m3fn and v_cache.dtype == torch.float8_e4m3fn
    assert k_cache.shape[2:] == (hk, d) and v_cache.shape == k_cache.shape
    assert k_scale_cache.shape == k_cache.shape[:-1] and v_scale_cache.shape == k_cache.shape[:-1]
    _lib.on_device("qk_norm_rope_store", q, k, v, positions, q_norm_weight, k_norm_weight,
                   cos, sin, k_cache, v_cache, k_scale_cache, v_scale_cache, slot_mapping)
    q_out = torch.empty(n, hq, d, dtype=q.dtype, device=q.device)
    k_out = torch.empty(n, hk, d, dtype=q.dtype, device=q.device) if return_k else None
    lib = _lib.load()
    _lib.check(lib.mskv_qk_norm_rope_store(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), v.stride(0),
        positions.data_ptr(),
        None if q_norm_weight is None else q_norm_weight.data_ptr(),
        None if k_norm_weight is None else k_norm_weight.data_ptr(), float(eps),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], q_out.data_ptr(),
        None if k_out is None else k_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        k_scale_cache.data_ptr(), v_scale_cache.data_ptr(), slot_mapping.data_ptr(),
        _lib.INT64 if slot_mapping.dtype == torch.int64 else _lib.INT32,
        n, hq, hk, d, k_cache.shape[0] * k_cache.shape[1], dt, _lib.stream_of(q)),
        "mskv_qk_norm_rope_store")
    return q_out, k_out
