"""FP8 E4M3 paged KV-cache quantization and scatter (drop-in for
``microserve/layers/fp8_kv_cache.py``), backed by the gfx950 HIP kernel."""

from __future__ import annotations

import torch

from microserve_amd import _lib

FP8_MAX = 448.0


def store_fp8_kvcache(
    key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
    v_cache: torch.Tensor, k_scale_cache: torch.Tensor,
    v_scale_cache: torch.Tensor, slot_mapping: torch.Tensor,
) -> None:
    """Quantize ``key``/``value`` rows and write them at ``slot_mapping``.

    Same signature, assertions and in-place effect as the reference
    (``fp8_kv_cache.py:42-61``): per (token, kv head) the scale is
    ``max(amax, 1e-8) / 448`` and the bytes are
    ``e4m3fn(clamp(x / scale, -448, 448))``; token ``t`` lands at cache row
    ``slot_mapping[t]``.  ``key``/``value`` may be fp16, bf16 or fp32 (the
    reference upcasts any float to fp32, ``:22-23``); ``slot_mapping`` may be
    int32 or int64.
    """
    key = key.contiguous()
    value = value.contiguous()
    slot_mapping = slot_mapping.contiguous()
    num_tokens, num_kv_heads, head_dim = key.shape
    assert value.shape == key.shape
    assert value.dtype == key.dtype
    assert k_cache.dtype == v_cache.dtype == torch.float8_e4m3fn
    assert k_scale_cache.dtype == v_scale_cache.dtype == torch.float32
    assert k_cache.shape[2:] == (num_kv_heads, head_dim)
    assert v_cache.shape == k_cache.shape
    assert k_scale_cache.shape == k_cache.shape[:-1]
    assert v_scale_cache.shape == k_scale_cache.shape
    assert slot_mapping.dtype in (torch.int32, torch.int64)
    assert slot_mapping.numel() == num_tokens
    for t in (k_cache, v_cache, k_scale_cache, v_scale_cache):
        assert t.is_contiguous(), "caches must be contiguous"
    _lib.on_device("store_fp8_kvcache", key, value, k_cache, v_cache, k_scale_cache,
                   v_scale_cache, slot_mapping)
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    lib = _lib.load()
    status = lib.mskv_store_fp8_kvcache(
        key.data_ptr(), value.data_ptr(), k_cache.data_ptr(),
        v_cache.data_ptr(), k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        slot_mapping.data_ptr(),
        _lib.INT64 if slot_mapping.dtype == torch.int64 else _lib.INT32,
        num_tokens, num_kv_heads, head_dim, num_slots, _lib.store_dtype(key),
        _lib.stream_of(key))
    _lib.check(status, "store_fp8_kvcache")
