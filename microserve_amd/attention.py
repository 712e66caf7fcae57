"""Paged attention layer (drop-in for the FP8 branch of
``microserve/layers/attention.py``).

The runner injects ``k_cache``/``v_cache`` (fp8 ``[NB+1, BS, H_kv, D]``
views), ``k_scale_cache``/``v_scale_cache`` (fp32 ``[NB+1, BS, H_kv]``) and
``kv_cache_dtype`` as plain attributes (``model_runner.py:111-122``).
``forward`` stores the step's K/V first and then attends, dispatching on the
global ``Context``'s mode (``attention.py:36-61``).  ``forward_fused`` does
the same from the un-normalized projection outputs, with the model's q/k
norms, rotary embedding and the store fused into one launch.
"""

from __future__ import annotations

import torch
from torch import nn

from microserve_amd.context import AttentionMode, get_context
from microserve_amd.fp8_chunk_prefill_attention import fp8_chunk_prefill_attention
from microserve_amd.fp8_decode_attention import fp8_decode_attention
from microserve_amd.fp8_kv_cache import store_fp8_kvcache
from microserve_amd.qk_norm_rope import qk_norm_rope_store
from microserve_amd.varlen_attention import varlen_attention


class Attention(nn.Module):
    """Paged attention over an injected FP8 KV cache."""

    def __init__(self, num_heads: int, head_dim: int, scale: float,
                 num_kv_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.k_scale_cache = self.v_scale_cache = None
        self.kv_cache_dtype = "fp8_e4m3"

    def _check_cache(self):
        assert self.k_cache.numel(), "k_cache was not injected: allocate the KV cache first"
        if self.kv_cache_dtype != "fp8_e4m3":
            # The fp16-cache branch (attention.py:63-85) runs on flash-attn
            # and is outside this library.
            raise NotImplementedError(
                f"kv_cache_dtype {self.kv_cache_dtype!r}: only the fp8_e4m3 path is provided")

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        self._check_cache()
        store_fp8_kvcache(k, v, self.k_cache, self.v_cache, self.k_scale_cache,
                          self.v_scale_cache, ctx.slot_mapping)
        return self._attend(ctx, q, k, v)

    def forward_fused(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, q_norm_weight, k_norm_weight, eps: float,
                      cos_cache: torch.Tensor, sin_cache: torch.Tensor) -> torch.Tensor:
        """The attention block of microserve/models/qwen3.py:49-54 from the
        projection's q/k/v views: q/k RMSNorm, rotary embedding and the FP8
        store in one launch (``qk_norm_rope_store``), then the same
        mode dispatch as ``forward``.  Pass None weights for models without
        the per-head norms."""
        ctx = get_context()
        self._check_cache()
        q, k_embed = qk_norm_rope_store(
            positions, q, k, v, q_norm_weight, k_norm_weight, eps, cos_cache, sin_cache,
            self.k_cache, self.v_cache, self.k_scale_cache, self.v_scale_cache,
            ctx.slot_mapping, return_k=ctx.mode is AttentionMode.PREFILL)
        return self._attend(ctx, q, k_embed, v)

    def _attend(self, ctx, q, k, v):
        k_cache, v_cache = self.k_cache, self.v_cache
        if ctx.mode is AttentionMode.DECODE:
            return fp8_decode_attention(
                q, k_cache, v_cache, self.k_scale_cache, self.v_scale_cache,
                ctx.cache_seqlens, ctx.block_tables, self.scale)
        if ctx.mode is AttentionMode.PREFILL:
            # fresh prefill attends over the unquantized new tokens, as the
            # reference's flash_attn_varlen_func call does (attention.py:49-55)
            return varlen_attention(
                q, k, v, cu_seqlens_q=ctx.cu_seqlens_q,
                cu_seqlens_k=ctx.cu_seqlens_k, max_seqlen_q=ctx.max_seqlen_q,
                max_seqlen_k=ctx.max_seqlen_k, softmax_scale=self.scale, causal=True)
        if ctx.mode is AttentionMode.CHUNK_PREFILL:
            return fp8_chunk_prefill_attention(
                q, k_cache, v_cache, self.k_scale_cache, self.v_scale_cache,
                ctx.block_tables, ctx.prefix_len, self.scale)
        raise RuntimeError(f"unsupported attention mode: {ctx.mode}")
