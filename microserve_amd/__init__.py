"""MI355X-native FP8 paged-KV hot path of microserve.

Drop-in replacements for ``microserve.layers.fp8_kv_cache``,
``fp8_decode_attention``, ``fp8_chunk_prefill_attention``, the fresh-prefill
``flash_attn_varlen_func`` call,
``layers.attention.Attention`` (FP8 branch), ``utils.context``, the runner's
step-input builders (``step_inputs``) and the fused q/k norm + rotary + store
prologue (``qk_norm_rope_store``), backed by
hand-written gfx950 HIP kernels behind the C ABI in ``include/mskv.h``.
"""

from microserve_amd.context import (  # noqa: F401
    AttentionMode, Context, get_context, reset_context, set_context)
from microserve_amd.fp8_kv_cache import store_fp8_kvcache  # noqa: F401
from microserve_amd.fp8_decode_attention import (  # noqa: F401
    decode_num_splits, fp8_decode_attention)
from microserve_amd.fp8_chunk_prefill_attention import (  # noqa: F401
    fp8_chunk_prefill_attention, fp8_varlen_prefill_attention)
from microserve_amd.varlen_attention import (  # noqa: F401
    flash_attn_varlen_func, varlen_attention)
from microserve_amd.qk_norm_rope import qk_norm_rope_store  # noqa: F401
from microserve_amd.attention import Attention  # noqa: F401
