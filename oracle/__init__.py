"""CPU oracle for the FP8 paged-KV path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
path (``microserve_amd``) never imports it and fails loudly when its HIP
library is missing.
"""

from oracle.fp8_oracle import (  # noqa: F401
    E4M3_MAX,
    e4m3fn_decode,
    e4m3fn_encode,
    quantize_rows,
    store_fp8_kvcache,
    dequant_gather,
    decode_attention,
    decode_attention_loop,
    chunk_prefill_attention,
    varlen_prefill_attention,
    varlen_prefill_attention_loop,
)
