"""ctypes binding of the mskv C ABI (``include/mskv.h``).

The library is ``microserve_amd/libmskv.so``, built in-tree by
``python -m microserve_amd.build``.  There is no fallback: if the library is
missing or cannot be loaded every entry point raises, so a GPU run can never
silently take another path.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmskv.so")

FLOAT16 = 0
BFLOAT16 = 1
FLOAT32 = 2  # key/value rows of the store only
INT32 = 0
INT64 = 1

_c_int, _c_i64, _c_f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/mskv.h
_PROTOS = {
    "mskv_version": (_c_int, []),
    "mskv_status_string": (ctypes.c_char_p, [_c_int]),
    "mskv_store_fp8_kvcache": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
        _c_i64, _c_int, _c_int, _c_i64, _c_int, _vp]),
    "mskv_decode_num_splits": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "mskv_decode_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "mskv_fp8_decode_attention": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_f32,
        _c_int, _c_int, _vp, _c_size, _vp]),
    "mskv_fp8_decode_attention_noalloc": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_f32,
        _c_int, _c_int, _vp]),
    "mskv_fp8_prefill_attention": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
        _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_i64,
        _c_int, _c_f32, _c_int, _vp]),
    "mskv_prefill_attention": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_i64, _c_int,
        _c_int, _c_int, _c_int, _c_f32, _c_int, _vp]),
    "mskv_build_step_inputs": (_c_int, [
        _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_i64, _c_int, _c_int, _c_i64,
        _vp, _vp, _vp, _vp, _vp, _c_int, _vp]),
    "mskv_qk_norm_rope_store": (_c_int, [
        _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_f32, _vp, _vp, _c_i64,
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_i64,
        _c_int, _vp]),
}

EXPORTED = tuple(_PROTOS)

_lib = None


def load() -> ctypes.CDLL:
    """Load libmskv.so once; raise with a build hint if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"mskv HIP library not found at {LIB_PATH}; build it with "
            "`python -m microserve_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status, as the reference's launcher would."""
    if status != 0:
        msg = load().mskv_status_string(status).decode()
        raise RuntimeError(f"{what} failed: status {status} ({msg})")


def act_dtype(t) -> int:
    import torch
    if t.dtype == torch.float16:
        return FLOAT16
    if t.dtype == torch.bfloat16:
        return BFLOAT16
    raise AssertionError(f"activation dtype must be float16 or bfloat16, got {t.dtype}")


def store_dtype(t) -> int:
    """Element type of the store's key/value rows: fp16, bf16 or fp32 (the
    reference upcasts any float input to fp32, fp8_kv_cache.py:22-23)."""
    import torch
    if t.dtype == torch.float32:
        return FLOAT32
    if t.dtype in (torch.float16, torch.bfloat16):
        return act_dtype(t)
    raise AssertionError(f"key/value dtype must be float16, bfloat16 or float32, got {t.dtype}")


def on_device(what: str, ref, *tensors) -> None:
    """Every tensor argument must live on ``ref``'s GPU: a kernel handed a
    host pointer faults instead of raising, so mixed placement is rejected
    here (AssertionError, like the reference's argument checks)."""
    assert ref.is_cuda, f"{what} runs on the GPU"
    for t in tensors:
        if t is not None:
            assert t.device == ref.device, (
                f"{what}: every tensor must be on {ref.device}, got one on {t.device}")


def stream_of(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream
