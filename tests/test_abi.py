"""CPU checks of the C ABI: the library loads, exports every symbol that
include/mskv.h declares, and rejects bad arguments before touching a GPU."""

import ctypes
import os
import re

import pytest

from microserve_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mskv.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mskv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert _declared() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert getattr(lib, name) is not None
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(raw, name), name


def test_status_strings_and_version():
    lib = _lib.load()
    assert lib.mskv_version() >= 100
    assert lib.mskv_status_string(0) == b"ok"
    for code in (-1, -2, -3, 1):
        assert lib.mskv_status_string(code)


def test_split_policy_depends_on_shapes_only():
    lib = _lib.load()
    # Qwen3-8B decode, batch 64 x 4096 tokens: 16 pages per sequence
    s = lib.mskv_decode_num_splits(64, 32, 8, 16, 256)
    assert 1 < s <= 16
    assert lib.mskv_decode_num_splits(64, 32, 8, 16, 256) == s
    # long single sequence is split across many waves, at most 4 pages each
    s = lib.mskv_decode_num_splits(1, 64, 8, 512, 256)
    assert s >= 128
    # a huge batch needs no split
    assert lib.mskv_decode_num_splits(4096, 32, 8, 4, 256) == 1
    assert lib.mskv_decode_workspace_bytes(64, 32, 8, 128, 1) == 0
    assert lib.mskv_decode_workspace_bytes(64, 32, 8, 128, 8) == 64 * 32 * 8 * 129 * 4
    # 256 x 31 splits runs longest-first work items: the partials (padded to
    # 256 bytes), a 16-byte item count, then 16 bytes per (sequence, split)
    part = (256 * 32 * 31 * 129 * 4 + 255) // 256 * 256
    assert lib.mskv_decode_workspace_bytes(256, 32, 8, 128, 31) == part + 16 + 256 * 31 * 16


def test_argument_validation_without_launch():
    lib = _lib.load()
    EINVAL, EUNSUP, EWS = -1, -2, -3
    # unsupported head_dim
    assert lib.mskv_store_fp8_kvcache(1, 1, 1, 1, 1, 1, 1, 1, 4, 8, 64, 100, 1, None) == EUNSUP
    # bad dtype codes
    assert lib.mskv_store_fp8_kvcache(1, 1, 1, 1, 1, 1, 1, 7, 4, 8, 128, 100, 1, None) == EINVAL
    assert lib.mskv_store_fp8_kvcache(1, 1, 1, 1, 1, 1, 1, 1, 4, 8, 128, 100, 9, None) == EINVAL
    # zero tokens is a no-op
    assert lib.mskv_store_fp8_kvcache(None, None, None, None, None, None, None, 1, 0, 8, 128, 100, 1, None) == 0
    # null pointer with work to do
    assert lib.mskv_store_fp8_kvcache(None, 1, 1, 1, 1, 1, 1, 1, 4, 8, 128, 100, 1, None) == EINVAL
    # decode: heads not divisible, block size not a multiple of 32
    args = [1] * 8
    assert lib.mskv_fp8_decode_attention(*args, 2, 30, 8, 128, 256, 10, 4, 0.1, 1, 1, None, 0, None) == EINVAL
    assert lib.mskv_fp8_decode_attention(*args, 2, 32, 8, 128, 48, 10, 4, 0.1, 1, 1, None, 0, None) == EUNSUP
    # decode: any GQA divisor is accepted (group 24: the last 16-head unit of
    # each kv head is partly idle); with the right split count the call gets
    # past the shape checks to the workspace check
    s24 = lib.mskv_decode_num_splits(2, 48, 2, 4, 256)
    assert s24 > 1
    assert lib.mskv_fp8_decode_attention(*args, 2, 48, 2, 128, 256, 10, 4, 0.1, 1, s24, None, 0, None) == EWS
    # store: fp32 key/value rows are accepted (zero tokens: a no-op)
    assert lib.mskv_store_fp8_kvcache(None, None, None, None, None, None, None, 1, 0, 8, 128, 100, _lib.FLOAT32, None) == 0
    assert lib.mskv_store_fp8_kvcache(1, 1, 1, 1, 1, 1, 1, 1, 4, 8, 128, 100, 3, None) == EINVAL
    # decode: wrong split count, missing workspace
    s = lib.mskv_decode_num_splits(2, 32, 8, 4, 256)
    assert lib.mskv_fp8_decode_attention(*args, 2, 32, 8, 128, 256, 10, 4, 0.1, 1, s + 1, None, 0, None) == EINVAL
    if s > 1:
        assert lib.mskv_fp8_decode_attention(*args, 2, 32, 8, 128, 256, 10, 4, 0.1, 1, s, None, 0, None) == EWS
    # prefill: only one of the two cu_seqlens pointers
    assert lib.mskv_fp8_prefill_attention(1, 1, 1, 1, 1, 1, 1, None, 0, 1, 2, 10, 5, 32, 8, 128, 256, 10, 4, 0.1, 1, None) == EINVAL
    # prefill: block size not a multiple of 128
    assert lib.mskv_fp8_prefill_attention(1, 1, 1, 1, 1, 1, None, None, 0, 1, 1, 10, 10, 32, 8, 128, 64, 10, 4, 0.1, 1, None) == EUNSUP
    # prefill: more query blocks than a grid dimension holds (GQA 16: 8 tokens per block)
    big_q = 8 * 65535 + 1
    assert lib.mskv_fp8_prefill_attention(1, 1, 1, 1, 1, 1, None, None, 0, 1, 1, big_q, big_q, 128, 8, 128, 256, 10, 4, 0.1, 1, None) == EUNSUP
    assert lib.mskv_prefill_attention(1, 1, 1, 1, 1, 1, 1, big_q, big_q, 4 * 65535 * 48 + 1, 32, 8, 128, 0.1, 1, None) == EUNSUP
    # prefills: the row maxima are taken before a positive, finite softmax scale
    for sc in (0.0, -0.1, float("nan"), float("inf"), 3e38):
        assert lib.mskv_fp8_prefill_attention(1, 1, 1, 1, 1, 1, None, None, 0, 1, 1, 10, 10, 32, 8, 128, 256, 10, 4, sc, 1, None) == EUNSUP
        assert lib.mskv_prefill_attention(1, 1, 1, 1, 1, 1, 1, 10, 10, 10, 32, 8, 128, sc, 1, None) == EUNSUP


def test_new_entry_points_validate_without_launch():
    lib = _lib.load()
    EINVAL, EUNSUP = -1, -2
    A = 1 << 20  # a 16-byte aligned stand-in address; nothing is launched
    # fused prologue: args before (q, k, v, strides, positions, weights, eps, cos, sin, maxpos)
    def nr(head_dim=128, qw=A, kw=A, q=A, qs=48 * 128, n=4, eps=1e-6, slot_dtype=1, act=1):
        return lib.mskv_qk_norm_rope_store(
            q, A, A, qs, 48 * 128, 48 * 128, A, qw, kw, eps, A, A, 4096, A, None, A, A, A, A, A,
            slot_dtype, n, 32, 8, head_dim, 1 << 16, act, None)
    assert nr(head_dim=64) == EUNSUP
    assert nr(kw=None) == EINVAL            # one weight without the other
    assert nr(q=A + 8) == EINVAL            # q not 16-byte aligned
    assert nr(qs=32 * 128 - 8) == EINVAL    # token stride shorter than the q heads
    assert nr(eps=-1.0) == EINVAL
    assert nr(slot_dtype=5) == EINVAL
    assert nr(act=3) == EINVAL
    assert nr(n=0) == 0                     # nothing to do
    # step inputs: (token_ids, starts, cu_q, table_off, tables, num_seqs, pad_seqs, total_q,
    #               block_size, table_width, garbage, ids, pos, slot, lens, tables_out, max_q)
    def si(num_seqs=2, pad=2, total_q=3, bs=256, width=4, ids=A, max_q=2):
        return lib.mskv_build_step_inputs(A, A, A, A, A, num_seqs, pad, total_q, bs, width, 0,
                                          ids, A, A, A, A, max_q, None)
    assert si(pad=1) == EINVAL              # fewer padded rows than sequences
    assert si(bs=0) == EINVAL
    assert si(width=-1) == EINVAL
    assert si(ids=None) == EINVAL           # rows to write but no output
    assert si(num_seqs=70000, pad=70000) == EUNSUP  # grid y limit
    assert si(num_seqs=0, pad=0, total_q=0) == 0


def test_python_wrappers_reject_like_the_reference():
    torch = pytest.importorskip("torch")
    from microserve_amd import fp8_decode_attention, store_fp8_kvcache
    kc = torch.zeros(2, 256, 8, 128, dtype=torch.float8_e4m3fn)
    ks = torch.ones(2, 256, 8)
    k = torch.zeros(3, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):       # wrong scale dtype
        store_fp8_kvcache(k, k, kc, kc, ks.double(), ks.double(), torch.zeros(3, dtype=torch.int64))
    with pytest.raises(AssertionError):       # wrong head_dim layout
        store_fp8_kvcache(k[..., :64], k[..., :64], kc, kc, ks, ks, torch.zeros(3, dtype=torch.int64))
    q = torch.zeros(2, 16, 128, dtype=torch.float32)
    with pytest.raises(AssertionError):       # fp32 query
        fp8_decode_attention(q, kc, kc, ks, ks, torch.ones(2, dtype=torch.int32),
                             torch.zeros(2, 1, dtype=torch.int32), 0.1)
    with pytest.raises(AssertionError):       # int64 lengths
        fp8_decode_attention(q.bfloat16(), kc, kc, ks, ks, torch.ones(2, dtype=torch.int64),
                             torch.zeros(2, 1, dtype=torch.int32), 0.1)


def test_wrappers_reject_tensors_off_the_gpu():
    """A host tensor among GPU arguments is rejected before any launch (a
    kernel given a host pointer would fault).  Checked with CPU tensors only:
    the first check (the reference tensor on the GPU) already fails here."""
    import torch
    from microserve_amd import _lib as L
    with pytest.raises(AssertionError, match="runs on the GPU"):
        L.on_device("x", torch.zeros(1))
