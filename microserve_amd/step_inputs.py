"""Device-side builder of one step's attention inputs.

Drop-in for the context builders of ``microserve/engine/model_runner.py``:
``compile_decode`` (``_compile_decode``, :124-142), ``compile_prefill``
(``_compile_prefill``, :144-172), ``compile_chunk_prefill``
(``_compile_chunk_prefill``, :174-193) and ``make_block_tables``
(``_make_block_tables``, :208-216), with the same asserts, the same
``Context`` fields and the same return tuples.  ``compile_decode`` also takes
the graph padding of ``_run_decode`` (:264-272): with ``pad_to`` rows it
writes the garbage slot, zero lengths and -1 tables of the padding rows, and
with ``out`` it writes into the caller's fixed graph buffers.

The reference writes every element with its own host-to-device copy.  Here
the per-sequence state (scheduled token ids, first positions, token and table
offsets, concatenated block tables) is packed by the host extension
``microserve_amd._step_pack`` (``csrc/host/step_pack.cpp``) in one pass over
the sequences' lists, copied once through a pinned buffer, and
``mskv_build_step_inputs`` expands it on the GPU.
Sequences are duck-typed: anything with ``token_ids``,
``num_computed_tokens``, ``num_scheduled_tokens``, ``block_table`` and
``gap`` (``microserve/engine/sequence.py:19-50``).
"""

from __future__ import annotations

import numpy as np
import torch

from microserve_amd import _lib
from microserve_amd.context import AttentionMode, Context

try:
    from microserve_amd import _step_pack
except ImportError as e:  # pragma: no cover - raised on use, with the build command
    raise ImportError("microserve_amd._step_pack is not built: run "
                      "`python -m microserve_amd.build`") from e

__all__ = ["compile_decode", "compile_prefill", "compile_chunk_prefill",
           "make_block_tables", "build_step_inputs"]


def build_step_inputs(seqs, block_size: int, device, *, pad_to: int | None = None,
                      table_width: int | None = None, garbage_slot: int = -1,
                      with_tables: bool = True, out: dict | None = None) -> dict:
    """Expand ``seqs`` (scheduled positions ``num_computed_tokens`` ..
    ``+ num_scheduled_tokens``) into device tensors.

    Returns a dict with ``input_ids``, ``positions``, ``slot_mapping`` (int64,
    one row per scheduled token plus one per padding row), ``cache_seqlens``
    (int32 [pad_to]), ``block_tables`` (int32 [pad_to, table_width], -1
    padded; absent when ``with_tables`` is false), ``cu_seqlens_q`` (int32
    [len(seqs) + 1]) and the host ints ``total_q`` / ``max_seqlen_q``.

    Raises IndexError where the reference's list indexing would: a scheduled
    position past the sequence's tokens or past its block table.
    """
    dev = torch.device(device)
    nseq = len(seqs)
    pad = nseq if pad_to is None else int(pad_to)
    if pad < nseq:
        raise ValueError(f"pad_to={pad} is smaller than the batch ({nseq})")
    # staging: int64 token ids, then int32 starts | cu_q | table offsets | tables
    packed, total_q, max_q, _, max_tlen = _step_pack.pack(seqs, block_size)
    width = max_tlen if table_width is None else int(table_width)
    if width < max_tlen:
        raise ValueError(f"table_width={width} is narrower than a block table")
    o_tok = 0
    o_start = 8 * total_q
    o_cu = o_start + 4 * nseq
    o_toff = o_cu + 4 * (nseq + 1)
    o_tab = o_toff + 4 * (nseq + 1)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    host = torch.empty(len(packed), dtype=torch.uint8, pin_memory=True)
    host.numpy()[:] = np.frombuffer(packed, np.uint8)
    staged = torch.empty(host.numel(), dtype=torch.uint8, device=dev)
    staged.copy_(host, non_blocking=True)

    rows = total_q + (pad - nseq)
    if out is None:
        i64 = torch.empty(3, max(rows, 1), dtype=torch.int64, device=dev)
        i32 = torch.empty(pad + (pad * width if with_tables else 0), dtype=torch.int32,
                          device=dev)
        res = {"input_ids": i64[0, :rows], "positions": i64[1, :rows],
               "slot_mapping": i64[2, :rows], "cache_seqlens": i32[:pad]}
        if with_tables:
            res["block_tables"] = i32[pad:].view(pad, width)
    else:
        res = {}
        for name, dt, n in (("input_ids", torch.int64, rows), ("positions", torch.int64, rows),
                            ("slot_mapping", torch.int64, rows),
                            ("cache_seqlens", torch.int32, pad)):
            t = out[name]
            assert t.dtype == dt and t.is_contiguous() and t.device == dev and t.numel() >= n, name
            res[name] = t[:n]
        if with_tables:
            t = out["block_tables"]
            assert (t.dtype == torch.int32 and t.is_contiguous() and t.device == dev
                    and t.dim() == 2 and t.size(1) == width and t.size(0) >= pad), "block_tables"
            res["block_tables"] = t[:pad]
    if pad:
        lib = _lib.load()
        _lib.check(lib.mskv_build_step_inputs(
            staged.data_ptr() + o_tok, staged.data_ptr() + o_start,
            staged.data_ptr() + o_cu, staged.data_ptr() + o_toff,
            staged.data_ptr() + o_tab, nseq, pad, total_q, block_size, width,
            int(garbage_slot), res["input_ids"].data_ptr(), res["positions"].data_ptr(),
            res["slot_mapping"].data_ptr(), res["cache_seqlens"].data_ptr(),
            res["block_tables"].data_ptr() if with_tables else None, max_q,
            torch.cuda.current_stream(dev).cuda_stream), "mskv_build_step_inputs")
    res["cu_seqlens_q"] = staged[o_cu:o_toff].view(torch.int32)
    res["total_q"] = total_q
    res["max_seqlen_q"] = max_q
    return res


class _TableOnly:
    """A sequence reduced to its block table (no scheduled tokens)."""
    __slots__ = ("block_table",)
    token_ids = ()
    num_computed_tokens = 0
    num_scheduled_tokens = 0

    def __init__(self, block_table):
        self.block_table = block_table


def make_block_tables(seqs, device) -> torch.Tensor:
    """int32 [len(seqs), max table length], -1 padded (model_runner.py:208-216)."""
    return build_step_inputs([_TableOnly(s.block_table) for s in seqs], 1,
                             device)["block_tables"]


def compile_decode(seqs, block_size: int, device, *, pad_to: int | None = None,
                   table_width: int | None = None, garbage_slot: int | None = None,
                   out: dict | None = None):
    """One token per sequence at position ``num_computed_tokens``
    (model_runner.py:124-142); returns ``(ctx, input_ids, positions)``.

    With ``pad_to`` (a captured graph's batch) the ``pad_to - len(seqs)``
    padding rows get ``garbage_slot``, length 0 and -1 tables
    (model_runner.py:264-272), and the returned tensors have ``pad_to`` rows.
    """
    for seq in seqs:
        assert seq.gap == 1 and seq.num_scheduled_tokens == 1
    if pad_to is not None and pad_to > len(seqs) and garbage_slot is None:
        raise ValueError("padding rows need the garbage slot (num_blocks * block_size)")
    r = build_step_inputs(seqs, block_size, device, pad_to=pad_to, table_width=table_width,
                          garbage_slot=-1 if garbage_slot is None else garbage_slot, out=out)
    ctx = Context(mode=AttentionMode.DECODE, slot_mapping=r["slot_mapping"],
                  cache_seqlens=r["cache_seqlens"], block_tables=r["block_tables"])
    return ctx, r["input_ids"], r["positions"]


def compile_prefill(seqs, block_size: int, device):
    """Fresh prompts, positions 0 .. n-1 (model_runner.py:144-172); returns
    ``(ctx, cu_q, input_ids, positions)``."""
    for seq in seqs:
        assert seq.num_computed_tokens == 0 and seq.gap > 1
    r = build_step_inputs(seqs, block_size, device, with_tables=False)
    cu_q = r["cu_seqlens_q"]
    ctx = Context(mode=AttentionMode.PREFILL, cu_seqlens_q=cu_q, cu_seqlens_k=cu_q,
                  max_seqlen_q=r["max_seqlen_q"], max_seqlen_k=r["max_seqlen_q"],
                  slot_mapping=r["slot_mapping"])
    return ctx, cu_q, r["input_ids"], r["positions"]


def compile_chunk_prefill(seq, block_size: int, device):
    """One sequence's next chunk over its cached prefix
    (model_runner.py:174-193); returns ``(ctx, input_ids, positions)``."""
    start = seq.num_computed_tokens
    n = seq.num_scheduled_tokens
    assert start > 0 and seq.gap > 1 and n > 0
    r = build_step_inputs([seq], block_size, device)
    dev = torch.device(device)
    cu_k = torch.tensor([0, start + n], dtype=torch.int32).pin_memory().to(dev, non_blocking=True)
    ctx = Context(mode=AttentionMode.CHUNK_PREFILL, slot_mapping=r["slot_mapping"],
                  block_tables=r["block_tables"], cache_seqlens=r["cache_seqlens"],
                  prefix_len=start, query_len=n, cu_seqlens_q=r["cu_seqlens_q"],
                  cu_seqlens_k=cu_k, max_seqlen_q=n, max_seqlen_k=start + n)
    return ctx, r["input_ids"], r["positions"]
