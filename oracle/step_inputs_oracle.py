"""CPU restatement of the runner's per-step input builders (test infrastructure).

Only the tests, ``__graft_entry__.smoke()`` and the benchmark's CPU baseline
may use this module, and only as the checker.  The product path is
``microserve_amd.step_inputs`` over the HIP kernel ``step_inputs_kernel``.

Each function follows the reference loop it names, element by element, in
plain Python over lists, and returns numpy arrays:

* ``compile_decode``        -- ``ModelRunner._compile_decode``,
  ``microserve/engine/model_runner.py:124-142``
* ``compile_prefill``       -- ``ModelRunner._compile_prefill``, :144-172
* ``compile_chunk_prefill`` -- ``ModelRunner._compile_chunk_prefill``, :174-193
* ``make_block_tables``     -- ``ModelRunner._make_block_tables``, :208-216
* ``pad_decode``            -- the graph-buffer padding of
  ``ModelRunner._run_decode``, :264-272

Pinned by ``tests/test_oracle.py``: hand-computed cases (block boundaries,
empty tables, a chunk over a cached prefix, graph padding) and a brute-force
restatement of the slot formula that enumerates every slot of a table in
order and indexes it by position.
"""

from __future__ import annotations

import numpy as np


def _slot(table, p: int, block_size: int) -> int:
    # model_runner.py:135, 160, 182
    return table[p // block_size] * block_size + p % block_size


def make_block_tables(seqs) -> np.ndarray:
    """model_runner.py:208-216: -1-padded int32 [B, max table length]."""
    max_len = max(len(s.block_table) for s in seqs)
    bt = np.full((len(seqs), max_len), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        if s.block_table:
            bt[i, :len(s.block_table)] = s.block_table
    return bt


def compile_decode(seqs, block_size: int) -> dict:
    """model_runner.py:124-142."""
    bs = len(seqs)
    input_ids = np.empty(bs, np.int64)
    positions = np.empty(bs, np.int64)
    slot = np.empty(bs, np.int64)
    cache_seqlens = np.empty(bs, np.int32)
    for i, seq in enumerate(seqs):
        p = seq.num_computed_tokens
        assert seq.gap == 1 and seq.num_scheduled_tokens == 1
        input_ids[i] = seq.token_ids[p]
        positions[i] = p
        slot[i] = _slot(seq.block_table, p, block_size)
        cache_seqlens[i] = p + 1
    return {"input_ids": input_ids, "positions": positions, "slot_mapping": slot,
            "cache_seqlens": cache_seqlens, "block_tables": make_block_tables(seqs)}


def compile_prefill(seqs, block_size: int) -> dict:
    """model_runner.py:144-172."""
    bs = len(seqs)
    total_q = sum(s.num_scheduled_tokens for s in seqs)
    input_ids = np.empty(total_q, np.int64)
    positions = np.empty(total_q, np.int64)
    slot = np.empty(total_q, np.int64)
    cu_q = np.zeros(bs + 1, np.int32)
    max_q = 0
    off = 0
    for i, seq in enumerate(seqs):
        assert seq.num_computed_tokens == 0 and seq.gap > 1
        n = seq.num_scheduled_tokens
        for j in range(n):
            p = j
            input_ids[off + j] = seq.token_ids[p]
            positions[off + j] = p
            slot[off + j] = _slot(seq.block_table, p, block_size)
        cu_q[i + 1] = cu_q[i] + n
        max_q = max(max_q, n)
        off += n
    return {"input_ids": input_ids, "positions": positions, "slot_mapping": slot,
            "cu_seqlens_q": cu_q, "cu_seqlens_k": cu_q, "max_seqlen_q": max_q,
            "max_seqlen_k": max_q}


def compile_chunk_prefill(seq, block_size: int) -> dict:
    """model_runner.py:174-193."""
    start = seq.num_computed_tokens
    n = seq.num_scheduled_tokens
    assert start > 0 and seq.gap > 1 and n > 0
    input_ids = np.empty(n, np.int64)
    positions = np.empty(n, np.int64)
    slot = np.empty(n, np.int64)
    for j in range(n):
        p = start + j
        input_ids[j] = seq.token_ids[p]
        positions[j] = p
        slot[j] = _slot(seq.block_table, p, block_size)
    return {"input_ids": input_ids, "positions": positions, "slot_mapping": slot,
            "block_tables": make_block_tables([seq]),
            "cache_seqlens": np.array([start + n], np.int32),
            "prefix_len": start, "query_len": n,
            "cu_seqlens_q": np.array([0, n], np.int32),
            "cu_seqlens_k": np.array([0, start + n], np.int32),
            "max_seqlen_q": n, "max_seqlen_k": start + n}


def pad_decode(d: dict, pad_to: int, table_width: int, garbage_slot: int) -> dict:
    """model_runner.py:264-272: the rows a captured graph of batch ``pad_to``
    sees.  Slots of padding rows are the garbage slot, their lengths 0, their
    table rows -1; input ids and positions of padding rows are 0 here (the
    reference leaves stale values there, which no output depends on)."""
    bs = d["slot_mapping"].shape[0]
    out = {
        "input_ids": np.zeros(pad_to, np.int64),
        "positions": np.zeros(pad_to, np.int64),
        "slot_mapping": np.full(pad_to, garbage_slot, np.int64),
        "cache_seqlens": np.zeros(pad_to, np.int32),
        "block_tables": np.full((pad_to, table_width), -1, np.int32),
    }
    out["input_ids"][:bs] = d["input_ids"]
    out["positions"][:bs] = d["positions"]
    out["slot_mapping"][:bs] = d["slot_mapping"]
    out["cache_seqlens"][:bs] = d["cache_seqlens"]
    w = d["block_tables"].shape[1]
    out["block_tables"][:bs, :w] = d["block_tables"]
    return out
