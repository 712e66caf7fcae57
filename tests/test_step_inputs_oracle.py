"""CPU checks that pin the step-input oracle (``oracle/step_inputs_oracle.py``)
and the host-side validation of the builder.  No GPU is needed."""

import numpy as np
import pytest

from oracle import step_inputs_oracle as SO
from tests.seqs import Seq, random_batch


def test_decode_hand_computed():
    bs = 4
    seqs = [Seq(range(10, 20), 9, 1, [7, 2, 5]),   # p=9 -> block 5, offset 1
            Seq(range(100, 104), 3, 1, [6]),       # p=3 -> block 6, offset 3
            Seq(range(40, 45), 4, 1, [1, 0])]      # p=4 -> block 0, offset 0
    d = SO.compile_decode(seqs, bs)
    assert d["input_ids"].tolist() == [19, 103, 44]
    assert d["positions"].tolist() == [9, 3, 4]
    assert d["slot_mapping"].tolist() == [21, 27, 0]
    assert d["cache_seqlens"].tolist() == [10, 4, 5]
    assert d["block_tables"].tolist() == [[7, 2, 5], [6, -1, -1], [1, 0, -1]]
    p = SO.pad_decode(d, 5, 4, 1000)
    assert p["slot_mapping"].tolist() == [21, 27, 0, 1000, 1000]
    assert p["cache_seqlens"].tolist() == [10, 4, 5, 0, 0]
    assert p["block_tables"].tolist() == [[7, 2, 5, -1], [6, -1, -1, -1], [1, 0, -1, -1],
                                          [-1] * 4, [-1] * 4]


def test_prefill_and_chunk_hand_computed():
    bs = 4
    d = SO.compile_prefill([Seq([1, 2, 3, 4, 5, 6], 0, 6, [3, 8]), Seq([9, 9], 0, 2, [0])], bs)
    assert d["slot_mapping"].tolist() == [12, 13, 14, 15, 32, 33, 0, 1]
    assert d["positions"].tolist() == [0, 1, 2, 3, 4, 5, 0, 1]
    assert d["input_ids"].tolist() == [1, 2, 3, 4, 5, 6, 9, 9]
    assert d["cu_seqlens_q"].tolist() == [0, 6, 8] and d["max_seqlen_q"] == 6
    c = SO.compile_chunk_prefill(Seq(range(20), 5, 4, [9, 4, 11]), bs)
    assert c["slot_mapping"].tolist() == [17, 18, 19, 44]
    assert c["positions"].tolist() == [5, 6, 7, 8]
    assert c["cu_seqlens_k"].tolist() == [0, 9] and c["cache_seqlens"].tolist() == [9]
    assert c["prefix_len"] == 5 and c["query_len"] == 4 and c["max_seqlen_k"] == 9


def test_empty_table_row_is_all_minus_one():
    bt = SO.make_block_tables([Seq([], 0, 0, []), Seq([], 0, 0, [3, 1])])
    assert bt.tolist() == [[-1, -1], [3, 1]]


@pytest.mark.parametrize("kind", ["decode", "prefill", "chunk"])
def test_slot_formula_matches_enumerated_slots(kind):
    """Brute force: list every slot of a table in order (block by block,
    offsets 0..bs-1) and index it by position."""
    rng = np.random.default_rng(3)
    bs = 16
    seqs = random_batch(rng, kind, 12, bs, 400, 200)
    if kind == "decode":
        d = SO.compile_decode(seqs, bs)
    elif kind == "prefill":
        d = SO.compile_prefill(seqs, bs)
    else:
        d = {k: np.concatenate([SO.compile_chunk_prefill(s, bs)[k] for s in seqs])
             for k in ("slot_mapping", "positions")}
    row = 0
    for s in seqs:
        full = [t * bs + o for t in s.block_table for o in range(bs)]
        for j in range(s.num_scheduled_tokens):
            p = s.num_computed_tokens + j
            assert d["positions"][row] == p
            assert d["slot_mapping"][row] == full[p]
            row += 1
    assert row == d["slot_mapping"].shape[0]


def test_builder_raises_like_the_reference_on_short_tables():
    from microserve_amd import step_inputs
    with pytest.raises(IndexError):
        step_inputs.build_step_inputs([Seq(range(9), 8, 1, [0, 1])], 4, "cpu")
    with pytest.raises(IndexError):
        step_inputs.build_step_inputs([Seq(range(5), 4, 2, [0, 1])], 4, "cpu")
    with pytest.raises(AssertionError):
        step_inputs.compile_decode([Seq(range(9), 7, 1, [0, 1])], 4, "cpu")  # gap 2


def _numpy_pack(seqs):
    """The staging layout written out with numpy: int64 token ids of the
    scheduled positions, then int32 first positions, cu_seqlens_q, table
    offsets and the concatenated tables."""
    ids = [t for s in seqs for t in s.token_ids[s.num_computed_tokens:
                                                 s.num_computed_tokens + s.num_scheduled_tokens]]
    ns = [s.num_scheduled_tokens for s in seqs]
    tl = [len(s.block_table) for s in seqs]
    parts = [np.asarray(ids, np.int64).tobytes(),
             np.asarray([s.num_computed_tokens for s in seqs], np.int32).tobytes(),
             np.concatenate([[0], np.cumsum(ns)]).astype(np.int32).tobytes(),
             np.concatenate([[0], np.cumsum(tl)]).astype(np.int32).tobytes(),
             np.asarray([b for s in seqs for b in s.block_table], np.int32).tobytes()]
    raw = b"".join(parts)
    return raw + bytes(max(0, 8 - len(raw)))


@pytest.mark.parametrize("kind", ["decode", "prefill", "chunk"])
def test_host_packer_layout(kind):
    """The packer's bytes and sizes equal the layout written out with numpy,
    on random batches, with tuple tables and an empty batch too."""
    from microserve_amd import _step_pack
    rng = np.random.default_rng(7)
    for n_seqs in (0, 1, 5, 64):
        seqs = random_batch(rng, kind, n_seqs, 16, 4096, 300)
        if n_seqs > 1:
            seqs[1].block_table = tuple(seqs[1].block_table)
        raw, total_q, max_q, ntab, max_tlen = _step_pack.pack(seqs, 16)
        assert raw == _numpy_pack(seqs), (kind, n_seqs)
        assert total_q == sum(s.num_scheduled_tokens for s in seqs)
        assert max_q == max((s.num_scheduled_tokens for s in seqs), default=0)
        assert ntab == sum(len(s.block_table) for s in seqs)
        assert max_tlen == max((len(s.block_table) for s in seqs), default=0)


def test_host_packer_errors():
    from microserve_amd import _step_pack
    with pytest.raises(IndexError, match="block_table"):
        _step_pack.pack([Seq(range(9), 8, 1, [0, 1])], 4)
    with pytest.raises(IndexError, match="token_ids"):
        _step_pack.pack([Seq(range(5), 4, 2, [0, 1])], 4)
    with pytest.raises(ValueError, match="negative"):
        _step_pack.pack([Seq(range(5), -1, 1, [0, 1])], 4)
    with pytest.raises(OverflowError):
        _step_pack.pack([Seq(range(5), 4, 1, [0, 1 << 40])], 4)
    with pytest.raises(AttributeError):
        _step_pack.pack([object()], 4)
