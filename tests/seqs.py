"""A stand-in for the runner's Sequence (``microserve/engine/sequence.py:19-50``):
the attributes the step-input builders read, and ``gap`` as the reference
defines it (tokens known, speculative ones included, minus tokens computed)."""

from __future__ import annotations


class Seq:
    def __init__(self, token_ids, num_computed_tokens, num_scheduled_tokens, block_table,
                 num_tokens_with_spec=None):
        self.token_ids = list(token_ids)
        self.num_computed_tokens = num_computed_tokens
        self.num_scheduled_tokens = num_scheduled_tokens
        self.block_table = list(block_table)
        self.num_tokens_with_spec = (len(self.token_ids) if num_tokens_with_spec is None
                                     else num_tokens_with_spec)

    @property
    def gap(self) -> int:
        return self.num_tokens_with_spec - self.num_computed_tokens


def decode_seq(ctx_len, table, first_token=0):
    """A sequence about to decode its token at position ctx_len - 1."""
    return Seq(range(first_token, first_token + ctx_len), ctx_len - 1, 1, table)


def random_batch(rng, kind, n_seqs, block_size, pool, max_len, vocab=151936):
    """Seeded sequences with tables drawn without replacement from a pool of
    ``pool`` blocks.  kind: "decode" (one scheduled token at the end),
    "prefill" (a fresh prompt), "chunk" (a chunk after a cached prefix)."""
    perm = rng.permutation(pool)
    at = 0
    seqs = []
    for _ in range(n_seqs):
        length = int(rng.integers(2, max_len + 1))
        pages = -(-length // block_size)
        table = [int(x) for x in perm[at:at + pages]]
        at += pages
        toks = [int(x) for x in rng.integers(0, vocab, length)]
        if kind == "decode":
            seqs.append(Seq(toks, length - 1, 1, table))
        elif kind == "prefill":
            seqs.append(Seq(toks, 0, length, table))
        else:
            start = int(rng.integers(1, length))
            seqs.append(Seq(toks, start, length - start, table, num_tokens_with_spec=length + 1))
    return seqs
