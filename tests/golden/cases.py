"""Seeded inputs of the reference kernel test's two known-answer cases.

``tests/test_fp8_kv_attention.py:39-73`` (decode: lengths [1, 73, 300],
tables [[0,1],[2,3],[4,5]], K/V/Q ``randn * 0.2`` fp16, H_q 16, H_kv 8,
D 128, block 256) and ``:76-108`` (chunk prefill: prefix 273, 31 queries,
table [[1,0]], K and Q ``randn * 0.2``, V unscaled ``randn``).  The
reference draws on the CUDA generator; these draw on a seeded CPU generator,
which gives the same tensors on every machine with this torch build.
"""

import torch

BLOCK, QH, KVH, D = 256, 16, 8, 128


def decode_case():
    g = torch.Generator().manual_seed(1)
    lengths = [1, 73, 300]
    tables = torch.tensor([[0, 1], [2, 3], [4, 5]], dtype=torch.int32)
    keys, values, slots = [], [], []
    for b, n in enumerate(lengths):
        keys.append((torch.randn(n, KVH, D, generator=g) * 0.2).half())
        values.append((torch.randn(n, KVH, D, generator=g) * 0.2).half())
        for p in range(n):
            slots.append(int(tables[b, p // BLOCK]) * BLOCK + p % BLOCK)
    query = (torch.randn(len(lengths), QH, D, generator=g) * 0.2).half()
    return dict(key=torch.cat(keys), value=torch.cat(values),
                slots=torch.tensor(slots, dtype=torch.int64), query=query,
                lengths=lengths, tables=tables, num_blocks=6)


def chunk_case():
    g = torch.Generator().manual_seed(2)
    prefix, lq = 273, 31
    total = prefix + lq
    table = torch.tensor([[1, 0]], dtype=torch.int32)
    key = (torch.randn(total, KVH, D, generator=g) * 0.2).half()
    value = torch.randn(total, KVH, D, generator=g).half()
    slots = torch.tensor([int(table[0, p // BLOCK]) * BLOCK + p % BLOCK
                          for p in range(total)], dtype=torch.int64)
    query = (torch.randn(lq, QH, D, generator=g) * 0.2).half()
    return dict(key=key, value=value, slots=slots, query=query,
                prefix=prefix, table=table, num_blocks=2)
