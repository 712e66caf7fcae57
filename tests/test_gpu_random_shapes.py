"""Seeded random-shape parity sweeps of decode and varlen prefill against
the oracle: batch sizes, context and query lengths (zero included), GQA
groups 1-16 (5 and 6 among them, whose 16-row blocks are partly filled) and
block sizes 256/512 drawn from fixed seeds, so every run checks the same
cases."""

import random

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from tests import gpu_helpers as H
from microserve_amd import (decode_num_splits, fp8_decode_attention,
                            fp8_varlen_prefill_attention, store_fp8_kvcache)

pytestmark = pytest.mark.gpu

HEADS = [(16, 16), (16, 8), (32, 8), (64, 8), (32, 2), (16, 1), (48, 8), (40, 8)]


def _fill(gen, lens, hk, bs, dtype):
    nb = sum((n + bs - 1) // bs for n in lens) + 2
    tables, slots = H.paged_layout(gen, lens, nb, bs)
    n = slots.numel()
    caches = H.alloc_cache(nb, bs, hk)
    if n:
        key = H.randn(gen, (n, hk, H.D), dtype)
        value = H.randn(gen, (n, hk, H.D), dtype)
        store_fp8_kvcache(key.to(H.DEV), value.to(H.DEV), *caches, slots.to(H.DEV))
    return tables, caches


@pytest.mark.parametrize("case", range(12))
def test_decode_random_shapes(case):
    rng = random.Random(1000 + case)
    hq, hk = rng.choice(HEADS)
    bs = rng.choice([256, 512])
    dtype = rng.choice([torch.bfloat16, torch.float16])
    batch = rng.randint(1, 24)
    lens = [rng.choice([0, 1, rng.randint(1, 3000)]) for _ in range(batch)]
    print(f"decode case {case}: hq {hq} hk {hk} bs {bs} {dtype} lens {lens}", flush=True)
    gen = torch.Generator().manual_seed(2000 + case)
    tables, caches = _fill(gen, lens, hk, bs, dtype)
    query = H.randn(gen, (batch, hq, H.D), dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32)
    scale = H.D ** -0.5
    out = fp8_decode_attention(query.to(H.DEV), *caches, seqlens.to(H.DEV), tables.to(H.DEV), scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.decode_attention(query, kc, vc, ks, vs, seqlens, tables, scale)
    H.assert_attention_close(out, ref)


@pytest.mark.parametrize("case", range(6))
def test_decode_random_shapes_work_items(case):
    """Grids of over 512 eight-wave workgroups, so the pre-pass ranks the
    sequences and lists their splits as work items (8-wave workgroups, or
    4-wave ones when a kv head group has fewer than eight units): random
    batches with zero, one-token, short and long contexts, ties included."""
    rng = random.Random(5000 + case)
    hq, hk = HEADS[case % len(HEADS)]
    dtype = rng.choice([torch.bfloat16, torch.float16])
    batch = rng.randint(40, 120)
    lens = [rng.choice([0, 1, 700, rng.randint(1, 3000)]) for _ in range(batch)]
    lens[rng.randrange(batch)] = rng.randint(16384, 24576)
    gen = torch.Generator().manual_seed(6000 + case)
    tables, caches = _fill(gen, lens, hk, H.BLOCK, dtype)
    units = hk * (1 if hq // hk <= 16 else hq // hk // 16)
    splits = decode_num_splits(batch, hq, hk, tables.shape[1], H.BLOCK)
    assert (units + 7) // 8 * splits * batch > 512 and batch * splits <= 65536
    print(f"decode work-item case {case}: hq {hq} hk {hk} {dtype} batch {batch} "
          f"splits {splits} lens {lens}", flush=True)
    query = H.randn(gen, (batch, hq, H.D), dtype)
    seqlens = torch.tensor(lens, dtype=torch.int32)
    scale = H.D ** -0.5
    out = fp8_decode_attention(query.to(H.DEV), *caches, seqlens.to(H.DEV), tables.to(H.DEV), scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.decode_attention(query, kc, vc, ks, vs, seqlens, tables, scale)
    H.assert_attention_close(out, ref)
    assert (out[seqlens.to(H.DEV) == 0] == 0).all()


@pytest.mark.parametrize("case", range(8))
def test_varlen_prefill_random_shapes(case):
    rng = random.Random(3000 + case)
    hq, hk = rng.choice(HEADS)
    bs = rng.choice([256, 512])
    dtype = rng.choice([torch.bfloat16, torch.float16])
    nseq = rng.randint(1, 5)
    lq = [rng.choice([0, 1, rng.randint(1, 400)]) for _ in range(nseq)]
    lk = [q + rng.choice([0, rng.randint(1, 1200)]) for q in lq]
    print(f"prefill case {case}: hq {hq} hk {hk} bs {bs} {dtype} lq {lq} lk {lk}", flush=True)
    gen = torch.Generator().manual_seed(4000 + case)
    tables, caches = _fill(gen, lk, hk, bs, dtype)
    query = H.randn(gen, (sum(lq), hq, H.D), dtype)
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    scale = H.D ** -0.5
    out = fp8_varlen_prefill_attention(query.to(H.DEV), *caches, tables.to(H.DEV),
                                       cu_q.to(H.DEV), cu_k.to(H.DEV), max(max(lq), 1), scale)
    torch.cuda.synchronize()
    kc, vc, ks, vs = H.cache_to_numpy(*caches)
    ref = O.varlen_prefill_attention(query, kc, vc, ks, vs, tables, cu_q, cu_k, scale)
    if sum(lq):
        H.assert_attention_close(out, ref)
