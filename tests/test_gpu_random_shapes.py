"""Seeded random-shape parity sweeps of decode and varlen prefill against
the oracle: batch sizes, context and query lengths (zero included), GQA
groups 1-16 and block sizes 256/512 drawn from fixed seeds, so every run
checks the same cases."""

import random

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from tests import gpu_helpers as H
from microserve_amd import (fp8_decode_attention, fp8_varlen_prefill_attention,
                            store_fp8_kvcache)

pytestmark = pytest.mark.gpu

HEADS = [(16, 16), (16, 8), (32, 8), (64, 8), (32, 2), (16, 1)]


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
