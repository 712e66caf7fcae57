"""GPU parity of the fresh PREFILL (``varlen_attention``, the
``flash_attn_varlen_func`` call at ``attention.py:49-55``) against the dense
oracle: outputs within 2e-2 max-abs and 1e-2 relative (Frobenius) error."""

import pytest
import torch

from oracle import fp8_oracle as O
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu

from microserve_amd import flash_attn_varlen_func, varlen_attention  # noqa: E402


def _setup(seed, lq, lk, hq, hk, dtype=torch.bfloat16, outliers=0.0):
    gen = torch.Generator().manual_seed(seed)
    q = H.randn(gen, (sum(lq), hq, H.D), dtype)
    k = torch.randn(sum(lk), hk, H.D, generator=gen)
    if outliers:
        k = torch.where(torch.rand(k.shape, generator=gen) < outliers, k * 20, k)
    k = k.to(dtype)
    v = H.randn(gen, (sum(lk), hk, H.D), dtype)
    cu_q = torch.tensor([0] + list(torch.tensor(lq).cumsum(0)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lk).cumsum(0)), dtype=torch.int32)
    return q, k, v, cu_q, cu_k


def _check(q, k, v, cu_q, cu_k, lq, lk):
    scale = H.D ** -0.5
    out = varlen_attention(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV), cu_q.to(H.DEV),
                           cu_k.to(H.DEV), max(lq), max(lk), scale)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, scale)
    return H.assert_attention_close(out, ref), out


@pytest.mark.parametrize("scale", [0.0, -0.088, float("nan"), float("inf")])
def test_fresh_prefill_rejects_a_softmax_scale_that_is_not_positive(scale):
    """The row maxima are taken before the softmax scale, so a scale that is
    not positive and finite raises (MSKV_EUNSUPPORTED) instead of returning
    rows normalized against the wrong maximum."""
    q, k, v, cu_q, cu_k = _setup(6, [40], [40], 8, 2)
    with pytest.raises(RuntimeError, match="status -2"):
        varlen_attention(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV), cu_q.to(H.DEV),
                         cu_k.to(H.DEV), 40, 40, scale)


def test_fresh_prefill_empty_sequences_and_oversized_max_seqlen():
    """Empty sequences at the start and in the middle of the batch, and
    max_seqlen_q far above the longest sequence."""
    lens = [0, 40, 0, 300]
    q, k, v, cu_q, cu_k = _setup(409, lens, lens, 32, 8)
    scale = H.D ** -0.5
    out = varlen_attention(q.to(H.DEV), k.to(H.DEV), v.to(H.DEV), cu_q.to(H.DEV),
                           cu_k.to(H.DEV), max(lens) + 1000, max(lens), scale)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, scale)
    H.assert_attention_close(out, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fresh_prefill_ragged_batch(dtype):
    """Fresh sequences (Lq == Lk) of ragged lengths, including 1 and lengths
    that are not multiples of the 64-key tile, in one launch."""
    lens = [1, 17, 64, 100, 300, 513]
    q, k, v, cu_q, cu_k = _setup(401, lens, lens, 32, 8, dtype)
    _check(q, k, v, cu_q, cu_k, lens, lens)


@pytest.mark.parametrize("hq,hk", [(16, 8), (8, 8), (64, 8), (32, 2), (16, 1), (24, 8), (40, 2),
                                   (20, 1), (48, 2)])
def test_fresh_prefill_gqa_groups(hq, hk):
    lens = [70, 129]
    q, k, v, cu_q, cu_k = _setup(411 + hq, lens, lens, hq, hk)
    _check(q, k, v, cu_q, cu_k, lens, lens)


def test_fresh_prefill_bottom_right_causal_alignment():
    """Lq < Lk (a prefix of keys before the queries) and Lq > Lk (the first
    rows see no key and are zero), flash-attn's causal convention."""
    lq = [40, 90]
    lk = [200, 30]
    q, k, v, cu_q, cu_k = _setup(421, lq, lk, 32, 8)
    _, out = _check(q, k, v, cu_q, cu_k, lq, lk)
    assert torch.all(out[40:100].float() == 0)          # rows 0..59 of seq 1 see nothing
    assert out[100:130].float().abs().amax() > 0


def test_fresh_prefill_qwen3_8b_with_outliers():
    """Two Qwen3-8B sequences of 2048 fresh tokens, 1% of K entries x20."""
    lens = [2048, 2048]
    q, k, v, cu_q, cu_k = _setup(431, lens, lens, 32, 8, outliers=0.01)
    max_abs, rel = _check(q, k, v, cu_q, cu_k, lens, lens)[0]
    print(f"fresh prefill with outliers: max_abs {max_abs:.4e} rel {rel:.4e}")


def test_fresh_prefill_batch_equals_alone_and_alias():
    """A sequence's rows do not depend on the other sequences of the batch
    (bitwise), and flash_attn_varlen_func is the same entry point."""
    lens = [33, 150, 77]
    q, k, v, cu_q, cu_k = _setup(441, lens, lens, 32, 8)
    d = [t.to(H.DEV) for t in (q, k, v, cu_q, cu_k)]
    batch = varlen_attention(*d, 150, 150, 0.1)
    one = flash_attn_varlen_func(d[0][33:183], d[1][33:183], d[2][33:183],
                                 torch.tensor([0, 150], dtype=torch.int32, device=H.DEV),
                                 torch.tensor([0, 150], dtype=torch.int32, device=H.DEV),
                                 max_seqlen_q=150, max_seqlen_k=150, softmax_scale=0.1,
                                 causal=True)
    torch.cuda.synchronize()
    assert torch.equal(batch[33:183], one)


HEADS = [(16, 16), (16, 8), (32, 8), (64, 8), (32, 2), (16, 1), (48, 8), (40, 8)]


@pytest.mark.parametrize("case", range(8))
def test_fresh_prefill_random_shapes(case):
    """Seeded random sweep: batch, query and key lengths (zero, one, short,
    multi-tile; Lk >= Lq, so the causal diagonal sits bottom-right), GQA
    groups 1-16 including groups that do not divide 16, both 16-bit types."""
    import random
    rng = random.Random(7000 + case)
    hq, hk = HEADS[case % len(HEADS)]
    dtype = rng.choice([torch.bfloat16, torch.float16])
    nseq = rng.randint(1, 6)
    lq = [rng.choice([0, 1, rng.randint(2, 200), rng.randint(200, 900)]) for _ in range(nseq)]
    lk = [q + rng.choice([0, 0, rng.randint(1, 700)]) for q in lq]
    print(f"fresh prefill case {case}: hq {hq} hk {hk} {dtype} lq {lq} lk {lk}", flush=True)
    q, k, v, cu_q, cu_k = _setup(8000 + case, lq, lk, hq, hk, dtype)
    if sum(lq):
        _check(q, k, v, cu_q, cu_k, [max(1, x) for x in lq], [max(1, x) for x in lk])
