"""GPU parity of the fused q/k RMSNorm + rotary + FP8 store
(``qk_norm_rope_store_kernel`` through ``mskv_qk_norm_rope_store``) against
the oracle: q/k outputs, cache bytes and scales bit-exact."""

import numpy as np
import pytest
import torch

from microserve_amd import Attention, qk_norm_rope_store, reset_context, set_context
from microserve_amd.context import AttentionMode, Context
from oracle import fp8_oracle as O
from oracle import norm_rope_oracle as NR
from tests.gpu_helpers import alloc_cache

DEV = "cuda"
D = 128
MAXPOS = 40960
EPS = 1e-6


def _inputs(n, hq, hk, dtype, seed, pool_blocks=64, bs=256, garbage=0):
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(n, (hq + 2 * hk) * D, generator=gen) * 2).to(dtype)
    pos = torch.randint(0, MAXPOS, (n,), generator=gen)
    slots = torch.randperm(pool_blocks * bs, generator=gen)[:n].long()
    if garbage:
        slots[:garbage] = pool_blocks * bs + torch.arange(garbage)  # out of range: skipped
    qw = (1 + 0.2 * torch.randn(D, generator=gen)).to(dtype)
    kw = (1 + 0.2 * torch.randn(D, generator=gen)).to(dtype)
    return qkv, pos, slots, qw, kw


def _split(qkv, hq, hk):
    n = qkv.shape[0]
    q, k, v = qkv.split([hq * D, hk * D, hk * D], dim=-1)
    return q.view(n, hq, D), k.view(n, hk, D), v.view(n, hk, D)


def _oracle_cache(k_embed, v, slots, pool_blocks, bs, hk):
    kc = np.zeros((pool_blocks, bs, hk, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((pool_blocks, bs, hk), np.float32)
    vs = np.ones_like(ks)
    keep = (slots >= 0) & (slots < pool_blocks * bs)
    O.store_fp8_kvcache(k_embed[keep].float().numpy(), v[keep].float().numpy(), kc, vc, ks, vs,
                        slots[keep].numpy())
    return kc, vc, ks, vs


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hk,n", [(32, 8, 1000), (64, 8, 77), (16, 8, 5)])
def test_fused_prologue_matches_oracle(dtype, hq, hk, n):
    print(f"fused prologue {dtype} hq {hq} hk {hk} n {n}", flush=True)
    qkv, pos, slots, qw, kw = _inputs(n, hq, hk, dtype, seed=hq + n, garbage=min(3, n - 1))
    cos, sin = NR.rope_tables(MAXPOS, 1e6, dtype)
    kc, vc, ks, vs = alloc_cache(64, kv_heads=hk)
    q, k, v = _split(qkv.to(DEV), hq, hk)
    q_out, k_out = qk_norm_rope_store(pos.to(DEV), q, k, v, qw.to(DEV), kw.to(DEV), EPS,
                                      cos.to(DEV), sin.to(DEV), kc, vc, ks, vs, slots.to(DEV))
    torch.cuda.synchronize()
    qc, kcpu, vcpu = _split(qkv, hq, hk)
    rq, rk = NR.qk_norm_rope(qc, kcpu, pos, qw, kw, EPS, cos, sin)
    assert torch.equal(q_out.cpu(), rq), "q differs"
    assert torch.equal(k_out.cpu(), rk), "k differs"
    okc, ovc, oks, ovs = _oracle_cache(rk, vcpu, slots, 64, 256, hk)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), okc), "k cache bytes differ"
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), ovc), "v cache bytes differ"
    assert np.array_equal(ks.cpu().numpy(), oks) and np.array_equal(vs.cpu().numpy(), ovs)


@pytest.mark.gpu
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_store_equals_store_kernel_on_the_rotated_k(dtype, slot_dtype):
    """Composition: the fused store writes the bytes the standalone store
    kernel writes from the same rotated k, with int64 slots and with the
    int32 slots the runner's warmup passes."""
    from microserve_amd import store_fp8_kvcache
    hq, hk, n = 32, 8, 512
    qkv, pos, slots, qw, kw = _inputs(n, hq, hk, dtype, seed=9)
    slots = slots.to(slot_dtype)
    cos, sin = NR.rope_tables(MAXPOS, 1e6, dtype)
    q, k, v = _split(qkv.to(DEV), hq, hk)
    a = alloc_cache(64, kv_heads=hk)
    _, k_out = qk_norm_rope_store(pos.to(DEV), q, k, v, qw.to(DEV), kw.to(DEV), EPS,
                                  cos.to(DEV), sin.to(DEV), *a, slots.to(DEV))
    b = alloc_cache(64, kv_heads=hk)
    store_fp8_kvcache(k_out, v, *b, slots.to(DEV))
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8) if x.dtype == torch.float8_e4m3fn else x,
                           y.view(torch.uint8) if y.dtype == torch.float8_e4m3fn else y)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("with_norm", [True, False])
def test_fused_prologue_edge_values(dtype, with_norm):
    """Bit-exact at the edges of the 16-bit types, where the fp16 form's
    packed multiplies and adds must round as torch's fp32 op + cast does:
    rows of tiny magnitudes (the rotary products go subnormal), rows near
    the type's largest values, signed zeros, rows of one repeated value,
    and tiny / large norm weights; with and without the norm."""
    hq, hk, n = 16, 8, 400
    gen = torch.Generator().manual_seed(31 + with_norm)
    heads = hq + 2 * hk
    base = torch.randn(n, heads, D, generator=gen)
    # large rows stay below max / 16, so a rotated sum cannot overflow; the
    # smallest magnitudes give subnormal products (in fp16 the 1e-37 rows
    # are zeros)
    big = (6.0e4 if dtype == torch.float16 else 3.0e38) / 16
    mag = torch.tensor([1.0, 1e-5, 3e-7, 6e-8, big / 4, 1e-37, 1e-3, 2.0])
    rowscale = mag[torch.randint(0, len(mag), (n, heads), generator=gen)]
    x = base * rowscale[..., None]
    x[0::7, :, 5:9] = 0.0
    x[1::7, :, 5:9] = -0.0
    x[2::11] = 0.75                       # rows of one repeated value
    qkv = x.reshape(n, heads * D).to(dtype)
    pos = torch.randint(0, MAXPOS, (n,), generator=gen)
    pos[:8] = torch.tensor([0, 1, 2, 3, MAXPOS - 1, MAXPOS - 2, 12345, 7])
    slots = torch.randperm(64 * 256, generator=gen)[:n].long()
    if with_norm:
        qw = (1 + 0.2 * torch.randn(D, generator=gen))
        qw[:4] = torch.tensor([1e-4, 3e-6, 50.0, -7.0])
        kw = qw.flip(0).clone()
        qw, kw = qw.to(dtype), kw.to(dtype)
    else:
        qw = kw = None
    cos, sin = NR.rope_tables(MAXPOS, 1e6, dtype)
    kc, vc, ks, vs = alloc_cache(64, kv_heads=hk)
    q, k, v = _split(qkv.to(DEV), hq, hk)
    q_out, k_out = qk_norm_rope_store(
        pos.to(DEV), q, k, v, None if qw is None else qw.to(DEV),
        None if kw is None else kw.to(DEV), EPS, cos.to(DEV), sin.to(DEV), kc, vc, ks, vs,
        slots.to(DEV))
    torch.cuda.synchronize()
    qc, kcpu, vcpu = _split(qkv, hq, hk)
    rq, rk = NR.qk_norm_rope(qc, kcpu, pos, qw, kw, EPS, cos, sin)
    assert torch.isfinite(rq.float()).all() and torch.isfinite(rk.float()).all()
    gq, gk = q_out.cpu(), k_out.cpu()
    assert torch.equal(gq.view(torch.int16), rq.view(torch.int16)), "q bits differ"
    assert torch.equal(gk.view(torch.int16), rk.view(torch.int16)), "k bits differ"
    okc, ovc, oks, ovs = _oracle_cache(rk, vcpu, slots, 64, 256, hk)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), okc), "k cache bytes differ"
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), ovc), "v cache bytes differ"
    assert np.array_equal(ks.cpu().numpy(), oks) and np.array_equal(vs.cpu().numpy(), ovs)


@pytest.mark.gpu
def test_no_norm_no_k_and_invalid_positions():
    dtype, hq, hk, n = torch.bfloat16, 32, 8, 300
    qkv, pos, slots, qw, kw = _inputs(n, hq, hk, dtype, seed=21)
    pos[:4] = torch.tensor([-1, MAXPOS, MAXPOS + 5, -100])
    cos, sin = NR.rope_tables(MAXPOS, 1e6, dtype)
    kc, vc, ks, vs = alloc_cache(64, kv_heads=hk)
    q, k, v = _split(qkv.to(DEV), hq, hk)
    q_out, k_out = qk_norm_rope_store(pos.to(DEV), q, k, v, None, None, EPS, cos.to(DEV),
                                      sin.to(DEV), kc, vc, ks, vs, slots.to(DEV),
                                      return_k=False)
    torch.cuda.synchronize()
    assert k_out is None
    qc, kcpu, vcpu = _split(qkv, hq, hk)
    ok = slice(4, None)
    rq, rk = NR.qk_norm_rope(qc[ok], kcpu[ok], pos[ok], None, None, EPS, cos, sin)
    got = q_out.cpu()
    assert torch.equal(got[ok], rq)
    assert (got[:4] == 0).all(), "rows with invalid positions must be zero"
    okc, ovc, oks, ovs = _oracle_cache(rk, vcpu[ok], slots[ok], 64, 256, hk)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), okc)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), ovc)
    assert np.array_equal(ks.cpu().numpy(), oks) and np.array_equal(vs.cpu().numpy(), ovs)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["decode", "prefill"])
def test_attention_forward_fused_equals_unfused(mode):
    """Attention.forward_fused gives bitwise the output of forward() on the
    oracle's normalized and rotated q/k, and the same cache."""
    dtype, hq, hk = torch.bfloat16, 32, 8
    bs, nb = 256, 32
    gen = torch.Generator().manual_seed(5)
    cos, sin = NR.rope_tables(MAXPOS, 1e6, dtype)
    if mode == "decode":
        lens = [300, 1, 700, 256]
        tables = torch.full((4, 3), -1, dtype=torch.int32)
        perm = torch.randperm(nb, generator=gen)
        at = 0
        for b, L in enumerate(lens):
            p = -(-L // bs)
            tables[b, :p] = perm[at:at + p].to(torch.int32)
            at += p
        pos = torch.tensor([L - 1 for L in lens])
        slots = torch.stack([tables[b, (L - 1) // bs].long() * bs + (L - 1) % bs
                             for b, L in enumerate(lens)])
        n = 4
    else:
        cu = torch.tensor([0, 100, 357], dtype=torch.int32)
        n = 357
        pos = torch.cat([torch.arange(100), torch.arange(257)])
        slots = torch.randperm(nb * bs, generator=gen)[:n].long()
    qkv = torch.randn(n, (hq + 2 * hk) * D, generator=gen).to(dtype)
    qw = (1 + 0.2 * torch.randn(D, generator=gen)).to(dtype)
    kw = (1 + 0.2 * torch.randn(D, generator=gen)).to(dtype)
    outs, caches = [], []
    for fused in (True, False):
        cache = alloc_cache(nb, kv_heads=hk)
        if mode == "decode":
            # earlier tokens of each sequence already cached (same for both)
            gen2 = torch.Generator().manual_seed(6)
            for c in cache[:2]:
                c.view(torch.uint8).copy_(torch.randint(0, 120, c.shape, generator=gen2,
                                                        dtype=torch.uint8).to(DEV))
        attn = Attention(hq, D, D ** -0.5, hk)
        attn.k_cache, attn.v_cache, attn.k_scale_cache, attn.v_scale_cache = cache
        if mode == "decode":
            ctx = Context(mode=AttentionMode.DECODE, slot_mapping=slots.to(DEV),
                          cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=DEV),
                          block_tables=tables.to(DEV))
        else:
            ctx = Context(mode=AttentionMode.PREFILL, cu_seqlens_q=cu.to(DEV),
                          cu_seqlens_k=cu.to(DEV), max_seqlen_q=257, max_seqlen_k=257,
                          slot_mapping=slots.to(DEV))
        set_context(ctx)
        try:
            q, k, v = _split(qkv.to(DEV), hq, hk)
            if fused:
                o = attn.forward_fused(pos.to(DEV), q, k, v, qw.to(DEV), kw.to(DEV), EPS,
                                       cos.to(DEV), sin.to(DEV))
            else:
                rq, rk = NR.qk_norm_rope(*[t.cpu() for t in _split(qkv, hq, hk)[:2]], pos,
                                         qw, kw, EPS, cos, sin)
                o = attn(rq.to(DEV), rk.to(DEV), v.contiguous())
        finally:
            reset_context()
        torch.cuda.synchronize()
        outs.append(o.cpu())
        caches.append([c.view(torch.uint8).cpu() if c.dtype == torch.float8_e4m3fn else c.cpu()
                       for c in cache])
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(*caches):
        assert torch.equal(a, b)
