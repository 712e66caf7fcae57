"""Shared helpers for the GPU parity tests: seeded inputs drawn on the CPU,
paged caches on the GPU, and the tolerance checks."""

from __future__ import annotations

import numpy as np
import torch

from oracle import fp8_oracle as O

DEV = "cuda"
BLOCK = 256
D = 128


def alloc_cache(num_blocks, block_size=BLOCK, kv_heads=8, device=DEV):
    """Zero fp8 caches and unit scale caches, the runner's initial state
    (``model_runner.py:76-83``)."""
    kc = torch.zeros(num_blocks, block_size, kv_heads, D, dtype=torch.float8_e4m3fn, device=device)
    vc = torch.zeros_like(kc)
    ks = torch.ones(num_blocks, block_size, kv_heads, dtype=torch.float32, device=device)
    vs = torch.ones_like(ks)
    return kc, vc, ks, vs


def paged_layout(gen, lens, num_blocks, block_size=BLOCK):
    """Block tables (-1 padded) drawn without replacement from the pool, and
    the slot of every token (``model_runner.py:135,160,182``)."""
    pages = [(n + block_size - 1) // block_size for n in lens]
    width = max(1, max(pages))
    assert sum(pages) <= num_blocks
    perm = torch.randperm(num_blocks, generator=gen)
    tables = torch.full((len(lens), width), -1, dtype=torch.int32)
    slots = []
    at = 0
    for b, (n, p) in enumerate(zip(lens, pages)):
        tables[b, :p] = perm[at:at + p].to(torch.int32)
        at += p
        pos = torch.arange(n)
        slots.append(tables[b, pos // block_size].long() * block_size + pos % block_size)
    return tables, torch.cat(slots) if slots else torch.zeros(0, dtype=torch.int64)


def randn(gen, shape, dtype, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(dtype)


def cache_to_numpy(kc, vc, ks, vs):
    return (kc.view(torch.uint8).cpu().numpy(), vc.view(torch.uint8).cpu().numpy(),
            ks.cpu().numpy(), vs.cpu().numpy())


def attention_errors(actual: torch.Tensor, expected: torch.Tensor):
    a = actual.float().cpu()
    e = expected.float().cpu()
    assert torch.isfinite(a).all(), "non-finite output"
    max_abs = (a - e).abs().max().item()
    rel = ((a - e).norm() / e.norm().clamp_min(1e-30)).item()
    return max_abs, rel


def assert_attention_close(actual, expected, atol=2e-2, rtol=1e-2):
    """The gate for attention outputs: max-abs error below ``atol`` and the
    relative (Frobenius) error below ``rtol``."""
    max_abs, rel = attention_errors(actual, expected)
    assert max_abs < atol and rel < rtol, f"max_abs {max_abs:.3e} rel {rel:.3e}"
    return max_abs, rel


def oracle_store_numpy(key, value, slots, num_blocks, block_size=BLOCK, kv_heads=8):
    kc = np.zeros((num_blocks, block_size, kv_heads, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((num_blocks, block_size, kv_heads), np.float32)
    vs = np.ones_like(ks)
    O.store_fp8_kvcache(key.float().numpy(), value.float().numpy(), kc, vc, ks, vs,
                        slots.numpy())
    return kc, vc, ks, vs


def oracle_quantize_threaded(x: torch.Tensor, chunk: int = 4096):
    """The oracle's ``quantize_rows`` over a large [N, H, D] tensor (any
    device), in chunks on a thread pool (numpy's array operations release
    the GIL).  Returns (uint8 bytes [N, H, D], float32 scales [N, H])."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    n = x.shape[0]
    q = np.empty(tuple(x.shape), np.uint8)
    s = np.empty(tuple(x.shape[:-1]), np.float32)

    def work(i):
        qi, si = O.quantize_rows(x[i:i + chunk].float().cpu().numpy())
        q[i:i + chunk] = qi
        s[i:i + chunk] = si

    with ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(work, range(0, n, chunk)))
    return q, s


def compact_cache(caches, tables):
    """The blocks ``tables`` uses, copied to the host as uint8 / float32 numpy
    arrays, and the tables renumbered to them (a block relabelling, which
    leaves every attention output unchanged)."""
    t = tables.cpu().long()
    used = t[t >= 0].unique()
    remap = torch.full((int(used.max()) + 1 if used.numel() else 1,), -1, dtype=torch.long)
    remap[used] = torch.arange(used.numel())
    new = torch.where(t >= 0, remap[t.clamp_min(0)], torch.full_like(t, -1)).to(torch.int32)
    idx = used.to(caches[0].device)
    kc, vc, ks, vs = caches
    return (kc.view(torch.uint8)[idx].cpu().numpy(), vc.view(torch.uint8)[idx].cpu().numpy(),
            ks[idx].cpu().numpy(), vs[idx].cpu().numpy()), new
