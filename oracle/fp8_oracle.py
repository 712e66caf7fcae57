"""CPU restatement of microserve's FP8 paged-KV path -- test infrastructure only.

This module is the checker for the HIP kernels in ``microserve_amd``.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product path never does.

Byte work (the e4m3fn encoder, the per-(token, kv_head) quantizer and the
slot scatter) is numpy integer/fp32 arithmetic.  Attention is float32 torch on
the CPU, written the way the reference's own kernel test restates it
(``tests/test_fp8_kv_attention.py:30-36,63-70,96-105``), plus pure-loop
float64 restatements for tiny cases.

How each function is pinned (the checks live in ``tests/test_oracle.py``):

* ``e4m3fn_encode`` / ``e4m3fn_decode`` -- written from the OCP FP8 E4M3FN
  definition (bias 7, 3 mantissa bits, subnormals m*2^-9, max 448 = 0x7E,
  0x7F/0xFF NaN, no infinities, round-to-nearest-even).  Pinned against
  torch's CPU ``.to(torch.float8_e4m3fn)`` over every bf16 and every fp16
  bit pattern in [-448, 448] and a structured fp32 set (all exponents x all
  leading mantissa bits x tie/sticky low bits), and against hand-derived
  known answers (1.0625 -> 0x38, 17 -> 0x58, 0.001 -> 0x01, -0.0 -> 0x80).
* ``quantize_rows`` -- the formula at ``fp8_kv_cache.py:24-27`` (also
  ``tests/test_fp8.py:25-26``, ``fp8_linear.py:51-54``).  Pinned against the
  same formula evaluated with torch CPU ops, and by closed forms (a row whose
  amax is 448 has scale exactly 1 and bytes equal to the plain cast; an
  all-zero row has scale 1e-8/448 and bytes 0x00 / 0x80 for -0.0).
* ``store_fp8_kvcache_torch`` -- the same store vectorized in torch CPU ops
  (the bench's multi-core baseline).  Pinned against ``store_fp8_kvcache``
  byte for byte on edge rows and random rows with skipped slots.
* ``store_fp8_kvcache`` -- placement ``row = (slot // BS) * BS + slot % BS``
  (``fp8_kv_cache.py:29-39``), which equals the fp16 path's
  ``index_copy_`` row (``attention.py:11-21``).  Pinned by brute-force
  per-element placement on tiny inputs and by the permutation invariant.
* ``decode_attention`` -- pinned against ``decode_attention_loop`` (the
  Triton kernel's online-softmax tile loop, ``fp8_decode_attention.py:16-58``,
  restated token by token in float64), against
  ``torch.nn.functional.scaled_dot_product_attention`` on the dequantized
  rows, and by invariants: block relabelling, ``seq_len == 0 -> 0``, a
  one-token context returns that token's dequantized V, equal scores return
  the mean of V.
* ``dense_varlen_attention`` -- the fresh PREFILL over unquantized q/k/v
  (flash-attn's causal convention, bottom-right aligned).  Pinned against
  ``dense_varlen_attention_loop`` (float64 per-query softmax), against
  ``scaled_dot_product_attention(is_causal=True)`` where ``Lq == Lk``, and
  against ``varlen_prefill_attention`` on a cache that holds the same K/V
  exactly (e4m3-representable rows with unit scale), which ties the two
  causal conventions together.
* ``chunk_prefill_attention`` / ``varlen_prefill_attention`` -- pinned
  against ``varlen_prefill_attention_loop`` (per-query direct softmax in
  float64, causal ``visible = prefix + i + 1`` from
  ``fp8_chunk_prefill_attention.py:52-54``), against SDPA with an explicit
  mask, and against ``decode_attention`` for the last query row.
"""

from __future__ import annotations

import math

import numpy as np
import torch

E4M3_MAX = 448.0
_F32_EPS_FLOOR = np.float32(1e-8)
_F32_MAX = np.float32(E4M3_MAX)


# --------------------------------------------------------------------------
# FP8 E4M3FN encode / decode (OCP definition)
# --------------------------------------------------------------------------

def e4m3fn_encode(x) -> np.ndarray:
    """Round fp32 values to OCP FP8 E4M3FN bytes, round-to-nearest-even.

    Magnitudes that round beyond 448 become NaN (0x7F | sign), which is what
    torch's cast does; the store path clamps to +-448 first, so it never
    reaches that case.  The sign is kept on zero: -0.0 and negative values
    that round to zero give 0x80.
    """
    x = np.asarray(x, dtype=np.float32)
    mag = np.abs(x).astype(np.float64)
    sign = (np.signbit(x).astype(np.uint8)) << 7
    out = np.zeros(x.shape, dtype=np.uint8)

    nan = np.isnan(x)
    # Normal range: |x| >= 2^-6.  |x| = f * 2^e2 with f in [0.5, 1).
    normal = (~nan) & (mag >= 2.0 ** -6)
    f, e2 = np.frexp(mag)
    e = e2.astype(np.int64) - 1                       # |x| = 1.m * 2^e
    ulp = np.ldexp(1.0, (e - 3).clip(-200, 200))       # 3 mantissa bits
    m = np.rint(np.where(normal, mag / ulp, 0.0))      # exact: ulp is 2^k
    carry = m >= 16.0
    e = np.where(carry, e + 1, e)
    m = np.where(carry, 8.0, m)
    biased = e + 7
    code = (biased << 3) | (m.astype(np.int64) - 8)
    over = normal & ((biased > 15) | (code > 0x7E))
    code = np.where(over, 0x7F, code)
    out = np.where(normal, code.astype(np.uint8), out)

    # Subnormal range: value = k * 2^-9, k in 0..8 (k == 8 is 2^-6, code 0x08).
    sub = (~nan) & (~normal)
    k = np.rint(np.where(sub, mag * 512.0, 0.0))       # exact scaling by 2^9
    out = np.where(sub, k.astype(np.uint8), out)

    out = np.where(nan, np.uint8(0x7F), out)
    return (out | sign).astype(np.uint8)


def e4m3fn_decode(b) -> np.ndarray:
    """Exact fp32 value of E4M3FN bytes (0x7F / 0xFF decode to NaN)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    ex = (b >> 3) & 0xF
    mt = b & 0x7
    val = np.where(ex == 0, mt * 2.0 ** -9,
                   np.ldexp(1.0 + mt / 8.0, ex - 7))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


_DECODE_LUT = e4m3fn_decode(np.arange(256, dtype=np.uint8))


# --------------------------------------------------------------------------
# store_kvcache
# --------------------------------------------------------------------------

def quantize_rows(x):
    """Per-row FP8 quantization: ``fp8_kv_cache.py:22-27``.

    ``x`` holds float32 values (an exact upcast of the fp16/bf16 input) with
    the head dimension last.  Returns ``(bytes uint8[..., D], scale f32[...])``
    with ``scale = max(amax, 1e-8) / 448`` and
    ``bytes = e4m3fn(clamp(x / scale, -448, 448))`` -- an IEEE fp32 division
    per element, not a multiply by the reciprocal.
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1)
    scale = (np.maximum(amax, _F32_EPS_FLOOR) / _F32_MAX).astype(np.float32)
    y = (x / scale[..., None]).astype(np.float32)
    y = np.minimum(np.maximum(y, -_F32_MAX), _F32_MAX)
    return e4m3fn_encode(y), scale


def store_fp8_kvcache(key, value, k_cache, v_cache, k_scale_cache,
                      v_scale_cache, slot_mapping) -> None:
    """In-place restatement of ``store_fp8_kvcache`` (``fp8_kv_cache.py:42-61``).

    ``key``/``value``: float32 ``[N, H_kv, D]``.  ``k_cache``/``v_cache``:
    uint8 ``[NB, BS, H_kv, D]`` (the fp8 cache viewed as bytes).  Scale caches:
    float32 ``[NB, BS, H_kv]``.  Token ``t`` lands in cache row
    ``(slot // BS) * BS + slot % BS`` (``fp8_kv_cache.py:29-33``), i.e. row
    ``slot`` of the cache flattened to ``[NB*BS, H_kv, D]``.  Slots outside
    ``[0, NB*BS)`` are skipped (the reference never produces them).
    """
    nb, bs, h, d = k_cache.shape
    slots = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    kq, ks = quantize_rows(key)
    vq, vs = quantize_rows(value)
    valid = (slots >= 0) & (slots < nb * bs)
    rows = (slots // bs) * bs + slots % bs
    kc = k_cache.reshape(nb * bs, h, d)
    vc = v_cache.reshape(nb * bs, h, d)
    ksc = k_scale_cache.reshape(nb * bs, h)
    vsc = v_scale_cache.reshape(nb * bs, h)
    for t in np.nonzero(valid)[0]:
        r = rows[t]
        kc[r] = kq[t]
        vc[r] = vq[t]
        ksc[r] = ks[t]
        vsc[r] = vs[t]


def store_fp8_kvcache_torch(key, value, k_cache, v_cache, k_scale_cache,
                            v_scale_cache, slot_mapping) -> None:
    """``store_fp8_kvcache`` vectorized in torch CPU ops, for timing on the
    host's cores (torch's intra-op threads): the reference's formula as its
    own tests write it (``tests/test_fp8.py:25-26``; ``fp8_kv_cache.py:24-27``)
    -- ``s = max(amax, 1e-8) / 448``, ``q = e4m3fn(clamp(x / s, -448, 448))``
    -- and one ``index_copy_`` per cache at rows ``slot``
    (``attention.py:11-21``).  Same arguments and effect as
    ``store_fp8_kvcache``, with torch tensors: ``key``/``value`` float
    ``[N, H_kv, D]``, uint8 byte caches, float32 scale caches, int64 slots.
    """
    nb, bs, h, d = k_cache.shape
    slots = slot_mapping.reshape(-1).to(torch.int64)
    valid = (slots >= 0) & (slots < nb * bs)
    rows = slots[valid]
    for x, cache, scales in ((key, k_cache, k_scale_cache), (value, v_cache, v_scale_cache)):
        x = x.float()
        sc = x.abs().amax(-1).clamp_min(_F32_EPS_FLOOR) / _F32_MAX
        q = (x / sc[..., None]).clamp(-_F32_MAX, _F32_MAX).to(torch.float8_e4m3fn)
        cache.view(nb * bs, h, d).index_copy_(0, rows, q.view(torch.uint8)[valid])
        scales.view(nb * bs, h).index_copy_(0, rows, sc[valid])


# --------------------------------------------------------------------------
# Attention (float32 torch, vectorized) -- the checker for the HIP kernels
# --------------------------------------------------------------------------

def _as_t(a, dtype=None):
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.asarray(a))
    return t if dtype is None else t.to(dtype)


def dequant_gather(cache_u8, scales, table_row, length) -> torch.Tensor:
    """Rows ``0..length-1`` of one sequence, dequantized to float32.

    ``tests/test_fp8_kv_attention.py:30-36``: position ``p`` lives in block
    ``table[p // BS]`` at offset ``p % BS``; its value is
    ``fp8(cache).float() * scale``.  Returns ``[length, H_kv, D]``.
    """
    cache_u8 = _as_t(cache_u8)
    scales = _as_t(scales, torch.float32)
    bs = cache_u8.shape[1]
    pos = torch.arange(length, dtype=torch.int64)
    table = _as_t(table_row, torch.int64).reshape(-1)
    blocks = table[pos // bs]
    offs = pos % bs
    raw = cache_u8[blocks, offs].to(torch.int64)                 # [L, H, D]
    vals = torch.from_numpy(_DECODE_LUT)[raw]
    return vals * scales[blocks, offs][..., None]


def decode_attention(query, k_cache, v_cache, k_scale_cache, v_scale_cache,
                     cache_seqlens, block_tables, softmax_scale) -> torch.Tensor:
    """``fp8_decode_attention`` restated (``fp8_decode_attention.py:16-58``).

    One query token per sequence; q head ``hq`` reads kv head
    ``hq // (H_q / H_kv)`` (``:18``); scores are ``q . k_deq * scale`` and the
    result is ``softmax(scores) @ v_deq`` in float32, or zeros for a sequence
    of length 0 (``:58``).  Returns float32 ``[B, H_q, D]``.
    """
    q = _as_t(query).float()
    b, hq, d = q.shape
    hk = k_cache.shape[2]
    group = hq // hk
    lens = [int(x) for x in _as_t(cache_seqlens).reshape(-1).tolist()]
    tables = _as_t(block_tables, torch.int64)
    out = torch.zeros(b, hq, d, dtype=torch.float32)
    for i, n in enumerate(lens):
        if n <= 0:
            continue
        k = dequant_gather(k_cache, k_scale_cache, tables[i], n)   # [L, H_kv, D]
        v = dequant_gather(v_cache, v_scale_cache, tables[i], n)
        qg = q[i].view(hk, group, d)            # q head h -> kv head h // group
        scores = torch.einsum("kgd,lkd->kgl", qg, k) * softmax_scale
        out[i] = torch.einsum("kgl,lkd->kgd", scores.softmax(-1), v).reshape(hq, d)
    return out


def decode_attention_loop(query, k_cache, v_cache, k_scale_cache,
                          v_scale_cache, cache_seqlens, block_tables,
                          softmax_scale) -> np.ndarray:
    """Token-by-token online-softmax loop in float64 (tiny inputs only).

    Follows the running-max recurrence of ``fp8_decode_attention.py:50-58``
    one token at a time, reading each row straight from the byte cache, so it
    shares no code with ``decode_attention``.
    """
    q = np.asarray(_as_t(query).float().numpy(), dtype=np.float64)
    kc = np.asarray(_as_t(k_cache).numpy())
    vc = np.asarray(_as_t(v_cache).numpy())
    ks = np.asarray(_as_t(k_scale_cache).numpy(), dtype=np.float64)
    vs = np.asarray(_as_t(v_scale_cache).numpy(), dtype=np.float64)
    lens = np.asarray(_as_t(cache_seqlens).numpy()).reshape(-1)
    tables = np.asarray(_as_t(block_tables).numpy())
    b, hq, d = q.shape
    bs, hk = kc.shape[1], kc.shape[2]
    out = np.zeros((b, hq, d))
    for i in range(b):
        for h in range(hq):
            kvh = h // (hq // hk)
            m, l = -math.inf, 0.0
            acc = np.zeros(d)
            for p in range(int(lens[i])):
                blk, off = int(tables[i, p // bs]), p % bs
                k = _DECODE_LUT[kc[blk, off, kvh]].astype(np.float64)
                v = _DECODE_LUT[vc[blk, off, kvh]].astype(np.float64)
                s = float(np.dot(k, q[i, h])) * ks[blk, off, kvh] * softmax_scale
                m_new = max(m, s)
                alpha = math.exp(m - m_new) if m != -math.inf else 0.0
                pr = math.exp(s - m_new)
                acc = acc * alpha + pr * v * vs[blk, off, kvh]
                l = l * alpha + pr
                m = m_new
            if lens[i] > 0:
                out[i, h] = acc / l
    return out


def varlen_prefill_attention(query, k_cache, v_cache, k_scale_cache,
                             v_scale_cache, block_tables, cu_seqlens_q,
                             cu_seqlens_k, softmax_scale, rows=None) -> torch.Tensor:
    """Causal paged prefill over a varlen batch, float32.

    Sequence ``s`` owns query rows ``cu_q[s]..cu_q[s+1]`` and a context of
    ``Lk = cu_k[s+1] - cu_k[s]`` cached tokens that already include the new
    ones (they are stored before attention, ``attention.py:41-43,56-60``).
    Query ``i`` sees positions ``< prefix + i + 1`` with
    ``prefix = Lk - Lq`` (``fp8_chunk_prefill_attention.py:52-54``).
    Returns float32 ``[total_q, H_q, D]``; with ``rows`` (ascending query
    row indices into ``total_q``), only those rows, ``[len(rows), H_q, D]``,
    each computed exactly as in the full result.
    """
    q = _as_t(query).float()
    tq, hq, d = q.shape
    hk = k_cache.shape[2]
    group = hq // hk
    cu_q = [int(x) for x in _as_t(cu_seqlens_q).reshape(-1).tolist()]
    cu_k = [int(x) for x in _as_t(cu_seqlens_k).reshape(-1).tolist()]
    tables = _as_t(block_tables, torch.int64)
    if rows is None:
        sel_all = torch.arange(tq)
    else:
        sel_all = _as_t(rows, torch.int64).reshape(-1)
        assert bool((sel_all[1:] > sel_all[:-1]).all()), "rows must be ascending"
    out = torch.zeros(sel_all.numel(), hq, d, dtype=torch.float32)
    for s in range(len(cu_q) - 1):
        lq = cu_q[s + 1] - cu_q[s]
        lk = cu_k[s + 1] - cu_k[s]
        if lq <= 0:
            continue
        at = ((sel_all >= cu_q[s]) & (sel_all < cu_q[s + 1])).nonzero().view(-1)
        if at.numel() == 0:
            continue
        i = sel_all[at] - cu_q[s]                                    # query index in the sequence
        prefix = lk - lq
        k = dequant_gather(k_cache, k_scale_cache, tables[s], lk)   # [Lk, H_kv, D]
        v = dequant_gather(v_cache, v_scale_cache, tables[s], lk)
        qs = q[cu_q[s] + i].view(i.numel(), hk, group, d)
        scores = torch.einsum("ikgd,lkd->kgil", qs, k) * softmax_scale
        pos = torch.arange(lk)[None, :]
        visible = (prefix + i + 1)[:, None]
        scores = scores.masked_fill(~(pos < visible)[None, None], float("-inf"))
        o = torch.einsum("kgil,lkd->ikgd", scores.softmax(-1), v)
        out[at] = o.reshape(i.numel(), hq, d)
    return out


def chunk_prefill_attention(query, k_cache, v_cache, k_scale_cache,
                            v_scale_cache, block_table, prefix_len,
                            softmax_scale) -> torch.Tensor:
    """Single-sequence chunk prefill (``fp8_chunk_prefill_attention.py:16-67``).

    The reference flattens ``block_table`` (``:77``) and runs ``query_len``
    rows over ``prefix_len + query_len`` cached positions.
    """
    q = _as_t(query)
    lq = q.shape[0]
    table = _as_t(block_table, torch.int64).reshape(1, -1)
    cu_q = torch.tensor([0, lq], dtype=torch.int32)
    cu_k = torch.tensor([0, int(prefix_len) + lq], dtype=torch.int32)
    return varlen_prefill_attention(q, k_cache, v_cache, k_scale_cache,
                                    v_scale_cache, table, cu_q, cu_k,
                                    softmax_scale)


def dense_varlen_attention(query, key, value, cu_seqlens_q, cu_seqlens_k,
                           softmax_scale, rows=None) -> torch.Tensor:
    """Causal varlen attention over unquantized q/k/v, float32: the fresh
    PREFILL of the FP8 path, which the reference runs as
    ``flash_attn_varlen_func(q, k, v, ..., causal=True)`` on the new tokens
    (``attention.py:49-55``).

    ``key``/``value`` are ``[total_k, H_kv, D]``; sequence ``s`` owns query
    rows ``cu_q[s]..cu_q[s+1]`` and key rows ``cu_k[s]..cu_k[s+1]``.  The
    causal mask is flash-attn's bottom-right alignment: query ``i`` sees key
    ``j`` iff ``j <= i + Lk - Lq`` (the same bound as the paged prefill's
    ``prefix + i + 1`` with ``prefix = Lk - Lq``).  Rows that see no key are
    zero.  Returns float32 ``[total_q, H_q, D]``; with ``rows`` (ascending
    query row indices into ``total_q``), only those rows,
    ``[len(rows), H_q, D]``, each against the same keys as in the full result.
    """
    q = _as_t(query).float()
    k_all = _as_t(key).float()
    v_all = _as_t(value).float()
    tq, hq, d = q.shape
    hk = k_all.shape[1]
    group = hq // hk
    cu_q = [int(x) for x in _as_t(cu_seqlens_q).reshape(-1).tolist()]
    cu_k = [int(x) for x in _as_t(cu_seqlens_k).reshape(-1).tolist()]
    if rows is None:
        sel_all = torch.arange(tq)
    else:
        sel_all = _as_t(rows, torch.int64).reshape(-1)
        assert bool((sel_all[1:] > sel_all[:-1]).all()), "rows must be ascending"
    out = torch.zeros(sel_all.numel(), hq, d, dtype=torch.float32)
    for s in range(len(cu_q) - 1):
        lq = cu_q[s + 1] - cu_q[s]
        lk = cu_k[s + 1] - cu_k[s]
        if lq <= 0 or lk <= 0:
            continue
        at = ((sel_all >= cu_q[s]) & (sel_all < cu_q[s + 1])).nonzero().view(-1)
        if at.numel() == 0:
            continue
        i = sel_all[at] - cu_q[s]  # query index in the sequence
        k = k_all[cu_k[s]:cu_k[s + 1]]
        v = v_all[cu_k[s]:cu_k[s + 1]]
        qs = q[cu_q[s] + i].view(i.numel(), hk, group, d)
        scores = torch.einsum("ikgd,lkd->kgil", qs, k) * softmax_scale
        visible = torch.arange(lk)[None, :] <= (i + lk - lq)[:, None]
        scores = scores.masked_fill(~visible[None, None], float("-inf"))
        p = torch.nan_to_num(scores.softmax(-1), nan=0.0)  # rows that see nothing
        o = torch.einsum("kgil,lkd->ikgd", p, v)
        out[at] = o.reshape(i.numel(), hq, d)
    return out


def dense_varlen_attention_loop(query, key, value, cu_seqlens_q, cu_seqlens_k,
                                softmax_scale) -> np.ndarray:
    """Per-query direct softmax in float64 over unquantized q/k/v (tiny
    inputs only); shares no code with ``dense_varlen_attention``."""
    q = np.asarray(_as_t(query).float().numpy(), dtype=np.float64)
    k = np.asarray(_as_t(key).float().numpy(), dtype=np.float64)
    v = np.asarray(_as_t(value).float().numpy(), dtype=np.float64)
    cu_q = np.asarray(_as_t(cu_seqlens_q).numpy()).reshape(-1)
    cu_k = np.asarray(_as_t(cu_seqlens_k).numpy()).reshape(-1)
    tq, hq, d = q.shape
    hk = k.shape[1]
    group = hq // hk
    out = np.zeros((tq, hq, d))
    for s in range(len(cu_q) - 1):
        lq = int(cu_q[s + 1] - cu_q[s])
        lk = int(cu_k[s + 1] - cu_k[s])
        for i in range(lq):
            last = i + lk - lq  # keys 0..last are visible
            if last < 0:
                continue
            for h in range(hq):
                kv = h // group
                sc = [float(np.dot(q[cu_q[s] + i, h], k[cu_k[s] + j, kv])) * softmax_scale
                      for j in range(last + 1)]
                mx = max(sc)
                w = [np.exp(x - mx) for x in sc]
                tot = sum(w)
                acc = np.zeros(d)
                for j, wj in enumerate(w):
                    acc += wj * v[cu_k[s] + j, kv]
                out[cu_q[s] + i, h] = acc / tot
    return out


def varlen_prefill_attention_loop(query, k_cache, v_cache, k_scale_cache,
                                  v_scale_cache, block_tables, cu_seqlens_q,
                                  cu_seqlens_k, softmax_scale) -> np.ndarray:
    """Per-query direct softmax in float64 (tiny inputs only).

    Reads every visible row from the byte cache one position at a time
    (``tests/test_fp8_kv_attention.py:96-105`` spelled out), sharing no code
    with ``varlen_prefill_attention``.
    """
    q = np.asarray(_as_t(query).float().numpy(), dtype=np.float64)
    kc = np.asarray(_as_t(k_cache).numpy())
    vc = np.asarray(_as_t(v_cache).numpy())
    ks = np.asarray(_as_t(k_scale_cache).numpy(), dtype=np.float64)
    vs = np.asarray(_as_t(v_scale_cache).numpy(), dtype=np.float64)
    tables = np.asarray(_as_t(block_tables).numpy())
    cu_q = np.asarray(_as_t(cu_seqlens_q).numpy()).reshape(-1)
    cu_k = np.asarray(_as_t(cu_seqlens_k).numpy()).reshape(-1)
    tq, hq, d = q.shape
    bs, hk = kc.shape[1], kc.shape[2]
    out = np.zeros((tq, hq, d))
    for s in range(len(cu_q) - 1):
        lq = int(cu_q[s + 1] - cu_q[s])
        lk = int(cu_k[s + 1] - cu_k[s])
        prefix = lk - lq
        for i in range(lq):
            visible = prefix + i + 1
            for h in range(hq):
                kvh = h // (hq // hk)
                scores = np.empty(visible)
                vals = np.empty((visible, d))
                for p in range(visible):
                    blk, off = int(tables[s, p // bs]), p % bs
                    k = _DECODE_LUT[kc[blk, off, kvh]].astype(np.float64)
                    scores[p] = np.dot(k, q[cu_q[s] + i, h]) * ks[blk, off, kvh] * softmax_scale
                    vals[p] = _DECODE_LUT[vc[blk, off, kvh]] * vs[blk, off, kvh]
                w = np.exp(scores - scores.max())
                out[cu_q[s] + i, h] = (w[:, None] * vals).sum(0) / w.sum()
    return out
