"""Benchmark of the FP8 paged-KV hot path on one MI355X.

Workload (the Qwen3-8B layer decode): 32 q heads, 8 kv heads, head_dim 128,
block 256, batch 64, every sequence at context 4096, a 2048-block FP8 pool
filled by store_fp8_kvcache from bf16 N(0,1) K/V, block tables drawn from a
seeded permutation, bf16 N(0,1) queries.  One step is one decode-attention
pass over the batch; consecutive steps alternate between two disjoint halves
of the pool (each a valid draw of the workload), so the 1.1 GB footprint
keeps the 256 MB MALL from serving the reads.  Steps are launched eagerly
(graph replay measured slower on this stack: ~6 us per replay).

Printed JSON: ``value`` is decode-attention HBM GB/s on algorithmic bytes
(2112 B per context token for H_kv 8 -- fp8 K+V rows and their fp32 scales --
plus queries, outputs, tables and lengths), ``roofline`` compares the decode
op (split-KV kernel + combine) with the 8 TB/s HBM peak, ``store`` reports
store_kvcache tokens/s on the 262,144-token pool fill, and ``cpu_baseline``
times the oracle's torch-CPU decode on a bounded sample of the same workload.
The other objects (prefill, fresh prefill, ragged and long-context decode,
the step-input builder, the fused norm + rotary + store) are measured in the
same run; the last two carry CPU baselines of their own from the oracle.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
HQ, HK, D, BS = 32, 8, 128, 256
BATCH, CTX, POOL = 64, 4096, 2048


def decode_bytes(batch, ctx, hq, hk, d, act_bytes=2):
    """Algorithmic bytes of one decode pass: each K/V byte and scale once per
    kv head, the query and output once, the table entries and lengths."""
    kv = batch * ctx * (2 * hk * d + 2 * hk * 4)
    qo = batch * hq * d * act_bytes * 2
    tables = 4 * (batch * ((ctx + BS - 1) // BS) + batch)
    return kv + qo + tables


def store_bytes(n, hk, d, act_bytes=2, slot_bytes=8):
    return n * (2 * hk * d * act_bytes + 2 * hk * d + 2 * hk * 4 + slot_bytes)


def build_workload(dev, dtype=torch.bfloat16):
    from microserve_amd import store_fp8_kvcache
    gen = torch.Generator().manual_seed(2024)
    perm = torch.randperm(POOL, generator=gen).to(torch.int32)
    pages = CTX // BS
    tables = [perm[:BATCH * pages].view(BATCH, pages).contiguous(),
              perm[BATCH * pages:2 * BATCH * pages].view(BATCH, pages).contiguous()]
    kc = torch.zeros(POOL, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(POOL, BS, HK, device=dev)
    vs = torch.ones_like(ks)
    pos = torch.arange(CTX)
    fills = []
    for t in tables:
        slots = (t[:, pos // BS].long() * BS + pos % BS).reshape(-1)
        key = torch.randn(slots.numel(), HK, D, generator=gen).to(dtype)
        value = torch.randn(slots.numel(), HK, D, generator=gen).to(dtype)
        fills.append((key.to(dev), value.to(dev), slots.to(dev)))
        store_fp8_kvcache(fills[-1][0], fills[-1][1], kc, vc, ks, vs, fills[-1][2])
    query = torch.randn(BATCH, HQ, D, generator=gen).to(dtype).to(dev)
    seqlens = torch.full((BATCH,), CTX, dtype=torch.int32, device=dev)
    return dict(kc=kc, vc=vc, ks=ks, vs=vs, query=query, seqlens=seqlens,
                tables=[t.to(dev) for t in tables], fills=fills)


def time_store_fill(w, iters=5):
    from microserve_amd import store_fp8_kvcache
    key, value, slots = w["fills"][0]
    n = slots.numel()
    stream = torch.cuda.current_stream()
    store_fp8_kvcache(key, value, w["kc"], w["vc"], w["ks"], w["vs"], slots)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    for i in range(iters):
        key, value, slots = w["fills"][i % 2]
        start.record(stream)
        store_fp8_kvcache(key, value, w["kc"], w["vc"], w["ks"], w["vs"], slots)
        end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e-3)
    t = sorted(times)[len(times) // 2]
    return {"tokens": n, "tokens_per_s": n / t, "us": t * 1e6,
            "gbs": store_bytes(n, HK, D) / t / 1e9,
            "frac": store_bytes(n, HK, D) / t / 1e9 / HBM_PEAK_GBS}


def time_fp16(dev, iters=200, warmup=20):
    """The headline decode and store fill with fp16 activations, the dtype the
    reference requires for its FP8 cache (Config.py:35-36)."""
    from microserve_amd import fp8_decode_attention
    w = build_workload(dev, torch.float16)
    torch.cuda.synchronize()
    out = torch.empty_like(w["query"])

    def step(i):
        fp8_decode_attention(w["query"], w["kc"], w["vc"], w["ks"], w["vs"],
                             w["seqlens"], w["tables"][i % 2], D ** -0.5, out=out)

    us = _time_steps(step, iters, warmup)
    nbytes = decode_bytes(BATCH, CTX, HQ, HK, D)
    store = time_store_fill(w)
    return {"workload": "the Qwen3-8B batch 64 x 4096 decode and the 262,144-token store "
                        "fill, fp16 q/K/V",
            "decode_us": round(us, 2), "decode_gbs": round(nbytes / us / 1e3, 1),
            "decode_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "store_tokens_per_s": round(store["tokens_per_s"], 1),
            "store_us": round(store["us"], 3)}


def cpu_baseline(w, budget_s=10.0):
    """Oracle torch-CPU decode on a bounded sample of the same workload:
    whole sequences of the batch, cycled until about budget_s of CPU work."""
    import numpy as np
    from oracle import fp8_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    kc = w["kc"].view(torch.uint8).cpu()
    vc = w["vc"].view(torch.uint8).cpu()
    ks, vs = w["ks"].cpu(), w["vs"].cpu()
    q = w["query"].cpu()
    tables = w["tables"][0].cpu()
    lens = np.full(BATCH, CTX)
    done, t_total = 0, 0.0
    while t_total < budget_s:
        i = done % BATCH
        t0 = time.perf_counter()
        O.decode_attention(q[i:i + 1], kc, vc, ks, vs, lens[i:i + 1],
                           tables[i:i + 1], D ** -0.5)
        t_total += time.perf_counter() - t0
        done += 1
    gbs = decode_bytes(done, CTX, HQ, HK, D) / t_total / 1e9
    # the store on the host: the oracle's store vectorized in torch CPU ops
    # (torch's intra-op threads on every core) over a bounded sample of the
    # fill's tokens (the first 65,536 of them), best of three passes
    key, value, slots = (t[:65536].cpu() for t in w["fills"][0])
    skc = torch.zeros(tuple(w["kc"].shape), dtype=torch.uint8)
    svc = torch.zeros_like(skc)
    sks = torch.ones(tuple(w["ks"].shape))
    svs = torch.ones_like(sks)
    store_s = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        O.store_fp8_kvcache_torch(key, value, skc, svc, sks, svs, slots)
        store_s = min(store_s, time.perf_counter() - t0)
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "os_cpu_count": os.cpu_count(), "kind": "port",
            "sample": f"{done} single-sequence decodes (4096 tokens, 32 q / 8 kv heads) "
                      f"cycling over the Qwen3-8B batch, torch fp32 oracle, {t_total:.1f} s",
            "store": {"value": round(key.shape[0] / store_s, 1), "unit": "tokens/s",
                      "cores": torch.get_num_threads(), "kind": "port",
                      "sample": f"{key.shape[0]} tokens of the 262,144-token fill, the oracle's "
                                f"store vectorized in torch CPU ops, best of 3 passes, "
                                f"{store_s:.2f} s"}}


C1_HQ, C1_BATCH, C1_POOL, C1_MAXLEN = 16, 4, 64, 1024


def config1_workload(dev, seed=1):
    """The reference's CPU-runnable case at the Qwen3-0.6B layer shape: 16 q
    / 8 kv heads, head_dim 128, block 256, batch 4, context lengths uniform
    in [1, 1024], block tables from a seeded permutation of a 64-block pool,
    bf16 N(0,1) q/k/v.  One step stores every token of the batch with
    store_fp8_kvcache, then runs one decode step
    (tests/test_fp8_kv_attention.py:39-73 at this shape)."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, C1_MAXLEN + 1, (C1_BATCH,), generator=gen)
    pages = (lens + BS - 1) // BS
    perm = torch.randperm(C1_POOL, generator=gen).to(torch.int32)
    tables = torch.full((C1_BATCH, int(pages.max())), -1, dtype=torch.int32)
    slots, at = [], 0
    for b in range(C1_BATCH):
        tables[b, :pages[b]] = perm[at:at + pages[b]]
        at += int(pages[b])
        pos = torch.arange(int(lens[b]))
        slots.append(tables[b, pos // BS].long() * BS + pos % BS)
    slots = torch.cat(slots)
    n = slots.numel()
    key = torch.randn(n, HK, D, generator=gen).bfloat16()
    value = torch.randn(n, HK, D, generator=gen).bfloat16()
    q = torch.randn(C1_BATCH, C1_HQ, D, generator=gen).bfloat16()
    kc = torch.zeros(C1_POOL, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(C1_POOL, BS, HK, device=dev)
    vs = torch.ones_like(ks)
    return dict(lens=lens, tables=tables, slots=slots, key=key, value=value, q=q,
                kc=kc, vc=vc, ks=ks, vs=vs, key_d=key.to(dev), value_d=value.to(dev),
                slots_d=slots.to(dev), q_d=q.to(dev), tables_d=tables.to(dev),
                seqlens_d=lens.to(torch.int32).to(dev))


def config1_step(w, out=None):
    from microserve_amd import fp8_decode_attention, store_fp8_kvcache
    store_fp8_kvcache(w["key_d"], w["value_d"], w["kc"], w["vc"], w["ks"], w["vs"], w["slots_d"])
    return fp8_decode_attention(w["q_d"], w["kc"], w["vc"], w["ks"], w["vs"], w["seqlens_d"],
                                w["tables_d"], D ** -0.5, out=out)


def time_config1(dev, iters=200, warmup=20, cpu_budget_s=8.0, cpu=True):
    """The Qwen3-0.6B batch-4 store-then-decode step on the GPU (HIP events)
    and, on the host cores in the same run, the oracle's store (numpy) and
    decode (torch fp32) of the same step."""
    import numpy as np
    w = config1_workload(dev)
    out = torch.empty_like(w["q_d"])
    us = _time_steps(lambda i: config1_step(w, out), iters, warmup)
    n = w["slots"].numel()
    st_bytes = store_bytes(n, HK, D)
    dec_bytes = decode_bytes_ragged(w["lens"], C1_HQ, HK, D)
    res = {"workload": "Qwen3-0.6B layer, 16 q / 8 kv heads, batch 4, context U[1, 1024] "
                       f"(lengths {w['lens'].tolist()}), 64-block permuted pool: store of "
                       f"every token ({n}) then one decode step",
           "us": round(us, 2), "tokens_stored": n, "bytes": st_bytes + dec_bytes,
           "gbs": round((st_bytes + dec_bytes) / us / 1e3, 1),
           "store_tokens_per_s": round(n / us * 1e6, 1),
           "note": "a 32 MB pool: the step runs from the caches, so GB/s here is not an HBM "
                   "figure; device time per step, the steps queued behind a spin kernel so "
                   "that no host launch time is counted"}
    if not cpu:
        return res
    from oracle import fp8_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    kc = torch.zeros(C1_POOL, BS, HK, D, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ks = torch.ones(C1_POOL, BS, HK)
    vs = torch.ones_like(ks)
    kf, vf, sl = w["key"], w["value"], w["slots"]
    t_store = t_dec = 0.0
    reps = 0
    while t_store + t_dec < cpu_budget_s:
        t0 = time.perf_counter()
        O.store_fp8_kvcache_torch(kf, vf, kc, vc, ks, vs, sl)
        t1 = time.perf_counter()
        O.decode_attention(w["q"], kc, vc, ks, vs, w["lens"], w["tables"], D ** -0.5)
        t2 = time.perf_counter()
        t_store += t1 - t0
        t_dec += t2 - t1
        reps += 1
    res["cpu_baseline"] = {
        "store_tokens_per_s": round(reps * n / t_store, 1),
        "store_cores": torch.get_num_threads(),
        "decode_gbs": round(reps * dec_bytes / t_dec / 1e9, 3),
        "decode_cores": torch.get_num_threads(),
        "step_us": round((t_store + t_dec) / reps * 1e6, 1),
        "kind": "port",
        "sample": f"{reps} repetitions of the whole step: the oracle's store vectorized in "
                  f"torch CPU ops and its torch fp32 decode, {t_store + t_dec:.1f} s"}
    return res


PRE_SEQS, PRE_CACHED, PRE_NEW = 8, 8192, 2048
FP8_PEAK_TFLOPS = 5000.0


def prefill_flops(seqs, cached, new, hq, d):
    """Causal-exact QK^T + PV FLOP: query i of a sequence sees cached + i + 1
    positions."""
    visits = new * cached + new * (new + 1) // 2
    return 4 * d * visits * hq * seqs


def prefill_workload(dev, dtype=torch.bfloat16):
    """Varlen chunked prefill: 8 sequences x (8192 cached + 2048 new tokens),
    32 q / 8 kv heads, q/k/v N(0,1) (bf16 by default) with 1% of K entries
    x20, all 10240 tokens of each sequence stored first (as Attention
    does).  Returns the tensors one prefill call reads."""
    from microserve_amd import store_fp8_kvcache
    gen = torch.Generator().manual_seed(77)
    lk = PRE_CACHED + PRE_NEW
    pages = lk // BS
    pool = PRE_SEQS * pages + 1
    perm = torch.randperm(pool, generator=gen)[:PRE_SEQS * pages].to(torch.int32)
    tables = perm.view(PRE_SEQS, pages).contiguous()
    pos = torch.arange(lk)
    slots = (tables[:, pos // BS].long() * BS + pos % BS).reshape(-1)
    key = torch.randn(slots.numel(), HK, D, generator=gen)
    key = torch.where(torch.rand(key.shape, generator=gen) < 0.01, key * 20, key).to(dtype)
    value = torch.randn(slots.numel(), HK, D, generator=gen).to(dtype)
    kc = torch.zeros(pool, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(pool, BS, HK, device=dev)
    vs = torch.ones_like(ks)
    store_fp8_kvcache(key.to(dev), value.to(dev), kc, vc, ks, vs, slots.to(dev))
    q = torch.randn(PRE_SEQS * PRE_NEW, HQ, D, generator=gen).to(dtype).to(dev)
    cu_q = torch.arange(0, PRE_SEQS + 1, dtype=torch.int32, device=dev) * PRE_NEW
    cu_k = torch.arange(0, PRE_SEQS + 1, dtype=torch.int32, device=dev) * lk
    return dict(q=q, kc=kc, vc=vc, ks=ks, vs=vs, tables=tables.to(dev), cu_q=cu_q, cu_k=cu_k,
                max_seqlen_q=PRE_NEW)


def run_prefill(w):
    from microserve_amd import fp8_varlen_prefill_attention
    return fp8_varlen_prefill_attention(w["q"], w["kc"], w["vc"], w["ks"], w["vs"], w["tables"],
                                        w["cu_q"], w["cu_k"], w["max_seqlen_q"], D ** -0.5)


def _time_sustained(run, iters, warmup):
    """HIP-event times of a compute-bound call after a one-second idle:
    (mean of the last `iters` calls, mean of the first `iters`).  From idle
    the shader clock ramps up over the first ~50 ms of matrix-core load, so
    the first calls of a ~2.5 ms kernel run up to ~25% slower than later
    ones.  The ramp repeats after every idle second, and a 100 ms spin
    kernel beforehand does not shorten it.  The steady-state mean is the
    figure of a continuously loaded engine; the first-calls mean is
    reported beside it."""
    time.sleep(1.0)
    stream = torch.cuda.current_stream()
    n = warmup + iters
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n)]
    for e0, e1 in evs:
        e0.record(stream)
        run()
        e1.record(stream)
    torch.cuda.synchronize()
    d = [a.elapsed_time(b) * 1e3 for a, b in evs]
    return sum(d[warmup:]) / iters, sum(d[:iters]) / iters


def time_prefill(dev, iters=20, warmup=40, dtype=torch.bfloat16):
    """The varlen chunked prefill workload (prefill_workload), HIP-event time
    per call at steady clocks (_time_sustained)."""
    w = prefill_workload(dev, dtype)
    us, us_cold = _time_sustained(lambda: run_prefill(w), iters, warmup)
    flop = prefill_flops(PRE_SEQS, PRE_CACHED, PRE_NEW, HQ, D)
    tflops = flop / us / 1e6
    dname = "bf16" if dtype == torch.bfloat16 else "fp16"
    return _with_mfma({
        "workload": "varlen chunked prefill, 8 seqs x (8192 cached + 2048 new), "
                    f"32 q / 8 kv heads, fp8 cache, {str(dtype).split('.')[-1]} q",
        "us": round(us, 2), "flop": flop, "tflops": round(tflops, 1),
        "peak_tflops": FP8_PEAK_TFLOPS, "frac": round(tflops / FP8_PEAK_TFLOPS, 4),
        "timing": f"mean of calls {warmup + 1}-{warmup + iters} after a 1 s idle",
        "us_first_calls": round(us_cold, 2)}, f"prefill_fp8_{dname}")


_SPIN_CYCLES_PER_MS = None


def _spin(ms):
    """Keep the current stream busy for about `ms` milliseconds (torch's
    clock-spin kernel, its rate measured once)."""
    global _SPIN_CYCLES_PER_MS
    if _SPIN_CYCLES_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SPIN_CYCLES_PER_MS = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(_SPIN_CYCLES_PER_MS * ms))


def _time_steps(step, iters, warmup):
    """Average device time of step(i) on the current stream, in us.  The
    timed steps are queued behind a spin kernel long enough for the host to
    enqueue all of them, so each event pair brackets the step's kernels and
    the gaps between them, not the host's launch path (which is slower
    than the GPU for steps of a few tens of microseconds)."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(iters)]
    _spin(0.25 * iters + 5.0)
    for i, (e0, e1) in enumerate(evs):
        e0.record(stream)
        step(i)
        e1.record(stream)
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / iters * 1e3


def _fill_pages(dev, kc, vc, ks, vs, pages, gen, chunk_pages=512):
    """store_fp8_kvcache every token of the given pages from bf16 N(0,1)
    drawn on the device."""
    from microserve_amd import store_fp8_kvcache
    bs, hk, d = kc.shape[1], kc.shape[2], kc.shape[3]
    dgen = torch.Generator(device=dev).manual_seed(int(torch.randint(1 << 30, (1,), generator=gen)))
    for i in range(0, pages.numel(), chunk_pages):
        pg = pages[i:i + chunk_pages].to(dev).long()
        slots = (pg[:, None] * bs + torch.arange(bs, device=dev)[None]).reshape(-1)
        key = torch.randn(slots.numel(), hk, d, generator=dgen, device=dev, dtype=torch.bfloat16)
        value = torch.randn(slots.numel(), hk, d, generator=dgen, device=dev, dtype=torch.bfloat16)
        store_fp8_kvcache(key, value, kc, vc, ks, vs, slots)


def ragged_workload(dev):
    """Ragged decode stress at the Qwen3-8B shape: batch 256, context lengths
    log-uniform in [16, 32768], each sequence's blocks sampled without
    replacement from a 40,000-block pool, every page filled by
    store_fp8_kvcache from bf16 N(0,1); one step is the one-token
    store_kvcache append of every sequence (at its last position) followed
    by the decode.  Returns the step's tensors."""
    gen = torch.Generator().manual_seed(3)
    b, pool = 256, 40000
    lens = torch.exp(torch.empty(b).uniform_(float(torch.log(torch.tensor(16.0))),
                                             float(torch.log(torch.tensor(32768.0))),
                                             generator=gen)).long()
    pages = (lens + BS - 1) // BS
    width = int(pages.max())
    perm = torch.randperm(pool, generator=gen)
    tables = torch.full((b, width), -1, dtype=torch.int32)
    at = 0
    for i in range(b):
        tables[i, :pages[i]] = perm[at:at + pages[i]].to(torch.int32)
        at += int(pages[i])
    kc = torch.zeros(pool, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(pool, BS, HK, device=dev)
    vs = torch.ones_like(ks)
    _fill_pages(dev, kc, vc, ks, vs, perm[:at], gen)
    # the appended token of each sequence is its last position
    last = (lens - 1)
    slots = (tables[torch.arange(b), last // BS].long() * BS + last % BS)
    knew = torch.randn(b, HK, D, generator=gen).bfloat16()
    vnew = torch.randn(b, HK, D, generator=gen).bfloat16()
    q = torch.randn(b, HQ, D, generator=gen).bfloat16()
    return dict(lens=lens, tables=tables, tables_d=tables.to(dev),
                seqlens=lens.to(torch.int32).to(dev), kc=kc, vc=vc, ks=ks, vs=vs,
                slots=slots, slots_d=slots.to(dev), knew=knew, knew_d=knew.to(dev),
                vnew=vnew, vnew_d=vnew.to(dev), q=q, q_d=q.to(dev))


def ragged_append(w):
    from microserve_amd import store_fp8_kvcache
    store_fp8_kvcache(w["knew_d"], w["vnew_d"], w["kc"], w["vc"], w["ks"], w["vs"], w["slots_d"])


def ragged_decode(w, out=None):
    from microserve_amd import fp8_decode_attention
    return fp8_decode_attention(w["q_d"], w["kc"], w["vc"], w["ks"], w["vs"], w["seqlens"],
                                w["tables_d"], D ** -0.5, out=out)


def time_ragged(dev, iters=50, warmup=5):
    """The ragged step (ragged_workload): append + decode, and the append's
    store alone (256 tokens, a launch-latency-bound call)."""
    w = ragged_workload(dev)
    b = w["lens"].numel()
    out = torch.empty_like(w["q_d"])

    def step(i):
        ragged_append(w)
        ragged_decode(w, out)

    us = _time_steps(step, iters, warmup)
    append_us = _time_steps(lambda i: ragged_append(w), iters, warmup)
    lens = w["lens"]
    nbytes = decode_bytes_ragged(lens, HQ, HK, D) + store_bytes(b, HK, D)
    return {"workload": "ragged decode, batch 256, context log-uniform [16, 32768], "
                        "40k-block fragmented pool, with the one-token append store",
            "tokens": int(lens.sum()), "us": round(us, 2), "bytes": nbytes,
            "gbs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "append_us": round(append_us, 2),
            "append_tokens_per_s": round(b / append_us * 1e6, 1)}


def decode_bytes_ragged(lens, hq, hk, d, act_bytes=2):
    kv = int(lens.sum()) * (2 * hk * d + 2 * hk * 4)
    qo = len(lens) * hq * d * act_bytes * 2
    tables = 4 * (int(((lens + BS - 1) // BS).sum()) + len(lens))
    return kv + qo + tables


def long_workload(dev, batch):
    """Long-context decode inputs at the Qwen3-32B shape: 64 q / 8 kv heads,
    every sequence at context 131072 (512 blocks), and two disjoint block
    table sets over one filled pool."""
    gen = torch.Generator().manual_seed(5 + batch)
    hq, ctx = 64, 131072
    pages = ctx // BS
    pool = 2 * batch * pages
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    kc = torch.zeros(pool, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(pool, BS, HK, device=dev)
    vs = torch.ones_like(ks)
    _fill_pages(dev, kc, vc, ks, vs, perm, gen)
    tabs = [perm[:batch * pages].view(batch, pages).contiguous().to(dev),
            perm[batch * pages:].view(batch, pages).contiguous().to(dev)]
    seqlens = torch.full((batch,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn(batch, hq, D, generator=gen).bfloat16().to(dev)
    return dict(q=q, kc=kc, vc=vc, ks=ks, vs=vs, seqlens=seqlens, tables=tabs, hq=hq, ctx=ctx,
                pages=pages)


def time_long_context(dev, batch, iters=50, warmup=5):
    """Long-context decode (long_workload); the two block sets alternate
    between steps so the MALL cannot serve the reads."""
    from microserve_amd import decode_num_splits, fp8_decode_attention
    w = long_workload(dev, batch)
    hq, ctx, pages = w["hq"], w["ctx"], w["pages"]
    out = torch.empty_like(w["q"])

    def step(i):
        fp8_decode_attention(w["q"], w["kc"], w["vc"], w["ks"], w["vs"], w["seqlens"],
                             w["tables"][i % 2], D ** -0.5, out=out)

    us = _time_steps(step, iters, warmup)
    nbytes = decode_bytes(batch, ctx, hq, HK, D)
    return {"workload": f"Qwen3-32B long-context decode, batch {batch} x context 131072",
            "splits": decode_num_splits(batch, hq, HK, pages, BS),
            "us": round(us, 2), "bytes": nbytes, "gbs": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


FRESH_SEQS, FRESH_LEN = 8, 8192
BF16_PEAK_TFLOPS = 2500.0


def fresh_workload(dev, dtype=torch.bfloat16):
    """Fresh PREFILL inputs: 8 sequences x 8192 new tokens, 32 q / 8 kv
    heads, q/k/v N(0,1) in `dtype`, and their cu_seqlens."""
    gen = torch.Generator().manual_seed(88)
    n = FRESH_SEQS * FRESH_LEN
    q = torch.randn(n, HQ, D, generator=gen).to(dtype).to(dev)
    k = torch.randn(n, HK, D, generator=gen).to(dtype).to(dev)
    v = torch.randn(n, HK, D, generator=gen).to(dtype).to(dev)
    cu = torch.arange(0, FRESH_SEQS + 1, dtype=torch.int32, device=dev) * FRESH_LEN
    return dict(q=q, k=k, v=v, cu=cu)


def run_fresh_prefill(w):
    from microserve_amd import varlen_attention
    return varlen_attention(w["q"], w["k"], w["v"], w["cu"], w["cu"], FRESH_LEN, FRESH_LEN,
                            D ** -0.5)


def time_fresh_prefill(dev, iters=20, warmup=30, dtype=torch.bfloat16):
    """Fresh PREFILL (unquantized q/k/v, causal, the flash_attn_varlen_func
    call of the FP8 path): fresh_workload's 8 sequences x 8192 new tokens in
    bf16, or in fp16, the activation type the reference requires with an
    FP8 cache (Config.py:35-36)."""
    w = fresh_workload(dev, dtype)

    def run():
        return run_fresh_prefill(w)

    us, us_cold = _time_sustained(run, iters, warmup)
    flop = prefill_flops(FRESH_SEQS, 0, FRESH_LEN, HQ, D)
    tflops = flop / us / 1e6
    dname = "bf16" if dtype == torch.bfloat16 else "fp16"
    return _with_mfma({
        "workload": "fresh causal prefill, 8 seqs x 8192 tokens, 32 q / 8 kv heads, "
                    f"{dname} q/k/v (16-bit MFMA)",
        "us": round(us, 2), "flop": flop, "tflops": round(tflops, 1),
        "peak_tflops": BF16_PEAK_TFLOPS, "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
        "timing": f"mean of calls {warmup + 1}-{warmup + iters} after a 1 s idle",
        "us_first_calls": round(us_cold, 2)}, f"dense_prefill_{dname}")


class _Seq:
    """The attributes of the runner's Sequence that its builders read."""

    def __init__(self, token_ids, computed, scheduled, table, total=None):
        self.token_ids = token_ids
        self.num_computed_tokens = computed
        self.num_scheduled_tokens = scheduled
        self.block_table = table
        self.gap = (len(token_ids) if total is None else total) - computed


def _ragged_decode_seqs(seed=42, batch=256, pool=40000):
    import numpy as np
    rng = np.random.default_rng(seed)
    lens = np.exp(rng.uniform(np.log(16), np.log(32768), batch)).astype(np.int64)
    perm = rng.permutation(pool)
    seqs, at = [], 0
    for n in lens.tolist():
        pages = -(-n // BS)
        seqs.append(_Seq(rng.integers(0, 151936, n).tolist(), n - 1, 1,
                         perm[at:at + pages].tolist()))
        at += pages
    return seqs


def _elementwise_decode_inputs(seqs, dev):
    """The per-element device writes the runner's decode builder and block
    table builder make (model_runner.py:124-142, 208-216): one host-to-device
    copy per element and one per table row; timed as the path the device
    builder replaces."""
    n = len(seqs)
    ids = torch.empty(n, dtype=torch.int64, device=dev)
    pos = torch.empty(n, dtype=torch.int64, device=dev)
    slot = torch.empty(n, dtype=torch.int64, device=dev)
    lens = torch.empty(n, dtype=torch.int32, device=dev)
    for i, s in enumerate(seqs):
        p = s.num_computed_tokens
        ids[i] = s.token_ids[p]
        pos[i] = p
        slot[i] = s.block_table[p // BS] * BS + p % BS
        lens[i] = p + 1
    width = max(len(s.block_table) for s in seqs)
    tables = torch.full((n, width), -1, dtype=torch.int32, device=dev)
    for i, s in enumerate(seqs):
        if s.block_table:
            tables[i, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32,
                                                          device=dev)
    return ids, pos, slot, lens, tables


def _elementwise_prefill_inputs(seqs, dev):
    """The per-element device writes of the runner's prefill builder
    (model_runner.py:144-172)."""
    total = sum(s.num_scheduled_tokens for s in seqs)
    ids = torch.empty(total, dtype=torch.int64, device=dev)
    pos = torch.empty(total, dtype=torch.int64, device=dev)
    slot = torch.empty(total, dtype=torch.int64, device=dev)
    off = 0
    for s in seqs:
        for j in range(s.num_scheduled_tokens):
            ids[off + j] = s.token_ids[j]
            pos[off + j] = j
            slot[off + j] = s.block_table[j // BS] * BS + j % BS
        off += s.num_scheduled_tokens
    return ids, pos, slot


def _wall_us(fn, iters):
    import statistics
    times = []
    for _ in range(iters):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e6)
    return statistics.median(times)


def _cpu_step_inputs(seqs):
    """The oracle's restatement of the runner's decode builder on the host
    (host arrays, no device copies): microseconds for one step."""
    from oracle import step_inputs_oracle as SO
    t0 = time.perf_counter()
    SO.compile_decode(seqs, BS)
    return (time.perf_counter() - t0) * 1e6


def time_step_inputs(dev, iters=30):
    """Per-step input building: the device builder (one pinned copy + one
    step_inputs_kernel launch) against the runner's element-by-element device
    writes, each timed host wall clock to completion (median)."""
    import numpy as np
    from microserve_amd import step_inputs as SI
    seqs = _ragged_decode_seqs()
    SI.compile_decode(seqs, BS, dev)
    dec_us = _wall_us(lambda: SI.compile_decode(seqs, BS, dev), iters)
    width = max(len(s.block_table) for s in seqs)
    gv = {"input_ids": torch.zeros(256, dtype=torch.int64, device=dev),
          "positions": torch.zeros(256, dtype=torch.int64, device=dev),
          "slot_mapping": torch.zeros(256, dtype=torch.int64, device=dev),
          "cache_seqlens": torch.zeros(256, dtype=torch.int32, device=dev),
          "block_tables": torch.zeros(256, width, dtype=torch.int32, device=dev)}
    graph_us = _wall_us(lambda: SI.compile_decode(seqs[:200], BS, dev, pad_to=256,
                                                  table_width=width, garbage_slot=40000 * BS,
                                                  out=gv), iters)
    _elementwise_decode_inputs(seqs, dev)
    ref_dec_us = _wall_us(lambda: _elementwise_decode_inputs(seqs, dev), 3)
    rng = np.random.default_rng(43)
    pre = [_Seq(rng.integers(0, 151936, FRESH_LEN).tolist(), 0, FRESH_LEN,
                list(range(i * (FRESH_LEN // BS), (i + 1) * (FRESH_LEN // BS))))
           for i in range(FRESH_SEQS)]
    SI.compile_prefill(pre, BS, dev)
    pre_us = _wall_us(lambda: SI.compile_prefill(pre, BS, dev), 10)
    sample = [_Seq(s.token_ids[:256], 0, 256, s.block_table[:1]) for s in pre]
    _elementwise_prefill_inputs(sample, dev)
    ref_sample_us = _wall_us(lambda: _elementwise_prefill_inputs(sample, dev), 3)
    ref_pre_us = ref_sample_us * FRESH_LEN / 256
    cpu_dec_us = _cpu_step_inputs(seqs)
    return {"decode": {"workload": "decode step, batch 256, context log-uniform on "
                                   "[16, 32768], block 256, 40k-block pool",
                       "us": round(dec_us, 1), "graph_padded_us": round(graph_us, 1),
                       "elementwise_us": round(ref_dec_us, 1),
                       "speedup": round(ref_dec_us / dec_us, 1),
                       "cpu_baseline": {"value": round(cpu_dec_us, 1), "unit": "us", "cores": 1,
                                        "kind": "port",
                                        "sample": "the oracle's loops building the same step "
                                                  "into host arrays (no device copies)"}},
            "prefill": {"workload": "fresh prefill step, 8 prompts x 8192 tokens, block 256",
                        "us": round(pre_us, 1),
                        "elementwise_us": round(ref_pre_us, 1),
                        "elementwise_sample": "8 prompts x 256 tokens timed, scaled x32 "
                                              "(linear in tokens)",
                        "speedup": round(ref_pre_us / pre_us, 1)}}


def norm_rope_bytes(n, hq, hk, with_k, act=2):
    """Algorithmic HBM bytes of the fused prologue for n tokens: q/k/v rows
    read once, cos/sin rows once per token, positions and slots; q (and k)
    written once, k/v FP8 rows and their scales."""
    rd = n * ((hq + 2 * hk) * D * act + 2 * D * act + 8 + 8)
    wr = n * (hq * D * act + (hk * D * act if with_k else 0) + 2 * hk * D + 2 * hk * 4)
    return rd + wr


def _unfused_prologue(positions, q, k, v, qw, kw, eps, cos, sin, cache, slots):
    """The reference's chain on the GPU (microserve/models/qwen3.py:49-53 with
    layernorm.py:55-57,80-81 and rotary_embedding.py:24-31, then the store at
    attention.py:41-43): torch ops for the norms and the rotation, this
    library's store kernel for the cache."""
    from microserve_amd import store_fp8_kvcache

    def norm(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(x.dtype) * w

    def rot(x):
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((-x2, x1), dim=-1)

    q, k = norm(q, qw), norm(k, kw)
    c = cos[positions].unsqueeze(1)
    s_ = sin[positions].unsqueeze(1)
    q, k = (q * c) + (rot(q) * s_), (k * c) + (rot(k) * s_)
    store_fp8_kvcache(k, v, *cache, slots)
    return q, k


NORM_ROPE_STEPS = ((FRESH_SEQS * FRESH_LEN, "prefill", torch.bfloat16),
                   (BATCH, "decode", torch.bfloat16),
                   (FRESH_SEQS * FRESH_LEN, "prefill", torch.float16))


def norm_rope_workloads(dev, steps=len(NORM_ROPE_STEPS)):
    """The fused prologue's inputs, Qwen3-8B heads, one dict per step of
    NORM_ROPE_STEPS (the first `steps` of them, drawn in order from one
    generator): q/k/v N(0,1) viewed from one [n, (32 + 2 * 8) * 128]
    projection, random positions under 40960, weights 1 + N(0, 0.1), slots a
    random permutation of a pool of ceil(n / 256) blocks."""
    gen = torch.Generator().manual_seed(77)
    for n, mode, dt in NORM_ROPE_STEPS[:steps]:
        cos_t, sin_t = (t.to(dev) for t in _rope_tables(40960, dt))
        qkv = torch.randn(n, (HQ + 2 * HK) * D, generator=gen).to(dt).to(dev)
        q, k, v = (t.view(n, -1, D) for t in qkv.split([HQ * D, HK * D, HK * D], dim=-1))
        pos = torch.randint(0, 40960, (n,), generator=gen).to(dev)
        qw = (1 + 0.1 * torch.randn(D, generator=gen)).to(dt).to(dev)
        kw = (1 + 0.1 * torch.randn(D, generator=gen)).to(dt).to(dev)
        nb = max(1, -(-n // BS))
        slots = torch.randperm(nb * BS, generator=gen)[:n].to(dev)
        cache = (torch.zeros(nb, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev),
                 torch.zeros(nb, BS, HK, D, dtype=torch.float8_e4m3fn, device=dev),
                 torch.ones(nb, BS, HK, device=dev), torch.ones(nb, BS, HK, device=dev))
        yield dict(n=n, mode=mode, dtype=dt, cos=cos_t, sin=sin_t, qkv=qkv, q=q, k=k, v=v,
                   pos=pos, qw=qw, kw=kw, nb=nb, slots=slots, cache=cache)


def time_norm_rope(dev, iters=20, warmup=3):
    """Fused q/k RMSNorm + rotary + FP8 store against the reference's unfused
    torch chain (plus the store kernel), Qwen3-8B heads: the prefill and
    decode steps in bf16, and the prefill step in fp16, the activation type
    the reference requires with an FP8 cache (Config.py:35-36)."""
    from microserve_amd import qk_norm_rope_store
    out = []
    for w in norm_rope_workloads(dev):
        n, mode, dt = w["n"], w["mode"], w["dtype"]
        cos_t, sin_t, q, k, v, pos, qw, kw = (w[x] for x in
                                              ("cos", "sin", "q", "k", "v", "pos", "qw", "kw"))
        qkv, nb, slots, cache = w["qkv"], w["nb"], w["slots"], w["cache"]
        with_k = mode == "prefill"

        def fused():
            return qk_norm_rope_store(pos, q, k, v, qw, kw, 1e-6, cos_t, sin_t, *cache, slots,
                                      return_k=with_k)

        def unfused():
            return _unfused_prologue(pos, q, k, v, qw, kw, 1e-6, cos_t, sin_t, cache, slots)

        res = {}
        for name, fn in (("fused", fused), ("unfused", unfused)):
            # device time per call: the calls queued behind a spin kernel
            # (_time_steps), so no host launch time is counted
            res[name] = _time_steps(lambda i: fn(), iters, warmup)
        # the host's cost per fused call (ctypes and Python argument checks):
        # back-to-back calls with no spin ahead, wall clock per call
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fused()
        host_us = (time.perf_counter() - t0) / iters * 1e6
        torch.cuda.synchronize()
        nbytes = norm_rope_bytes(n, HQ, HK, with_k)
        cpu = (_cpu_norm_rope(qkv, pos, qw, kw, cos_t, sin_t, slots, nb)
               if mode == "prefill" and dt == torch.bfloat16 else None)
        dname = "bf16" if dt == torch.bfloat16 else "fp16"
        out.append({"workload": f"{mode}: {n} tokens, 32 q / 8 kv heads, {dname}, rotary table "
                                f"40960 x 128",
                    "us": round(res["fused"], 2), "unfused_us": round(res["unfused"], 2),
                    "speedup": round(res["unfused"] / res["fused"], 2),
                    "host_us_per_call": round(host_us, 2),
                    "bytes": nbytes, "gbs": round(nbytes / res["fused"] / 1e3, 1),
                    "frac": round(nbytes / res["fused"] / 1e3 / HBM_PEAK_GBS, 4),
                    **({"cpu_baseline": cpu} if cpu else {})})
    return out


def _cpu_norm_rope(qkv, pos, qw, kw, cos_t, sin_t, slots, nb, sample=4096):
    """The oracle's norm + rotary + FP8 store on the host cores, on the first
    ``sample`` tokens of the same step (a bounded sample)."""
    import numpy as np
    from oracle import fp8_oracle as O
    from oracle import norm_rope_oracle as NR
    torch.set_num_threads(os.cpu_count() or 1)
    x = qkv[:sample].cpu()
    p = pos[:sample].cpu()
    q, k, v = (t.view(sample, -1, D) for t in x.split([HQ * D, HK * D, HK * D], dim=-1))
    c, s_ = cos_t.cpu(), sin_t.cpu()
    w_q, w_k = qw.cpu(), kw.cpu()
    sl = slots[:sample].cpu().numpy()
    kc = np.zeros((nb, BS, HK, D), np.uint8)
    vc = np.zeros_like(kc)
    ks = np.ones((nb, BS, HK), np.float32)
    vs = np.ones_like(ks)
    kc, vc = torch.from_numpy(kc), torch.from_numpy(vc)
    ks, vs = torch.from_numpy(ks), torch.from_numpy(vs)
    t0 = time.perf_counter()
    _, rk = NR.qk_norm_rope(q, k, p, w_q, w_k, 1e-6, c, s_)
    O.store_fp8_kvcache_torch(rk, v, kc, vc, ks, vs, torch.from_numpy(sl))
    dt = time.perf_counter() - t0
    return {"value": round(sample / dt, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{sample} tokens of the prefill step, oracle in numpy/torch "
                                      f"on the host"}


def _rope_tables(max_position, dtype, base=1e6):
    """cos/sin tables as the reference builds them (rotary_embedding.py:16-22)
    after the runner's cast to the activation type."""
    inv_freq = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    freqs = torch.einsum("i,j -> ij", torch.arange(max_position, dtype=torch.float32), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def calibrate_copy(dev, nbytes=1 << 30, iters=5):
    """A plain device copy of known size, for scaling the FETCH_SIZE and
    WRITE_SIZE counters to bytes (run it under rocprofv3 --pmc)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "torch copy_", "bytes_read_per_launch": nbytes,
                      "bytes_written_per_launch": nbytes, "launches": iters}), flush=True)


def mfma_counters(name):
    """MFMA utilization of a prefill kernel from the committed rocprofv3
    --pmc summary: the busy fraction of the matrix pipe
    (SQ_VALU_MFMA_BUSY_CYCLES over the SIMDs' active cycles) and VALU
    instructions per MFMA.  frac / mfma_busy is the fraction of peak the
    kernel's own instruction mix would reach with the pipe always busy."""
    path = os.path.join(ROOT, "profiles", "prefill_kernel_trace_and_mfma.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"mfma_counters {name}:"):
                    kv = dict(x.split("=") for x in line.split(":", 1)[1].split())
                    return ({"mfma_busy": float(kv["mfma_busy"]),
                             "valu_per_mfma": float(kv["valu_per_mfma"]),
                             "mfma_source": os.path.relpath(path, ROOT)})
    except (OSError, ValueError, KeyError):
        pass
    return {}


def _with_mfma(res, name):
    """res plus the kernel's MFMA counters and the fraction of peak at a
    fully busy matrix pipe."""
    c = mfma_counters(name)
    if c:
        res.update(c)
        res["frac_at_full_mfma"] = round(res["frac"] / c["mfma_busy"], 4)
    return res


def measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = os.path.join(ROOT, "profiles", "decode_qwen3_8b_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1].strip()), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--decode-only", action="store_true",
                    help="time decode only (no store fill timing, no CPU baseline)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the varlen chunked prefill workload")
    ap.add_argument("--prefill-dtype", choices=["bf16", "fp16"], default="bf16",
                    help="activation type of the --prefill-only and --fresh-only workloads")
    ap.add_argument("--fresh-only", action="store_true",
                    help="time only the fresh (unquantized) prefill workload")
    ap.add_argument("--shapes-only", action="store_true",
                    help="time only the ragged and long-context decode workloads")
    ap.add_argument("--norm-rope-only", action="store_true",
                    help="time only the fused q/k norm + rotary + store prologue")
    ap.add_argument("--config1-only", action="store_true",
                    help="time only the Qwen3-0.6B batch-4 store + decode step")
    ap.add_argument("--step-inputs-only", action="store_true",
                    help="time only the per-step input builder")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run the 1 GiB copy used to calibrate rocprofv3 byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs the path on a single "
              "MI355X (multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)
    dev = "cuda:0"
    if args.calibrate_copy:
        calibrate_copy(dev)
        return
    if args.shapes_only:
        print(json.dumps({"ragged": time_ragged(dev),
                          "long_context": [time_long_context(dev, b) for b in (1, 2, 4)]}))
        return
    if args.fresh_only:
        dtype = torch.bfloat16 if args.prefill_dtype == "bf16" else torch.float16
        print(json.dumps({"fresh_prefill": time_fresh_prefill(dev, dtype=dtype)}))
        return
    if args.norm_rope_only:
        print(json.dumps({"qk_norm_rope_store": time_norm_rope(dev)}))
        return
    if args.config1_only:
        print(json.dumps({"config1": time_config1(dev, cpu=not args.no_cpu)}))
        return
    if args.step_inputs_only:
        print(json.dumps({"step_inputs": time_step_inputs(dev)}))
        return
    if args.prefill_only:
        dtype = torch.bfloat16 if args.prefill_dtype == "bf16" else torch.float16
        print(json.dumps({"prefill": time_prefill(dev, dtype=dtype)}))
        return
    from microserve_amd import decode_num_splits, fp8_decode_attention
    w = build_workload(dev)
    torch.cuda.synchronize()
    out = torch.empty_like(w["query"])
    scale = D ** -0.5

    def step(i):
        fp8_decode_attention(w["query"], w["kc"], w["vc"], w["ks"], w["vs"],
                             w["seqlens"], w["tables"][i % 2], scale, out=out)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # whole-job throughput: K back-to-back steps between two synchronizes
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # per-launch durations of the op, HIP events on its stream, own loop
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        evs[i][0].record(stream)
        step(i)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    per_launch = sorted(a.elapsed_time(b) * 1e-3 for a, b in evs)
    avg_launch = sum(per_launch) / len(per_launch)
    nbytes = decode_bytes(BATCH, CTX, HQ, HK, D)
    ms_per_step = wall / args.steps * 1e3
    value = nbytes / (wall / args.steps) / 1e9
    achieved = nbytes / avg_launch / 1e9
    store = None if args.decode_only else time_store_fill(w)
    traffic, traffic_src = measured_traffic()
    result = {
        "metric": "FP8 paged decode-attn HBM GB/s (% of peak) + store_kvcache tokens/s, Qwen3-8B",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 KV, bf16 q/out, fp32 softmax",
        "data": "synthetic: seeded N(0,1) bf16 K/V/q quantized by store_fp8_kvcache",
        "config": {"workload": "Qwen3-8B layer decode: 32 q / 8 kv heads, head_dim 128, "
                               "block 256, batch 64 x context 4096, 2048-block fp8 pool",
                   "splits": decode_num_splits(BATCH, HQ, HK, CTX // BS, BS),
                   "launch": "eager, one decode call per step",
                   "algorithmic_bytes_per_step": nbytes},
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "kernel": "decode_fp8_kernel + decode_combine_small_kernel",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(avg_launch * 1e6, 2),
                     "median_launch_us": round(per_launch[len(per_launch) // 2] * 1e6, 2),
                     "algorithmic_bytes": nbytes,
                     "traffic": traffic, "traffic_source": traffic_src},
    }
    if store is not None:
        result["store"] = {k: (round(v, 4) if isinstance(v, float) else v)
                           for k, v in store.items()}
    if not args.no_cpu and not args.decode_only:
        result["cpu_baseline"] = cpu_baseline(w)
    if not args.decode_only:
        result["config1"] = time_config1(dev, cpu=not args.no_cpu)
        result["prefill"] = time_prefill(dev)
        # fp16 activations, the type the reference requires with an FP8
        # cache (Config.py:35-36)
        result["prefill_fp16"] = time_prefill(dev, dtype=torch.float16)
        result["fresh_prefill"] = time_fresh_prefill(dev)
        result["fresh_prefill_fp16"] = time_fresh_prefill(dev, dtype=torch.float16)
        del w
        torch.cuda.empty_cache()
        result["fp16"] = time_fp16(dev)
        torch.cuda.empty_cache()
        result["ragged"] = time_ragged(dev)
        result["long_context"] = [time_long_context(dev, b) for b in (1, 2, 4)]
        result["step_inputs"] = time_step_inputs(dev)
        result["qk_norm_rope_store"] = time_norm_rope(dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
