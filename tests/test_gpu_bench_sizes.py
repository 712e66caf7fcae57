"""GPU parity at the sizes bench.py reports, on the very tensors it times
(its workload builders are imported, not restated):

* the Qwen3-8B pool fill (2 x 262,144 tokens): every cache byte and scale
  against the oracle's quantizer and the placement rule
  (``fp8_kv_cache.py:24-39``), and both decode table sets against the
  oracle's decode;
* the ragged batch-256 step over the 40,000-block pool: the one-token
  append's bytes, then every output row of the decode that follows it
  (``fp8_decode_attention.py:16-58``);
* the 8 x (8192 cached + 2048 new) chunked prefill with 1% x20 K outliers,
  bf16 and fp16: every output finite, and 512 query tokens per sequence (the
  first and last token of every 128-row workgroup block, the sequence's last
  token, the rest random) against the oracle over ``prefix + i + 1`` keys
  (``fp8_chunk_prefill_attention.py:52-54``);
* the 8 x 8192 fresh prefill, bf16 and fp16: every output finite, and 512
  query tokens per sequence (the first and last of every 192-row workgroup
  block, the rest random) against the unquantized oracle over keys 0..i
  (``attention.py:49-55``).

* the Qwen3-32B 131072-token decode at batch 2 and 4, both block table
  sets, against the oracle's decode (``fp8_decode_attention.py:16-58``);
* the 65,536-token fused prologue steps, bf16 and fp16: q, k, every cache
  byte and scale bit-exact against the oracle (``qwen3.py:49-53``,
  ``fp8_kv_cache.py:24-39``).

The fill and decode check runs in bf16 and in fp16, the activation type
the reference requires with an FP8 cache (``Config.py:35-36``).
"""

import numpy as np
import pytest
import torch

import bench
from oracle import fp8_oracle as O
from tests import gpu_helpers as H

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_store_fill_qwen3_8b_every_byte_and_decode(dtype):
    w = bench.build_workload(H.DEV, dtype)
    torch.cuda.synchronize()
    kc8 = w["kc"].view(torch.uint8).view(-1, bench.HK, bench.D)
    vc8 = w["vc"].view(torch.uint8).view(-1, bench.HK, bench.D)
    ksf = w["ks"].view(-1, bench.HK)
    vsf = w["vs"].view(-1, bench.HK)
    written = torch.zeros(kc8.shape[0], dtype=torch.bool)
    for half, (key, value, slots) in enumerate(w["fills"]):
        n = slots.numel()
        assert n == 262144
        print(f"fill half {half}: {n} tokens", flush=True)
        kq, kscale = H.oracle_quantize_threaded(key)
        vq, vscale = H.oracle_quantize_threaded(value)
        # row slot of the flattened cache holds token t (fp8_kv_cache.py:29-39)
        assert np.array_equal(kc8[slots].cpu().numpy(), kq), "k bytes"
        assert np.array_equal(vc8[slots].cpu().numpy(), vq), "v bytes"
        assert np.array_equal(ksf[slots].cpu().numpy().view(np.uint32), kscale.view(np.uint32))
        assert np.array_equal(vsf[slots].cpu().numpy().view(np.uint32), vscale.view(np.uint32))
        written[slots.cpu()] = True
    assert bool(written.all())  # the two halves tile the whole 2048-block pool
    scale = bench.D ** -0.5
    from microserve_amd import fp8_decode_attention
    for half in range(2):
        out = fp8_decode_attention(w["query"], w["kc"], w["vc"], w["ks"], w["vs"], w["seqlens"],
                                   w["tables"][half], scale)
        torch.cuda.synchronize()
        caches, tables = H.compact_cache((w["kc"], w["vc"], w["ks"], w["vs"]), w["tables"][half])
        ref = O.decode_attention(w["query"].cpu(), *caches, w["seqlens"].cpu(), tables, scale)
        max_abs, rel = H.assert_attention_close(out, ref)
        print(f"decode {dtype} half {half}: max_abs {max_abs:.3e} rel {rel:.3e}", flush=True)


def test_ragged_batch256_step_append_and_decode():
    w = bench.ragged_workload(H.DEV)
    lens = w["lens"]
    print(f"ragged: {lens.numel()} sequences, {int(lens.sum())} tokens, "
          f"table width {w['tables'].shape[1]}", flush=True)
    bench.ragged_append(w)
    out = bench.ragged_decode(w)
    torch.cuda.synchronize()
    # the appended rows: bit-exact at their slots
    kq, kscale = O.quantize_rows(w["knew"].float().numpy())
    vq, vscale = O.quantize_rows(w["vnew"].float().numpy())
    rows = w["slots_d"]
    assert np.array_equal(w["kc"].view(torch.uint8).view(-1, 8, 128)[rows].cpu().numpy(), kq)
    assert np.array_equal(w["vc"].view(torch.uint8).view(-1, 8, 128)[rows].cpu().numpy(), vq)
    assert np.array_equal(w["ks"].view(-1, 8)[rows].cpu().numpy().view(np.uint32),
                          kscale.view(np.uint32))
    assert np.array_equal(w["vs"].view(-1, 8)[rows].cpu().numpy().view(np.uint32),
                          vscale.view(np.uint32))
    # every output row against the oracle's decode over the same cache
    caches, tables = H.compact_cache((w["kc"], w["vc"], w["ks"], w["vs"]), w["tables"])
    ref = O.decode_attention(w["q"], *caches, lens, tables, bench.D ** -0.5)
    max_abs, rel = H.assert_attention_close(out, ref)
    print(f"ragged decode: max_abs {max_abs:.3e} rel {rel:.3e}", flush=True)


def _sampled_rows(gen, seqs, lq, per_seq=512, block_tokens=32):
    rows = []
    for s in range(seqs):
        pick = set()
        for j in range(0, lq, block_tokens):
            pick.update((j, min(lq, j + block_tokens) - 1))
        pick.add(lq - 1)
        rest = torch.randperm(lq, generator=gen).tolist()
        for i in rest:
            if len(pick) >= per_seq:
                break
            pick.add(i)
        rows.extend(s * lq + i for i in sorted(pick))
    return torch.tensor(rows)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunked_prefill_full_size_sampled_rows(dtype):
    w = bench.prefill_workload(H.DEV, dtype)
    out = bench.run_prefill(w)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite output"
    rows = _sampled_rows(torch.Generator().manual_seed(5), bench.PRE_SEQS, bench.PRE_NEW)
    assert rows.numel() == bench.PRE_SEQS * 512
    # 128 rows of a workgroup block are 32 query tokens at GQA 4
    assert bench.HQ // bench.HK == 4
    kc = w["kc"].view(torch.uint8).cpu().numpy()
    vc = w["vc"].view(torch.uint8).cpu().numpy()
    ref = O.varlen_prefill_attention(w["q"].cpu(), kc, vc, w["ks"].cpu().numpy(),
                                     w["vs"].cpu().numpy(), w["tables"].cpu(), w["cu_q"].cpu(),
                                     w["cu_k"].cpu(), bench.D ** -0.5, rows=rows)
    max_abs, rel = H.assert_attention_close(out[rows.to(H.DEV)], ref)
    print(f"prefill {dtype}: {rows.numel()} rows, max_abs {max_abs:.3e} rel {rel:.3e}",
          flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fresh_prefill_full_size_sampled_rows(dtype):
    w = bench.fresh_workload(H.DEV, dtype)
    out = bench.run_fresh_prefill(w)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite output"
    # 192 rows of a workgroup block are 48 query tokens at GQA 4
    assert bench.HQ // bench.HK == 4
    rows = _sampled_rows(torch.Generator().manual_seed(6), bench.FRESH_SEQS, bench.FRESH_LEN,
                         block_tokens=48)
    assert rows.numel() == bench.FRESH_SEQS * 512
    ref = O.dense_varlen_attention(w["q"].cpu(), w["k"].cpu(), w["v"].cpu(), w["cu"].cpu(),
                                   w["cu"].cpu(), bench.D ** -0.5, rows=rows)
    max_abs, rel = H.assert_attention_close(out[rows.to(H.DEV)], ref)
    print(f"fresh prefill {dtype}: {rows.numel()} rows, max_abs {max_abs:.3e} rel {rel:.3e}",
          flush=True)


@pytest.mark.parametrize("step", [0, 2])
def test_fused_prologue_full_size_bit_exact(step):
    """The 65,536-token prologue steps bench.py times (step 0 in bf16, step 2
    in fp16): q, k, every cache byte and scale against the oracle."""
    from microserve_amd import qk_norm_rope_store
    from oracle import norm_rope_oracle as NR
    for w in bench.norm_rope_workloads(H.DEV, steps=step + 1):
        pass
    assert w["n"] == 65536 and w["mode"] == "prefill"
    q_out, k_out = qk_norm_rope_store(w["pos"], w["q"], w["k"], w["v"], w["qw"], w["kw"], 1e-6,
                                      w["cos"], w["sin"], *w["cache"], w["slots"], return_k=True)
    torch.cuda.synchronize()
    rq, rk = NR.qk_norm_rope(w["q"].cpu(), w["k"].cpu(), w["pos"].cpu(), w["qw"].cpu(),
                             w["kw"].cpu(), 1e-6, w["cos"].cpu(), w["sin"].cpu())
    assert torch.equal(q_out.cpu(), rq), "q differs"
    assert torch.equal(k_out.cpu(), rk), "k differs"
    kq, kscale = H.oracle_quantize_threaded(rk)
    vq, vscale = H.oracle_quantize_threaded(w["v"])
    slots = w["slots"].cpu()
    kc, vc, ks, vs = w["cache"]
    assert np.array_equal(kc.view(torch.uint8).view(-1, bench.HK, bench.D)[slots].cpu().numpy(), kq)
    assert np.array_equal(vc.view(torch.uint8).view(-1, bench.HK, bench.D)[slots].cpu().numpy(), vq)
    assert np.array_equal(ks.view(-1, bench.HK)[slots].cpu().numpy().view(np.uint32),
                          kscale.view(np.uint32))
    assert np.array_equal(vs.view(-1, bench.HK)[slots].cpu().numpy().view(np.uint32),
                          vscale.view(np.uint32))
    print(f"fused prologue {w['dtype']}: {w['n']} tokens bit-exact", flush=True)


@pytest.mark.parametrize("batch", [2, 4])
def test_long_context_decode_full_size(batch):
    """The Qwen3-32B 131072-token decode bench.py times at batch 2 and 4
    (128 splits per sequence), both block table sets, against the oracle's
    decode (``fp8_decode_attention.py:16-58``)."""
    from microserve_amd import fp8_decode_attention
    w = bench.long_workload(H.DEV, batch)
    scale = bench.D ** -0.5
    for half in range(2):
        out = fp8_decode_attention(w["q"], w["kc"], w["vc"], w["ks"], w["vs"], w["seqlens"],
                                   w["tables"][half], scale)
        torch.cuda.synchronize()
        caches, tables = H.compact_cache((w["kc"], w["vc"], w["ks"], w["vs"]), w["tables"][half])
        ref = O.decode_attention(w["q"].cpu(), *caches, w["seqlens"].cpu(), tables, scale)
        max_abs, rel = H.assert_attention_close(out, ref)
        print(f"131k decode batch {batch} half {half}: max_abs {max_abs:.3e} rel {rel:.3e}",
              flush=True)
