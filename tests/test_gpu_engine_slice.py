"""One Qwen3-shaped attention layer stepped the way the runner steps it, with
no model weights: the runner's FP8 engine test
(``tests/test_fp8_kv_engine.py:13-38`` -- a mixed batch, a chunk over a cached
prefix, eager tokens == graph tokens) restated at the attention layer.

Every step goes through this library only: the step-input builder
(``compile_prefill`` / ``compile_chunk_prefill`` / ``compile_decode``), the
fused q/k norm + rotary + FP8 store, and the three attention modes.  The
q/k/v projection of each token is seeded random data.  Checks:
- each step's attention output against the oracle, within 2e-2 / 1e-2;
- after every step, the whole FP8 pool byte-identical to the oracle's;
- a decode step captured in a HIP graph with the runner's padding (garbage
  slot, zero length, -1 tables) replays bitwise equal to the eager step.
"""

import numpy as np
import pytest
import torch

from microserve_amd import Attention, reset_context, set_context
from microserve_amd import step_inputs as SI
from oracle import fp8_oracle as O
from oracle import norm_rope_oracle as NR
from tests.gpu_helpers import alloc_cache, assert_attention_close
from tests.seqs import Seq

DEV = "cuda"
HQ, HK, D, BS, NB = 16, 8, 128, 256, 12  # Qwen3-0.6B attention shape
EPS, MAXPOS = 1e-6, 4096
DT = torch.bfloat16
SCALE = D ** -0.5


class Layer:
    """The layer, its cache, and the oracle's copy of everything stored."""

    def __init__(self):
        gen = torch.Generator().manual_seed(0)
        self.qw = (1 + 0.2 * torch.randn(D, generator=gen)).to(DT)
        self.kw = (1 + 0.2 * torch.randn(D, generator=gen)).to(DT)
        self.cos, self.sin = NR.rope_tables(MAXPOS, 1e6, DT)
        self.cache = alloc_cache(NB + 1, kv_heads=HK)  # block NB is the garbage block
        self.attn = Attention(HQ, D, SCALE, HK)
        (self.attn.k_cache, self.attn.v_cache, self.attn.k_scale_cache,
         self.attn.v_scale_cache) = self.cache
        self.ocache = [np.zeros((NB + 1, BS, HK, D), np.uint8),
                       np.zeros((NB + 1, BS, HK, D), np.uint8),
                       np.ones((NB + 1, BS, HK), np.float32),
                       np.ones((NB + 1, BS, HK), np.float32)]
        self.qkv = {}  # seq id -> [max_len, (HQ + 2 HK) D] projection rows

    def rows(self, sid, positions):
        if sid not in self.qkv:
            g = torch.Generator().manual_seed(100 + sid)
            self.qkv[sid] = torch.randn(1024, (HQ + 2 * HK) * D, generator=g).to(DT)
        return self.qkv[sid][positions]

    def run(self, ctx, positions, qkv):
        n = qkv.shape[0]
        q, k, v = (t.view(n, -1, D) for t in qkv.to(DEV).split([HQ * D, HK * D, HK * D], -1))
        set_context(ctx)
        try:
            return self.attn.forward_fused(positions, q, k, v, self.qw.to(DEV), self.kw.to(DEV),
                                           EPS, self.cos.to(DEV), self.sin.to(DEV))
        finally:
            reset_context()

    def oracle_store(self, qkv, positions, slots):
        n = qkv.shape[0]
        q, k, v = (t.view(n, -1, D) for t in qkv.split([HQ * D, HK * D, HK * D], -1))
        rq, rk = NR.qk_norm_rope(q, k, positions, self.qw, self.kw, EPS, self.cos, self.sin)
        O.store_fp8_kvcache(rk.float().numpy(), v.float().numpy(), *self.ocache, slots.numpy())
        return rq, rk, v

    def check_cache(self):
        torch.cuda.synchronize()
        for got, ref in zip(self.cache, self.ocache):
            got = got.view(torch.uint8) if got.dtype == torch.float8_e4m3fn else got
            assert np.array_equal(got.cpu().numpy(), ref), "cache differs from the oracle's"


def _batch_rows(layer, seqs, sids):
    rows, pos = [], []
    for s, sid in zip(seqs, sids):
        p = torch.arange(s.num_computed_tokens, s.num_computed_tokens + s.num_scheduled_tokens)
        rows.append(layer.rows(sid, p))
        pos.append(p)
    return torch.cat(rows), torch.cat(pos)


@pytest.mark.gpu
def test_mixed_steps_match_oracle_and_graph_replay_equals_eager():
    L = Layer()
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(1)).tolist()
    prompts = {0: 300, 1: 45, 2: 520}
    tables = {0: perm[0:2], 1: perm[2:3], 2: perm[3:6]}
    toks = {sid: list(range(1000 * sid, 1000 * sid + n + 8)) for sid, n in prompts.items()}

    # step 1: fresh prompts A, B and the first 256-token chunk of C (PREFILL)
    seqs = [Seq(toks[0], 0, 300, tables[0], 300), Seq(toks[1], 0, 45, tables[1], 45),
            Seq(toks[2], 0, 256, tables[2], 520)]
    print("step 1: prefill", flush=True)
    ctx, cu, _, positions = SI.compile_prefill(seqs, BS, DEV)
    qkv, pos = _batch_rows(L, seqs, [0, 1, 2])
    assert torch.equal(positions.cpu(), pos)
    out = L.run(ctx, positions, qkv)
    rq, rk, v = L.oracle_store(qkv, pos, ctx.slot_mapping.cpu())
    ref = O.dense_varlen_attention(rq, rk, v, cu.cpu(), cu.cpu(), SCALE)
    assert_attention_close(out, ref)
    L.check_cache()

    # step 2: the rest of C over its cached 256-token prefix (CHUNK_PREFILL)
    print("step 2: chunk prefill", flush=True)
    seq_c = Seq(toks[2], 256, 264, tables[2], 520)
    ctx, _, positions = SI.compile_chunk_prefill(seq_c, BS, DEV)
    qkv, pos = _batch_rows(L, [seq_c], [2])
    out = L.run(ctx, positions, qkv)
    rq, _, _ = L.oracle_store(qkv, pos, ctx.slot_mapping.cpu())
    ref = O.chunk_prefill_attention(rq, *L.ocache, torch.tensor(tables[2]), 256, SCALE)
    assert_attention_close(out, ref)
    L.check_cache()

    # steps 3-6: eager decode of all three
    done = {0: 300, 1: 45, 2: 520}
    for it in range(4):
        print(f"decode step {it}", flush=True)
        seqs = [Seq(toks[sid], done[sid], 1, tables[sid], done[sid] + 1) for sid in (0, 1, 2)]
        ctx, _, positions = SI.compile_decode(seqs, BS, DEV)
        qkv, pos = _batch_rows(L, seqs, [0, 1, 2])
        out = L.run(ctx, positions, qkv)
        rq, _, _ = L.oracle_store(qkv, pos, ctx.slot_mapping.cpu())
        ref = O.decode_attention(rq, *L.ocache, ctx.cache_seqlens.cpu(),
                                 ctx.block_tables.cpu(), SCALE)
        assert_attention_close(out, ref)
        L.check_cache()
        for sid in done:
            done[sid] += 1

    # one more decode step: eager, then as a captured graph padded to 4 rows
    print("graph decode", flush=True)
    seqs = [Seq(toks[sid], done[sid], 1, tables[sid], done[sid] + 1) for sid in (0, 1, 2)]
    qkv, pos = _batch_rows(L, seqs, [0, 1, 2])
    ctx, _, positions = SI.compile_decode(seqs, BS, DEV)
    eager = L.run(ctx, positions, qkv).clone()
    width = 4
    gv = {"input_ids": torch.zeros(8, dtype=torch.int64, device=DEV),
          "positions": torch.zeros(8, dtype=torch.int64, device=DEV),
          "slot_mapping": torch.zeros(8, dtype=torch.int64, device=DEV),
          "cache_seqlens": torch.zeros(8, dtype=torch.int32, device=DEV),
          "block_tables": torch.full((8, width), -1, dtype=torch.int32, device=DEV)}
    gctx, _, gpos = SI.compile_decode(seqs, BS, DEV, pad_to=4, table_width=width,
                                      garbage_slot=NB * BS, out=gv)
    static_qkv = torch.zeros(4, qkv.shape[1], dtype=DT, device=DEV)
    static_qkv[:3] = qkv.to(DEV)
    sq, sk, sv = (t.view(4, -1, D) for t in static_qkv.split([HQ * D, HK * D, HK * D], -1))
    args = (gpos, sq, sk, sv, L.qw.to(DEV), L.kw.to(DEV), EPS, L.cos.to(DEV), L.sin.to(DEV))
    set_context(gctx)
    try:
        L.attn.forward_fused(*args)  # warm-up at the padded shape
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gout = L.attn.forward_fused(*args)
    finally:
        reset_context()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout[:3], eager), f"replay {rep} differs from the eager step"
        assert (gout[3] == 0).all(), "the padding row (length 0) must be zero"
        _ = (static_qkv * 2).sum().item()  # eager work between replays
    # the replays stored the same bytes again, plus the padding row into the
    # garbage block, which the oracle's pool leaves as it was
    L.oracle_store(qkv, pos, gctx.slot_mapping[:3].cpu())
    torch.cuda.synchronize()
    for got, ref in zip(L.cache, L.ocache):
        got = got.view(torch.uint8) if got.dtype == torch.float8_e4m3fn else got
        assert np.array_equal(got[:NB].cpu().numpy(), ref[:NB])
