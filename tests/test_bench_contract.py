"""CPU checks of bench.py's contract: it refuses more than one GPU, and the
algorithmic byte and FLOP counts behind its roofline figures match closed
forms counted independently here."""

import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_decode_bytes_of_the_headline_step():
    """Qwen3-8B, batch 64 x 4096: per token and kv head 128 K + 128 V bytes
    and two fp32 scales; bf16 q and out; int32 table entries and lengths."""
    per_token = 8 * (128 + 128 + 4 + 4)
    kv = 64 * 4096 * per_token
    q_and_out = 2 * 64 * 32 * 128 * 2
    tables = 4 * (64 * (4096 // 256)) + 4 * 64
    assert kv + q_and_out + tables == 554_701_056
    assert bench.decode_bytes(64, 4096, 32, 8, 128) == 554_701_056


def test_store_bytes_of_the_fill():
    """bf16 K and V read, FP8 K and V written, two fp32 scales per token and
    kv head, one int64 slot per token."""
    per_token = 2 * 8 * 128 * 2 + 2 * 8 * 128 + 2 * 8 * 4 + 8
    assert bench.store_bytes(262_144, 8, 128) == 262_144 * per_token == 1_629_487_104


def test_prefill_flops_count_every_visible_key():
    """Brute force over the queries of the 8 x (8192 cached + 2048 new) step:
    query i sees 8192 + i + 1 keys, and each visible (query, key) pair costs
    2 * head_dim FLOP for QK^T and as many for PV, per q head."""
    visits = sum(8192 + i + 1 for i in range(2048))
    brute = 8 * 32 * visits * 4 * 128
    assert brute == 2_474_035_380_224
    assert bench.prefill_flops(8, 8192, 2048, 32, 128) == brute


def test_committed_profiles_feed_the_bench_line():
    """The roofline's traffic and each prefill object's MFMA fields are read
    from the committed rocprofv3 summaries; every name bench.py asks for is
    there, with a busy fraction in (0, 1]."""
    traffic, src = bench.measured_traffic()
    assert src == os.path.join("profiles", "decode_qwen3_8b_pmc.md")
    alg = bench.decode_bytes(64, 4096, 32, 8, 128)
    assert alg <= traffic < 1.1 * alg
    for name in ("prefill_fp8_bf16", "prefill_fp8_fp16", "dense_prefill_bf16",
                 "dense_prefill_fp16"):
        c = bench.mfma_counters(name)
        assert 0.0 < c["mfma_busy"] <= 1.0, name
        assert c["valu_per_mfma"] > 1.0, name
        res = bench._with_mfma({"frac": 0.25}, name)
        assert res["frac_at_full_mfma"] >= 0.25
