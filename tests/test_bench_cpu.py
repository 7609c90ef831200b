"""bench.py reads the committed profile summaries for its roofline line: the counter-derived
HBM traffic of the routed one-token gate/up launch and the kernel trace's average duration
of that launch.  Both must resolve (a key mismatch silently reported `traffic: null`)."""

import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [REPO, os.path.join(REPO, "pytorch-engine_amd")]

import bench  # noqa: E402

# 8 active experts x (gate + up) GGUF bytes of the qwen3_30b_a3b layer (Q4_K, 768 x 2048)
ALGO_BYTES = 8 * 2 * 884_736


def test_traffic_record_resolves():
    traffic, rec = bench.load_traffic("dec_gu_kernel")
    assert traffic is not None and rec is not None
    assert rec["source"].startswith("profiles/traffic_dec_gu_qwen3_m1.json")
    # counters see the weights once plus the router's fp32 rows and small writes
    assert ALGO_BYTES <= traffic <= 1.25 * ALGO_BYTES
    assert traffic == round(rec["fetch_bytes"] + rec["write_bytes"])


def test_trace_average_resolves():
    us = bench.load_trace_avg("dec_gu_kernel<12, 1, 1, 2, false>")
    assert us is not None and 1.0 < us < 100.0
