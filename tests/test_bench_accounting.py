"""bench.py's algorithmic-byte accounting against the per-unit figures the
BASELINE configs are measured on (HBM bytes a unit of work must move at
least once; the roofline fractions divide by these).  CPU only: the
synthetic model is built by the library's C code, no device is touched."""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_operator_bytes():
    # config 1: 8,765,440 payload + 273,920 scales + x 2,560 + y 13,696
    assert bench.algo_bytes_gemv_q8() == 9_055_616
    # config 3: router 163,840 + shared 3,655,680 + 6 experts 10,967,040 + I/O 5,120
    assert bench.algo_bytes_moe_q4() == 14_791_680
    # config 4: weights 6,758,400 + 5,120 per context slot + I/O
    assert bench.algo_bytes_attention_q8(1024) == 12_011_520
    assert bench.algo_bytes_attention_q8(4096) == 27_740_160


def test_decode_bytes_per_token_q4(q4_model):
    """Config 5, Q4 profile: 345,697,280 weight bytes per token (all
    non-expert tensors and 6 of 64 experts per MoE layer) plus one embedding
    row
    plus 61,440 B of K/V per context slot over the mean attention length of
    the 512 greedy steps after a 932-row prompt."""
    t = bench.tensor_table(q4_model)
    size = t["payload_size"] + t["scale_size"]
    experts = float(size[t["family"] == 8].sum()) * 6 / 64
    dense = float(size[(t["family"] != 8) & (t["family"] != 1)].sum())
    embed_row = float(size[t["family"] == 1].sum()) / 129280
    assert experts == 120_637_440  # routed: 11 layers x 6 experts x 1,827,840
    assert dense + experts == 345_697_280
    assert embed_row == 680  # one Q4 row of 1280 + its 20 scales
    total = bench.decode_bytes_per_token(q4_model, 932, 512)
    assert abs(total - 409_908_531) < 2048
    # roofline tok/s at 8 TB/s
    assert abs(8e12 / total - 19_516.5) < 1.0
