"""Pins the byte model every bandwidth figure divides by (kvq_decode_amd/roofline.py), and
the oracle's split heuristic, against what the reference itself recorded or the storage
itself fixes. CPU only.

  * the reference's results files: every row's kv_MB (bench/bench_triton_fp16.py:58 with
    the byte count of roofline.py) and every auto split count, extracted into
    tests/golden/reference_known_answers.json by tests/golden/make_known_answers.py;
  * the reference's notes (docs/NOTES.md:14-15): Llama-3-8B fp16 reads 128 KiB per token
    over its 32 layers, and INT4 reads 3.76x fewer bytes;
  * the quantized cache's own storage: bytes of the code and (scale, zero) tensors that
    allocate_quantized_cache creates, divided by the token-heads they hold.
"""
import json
import math
import os

import pytest
import torch

from kvq_decode_amd import roofline
from oracle.attention import choose_num_splits, normalize_splits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_known_answers.json")


def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def test_step_bytes_match_reference_kv_mb():
    """Every recorded (batch, ctx) row: the fp16 step bytes equal the reference's kv_MB."""
    g = golden()
    rows = g["kv_bytes"]
    assert len(rows) == 16
    for r in rows:
        got = roofline.step_bytes([r["ctx"]] * r["batch"], g["kv_heads"], g["head_dim"], "fp16")
        assert got == round(r["kv_MB"] * 1e6), r


def test_llama3_8b_bytes_per_token_and_int4_ratio():
    m = roofline.MODELS["llama3-8b"]
    assert roofline.kv_bytes_per_token(m, "fp16") == 128 * 1024
    ratio = roofline.kv_bytes_per_token(m, "fp16") / roofline.kv_bytes_per_token(m, "int4")
    assert f"{ratio:.2f}" == "3.76"


@pytest.mark.parametrize("fmt,want", [("fp16", 512), ("int8", 264), ("fp8_e4m3", 264),
                                      ("int4", 136), ("fp8", 256)])
def test_bytes_per_token_head(fmt, want):
    assert roofline.bytes_per_token_head(128, fmt) == want


@pytest.mark.parametrize("fmt", ["int8", "fp8_e4m3", "int4"])
@pytest.mark.parametrize("group", [16, 128, 256])
def test_quantized_bytes_equal_cache_storage(fmt, group):
    """The model's bytes per token-head equal what the cache stores per token-head: code
    bytes of both caches plus the V pairs of the V-group-leading blocks (one 32-token V
    group per 32/block_size blocks) plus the K pairs of the K-group-leading blocks (one
    group per group/block_size blocks), from the real tensors."""
    from kvq_decode_amd.quant import allocate_quantized_cache
    nb, bs, hkv, d = 64, 16, 2, 128
    qc = allocate_quantized_cache(nb, bs, hkv, d, fmt, "cpu", k_group=group)
    codes = (qc.k_codes.numel() + qc.v_codes.numel()) * qc.k_codes.element_size()
    v_pairs = qc.v_sz.numel() * qc.v_sz.element_size() * bs / max(bs, 32)  # leading blocks
    k_pairs = qc.k_sz.numel() * qc.k_sz.element_size() * bs / group  # leading blocks only
    token_heads = nb * bs * hkv
    assert (codes + v_pairs + k_pairs) / token_heads == roofline.bytes_per_token_head(d, fmt, group)


def test_fp16_bytes_equal_cache_storage():
    k = torch.empty(8, 16, 4, 64, dtype=torch.float16)
    per = 2 * k.numel() * k.element_size() / (8 * 16 * 4)
    assert per == roofline.bytes_per_token_head(64, "fp16")


def test_min_time_us():
    """C2's 1 GiB at 8 TB/s: 134.2 µs."""
    assert roofline.min_time_us(1 << 30) == pytest.approx(134.217728)


def test_oracle_choose_num_splits_known_answers():
    """The oracle's split heuristic (reference triton_fp16.py:175-180) reproduces the 16 auto
    split counts the reference recorded on A100 (108 SMs) and T4 (40 SMs)."""
    rows = golden()["auto_splits"]
    assert len(rows) == 16
    for r in rows:
        got = choose_num_splits(r["batch"], 8, r["block_size"], r["ctx"] // r["block_size"],
                                r["sms"])
        assert got == r["auto_splits"], r


@pytest.mark.parametrize("pages", [1, 2, 3, 7, 64, 100, 2047, 2048])
def test_oracle_normalize_splits_invariants(pages):
    """For every requested count: S splits of pps pages cover all pages, the last split of
    the longest sequence is not empty, and pps is the smallest page count that fits the
    clamped request (reference triton_fp16.py:211-217)."""
    for n in range(0, pages + 3):
        S, pps = normalize_splits(n, pages)
        want = max(1, min(n, pages))
        assert 1 <= S <= want
        assert S * pps >= pages and (S - 1) * pps < pages
        assert pps == (pages if want == 1 else math.ceil(pages / want))


def test_oracle_normalize_splits_matches_library():
    import ctypes

    from kvq_decode_amd import _lib
    L = _lib.lib()
    s, pps = ctypes.c_int32(), ctypes.c_int32()
    for pages in (1, 5, 33, 2048):
        for n in (0, 1, 2, 3, 7, 8, 31, 32, 64, 3000):
            assert L.kvq_normalize_splits(n, pages, ctypes.byref(s), ctypes.byref(pps)) == 0
            assert (s.value, pps.value) == normalize_splits(n, pages), (n, pages)
