"""Quantized-KV accuracy harness (kvq_decode_amd/accuracy.py) at a small size. Needs a GPU.

Needle in a haystack (ctx 4096): each quantized format must keep the fp16 cache's
retrieval decisions and outputs within bounds set from the harness's own full-size
measurements (ctx 16384, 2 seeds: INT8 agreement 1.0 / cosine >= 0.99995, FP8 >= 0.996 /
>= 0.9985, INT4 >= 0.984 / >= 0.987), with margin for the smaller sample. The fp16 row
checks the harness itself: the library's fp16 decode reproduces the float32 truth's
needle weights."""
import pytest

pytestmark = pytest.mark.gpu

BOUNDS = {  # format: (min retrieval agreement, min cosine vs fp16, max mean |dw|)
    "fp16": (1.0, 1.0, 1e-3),
    "int8": (0.98, 0.9995, 0.005),
    "fp8_e4m3": (0.97, 0.997, 0.02),
    "int4": (0.90, 0.97, 0.05),
}


def test_needle_retrieval_bounds():
    from kvq_decode_amd.accuracy import evaluate
    rows = evaluate(B=2, ctx=4096, deltas=(0.0, 4.0), seeds=(0,))
    assert len(rows) == 2 * len(BOUNDS)
    for r in rows:
        agree, cos, dw = BOUNDS[r["format"]]
        print(r, flush=True)
        assert r["retrieval_agreement"] >= agree, r
        assert r["cos_vs_fp16"] >= cos - 1e-6, r
        assert r["mean_abs_needle_weight_err"] <= dw, r
    # the planted margins produce both retrieving and non-retrieving heads
    fracs = {r["delta"]: r["retrieving_heads_true"] for r in rows}
    assert fracs[0.0] < fracs[4.0]
