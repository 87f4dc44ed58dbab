"""CPU oracle for the paged-KV GQA decode path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithm of the reference `bpt` package
(pawaryd/kvq-decode) for the decode hot path, plus the KIVI quantizer spec that the
reference plans but never wrote. It is the checker the HIP path is compared against.

Rules this package lives under:
  * Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
    may import it, and only to check or to time the CPU baseline. The product package
    `kvq_decode_amd` never imports it and has no CPU fallback.
  * Every function cites the reference file:line it follows (paths relative to the
    reference repository root).

Pinning status (what checks each function beyond re-typing its formula):
  attention.paged_decode_attention_ref  pinned: SDPA on contiguous K/V (torch library
      routine), float64 brute force, closed forms (len 1, q = 0, dominant key),
      permutation/garbage invariance.
  attention.build_paged_cache            pinned: gather-back round trip, garbage fill.
  attention.split_decode_ref / merge_ref pinned: merge(split(x)) == single pass for every
      split count, empty-split convention, LSE closed form on tiny inputs.
  attention.choose_num_splits            pinned: auto split counts the reference recorded
      in its own results files (A100 108 SMs, T4 40 SMs).
  roofline.*                             pinned: 128 KiB/token Llama-3-8B fp16, INT4 3.76x,
      kv_MB fields of the reference results files.
  kivi.*                                 pinned by the spec's mathematics (the reference
      has no quantizer code to compare with: quantized KV is "not started" upstream):
      hand-computed vectors, invariants (code range, extremes, error <= s/2, pack/unpack
      identity) and, for FP8, the library routine torch.float8_e4m3fn.
"""

from oracle.attention import (  # noqa: F401
    build_paged_cache,
    choose_num_splits,
    merge_ref,
    normalize_splits,
    paged_decode_attention_ref,
    split_decode_ref,
)
